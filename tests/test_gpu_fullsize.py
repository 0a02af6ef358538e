"""Full-size parity of the path bench.py times: fragment-layout weights through moe_forward
(router + expert path in one C-ABI call), at the BASELINE.json prefill shapes c4 (T=4096,
Zipf routing) and c5 (T=2048, H=4096, E=128, I=1536), and the c5 shape at decode.

The oracle checks an expert-stratified token set: a token of the first and of the last
slot of every touched expert (so every expert's weights, and the last live row of every
partial tile, are checked), plus every token of the hottest expert's last tile. A crafted
routing at the c4 shape makes the per-expert slot counts cover every residue mod 64, so
partial tiles with 1, 2, 3 and 4 live 16-row fragments all occur. The fragment layout must
also equal the op layout bit for bit. Bar: max|out - ref| / max|ref| <= 1e-2."""
import numpy as np
import pytest
import torch

import bench
import oracle as O
import w4a8_fp8_wmma as W

pytestmark = pytest.mark.gpu
DEV = "cuda"
REL_TOL = 1e-2
PREFILL_BLOCK_M = 64      # rows per prefill tile (one expert per tile)


def maxrel(got, ref):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.abs(got - ref).max() / max(np.abs(ref).max(), 1e-30))


def stratified_tokens(ids: np.ndarray, block_m: int = PREFILL_BLOCK_M):
    """Token set covering every touched expert's first and last slot and the whole last
    tile of the hottest expert; also returns the live-fragment counts of the partial tiles
    (slots of an expert are ordered by slot index, as the align orders them)."""
    T, k = ids.shape
    flat = ids.reshape(-1)
    toks, live_frags = set(), set()
    hottest, hot_count = -1, -1
    for e in np.unique(flat):
        slots = np.nonzero(flat == e)[0]            # ascending: align order within expert
        toks.add(int(slots[0] // k))
        toks.add(int(slots[-1] // k))
        rem = slots.size % block_m
        if rem:
            live_frags.add((rem + 15) // 16)
        if slots.size > hot_count:
            hottest, hot_count = e, slots.size
    slots = np.nonzero(flat == hottest)[0]
    last_tile = slots[(slots.size - 1) // block_m * block_m:]
    toks.update(int(s // k) for s in last_tile)
    return np.array(sorted(toks)), live_frags


def crafted_ids(T: int, E: int, k: int, seed: int) -> np.ndarray:
    """topk ids (T, k) without repeats in a token, whose per-expert slot counts take every
    residue 1..64 mod 64 (and some exact multiples): labels sorted by expert are dealt out
    with stride T, so a token's k labels are T apart and belong to k different experts."""
    r = np.random.default_rng(seed)
    n = T * k
    counts = np.array([64 * (1 + e % 3) + (e % 65) for e in range(E)], np.int64)
    counts = np.maximum(1, (counts * n) // counts.sum())
    counts[np.argmax(counts)] += n - counts.sum()
    assert counts.max() <= T and counts.sum() == n
    labels = np.repeat(r.permutation(E), counts)     # each expert's labels contiguous
    ids = labels.reshape(k, T).T.copy()
    assert all(np.unique(row).size == k for row in ids)
    return ids.astype(np.int32)


def host(ws):
    return {kk: (None if v is None else v.cpu().numpy()) for kk, v in ws.items()}


def check_tokens(cfg, h, x, tw, ids, out, toks):
    ref = O.moe_layer(x.float().cpu().numpy()[toks], h["w13"], h["s13"], h["z13"], h["w2"],
                      h["s2"], h["z2"], tw.cpu().numpy()[toks], ids.cpu().numpy()[toks],
                      cfg["g"], round_y_fp16=cfg["T"] > 96)
    got = out.float().cpu().numpy()[toks]
    rel = maxrel(got, ref)
    print(f"  {len(toks)} tokens checked, max_rel_err={rel:.3e}", flush=True)
    assert rel <= REL_TOL
    assert torch.isfinite(out.float()).all()


@pytest.mark.parametrize("name", ["c4", "c5"])
def test_benched_path_full_size_stratified(name):
    """moe_forward on fragment-layout weights, exactly as bench.py runs it."""
    cfg = dict(bench.CONFIGS[name])
    cfgno = int(name[1:])
    print(f"\n[{name}] T={cfg['T']} H={cfg['H']} E={cfg['E']} I={cfg['I']}", flush=True)
    ws = bench.make_weights(cfg, 1000 + cfgno * 17, DEV)
    x, logits = bench.make_inputs(cfg, 1000 + cfgno, DEV)
    f13, f2 = W.repack_fragments(ws["w13"], ws["s13"], ws["z13"]), W.repack_fragments(ws["w2"], ws["s2"], ws["z2"])
    out, tw, ids = W.moe_forward(x, logits, cfg["k"], f13, f2, ws["s13"], ws["s2"], ws["z13"],
                                 ws["z2"])
    out_op, tw_op, ids_op = W.moe_forward(x, logits, cfg["k"], ws["w13"], ws["w2"], ws["s13"],
                                          ws["s2"], ws["z13"], ws["z2"])
    assert torch.equal(ids, ids_op) and torch.equal(tw, tw_op)
    assert torch.equal(out, out_op), "fragment layout must equal the op layout bit for bit"
    toks, live = stratified_tokens(ids.cpu().numpy())
    print(f"  partial-tile live fragments present: {sorted(live)}", flush=True)
    check_tokens(cfg, host(ws), x, tw, ids, out, toks)


def test_crafted_counts_cover_every_partial_tile_c4_shape():
    """Every residue of the per-expert slot count mod 64 (live fragments 1..4, and the last
    live row at every position of a partial tile) at the c4 shape, fragment layout."""
    cfg = dict(bench.CONFIGS["c4"])
    ws = bench.make_weights(cfg, 4242, DEV)
    x, _ = bench.make_inputs(cfg, 4243, DEV)
    ids_np = crafted_ids(cfg["T"], cfg["E"], cfg["k"], 4244)
    r = np.random.default_rng(4245)
    tw_np = r.random(ids_np.shape).astype(np.float32)
    tw_np /= tw_np.sum(1, keepdims=True)
    ids = torch.from_numpy(ids_np).to(DEV)
    tw = torch.from_numpy(tw_np).to(DEV)
    f13, f2 = W.repack_fragments(ws["w13"], ws["s13"], ws["z13"]), W.repack_fragments(ws["w2"], ws["s2"], ws["z2"])
    out = W.moe_apply(x, f13, f2, ws["s13"], ws["s2"], ws["z13"], ws["z2"], tw, ids)
    out_op = W.moe_apply(x, ws["w13"], ws["w2"], ws["s13"], ws["s2"], ws["z13"], ws["z2"], tw, ids)
    assert torch.equal(out, out_op)
    toks, live = stratified_tokens(ids_np)
    rems = {int((ids_np == e).sum()) % 64 for e in range(cfg["E"])}
    assert live == {1, 2, 3, 4} and len(rems) == 64, (live, len(rems))
    check_tokens(cfg, host(ws), x, tw, ids, out, toks)


@pytest.mark.parametrize("T", [1, 32])
def test_c5_shape_decode_fragments(T):
    """H=4096 (K/128 = 32) and I=1536 (K/128 = 12) through the decode GEMV on fragments."""
    cfg = dict(bench.CONFIGS["c5"])
    cfg["T"] = T
    ws = bench.make_weights(cfg, 5150 + T, DEV)
    x, logits = bench.make_inputs(cfg, 5151 + T, DEV)
    f13, f2 = W.repack_fragments(ws["w13"], ws["s13"], ws["z13"]), W.repack_fragments(ws["w2"], ws["s2"], ws["z2"])
    out, tw, ids = W.moe_forward(x, logits, cfg["k"], f13, f2, ws["s13"], ws["s2"], ws["z13"],
                                 ws["z2"])
    out_op, _, _ = W.moe_forward(x, logits, cfg["k"], ws["w13"], ws["w2"], ws["s13"], ws["s2"],
                                 ws["z13"], ws["z2"])
    assert torch.equal(out, out_op)
    check_tokens(cfg, host(ws), x, tw, ids, out, np.arange(T))
