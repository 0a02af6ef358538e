"""GPU parity of the whole expert path (w4a8_moe_apply / _run_grouped_moe) against the
CPU oracle, at small shapes and at the BASELINE.json shapes (sampled tokens), plus
size-independent properties at full size. Bar: max|out - ref| / max|ref| <= 1e-2."""
import numpy as np
import pytest
import torch

import bench
import oracle as O
import w4a8_fp8_wmma as W
from w4a8_fp8_wmma import moe_experts

pytestmark = pytest.mark.gpu
DEV = "cuda"
REL_TOL = 1e-2


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    assert torch.cuda.is_available(), "GPU tests need a visible MI355X"


def maxrel(got, ref):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.abs(got - ref).max() / max(np.abs(ref).max(), 1e-30))


def small_layer(seed, T, E, H, I, k, g=128, asym=True, dtype=torch.bfloat16):
    cfg = dict(T=T, H=H, E=E, k=k, I=I, g=g, routing="uniform")
    ws = bench.make_weights(cfg, seed, DEV)
    if not asym:
        ws["z13"] = None
        ws["z2"] = None
    x, logits = bench.make_inputs(cfg, seed + 1, DEV)
    tw, ids = W.fused_topk(None, logits, k, True)
    return cfg, ws, x.to(dtype), tw, ids


def oracle_layer(cfg, ws, x, tw, ids, tokens=None, round_y=False):
    sel = slice(None) if tokens is None else tokens
    h = {kk: (None if v is None else v.cpu().numpy()) for kk, v in ws.items()}
    return O.moe_layer(x.float().cpu().numpy()[sel], h["w13"], h["s13"], h["z13"], h["w2"],
                       h["s2"], h["z2"], tw.cpu().numpy()[sel], ids.cpu().numpy()[sel],
                       cfg["g"], round_y_fp16=round_y)


@pytest.mark.parametrize("T", [1, 7, 32, 96, 97, 300])
@pytest.mark.parametrize("asym", [True, False])
def test_moe_apply_small(T, asym):
    cfg, ws, x, tw, ids = small_layer(100 + T, T, 16, 512, 256, 4, asym=asym)
    out = W.moe_apply(x, ws["w13"], ws["w2"], ws["s13"], ws["s2"], ws["z13"], ws["z2"], tw, ids)
    ref = oracle_layer(cfg, ws, x, tw, ids)
    assert out.dtype == torch.bfloat16 and out.shape == x.shape
    assert maxrel(out.float().cpu().numpy(), ref) <= REL_TOL


@pytest.mark.parametrize("kernel", ["scalar", "wmma", "gemv"])
@pytest.mark.parametrize("T", [4, 160])
def test_run_grouped_moe_kernels(kernel, T):
    cfg, ws, x, tw, ids = small_layer(200 + T, T, 8, 256, 128, 2)
    out = moe_experts._run_grouped_moe(x, ws["w13"], ws["w2"], ws["s13"], ws["s2"], ws["z13"],
                                       ws["z2"], tw, ids, "silu", 8, None, False, kernel)
    ref = oracle_layer(cfg, ws, x, tw, ids, round_y=(kernel == "scalar"))
    assert out.dtype == x.dtype
    assert maxrel(out.float().cpu().numpy(), ref) <= REL_TOL


def test_fp16_input_and_router_weight_on_input():
    cfg, ws, x, tw, ids = small_layer(300, 12, 8, 256, 128, 1, dtype=torch.float16)
    out = moe_experts._run_grouped_moe(x, ws["w13"], ws["w2"], ws["s13"], ws["s2"], ws["z13"],
                                       ws["z2"], tw, ids, "silu", 8, None, True, "wmma")
    xin = (x * tw.to(x.dtype)).float()
    ref = oracle_layer(cfg, ws, xin, torch.ones_like(tw), ids)
    assert out.dtype == torch.float16
    assert maxrel(out.float().cpu().numpy(), ref) <= REL_TOL


def test_expert_map_drops_non_local_experts():
    cfg, ws, x, tw, ids = small_layer(400, 16, 8, 256, 128, 2)
    emap = torch.tensor([0, 1, 2, 3, -1, -1, -1, -1], dtype=torch.int32, device=DEV)
    out = W.moe_apply(x, ws["w13"], ws["w2"], ws["s13"], ws["s2"], ws["z13"], ws["z2"], tw, ids,
                      expert_map=emap)
    # reference: local experts keep their weights; non-local slots get weight 0
    twm = tw.clone()
    twm[ids >= 4] = 0
    ref = oracle_layer(cfg, ws, x, twm, ids.clamp(max=3))
    assert maxrel(out.float().cpu().numpy(), ref) <= REL_TOL


@pytest.mark.parametrize("T,frag", [(16, False), (16, True), (200, False), (200, True)])
def test_expert_map_global_ids_beyond_local_count(T, frag):
    """EP layout: 4 local experts, 8 global ids, experts 4..7 local (as 0..3). Ids >= the
    local count must be mapped, not dropped (decode and prefill schedules, both layouts)."""
    cfg = dict(T=T, H=256, E=4, k=3, I=128, g=128, routing="uniform")
    ws = bench.make_weights(cfg, 410 + T, DEV)
    g_cfg = dict(cfg, E=8)
    x, logits = bench.make_inputs(g_cfg, 411 + T, DEV)
    emap_np = np.array([-1, -1, -1, -1, 0, 1, 2, 3], np.int32)
    emap = torch.from_numpy(emap_np).to(DEV)
    w13, w2 = ws["w13"], ws["w2"]
    if frag:
        w13, w2 = W.repack_fragments(w13, ws["s13"], ws["z13"]), W.repack_fragments(w2, ws["s2"], ws["z2"])
    out, tw, ids = W.moe_forward(x, logits, 3, w13, w2, ws["s13"], ws["s2"], ws["z13"], ws["z2"],
                                 expert_map=emap)
    assert int(ids.max()) >= 4 and int(ids.min()) < 4
    h = {kk: v.cpu().numpy() for kk, v in ws.items()}
    ref = O.moe_layer(x.float().cpu().numpy(), h["w13"], h["s13"], h["z13"], h["w2"], h["s2"],
                      h["z2"], tw.cpu().numpy(), ids.cpu().numpy(), 128, round_y_fp16=T > 96,
                      expert_map=emap_np)
    assert maxrel(out.float().cpu().numpy(), ref) <= REL_TOL
    # _run_grouped_moe with global_num_experts = 8 takes the same path
    out2 = moe_experts._run_grouped_moe(x, w13, w2, ws["s13"], ws["s2"], ws["z13"], ws["z2"], tw,
                                        ids, "silu", 8, emap, False, "wmma")
    assert torch.equal(out2, out)


def _oracle_after_gemm1(g1, ids, tw, w2, s2, g, round_y):
    """The oracle layer from gemm1's fp16 output on (slot, 2*inter) rows: SiLU-mul, act-quant,
    gemm2 over the E2M1 codebook, y, and the top-k weighted sum (the second half of
    oracle.moe_layer)."""
    T, k = ids.shape
    inter = g1.shape[1] // 2
    h = O.silu_and_mul(g1[:, :inter], g1[:, inter:])
    a2, sc2 = O.act_quant(h)
    y = (O.grouped_run(a2, ids.reshape(-1), w2, s2, None, g, True) * sc2[:, None]).astype(np.float32)
    if round_y:
        y = y.astype(np.float16).astype(np.float32)
    y = y.reshape(T, k, -1)
    acc = np.zeros((T, y.shape[2]), np.float32)
    for j in range(k):
        acc = O.fma32(tw[:, j:j + 1].astype(np.float32), y[:, j], acc)
    return acc


@pytest.mark.parametrize("g,T", [(128, 8), (128, 160), (32, 8), (32, 160), (64, 40), (64, 200)])
def test_e2m1_layer(g, T):
    """mxfp4 (OCP E2M1 codebook, symmetric) weights through the whole layer
    (moe_experts.py:1351-1450, tile_config.h:47-71): fp4-operand matrix-core tiles at the
    mxfp4 block size 32, at 64 and at 128, decode and prefill schedules.

    The fp4 MFMA forms a group's 32..128-term sum of e4m3 x e2m1 products inside the matrix
    core; where the exact sum needs more than fp32's 24 bits it may round differently from
    the scalar fmaf chain, so gemm1 can differ from the oracle by one fp16 ulp (bounded at
    2e-3 below). When that element is its row's absmax, act-quant rescales the whole h row
    and every e4m3 byte of it re-rounds (3-bit mantissa), which moves that token's output by
    up to ~2e-2 of the layer's range (measured 1.7e-2 on one token of 160). So the layer is
    pinned in two steps: gemm1 through the same tiles against the oracle's gemm1, then the
    layer against the oracle's second half run from the kernel's own gemm1 bits, at the
    usual 1e-2; the end-to-end oracle is held to 3e-2."""
    cfg = dict(T=T, H=256, E=8, k=2, I=128, g=g, routing="uniform")
    ws = bench.make_weights(cfg, 420 + g + T, DEV)
    x, logits = bench.make_inputs(cfg, 421 + g + T, DEV)
    tw, ids = W.fused_topk(None, logits, 2, True)
    out = moe_experts._run_grouped_moe(x, ws["w13"], ws["w2"], ws["s13"], ws["s2"], None, None,
                                       tw, ids, "silu", 8, None, False, "wmma",
                                       weight_is_e2m1=True).float().cpu().numpy()
    h = {kk: v.cpu().numpy() for kk, v in ws.items()}
    ids_np, tw_np = ids.cpu().numpy(), tw.cpu().numpy()
    round_y = T > 96   # prefill rows leave gemm2 as fp16; decode slots stay fp32
    ref, st = O.moe_layer(x.float().cpu().numpy(), h["w13"], h["s13"], None, h["w2"], h["s2"],
                          None, tw_np, ids_np, g, round_y_fp16=round_y, e2m1=True,
                          return_stages=True)
    # gemm1 on the same fp4 tiles, op by op, rows back in slot order
    bm = 16
    sti, eid, ntp = O.moe_align(ids_np.astype(np.int32), bm, 8)
    n = int(ntp[0])
    g1 = W.mmq_fp8_moe_gemm(x.half(), ws["w13"], ws["s13"], *[torch.from_numpy(a).to(DEV) for a in (sti, eid, ntp)],
                            2, bm, kernel="wmma", weight_is_e2m1=True).cpu().numpy()
    real = np.nonzero(sti[:n] < T * 2)[0]
    g1_slots = np.empty((T * 2, g1.shape[1]), np.float16)
    g1_slots[sti[real]] = g1[real]
    assert maxrel(g1_slots, st["g1"]) <= 2e-3
    ref2 = _oracle_after_gemm1(g1_slots, ids_np, tw_np, h["w2"], h["s2"], g, round_y)
    assert maxrel(out, ref2) <= REL_TOL
    assert maxrel(out, ref) <= 3e-2


@pytest.mark.parametrize("e2m1", [False, True])
@pytest.mark.parametrize("T", [6, 130])
def test_per_expert_biases(e2m1, T):
    """gpt-oss style per-expert biases (moe_experts.py:565-575,654-655): added to gemm1's fp16
    output before the activation and to gemm2's fp16 rows before the weighted reduce."""
    cfg = dict(T=T, H=256, E=8, k=2, I=128, g=128, routing="uniform")
    ws = bench.make_weights(cfg, 430 + T, DEV)
    x, logits = bench.make_inputs(cfg, 431 + T, DEV)
    tw, ids = W.fused_topk(None, logits, 2, True)
    r = np.random.default_rng(432 + T)
    b1 = (r.standard_normal((8, 256)) * 0.1).astype(np.float16)
    b2 = (r.standard_normal((8, 256)) * 0.1).astype(np.float16)
    z13, z2 = (None, None) if e2m1 else (ws["z13"], ws["z2"])
    out = moe_experts._run_grouped_moe(
        x, ws["w13"], ws["w2"], ws["s13"], ws["s2"], z13, z2, tw, ids, "silu", 8, None, False,
        "wmma", weight_is_e2m1=e2m1, w1_bias=torch.from_numpy(b1).to(DEV),
        w2_bias=torch.from_numpy(b2).to(DEV))
    h = {kk: v.cpu().numpy() for kk, v in ws.items()}
    ref = O.moe_layer(x.float().cpu().numpy(), h["w13"], h["s13"], None if e2m1 else h["z13"],
                      h["w2"], h["s2"], None if e2m1 else h["z2"], tw.cpu().numpy(),
                      ids.cpu().numpy(), 128, e2m1=e2m1, w1_bias=b1, w2_bias=b2)
    assert maxrel(out.float().cpu().numpy(), ref) <= REL_TOL


@pytest.mark.parametrize("T,frag", [(160, False), (300, True), (1024, True)])
def test_prefill_layer_equals_op_composition(T, frag):
    """The whole-layer prefill tiles (fused gemm1+SiLU, gemm2 quantising its own rows, row
    reduce) against the op-by-op composition of the reference's ops (gemm1, silu_and_mul,
    gemm2, gather-reduce; moe_experts.py:587-665). The fused SiLU is silu_mul_h, the
    unfused kernel's own function (test_moe_experts.py:283-315 property)."""
    cfg = dict(bench.CONFIGS["c4"])
    cfg["T"] = T
    ws = bench.make_weights(cfg, 440 + T, DEV)
    x, logits = bench.make_inputs(cfg, 441 + T, DEV)
    tw, ids = W.fused_topk(None, logits, cfg["k"], True)
    w13, w2 = ws["w13"], ws["w2"]
    if frag:
        w13, w2 = W.repack_fragments(w13, ws["s13"], ws["z13"]), W.repack_fragments(w2, ws["s2"], ws["z2"])
    fused = W.moe_apply(x, w13, w2, ws["s13"], ws["s2"], ws["z13"], ws["z2"], tw, ids)
    unfused = moe_experts._run_unfused(
        x.to(torch.float16), ws["w13"], ws["w2"], ws["s13"], ws["s2"], ws["z13"], ws["z2"],
        tw.reshape(-1).contiguous(), ids, cfg["k"], cfg["E"], None, "wmma", False, None, None,
        64).to(x.dtype)
    same = (fused == unfused).float().mean().item()
    print(f"  identical elements: {same:.6f}")
    assert torch.equal(fused, unfused)


def test_decode_1024_experts_1024_slots():
    """The decode schedule at its list limits (1024 experts, 64 tokens x top-16 = 1024 slots):
    gemm2 reads the lists gemm1 hands over whole. moe_forward (router launch, prequantised
    rows) equals fused_topk + moe_apply bit for bit, and the oracle agrees."""
    cfg = dict(T=64, H=256, E=1024, k=16, I=128, g=128, routing="uniform")
    ws = bench.make_weights(cfg, 990, DEV)
    x, logits = bench.make_inputs(cfg, 991, DEV)
    f13 = W.repack_fragments(ws["w13"], ws["s13"], ws["z13"])
    f2 = W.repack_fragments(ws["w2"], ws["s2"], ws["z2"])
    tw, ids = W.fused_topk(None, logits, cfg["k"], True)
    a = W.moe_apply(x, f13, f2, ws["s13"], ws["s2"], ws["z13"], ws["z2"], tw, ids)
    b, tw2, ids2 = W.moe_forward(x, logits, cfg["k"], f13, f2, ws["s13"], ws["s2"], ws["z13"],
                                 ws["z2"])
    assert torch.equal(ids, ids2) and torch.equal(tw, tw2)
    assert torch.equal(a, b)
    ref = oracle_layer(cfg, ws, x, tw, ids)
    assert maxrel(a.float().cpu().numpy(), ref) <= REL_TOL


@pytest.mark.parametrize("T,frag,emap", [(100, True, False), (129, True, False), (160, False, False),
                                         (300, True, False), (1024, True, True), (4096, True, False)])
def test_prefill_pair_equals_two_launches(T, frag, emap):
    """gemm1+SiLU and gemm2 of each 64-row tile in one work-group (prefill_ares_pair_kernel,
    the default where both tiles apply) give the two launches' output bit for bit, with
    partial tiles (T = 100 and 129: a few tiles, 800 and 1032 slots), an expert map that
    drops experts, and at the c4 size."""
    cfg = dict(bench.CONFIGS["c4"])
    cfg["T"] = T
    ws = bench.make_weights(cfg, 470 + T, DEV)
    x, logits = bench.make_inputs(cfg, 471 + T, DEV)
    tw, ids = W.fused_topk(None, logits, cfg["k"], True)
    w13, w2 = ws["w13"], ws["w2"]
    if frag:
        w13, w2 = W.repack_fragments(w13, ws["s13"], ws["z13"]), W.repack_fragments(w2, ws["s2"], ws["z2"])
    em = None
    if emap:   # the first 200 global experts map onto local experts 0..199, the rest dropped
        em = torch.full((cfg["E"],), -1, dtype=torch.int32, device=DEV)
        em[:200] = torch.arange(200, dtype=torch.int32, device=DEV)
    prev = W.set_prefill_pair(True)
    try:
        a = W.moe_apply(x, w13, w2, ws["s13"], ws["s2"], ws["z13"], ws["z2"], tw, ids, expert_map=em)
        W.set_prefill_pair(False)
        b = W.moe_apply(x, w13, w2, ws["s13"], ws["s2"], ws["z13"], ws["z2"], tw, ids, expert_map=em)
    finally:
        W.set_prefill_pair(prev)
    assert torch.isfinite(a.float()).all()
    assert torch.equal(a, b)


@pytest.mark.parametrize("H,T,frag", [(2048, 300, True), (2048, 170, False), (4096, 260, True)])
def test_prefill_intermediate_1536(H, T, frag):
    """Intermediate size 1536 (as c5): gemm2 tiles take the rows act_quant_kernel quantised
    (above the self-quantising tiles' K <= 1024), so the layer runs gemm1 and gemm2 as two
    launches whatever the pair switch says; it equals the op-by-op composition bit for bit,
    and the oracle agrees."""
    cfg = dict(T=T, H=H, E=32, k=4, I=1536, g=128, routing="uniform")
    ws = bench.make_weights(cfg, 650 + T, DEV)
    x, logits = bench.make_inputs(cfg, 651 + T, DEV)
    tw, ids = W.fused_topk(None, logits, cfg["k"], True)
    w13, w2 = ws["w13"], ws["w2"]
    if frag:
        w13, w2 = W.repack_fragments(w13, ws["s13"], ws["z13"]), W.repack_fragments(w2, ws["s2"], ws["z2"])
    prev = W.set_prefill_pair(True)
    try:
        out = W.moe_apply(x, w13, w2, ws["s13"], ws["s2"], ws["z13"], ws["z2"], tw, ids)
        W.set_prefill_pair(False)
        two = W.moe_apply(x, w13, w2, ws["s13"], ws["s2"], ws["z13"], ws["z2"], tw, ids)
    finally:
        W.set_prefill_pair(prev)
    assert torch.equal(out, two)
    unfused = moe_experts._run_unfused(
        x.to(torch.float16), ws["w13"], ws["w2"], ws["s13"], ws["s2"], ws["z13"], ws["z2"],
        tw.reshape(-1).contiguous(), ids, cfg["k"], cfg["E"], None, "wmma", False, None, None,
        64).to(x.dtype)
    assert torch.equal(out, unfused)
    ref = oracle_layer(cfg, ws, x, tw, ids)
    err = maxrel(out.float().cpu().numpy(), ref)
    print(f"  H={H} T={T} frag={frag} max rel err {err:.2e}")
    assert err <= REL_TOL


@pytest.mark.parametrize("H,T,frag", [(4096, 200, True), (3072, 130, False)])
def test_prefill_wide_k_tiles(H, T, frag):
    """Hidden sizes above 2048 run gemm1 on the 32-row activation tiles, whose per-range
    tables are rebuilt in the middle of K (H = 3072: a partial second half of 8 groups):
    against the oracle, and equal to the op-by-op composition bit for bit."""
    cfg = dict(T=T, H=H, E=16, k=4, I=512, g=128, routing="uniform")
    ws = bench.make_weights(cfg, 600 + H, DEV)
    x, logits = bench.make_inputs(cfg, 601 + H, DEV)
    tw, ids = W.fused_topk(None, logits, cfg["k"], True)
    w13, w2 = ws["w13"], ws["w2"]
    if frag:
        w13, w2 = W.repack_fragments(w13, ws["s13"], ws["z13"]), W.repack_fragments(w2, ws["s2"], ws["z2"])
    out = W.moe_apply(x, w13, w2, ws["s13"], ws["s2"], ws["z13"], ws["z2"], tw, ids)
    ref = oracle_layer(cfg, ws, x, tw, ids)
    err = maxrel(out.float().cpu().numpy(), ref)
    print(f"  H={H} T={T} frag={frag} max rel err {err:.2e}")
    assert err <= REL_TOL
    unfused = moe_experts._run_unfused(
        x.to(torch.float16), ws["w13"], ws["w2"], ws["s13"], ws["s2"], ws["z13"], ws["z2"],
        tw.reshape(-1).contiguous(), ids, cfg["k"], cfg["E"], None, "wmma", False, None, None,
        64).to(x.dtype)
    assert torch.equal(out, unfused)


@pytest.mark.parametrize("name", ["c2", "c3", "c4", "c5"])
def test_baseline_configs_sampled_tokens(name):
    """Full-size BASELINE.json layers; the oracle checks 3 tokens (first, middle, last)."""
    cfg = dict(bench.CONFIGS[name])
    ws = bench.make_weights(cfg, 1000 + int(name[1:]) * 17, DEV)
    x, logits = bench.make_inputs(cfg, 1000 + int(name[1:]), DEV)
    tw, ids = W.fused_topk(None, logits, cfg["k"], True)
    out = W.moe_apply(x, ws["w13"], ws["w2"], ws["s13"], ws["s2"], ws["z13"], ws["z2"], tw, ids)
    T = cfg["T"]
    tok = sorted({0, T // 2, T - 1})
    ref = oracle_layer(cfg, ws, x, tw, ids, tokens=tok)
    got = out.float().cpu().numpy()[tok]
    assert maxrel(got, ref) <= REL_TOL
    assert torch.isfinite(out.float()).all()


@pytest.mark.parametrize("T,asym", [(1, True), (32, True), (32, False), (97, True), (300, False)])
def test_fragment_layout_bit_identical(T, asym):
    """Weights repacked into the fragment layout give the op-layout results bit for bit
    (decode GEMV and prefill tiles), and the repack equals the oracle permutation."""
    cfg, ws, x, tw, ids = small_layer(300 + T, T, 16, 512, 256, 4, asym=asym)
    a = W.moe_apply(x, ws["w13"], ws["w2"], ws["s13"], ws["s2"], ws["z13"], ws["z2"], tw, ids)
    f13, f2 = W.repack_fragments(ws["w13"], ws["s13"], ws["z13"]), W.repack_fragments(ws["w2"], ws["s2"], ws["z2"])
    assert np.array_equal(f13.cpu().numpy(), O.repack_fragments(*_host(ws, "13")))
    assert np.array_equal(f2.cpu().numpy(), O.repack_fragments(*_host(ws, "2")))
    b = W.moe_apply(x, f13, f2, ws["s13"], ws["s2"], ws["z13"], ws["z2"], tw, ids)
    assert torch.equal(a, b)


@pytest.mark.parametrize("name,T", [("c3", None), ("c4", 512)])
def test_fragment_layout_full_size(name, T):
    cfg = dict(bench.CONFIGS[name])
    if T is not None:
        cfg["T"] = T
    ws = bench.make_weights(cfg, 555, DEV)
    x, logits = bench.make_inputs(cfg, 556, DEV)
    tw, ids = W.fused_topk(None, logits, cfg["k"], True)
    a = W.moe_apply(x, ws["w13"], ws["w2"], ws["s13"], ws["s2"], ws["z13"], ws["z2"], tw, ids)
    b = W.moe_apply(x, W.repack_fragments(ws["w13"], ws["s13"], ws["z13"]), W.repack_fragments(ws["w2"], ws["s2"], ws["z2"]), ws["s13"],
                    ws["s2"], ws["z13"], ws["z2"], tw, ids)
    assert torch.equal(a, b)


@pytest.mark.parametrize("T,frag,E", [(1, True, 64), (32, True, 64), (32, False, 64),
                                      (96, True, 64), (300, True, 64), (4, True, 256),
                                      (5, True, 256), (3, True, 16), (2, True, 512)])
def test_moe_forward_equals_router_then_apply(T, frag, E):
    """moe_forward (router + expert path in one call) gives the fused_topk ids / weights and
    the moe_apply output bit for bit. On fragment weights with T <= 4 and E <= 256 the decode
    gemm1 launch routes the tokens itself (same selection code, every work-group); T = 5 and
    E = 512 go through the router kernel."""
    cfg = dict(T=T, H=512, E=E, k=8, I=256, g=128, routing="uniform")
    ws = bench.make_weights(cfg, 700 + T, DEV)
    x, logits = bench.make_inputs(cfg, 701 + T, DEV)
    x = x.to(torch.bfloat16)
    w13, w2 = ws["w13"], ws["w2"]
    if frag:
        w13, w2 = W.repack_fragments(w13, ws["s13"], ws["z13"]), W.repack_fragments(w2, ws["s2"], ws["z2"])
    tw, ids = W.fused_topk(None, logits, cfg["k"], True)
    a = W.moe_apply(x, w13, w2, ws["s13"], ws["s2"], ws["z13"], ws["z2"], tw, ids)
    b, tw2, ids2 = W.moe_forward(x, logits, cfg["k"], w13, w2, ws["s13"], ws["s2"], ws["z13"],
                                 ws["z2"])
    assert torch.equal(ids2, ids.to(torch.int32)) and torch.equal(tw2, tw)
    assert torch.equal(a, b)


@pytest.mark.parametrize("T,E,k,frag,emap", [(129, 256, 8, True, False), (1000, 256, 8, True, False),
                                              (513, 128, 4, False, False), (700, 64, 6, True, False),
                                              (600, 4, 4, True, True), (2048, 128, 8, True, False)])
def test_router_many_tokens_equals_router_then_apply(T, E, k, frag, emap):
    """Many tokens (T * k > 1024, the multi-chunk align): moe_forward (router launch that
    also quantises x, then the align from the ids in memory) equals fused_topk + moe_apply bit
    for bit: partial last chunks (129 * 8 = 1032 slots), top-k that does not divide a chunk
    (k = 6), both layouts, and an expert map (8 routed ids, 4 local experts)."""
    cfg = dict(T=T, H=256, E=E, k=k, I=128, g=128, routing="uniform")
    ws = bench.make_weights(cfg, 900 + T, DEV)
    emap_t = None
    if emap:
        x, logits = bench.make_inputs(dict(cfg, E=2 * E), 901 + T, DEV)
        emap_t = torch.tensor([-1] * E + list(range(E)), dtype=torch.int32, device=DEV)
    else:
        x, logits = bench.make_inputs(cfg, 901 + T, DEV)
    x = x.to(torch.bfloat16)
    w13, w2 = ws["w13"], ws["w2"]
    if frag:
        w13, w2 = W.repack_fragments(w13, ws["s13"], ws["z13"]), W.repack_fragments(w2, ws["s2"], ws["z2"])
    tw, ids = W.fused_topk(None, logits, k, True)
    a = W.moe_apply(x, w13, w2, ws["s13"], ws["s2"], ws["z13"], ws["z2"], tw, ids, expert_map=emap_t)
    b, tw2, ids2 = W.moe_forward(x, logits, k, w13, w2, ws["s13"], ws["s2"], ws["z13"], ws["z2"],
                                 expert_map=emap_t)
    assert torch.equal(ids2, ids.to(torch.int32)) and torch.equal(tw2, tw)
    assert torch.equal(a, b)
    if emap:
        assert int(ids.max()) >= E and int(ids.min()) < E


def test_decode_is_deterministic_and_token_local():
    """Decode schedule: bit-identical reruns; permuting tokens permutes outputs exactly."""
    cfg = dict(bench.CONFIGS["c3"])
    ws = bench.make_weights(cfg, 77, DEV)
    x, logits = bench.make_inputs(cfg, 78, DEV)
    tw, ids = W.fused_topk(None, logits, cfg["k"], True)
    a = W.moe_apply(x, ws["w13"], ws["w2"], ws["s13"], ws["s2"], ws["z13"], ws["z2"], tw, ids)
    b = W.moe_apply(x, ws["w13"], ws["w2"], ws["s13"], ws["s2"], ws["z13"], ws["z2"], tw, ids)
    assert torch.equal(a, b)
    perm = torch.randperm(cfg["T"], generator=torch.Generator().manual_seed(0)).to(DEV)
    c = W.moe_apply(x[perm].contiguous(), ws["w13"], ws["w2"], ws["s13"], ws["s2"], ws["z13"],
                    ws["z2"], tw[perm].contiguous(), ids[perm].contiguous())
    assert torch.equal(c, a[perm])


def test_prefill_linear_in_router_weights():
    """out(w) is linear in the top-k weights: out(2w) == 2 out(w) up to fp32 rounding."""
    cfg = dict(bench.CONFIGS["c4"])
    cfg["T"] = 512
    ws = bench.make_weights(cfg, 91, DEV)
    x, logits = bench.make_inputs(cfg, 92, DEV)
    tw, ids = W.fused_topk(None, logits, cfg["k"], True)
    a = W.moe_apply(x, ws["w13"], ws["w2"], ws["s13"], ws["s2"], ws["z13"], ws["z2"], tw, ids)
    b = W.moe_apply(x, ws["w13"], ws["w2"], ws["s13"], ws["s2"], ws["z13"], ws["z2"],
                    (2 * tw).contiguous(), ids)
    assert maxrel(b.float().cpu().numpy(), 2 * a.float().cpu().numpy()) <= 1e-2


def test_graph_replay_matches_eager():
    """The bench captures the layer in a HIP graph: every replay must equal eager."""
    cfg, ws, x, tw, ids = small_layer(500, 32, 16, 512, 256, 4)
    eager = W.moe_apply(x, ws["w13"], ws["w2"], ws["s13"], ws["s2"], ws["z13"], ws["z2"], tw, ids)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        W.moe_apply(x, ws["w13"], ws["w2"], ws["s13"], ws["s2"], ws["z13"], ws["z2"], tw, ids)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = W.moe_apply(x, ws["w13"], ws["w2"], ws["s13"], ws["s2"], ws["z13"], ws["z2"], tw,
                          ids)
    for _ in range(4):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
        W.moe_apply(x, ws["w13"], ws["w2"], ws["s13"], ws["s2"], ws["z13"], ws["z2"], tw, ids)
        torch.cuda.synchronize()


@pytest.mark.parametrize("T", [1, 4, 32, 300])
def test_graph_replay_forward_fragments_fresh_inputs(T):
    """moe_forward on fragment weights captured once and replayed with new hidden states and
    router logits copied in before each replay (how a serving loop uses the graph): every
    replay equals an eager call on the same inputs. T = 1 and 4 route inside the decode
    gemm1 launch, 32 has the router launch, 300 is the prefill schedule."""
    cfg = dict(T=T, H=512, E=64, k=8, I=256, g=128, routing="uniform")
    ws = bench.make_weights(cfg, 900 + T, DEV)
    f13, f2 = W.repack_fragments(ws["w13"], ws["s13"], ws["z13"]), W.repack_fragments(ws["w2"], ws["s2"], ws["z2"])
    x, logits = bench.make_inputs(cfg, 901 + T, DEV)
    xs, ls = x.clone(), logits.clone()

    def fwd(a, b):
        return W.moe_forward(a, b, cfg["k"], f13, f2, ws["s13"], ws["s2"], ws["z13"], ws["z2"])

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fwd(xs, ls)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out_g, tw_g, ids_g = fwd(xs, ls)
    for r in range(4):
        x_r, l_r = bench.make_inputs(cfg, 950 + 10 * T + r, DEV)
        xs.copy_(x_r)
        ls.copy_(l_r)
        g.replay()
        torch.cuda.synchronize()
        got = (out_g.clone(), tw_g.clone(), ids_g.clone())
        ref = fwd(x_r, l_r)
        torch.cuda.synchronize()
        assert torch.equal(got[2], ref[2]) and torch.equal(got[1], ref[1]), r
        assert torch.equal(got[0], ref[0]), r


@pytest.mark.parametrize("T", [1, 8, 32, 96])
@pytest.mark.parametrize("frag", [False, True])
def test_decode_six_group_intermediate(T, frag):
    """An intermediate size of 768 (K/128 = 6 for gemm2, Qwen3-30B-A3B-shaped) runs the decode
    GEMV (split table entry 6 = 3 groups per wave, two waves per team) against the oracle, on
    op-layout and fragment weights, and the two layouts agree bit for bit."""
    cfg, ws, x, tw, ids = small_layer(800 + T, T, 32, 512, 768, 4)
    assert W.fragments_supported(512, 768, 128)
    w13, w2 = ws["w13"], ws["w2"]
    if frag:
        w13, w2 = W.repack_fragments(w13, ws["s13"], ws["z13"]), W.repack_fragments(w2, ws["s2"], ws["z2"])
    out = W.moe_apply(x, w13, w2, ws["s13"], ws["s2"], ws["z13"], ws["z2"], tw, ids)
    ref = oracle_layer(cfg, ws, x, tw, ids)
    assert maxrel(out.float().cpu().numpy(), ref) <= REL_TOL
    if frag:
        op = W.moe_apply(x, ws["w13"], ws["w2"], ws["s13"], ws["s2"], ws["z13"], ws["z2"], tw, ids)
        assert torch.equal(out, op)


def _same_fp32_output(ob, oh):
    """ob (bf16) and oh (fp16) are the two roundings (RNE) of one fp32 value per element: the
    bf16 output lies between the bf16 roundings of the ends of the fp32 interval that rounds
    to the fp16 output (out_h +- half its spacing; rounding is monotone). NaN matches NaN."""
    nb, nh = torch.isnan(ob), torch.isnan(oh)
    if not torch.equal(nb, nh):
        return False, int((nb != nh).sum())
    hf = oh.float()
    a = hf.abs()
    e = torch.floor(torch.log2(torch.where(a > 0, a, torch.full_like(a, 2.0 ** -30)))).clamp(min=-14)
    half = torch.exp2(e - 11)                               # half an fp16 ulp (2^-25 floor)
    lo, hi = (hf - half).to(torch.bfloat16), (hf + half).to(torch.bfloat16)
    ok = ((ob >= lo) & (ob <= hi)) | nb
    return bool(ok.all()), int((~ok).sum())


def _host(ws, w):
    """Op-layout weights, scales and zero-points of weight w ("13" / "2") as numpy."""
    z = ws["z" + w]
    return ws["w" + w].cpu().numpy(), ws["s" + w].cpu().numpy(), None if z is None else z.cpu().numpy()


def _bf16_routes(cfg, ws, x, logits, frag):
    w13, w2 = ws["w13"], ws["w2"]
    if frag:
        w13, w2 = W.repack_fragments(w13, ws["s13"], ws["z13"]), W.repack_fragments(w2, ws["s2"], ws["z2"])
    ob, twb, idb = W.moe_forward(x, logits, cfg["k"], w13, w2, ws["s13"], ws["s2"], ws["z13"],
                                 ws["z2"])
    oh, twh, idh = W.moe_forward(x.to(torch.float16), logits, cfg["k"], w13, w2, ws["s13"],
                                 ws["s2"], ws["z13"], ws["z2"])
    assert ob.dtype == torch.bfloat16 and oh.dtype == torch.float16
    assert torch.equal(idb, idh) and torch.equal(twb, twh)
    return ob, oh, twb, idb


@pytest.mark.parametrize("T", [5, 32, 96, 97, 300])
@pytest.mark.parametrize("frag", [False, True])
def test_bf16_input_route_equals_fp16_cast(T, frag):
    """a3: a bf16 layer input is cast to fp16 before it is quantised, as the reference's
    x.to(fp16) (moe_experts.py:596). moe_forward(x_bf16) and moe_forward(x_bf16.to(fp16)) must
    then produce bf16(v) and fp16(v) of the same fp32 layer output v (bit-exact up to the two
    output casts). One row holds 65536 (fp16 infinity after the cast: the whole output row is
    NaN on both routes), one the largest finite bf16 below 65504 (finite through the cast;
    the layer then overflows fp16 in h on both routes alike). T covers the decode (<= 96) and
    prefill schedules; the fp16-subnormal range is the next test."""
    cfg = dict(T=T, H=512, E=16, k=4, I=256, g=128, routing="uniform")
    ws = bench.make_weights(cfg, 8100 + T, DEV)
    x, logits = bench.make_inputs(cfg, 8101 + T, DEV)
    x = x.to(torch.bfloat16)
    x[3, 17] = 65536.0                                       # fp16 overflow -> inf
    x[4, 5] = 65280.0                                        # largest finite bf16 < 65504
    ob, oh, _, _ = _bf16_routes(cfg, ws, x, logits, frag)
    nb = torch.isnan(ob)
    assert nb[3].all() and not nb[:3].any() and not nb[5:].any()
    ok, bad = _same_fp32_output(ob, oh)
    assert ok, bad


@pytest.mark.parametrize("T", [6, 130])
@pytest.mark.parametrize("frag", [False, True])
def test_bf16_input_route_fp16_subnormals(T, frag):
    """a3 where the cast is not the identity below fp16's normal range: rows of N(0,1) scaled
    to 1e-6 .. 5e-5 (fp16 quantum 2^-24 below 2^-14), so bf16 -> fp16 rounds them, and act
    scales at the 1e-8 floor. gemm1 scales x2000 keep the layer output of such rows above
    fp16 underflow. Both routes must give the same fp32 output (as above), and the fp16 route
    must match the oracle (x16 = fp16(x) first) on every row."""
    cfg = dict(T=T, H=512, E=16, k=4, I=256, g=128, routing="uniform")
    ws = bench.make_weights(cfg, 8200 + T, DEV)
    ws["s13"] = (ws["s13"].float() * 2000).to(torch.float16)
    x, logits = bench.make_inputs(cfg, 8201 + T, DEV)
    mag = torch.tensor([1e-6, 4e-6, 3e-5, 5e-5], device=DEV).repeat(T)[:T]
    x = (x.float() * mag[:, None]).to(torch.bfloat16)
    x16 = x.to(torch.float16)
    assert not torch.equal(x16.float(), x.float())          # the cast rounds these rows
    ob, oh, tw, ids = _bf16_routes(cfg, ws, x, logits, frag)
    assert not torch.isnan(ob).any()
    ok, bad = _same_fp32_output(ob, oh)
    assert ok, bad
    ref = oracle_layer(cfg, ws, x, tw, ids, round_y=T > 96)
    nz = np.abs(ref).max(axis=1) > 0
    assert nz.sum() >= T // 2, "the rows must not underflow to zero"
    # per row, within the layer bar of that row's own magnitude plus half the fp16 output's
    # quantum (2^-25: these outputs sit near fp16's subnormal range)
    got = oh.float().cpu().numpy()
    for r in np.nonzero(nz)[0]:
        err = float(np.abs(got[r].astype(np.float64) - ref[r]).max())
        assert err <= REL_TOL * float(np.abs(ref[r]).max()) + 2.0 ** -25, (r, err)
