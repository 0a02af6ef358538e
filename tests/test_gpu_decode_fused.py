"""The decode layer's two GEMVs fused into one launch (decode_layer_kernel, opt-in with
set_decode_fused / W4A8_DECODE_FUSED=1): gemm2 waits in the kernel for the gemm1 rows it
reads. Same arithmetic and partition as the two launches, so the outputs are bit-identical to
them; the oracle checks every token of the fused output at the c3 shape. Graph replays with
fresh inputs check that the completion flags are reset between calls (the slot reduce clears
them). The failure path is forced from the host (w4a8_decode_fused_test_fault: the waits wait
for a value nobody publishes, with a short spin limit, and every kernel ends normally): the
call's output is NaN, and the next call, or the next replay of the same graph, is clean."""
import numpy as np
import pytest
import torch

import bench
import oracle as O
import w4a8_fp8_wmma as W
from w4a8_fp8_wmma import _ops

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture
def fused_mode():
    old = W.set_decode_fused(False)
    yield
    _ops._decode_fused_test_fault(False)
    W.set_decode_fused(old)


def run(cfg, ws, x, logits, fused):
    W.set_decode_fused(fused)
    out, tw, ids = W.moe_forward(x, logits, cfg["k"], ws["f13"], ws["f2"], ws["s13"], ws["s2"],
                                 ws["z13"], ws["z2"])
    torch.cuda.synchronize()
    return out, tw, ids


def layer(name, T, seed):
    cfg = dict(bench.CONFIGS[name]) if isinstance(name, str) else dict(name)
    cfg["T"] = T
    ws = bench.make_weights(cfg, seed, DEV)
    ws["f13"], ws["f2"] = W.repack_fragments(ws["w13"], ws["s13"], ws["z13"]), W.repack_fragments(ws["w2"], ws["s2"], ws["z2"])
    x, logits = bench.make_inputs(cfg, seed + 1, DEV)
    return cfg, ws, x, logits


def oracle_rel(cfg, ws, x, tw, ids, out, sel):
    h = {kk: v.cpu().numpy() for kk, v in ws.items() if kk in ("w13", "s13", "z13", "w2", "s2", "z2")}
    ref = O.moe_layer(x.float().cpu().numpy()[sel], h["w13"], h["s13"], h["z13"], h["w2"],
                      h["s2"], h["z2"], tw.cpu().numpy()[sel], ids.cpu().numpy()[sel], cfg["g"],
                      round_y_fp16=False)
    got = out.float().cpu().numpy()[sel]
    return float(np.abs(got - ref).max() / np.abs(ref).max())


SMALL = dict(H=512, E=16, k=4, I=256, g=128, routing="uniform")


@pytest.mark.parametrize("name,T", [("c3", 32), ("c3", 1), ("c3", 96), ("c5", 32), ("c5", 1),
                                    (SMALL, 7), (SMALL, 64)])
def test_fused_decode_equals_two_launches(fused_mode, name, T):
    cfg, ws, x, logits = layer(name, T, 6100 + T)
    out2, tw, ids = run(cfg, ws, x, logits, fused=False)
    out1, tw1, ids1 = run(cfg, ws, x, logits, fused=True)
    assert torch.equal(ids1, ids) and torch.equal(tw1, tw)
    assert not torch.isnan(out1.float()).any()
    assert torch.equal(out1, out2)
    # the oracle on a few tokens here; every token at the c3 shape below
    assert oracle_rel(cfg, ws, x, tw, ids, out1, np.arange(min(T, 4))) <= 1e-2


def test_fused_decode_c3_every_token_vs_oracle(fused_mode):
    """All 32 tokens of the c3 shape (2048 hidden, 256 experts, top-8, 512 intermediate)
    through the fused launch, against the CPU oracle, max-rel <= 1e-2."""
    cfg, ws, x, logits = layer("c3", 32, 6150)
    out, tw, ids = run(cfg, ws, x, logits, fused=True)
    assert not torch.isnan(out.float()).any()
    assert oracle_rel(cfg, ws, x, tw, ids, out, np.arange(32)) <= 1e-2


def test_fused_decode_graph_replays(fused_mode):
    """Five replays of one captured fused layer, each after new inputs are copied in, against
    eager two-launch calls on the same inputs (the flags are cleared by each replay's slot
    reduce; a stale flag would let gemm2 read the previous replay's rows)."""
    cfg, ws, x, logits = layer("c3", 32, 6200)
    W.set_decode_fused(True)
    xs, ls = x.clone(), logits.clone()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        W.moe_forward(xs, ls, cfg["k"], ws["f13"], ws["f2"], ws["s13"], ws["s2"], ws["z13"], ws["z2"])
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out_g, _, _ = W.moe_forward(xs, ls, cfg["k"], ws["f13"], ws["f2"], ws["s13"], ws["s2"],
                                    ws["z13"], ws["z2"])
    for r in range(5):
        x_r, l_r = bench.make_inputs(cfg, 6300 + r, DEV)
        xs.copy_(x_r)
        ls.copy_(l_r)
        g.replay()
        torch.cuda.synchronize()
        got = out_g.clone()
        ref, _, _ = run(cfg, ws, x_r, l_r, fused=False)
        W.set_decode_fused(True)
        assert torch.equal(got, ref), r


def test_fused_decode_wait_gives_up_then_recovers(fused_mode):
    """Eager: a call whose waits give up returns a NaN layer (and no error); the next call
    with the hook off equals the two-launch result."""
    cfg, ws, x, logits = layer("c3", 32, 6400)
    ref, _, _ = run(cfg, ws, x, logits, fused=False)
    _ops._decode_fused_test_fault(True)
    bad, _, _ = run(cfg, ws, x, logits, fused=True)
    assert torch.isnan(bad.float()).all()
    _ops._decode_fused_test_fault(False)
    good, _, _ = run(cfg, ws, x, logits, fused=True)
    assert torch.equal(good, ref)


def test_fused_decode_graph_replay_after_a_timeout(fused_mode):
    """One captured graph (its nonce fixed at capture): a replay whose waits give up is NaN,
    and the replays after it are finite and exact again (each work-group clears its own
    timeout word when it starts)."""
    cfg, ws, x, logits = layer("c3", 32, 6500)
    ref, _, _ = run(cfg, ws, x, logits, fused=False)
    W.set_decode_fused(True)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        W.moe_forward(x, logits, cfg["k"], ws["f13"], ws["f2"], ws["s13"], ws["s2"], ws["z13"], ws["z2"])
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out_g, _, _ = W.moe_forward(x, logits, cfg["k"], ws["f13"], ws["f2"], ws["s13"], ws["s2"],
                                    ws["z13"], ws["z2"])
    g.replay()
    torch.cuda.synchronize()
    assert torch.equal(out_g, ref)
    _ops._decode_fused_test_fault(True)
    g.replay()
    torch.cuda.synchronize()
    assert torch.isnan(out_g.float()).all()
    _ops._decode_fused_test_fault(False)
    for r in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out_g, ref), r
