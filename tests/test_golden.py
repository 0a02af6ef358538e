"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py).

CPU: the oracle reproduces every fixture bit for bit (regression lock on the pinned
oracle). GPU: the HIP kernels reproduce the same fixtures through the C ABI, bit-exact
for dequant / act-quant / routing indices / align, weights to 2e-5 relative, and the
tiny layer to max|out - ref| / max|ref| <= 1e-2."""
import os

import numpy as np
import pytest
import torch

import oracle as O

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    with np.load(os.path.join(GOLD, name), allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


# --------------------------------------------------------------------------- #
# oracle == fixtures (CPU)
# --------------------------------------------------------------------------- #
def test_oracle_dequant_fixture():
    g = load("dequant_tables.npz")
    for z in range(16):
        assert np.array_equal(O.dequant_table(z), g["tables"][z])
    assert np.array_equal(O.dequant_table(0, e2m1=True), g["e2m1"])
    # closed form: e4m3 bytes of the small integers n - z decode back exactly
    n = np.arange(16)
    for z in range(16):
        assert np.array_equal(O.e4m3_decode(g["tables"][z]), (n - z).astype(np.float32))


def test_oracle_act_quant_fixture():
    g = load("act_quant.npz")
    q, s = O.act_quant(g["x_bits"].view(np.float16))
    assert np.array_equal(q, g["q"]) and np.array_equal(s, g["scales"])


def test_oracle_routing_fixture():
    g = load("routing.npz")
    w, ids = O.topk_softmax(g["logits"], int(g["top_k"]))
    assert np.array_equal(ids, g["ids"]) and np.array_equal(w, g["weights"])
    assert ids[0].tolist() == [0, 1, 2, 3]                 # full tie -> lowest ids
    assert sorted(ids[1][:3].tolist()) == [3, 9, 12]


def _align_cases():
    g = load("align.npz")
    for name in ("a", "b", "c", "d"):
        em = g[f"{name}_emap"]
        yield (name, g[f"{name}_ids"], int(g[f"{name}_E"]), int(g[f"{name}_bm"]),
               em if em.size else None, g[f"{name}_sorted"], g[f"{name}_experts"],
               g[f"{name}_ntp"])


def test_oracle_align_fixture():
    for name, ids, E, bm, em, so, eo, no in _align_cases():
        s, e, n = O.moe_align(ids, bm, E, expert_map=em)
        assert np.array_equal(s, so) and np.array_equal(e, eo) and np.array_equal(n, no), name


def test_oracle_layer_fixture():
    g = load("layer_tiny.npz")
    out = O.moe_layer(O.bf16_bits_to_f32(g["x_bf16_bits"]), g["w13"], g["s13_bits"].view(np.float16),
                      g["z13"], g["w2"], g["s2_bits"].view(np.float16), g["z2"], g["topk_weights"],
                      g["topk_ids"], int(g["group_size"]), round_y_fp16=False)
    assert np.array_equal(out, g["out"])


# --------------------------------------------------------------------------- #
# HIP kernels == fixtures (GPU)
# --------------------------------------------------------------------------- #
@pytest.fixture(scope="module")
def gpu():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a visible MI355X"
    import w4a8_fp8_wmma as W
    return torch, W


@pytest.mark.gpu
def test_gpu_dequant_fixture(gpu):
    torch, W = gpu
    g = load("dequant_tables.npz")
    # one row per zero-point, holding all 16 nibbles; group 128 -> zp constant per row
    N, K = 16, 128
    nib = np.tile(np.arange(16), (N, K // 16))
    w = O.pack_nibbles(nib)[None]
    z = O.pack_zeros(np.arange(16).reshape(N, 1))[None]
    got = W.dequant_fp8(torch.from_numpy(w).cuda(), 128, torch.from_numpy(z).cuda()).cpu().numpy()[0]
    assert np.array_equal(got, g["tables"][:, nib[0]])
    got2 = W.dequant_fp8(torch.from_numpy(w).cuda(), 128, None, weight_is_e2m1=True).cpu().numpy()[0]
    assert np.array_equal(got2[0], g["e2m1"][nib[0]])


@pytest.mark.gpu
def test_gpu_act_quant_fixture(gpu):
    torch, W = gpu
    g = load("act_quant.npz")
    q, s = W.act_quant_fp8(torch.from_numpy(g["x_bits"].view(np.float16)).cuda())
    assert np.array_equal(s.cpu().numpy(), g["scales"])
    assert np.array_equal(q.cpu().numpy(), g["q"])


@pytest.mark.gpu
def test_gpu_routing_fixture(gpu):
    torch, W = gpu
    g = load("routing.npz")
    w, ids = W.fused_topk(None, torch.from_numpy(g["logits"]).cuda(), int(g["top_k"]), True)
    assert np.array_equal(ids.cpu().numpy(), g["ids"])
    np.testing.assert_allclose(w.cpu().numpy(), g["weights"], rtol=2e-5, atol=1e-7)


@pytest.mark.gpu
def test_gpu_align_fixture(gpu):
    torch, W = gpu
    for name, ids, E, bm, em, so, eo, no in _align_cases():
        tm = None if em is None else torch.from_numpy(em).cuda()
        s, e, n = W.moe_align_block_size(torch.from_numpy(ids).cuda(), bm, E, tm)
        assert int(n.item()) == int(no[0]), name
        assert np.array_equal(s.cpu().numpy(), so), name
        assert np.array_equal(e.cpu().numpy(), eo), name


@pytest.mark.gpu
def test_gpu_layer_fixture(gpu):
    torch, W = gpu
    g = load("layer_tiny.npz")
    t = {k: torch.from_numpy(v).cuda() for k, v in g.items() if v.ndim > 0}
    x = t["x_bf16_bits"].view(torch.bfloat16)
    out = W.moe_apply(x, t["w13"], t["w2"], t["s13_bits"].view(torch.float16),
                      t["s2_bits"].view(torch.float16), t["z13"], t["z2"], t["topk_weights"],
                      t["topk_ids"])
    got = out.float().cpu().numpy()
    ref = g["out"]
    assert np.abs(got - ref).max() / np.abs(ref).max() <= 1e-2


def _conversion_cases():
    f = load("conversion_ref.npz")
    n = len({k.split("_")[0] for k in f})
    return f, n


def test_awq_conversion_matches_reference_vectors():
    """AWQ -> op layout: the oracle and the torch converter both reproduce the vectors the
    reference's own numpy conversion test wrote (tests/golden/make_conversion_golden.py),
    which pins the AWQ nibble order independently of this repository's packer."""
    from w4a8_fp8_wmma import moe_experts
    f, n = _conversion_cases()
    for i in range(n):
        c = lambda k: f[f"c{i}_{k}"]  # noqa: E731
        g = int(c("group"))
        w, s, z = O.awq_to_op_layout(c("awq_qweight"), c("scales"), c("awq_qzeros"))
        assert np.array_equal(w, c("awq_w_op")) and np.array_equal(z, c("awq_z_op"))
        assert np.array_equal(s, c("awq_s_op"))
        tw, ts, tz = moe_experts._awq_moe_to_op_layout(
            torch.from_numpy(c("awq_qweight")), torch.from_numpy(c("scales")),
            torch.from_numpy(c("awq_qzeros")), g)
        assert np.array_equal(tw.numpy(), c("awq_w_op")) and np.array_equal(tz.numpy(), c("awq_z_op"))
        # the converted nibbles are the ground-truth values the reference packed
        assert np.array_equal(O.unpack_nibbles(w), np.swapaxes(c("qvals"), 1, 2))
        assert np.array_equal(O.unpack_zeros(z, w.shape[1]), np.swapaxes(c("zeros"), 1, 2))
        # and our AWQ packer writes the reference's words
        assert np.array_equal(O.awq_pack(c("qvals")), c("awq_qweight"))


def test_ct_conversion_matches_reference_vectors():
    from w4a8_fp8_wmma import moe_experts
    f, n = _conversion_cases()
    for i in range(n):
        c = lambda k: f[f"c{i}_{k}"]  # noqa: E731
        cw, _ = moe_experts._ct_moe_to_op_layout(torch.from_numpy(c("gptq_qweight")),
                                                 torch.from_numpy(c("scales")))
        assert np.array_equal(cw.numpy(), c("ct_w_op"))
