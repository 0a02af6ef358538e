"""Pin the oracle's align, grouped GEMM, converters and full layer (CPU)."""
import numpy as np
import pytest

import oracle as O


# --------------------------------------------------------------------------- #
# moe_align
# --------------------------------------------------------------------------- #
def align_bruteforce(ids, block_m, E):
    """Pure-Python statement of the mirror's loop (expert asc, slot asc, pad)."""
    T, k = ids.shape
    flat = [int(v) for v in ids.reshape(-1)]
    out, eids = [], []
    for e in range(E):
        slots = [i for i, v in enumerate(flat) if v == e]
        npad = -(-len(slots) // block_m) * block_m
        out += slots + [T * k] * (npad - len(slots))
        eids += [e] * (npad // block_m)
    return out, eids


@pytest.mark.parametrize("T,k,E,bm", [(1, 8, 256, 16), (3, 2, 8, 4), (37, 4, 16, 8),
                                      (64, 8, 32, 64), (5, 1, 3, 1)])
def test_align_bruteforce(T, k, E, bm):
    r = np.random.default_rng(T * 131 + E)
    ids = np.stack([r.permutation(E)[:k] for _ in range(T)]).astype(np.int32)
    sti, eid, ntp = O.moe_align(ids, bm, E)
    bs, be = align_bruteforce(ids, bm, E)
    n = int(ntp[0])
    assert n == len(bs)
    assert sti[:n].tolist() == bs and eid[:n // bm].tolist() == be
    assert np.all(sti[n:] == T * k) and np.all(eid[n // bm:] == -1)
    assert sti.size == O.align_alloc_len(T * k, E, bm)


def test_align_invariants_with_duplicates_and_map():
    r = np.random.default_rng(9)
    T, k, E, bm = 40, 4, 12, 8
    ids = r.integers(0, E, (T, k)).astype(np.int32)      # duplicates inside a row allowed
    sti, eid, ntp = O.moe_align(ids, bm, E)
    n = int(ntp[0])
    real = sti[:n][sti[:n] < T * k]
    assert sorted(real.tolist()) == list(range(T * k))  # a permutation of all slots
    for b in range(n // bm):                              # single-expert blocks, slots asc
        blk = sti[b * bm:(b + 1) * bm]
        v = blk[blk < T * k]
        assert np.all(ids.reshape(-1)[v] == eid[b]) and np.all(np.diff(v) > 0)
    assert np.all(np.diff(eid[:n // bm]) >= 0)
    # expert_map: experts 0..5 local (as 0..5), others dropped
    emap = np.array([0, 1, 2, 3, 4, 5] + [-1] * 6, np.int32)
    sti2, eid2, ntp2 = O.moe_align(ids, bm, E, expert_map=emap)
    n2 = int(ntp2[0])
    kept = sti2[:n2][sti2[:n2] < T * k]
    assert sorted(kept.tolist()) == sorted(np.nonzero(ids.reshape(-1) < 6)[0].tolist())


# --------------------------------------------------------------------------- #
# grouped GEMM vs an independent dense float64 formulation
# --------------------------------------------------------------------------- #
def make_weights(r, E, N, K, g, asym=True):
    nib = r.integers(0, 16, (E, N, K))
    zp = r.integers(0, 16, (E, N, K // g)) if asym else np.full((E, N, K // g), 8)
    sc = r.uniform(0.005, 0.02, (E, N, K // g)).astype(np.float16)
    return nib, zp, sc, O.pack_nibbles(nib), (O.pack_zeros(zp) if asym else None)


def dense_ref(x16, nib, zp, sc, g, rows_expert):
    """out[r] = fp16(sum_k fp8(x)[k] * (nib-zp)[k] * scale[k//g] * s_r): one float64
    dot product over dequantised weights (no per-group partial sums)."""
    q, s = O.act_quant(x16)
    A = O.E4M3_TO_F64[q]
    W = (nib - np.repeat(zp, g, -1)) * np.repeat(sc.astype(np.float64), g, -1)
    out = np.stack([W[e] @ A[i] for i, e in enumerate(rows_expert)])
    return out * s[:, None]


@pytest.mark.parametrize("asym", [True, False])
@pytest.mark.parametrize("g", [128, 64, 32])
def test_grouped_gemm_vs_dense_f64(asym, g):
    r = np.random.default_rng(11 + g)
    T, E, N, K, k, bm = 12, 4, 32, 256, 2, 16
    nib, zp, sc, w, z = make_weights(r, E, N, K, g, asym)
    x = r.standard_normal((T, K)).astype(np.float16)
    ids = np.stack([r.permutation(E)[:k] for _ in range(T)]).astype(np.int32)
    sti, eid, ntp = O.moe_align(ids, bm, E)
    out, valid = O.grouped_gemm_padded(x, w, sc, z, sti, eid, ntp, k, bm)
    rows = np.nonzero(valid)[0]
    slots = sti[rows]
    ref = dense_ref(x[slots // k], nib, zp, sc, g, eid[rows // bm])
    got = out[rows].astype(np.float64)
    assert np.all(np.abs(got - ref) <= 2.0 ** -10 * np.abs(ref) + 1e-3 * np.abs(ref).max())
    assert np.all(np.isnan(out[~valid].astype(np.float32)))


def test_grouped_gemm_planted_mistakes_are_caught():
    """A transposed nibble order, a dropped zero-point and a wrong scale index each move
    the result far outside the parity tolerance used on the GPU."""
    r = np.random.default_rng(12)
    T, E, N, K, k, bm, g = 8, 2, 16, 256, 1, 8, 128
    nib, zp, sc, w, z = make_weights(r, E, N, K, g)
    x = r.standard_normal((T, K)).astype(np.float16)
    ids = r.integers(0, E, (T, k)).astype(np.int32)
    sti, eid, ntp = O.moe_align(ids, bm, E)
    good, valid = O.grouped_gemm_padded(x, w, sc, z, sti, eid, ntp, k, bm)

    def relerr(bad):
        a = good[valid].astype(np.float64)
        return np.abs(bad[valid].astype(np.float64) - a).max() / np.abs(a).max()

    swapped = O.pack_nibbles(nib[..., ::-1])
    assert relerr(O.grouped_gemm_padded(x, swapped, sc, z, sti, eid, ntp, k, bm)[0]) > 0.05
    assert relerr(O.grouped_gemm_padded(x, w, sc, None, sti, eid, ntp, k, bm)[0]) > 0.05
    sc_t = np.ascontiguousarray(sc[:, :, ::-1])
    assert relerr(O.grouped_gemm_padded(x, w, sc_t, z, sti, eid, ntp, k, bm)[0]) > 0.05


def test_dense_gemm_equals_grouped_identity():
    r = np.random.default_rng(13)
    M, N, K, g = 16, 64, 256, 128
    nib, zp, sc, w, z = make_weights(r, 1, N, K, g)
    x = r.standard_normal((M, K)).astype(np.float16)
    d = O.dense_gemm(x, w[0], sc[0], z[0])
    ref = dense_ref(x, nib, zp, sc, g, [0] * M)
    assert np.all(np.abs(d.astype(np.float64) - ref) <= 2.0 ** -10 * np.abs(ref) + 1e-3 * np.abs(ref).max())


def test_scatter_equals_gather_reduce_without_fp16_rounding():
    r = np.random.default_rng(14)
    T, E, N, K, k, bm, g = 6, 4, 32, 128, 2, 8, 128
    nib, zp, sc, w, z = make_weights(r, E, N, K, g)
    ids = np.stack([r.permutation(E)[:k] for _ in range(T)]).astype(np.int32)
    tw = r.random((T, k)).astype(np.float32)
    sti, eid, ntp = O.moe_align(ids, bm, E)
    P = sti.size
    hpad = r.standard_normal((P, K)).astype(np.float16)
    sc_out = O.gemm_scatter(hpad, w, sc, z, sti, eid, ntp, tw.reshape(-1),
                            np.zeros((T, N), np.float32), k, bm)
    ident = np.arange(P, dtype=np.int32)
    # identity gather with top_k=1 -> (P, N) fp16, then gather-reduce
    o2, _ = O.grouped_gemm_padded(hpad, w, sc, z, np.where(
        (sti < T * k) & (np.arange(P) < ntp[0]), ident, P).astype(np.int32), eid, ntp, 1, bm)
    gr = O.gather_reduce(np.nan_to_num(o2), sti, tw.reshape(-1), ntp, k)
    assert np.allclose(sc_out, gr, rtol=2e-3, atol=2e-3 * np.abs(gr).max())


# --------------------------------------------------------------------------- #
# converters
# --------------------------------------------------------------------------- #
def test_awq_to_op_layout_dequant_equality():
    """Reference property (test_moe_experts.py:115-130, test_moe_conversion_numpy.py:83-105)."""
    r = np.random.default_rng(0)
    for (E, K, N, g) in [(4, 256, 128, 32), (8, 512, 256, 128), (3, 256, 64, 16)]:
        q = r.integers(0, 16, (E, K, N))
        zz = r.integers(0, 16, (E, K // g, N))
        s = (np.abs(r.standard_normal((E, K // g, N))) * 0.02 + 0.001).astype(np.float16)
        w, sc, z = O.awq_to_op_layout(O.awq_pack(q), s, O.awq_pack(zz))
        assert w.shape == (E, N, K // 8) and sc.shape == (E, N, K // g) and z.shape == (E, N // 8, K // g)
        assert np.array_equal(O.unpack_nibbles(w), np.swapaxes(q, 1, 2))
        assert np.array_equal(O.unpack_zeros(z, N), np.swapaxes(zz, 1, 2))
        assert np.array_equal(sc, np.swapaxes(s, 1, 2))


def test_wna16_loader_then_view_matches_awq_conversion():
    """vLLM loader (convert_awq_tensor) + zero-copy view == direct AWQ conversion."""
    r = np.random.default_rng(2)
    K, N, g = 256, 64, 128
    q = r.integers(0, 16, (1, K, N))
    zz = r.integers(0, 16, (1, K // g, N))
    qw, qz = O.awq_pack(q)[0], O.awq_pack(zz)[0]
    u8w = O.convert_awq_tensor(qw, "qweight")            # (N, K/2)
    u8z = O.convert_awq_tensor(qz, "qzeros")             # (N/2, G)
    w, _, z = O.wna16_to_op_layout(u8w[None], np.ones((1, N, K // g), np.float16), u8z[None])
    w2, _, z2 = O.awq_to_op_layout(O.awq_pack(q), np.ones((1, K // g, N), np.float16),
                                   O.awq_pack(zz))
    assert np.array_equal(w, w2) and np.array_equal(z, z2)


# --------------------------------------------------------------------------- #
# full layer
# --------------------------------------------------------------------------- #
def layer_inputs(r, T=8, E=8, H=256, I=128, k=2, g=128, asym=True):
    n13, z13, s13, w13, zz13 = make_weights(r, E, 2 * I, H, g, asym)
    n2, z2, s2, w2, zz2 = make_weights(r, E, H, I, g, asym)
    x = r.standard_normal((T, H)).astype(np.float32)
    lg = r.standard_normal((T, E)).astype(np.float32)
    tw, ids = O.topk_softmax(lg, k)
    return dict(x=x, w13=w13, s13=s13, z13=zz13, w2=w2, s2=s2, z2=zz2, tw=tw, ids=ids)


def test_layer_close_to_unquantised_f64():
    r = np.random.default_rng(21)
    d = layer_inputs(r)
    got = O.moe_layer(d["x"], d["w13"], d["s13"], d["z13"], d["w2"], d["s2"], d["z2"],
                      d["tw"], d["ids"])
    ideal = O.moe_layer_f64(d["x"], d["w13"], d["s13"], d["z13"], d["w2"], d["s2"], d["z2"],
                            d["tw"], d["ids"])
    rel = np.abs(got - ideal).max() / np.abs(ideal).max()
    assert rel < 0.08, rel        # fp8 activation quantisation error only


def test_swigluoai_bias_layer_close_to_unquantised_f64():
    """The gpt-oss composition (per-expert biases on both GEMMs, swigluoai on interleaved
    gate/up) against the float64 model; taking gate/up as halves (the SiLU layout), or
    dropping either bias, moves the layer far outside the fp8 error."""
    r = np.random.default_rng(23)
    d = layer_inputs(r)
    E, I2, H = d["w13"].shape[0], d["w13"].shape[1], d["w2"].shape[1]
    b13 = (r.standard_normal((E, I2)) * 1.0).astype(np.float16)
    b2 = (r.standard_normal((E, H)) * 2.0).astype(np.float16)
    args = (d["x"], d["w13"], d["s13"], d["z13"], d["w2"], d["s2"], d["z2"], d["tw"], d["ids"])
    got = O.moe_layer(*args, activation="swigluoai", w1_bias=b13, w2_bias=b2)
    ideal = O.moe_layer_f64(*args, activation="swigluoai", w1_bias=b13, w2_bias=b2)
    scale = np.abs(ideal).max()
    assert np.abs(got - ideal).max() / scale < 0.05     # fp8 activation quantisation only
    for planted in (dict(activation="swigluoai", w1_bias=b13),
                    dict(activation="swigluoai", w2_bias=b2),
                    dict(activation="silu", w1_bias=b13, w2_bias=b2)):
        wrong = O.moe_layer_f64(*args, **planted)
        assert np.abs(got - wrong).max() / scale > 0.1, planted


def test_layer_equals_stage_chain():
    """The composed layer equals align -> padded gemm1 -> silu -> padded gemm2 (identity)
    -> gather-reduce built from the per-op oracle functions."""
    r = np.random.default_rng(22)
    d = layer_inputs(r, T=6, E=4, k=2)
    T, k = d["ids"].shape
    bm = 8
    sti, eid, ntp = O.moe_align(d["ids"], bm, 4)
    x16 = d["x"].astype(np.float16)
    o1, valid = O.grouped_gemm_padded(x16, d["w13"], d["s13"], d["z13"], sti, eid, ntp, k, bm)
    I = o1.shape[1] // 2
    h = O.silu_and_mul(np.nan_to_num(o1[:, :I]), np.nan_to_num(o1[:, I:]))
    P = sti.size
    ident = np.where(valid, np.arange(P), P).astype(np.int32)
    o2, _ = O.grouped_gemm_padded(h, d["w2"], d["s2"], d["z2"], ident, eid, ntp, 1, bm)
    chain = O.gather_reduce(np.nan_to_num(o2), sti, d["tw"].reshape(-1), ntp, k)
    lay = O.moe_layer(d["x"], d["w13"], d["s13"], d["z13"], d["w2"], d["s2"], d["z2"],
                      d["tw"], d["ids"], round_y_fp16=True)
    assert np.array_equal(chain, lay)


@pytest.mark.parametrize("asym", [True, False])
def test_integer_weights_equal_e4m3_round_trip(asym):
    """The oracle's fast weight path (n - z as integers) equals decoding the e4m3 bytes the
    kernels' tables produce, element for element."""
    r = np.random.default_rng(23)
    _, _, _, w, zz = make_weights(r, 2, 32, 512, 128, asym)
    for e in range(2):
        fast = O.expert_weights_f64(w[e], None if zz is None else zz[e], 128, False)
        codes = O.dequant_codes(w[e], None if zz is None else zz[e], 128)
        assert np.array_equal(fast, O.E4M3_TO_F64[codes])


def test_layer_biases_closed_form():
    """Zero weights: gemm1 gives exact zeros, so gate/up are the w1 bias itself and
    out[t] = sum_j w_j * fp16(0 + b2[e_j]) with h = silu(b_gate) * b_up ignored by gemm2."""
    r = np.random.default_rng(24)
    T, E, H, I, k = 5, 4, 256, 128, 2
    w13 = O.pack_nibbles(np.full((E, 2 * I, H), 8))
    w2 = O.pack_nibbles(np.full((E, H, I), 8))
    s13 = np.full((E, 2 * I, H // 128), 0.01, np.float16)
    s2 = np.full((E, H, I // 128), 0.01, np.float16)
    b1 = r.standard_normal((E, 2 * I)).astype(np.float16)
    b2 = r.standard_normal((E, H)).astype(np.float16)
    x = r.standard_normal((T, H)).astype(np.float32)
    tw, ids = O.topk_softmax(r.standard_normal((T, E)).astype(np.float32), k)
    out, st = O.moe_layer(x, w13, s13, None, w2, s2, None, tw, ids, w1_bias=b1, w2_bias=b2,
                          return_stages=True)
    e = ids.reshape(-1)
    assert np.array_equal(st["g1"], b1[e])
    exp = np.zeros((T, H), np.float32)
    for j in range(k):
        exp = O.fma32(tw[:, j:j + 1], b2[ids[:, j]].astype(np.float32), exp)
    assert np.array_equal(out, exp)


def test_layer_biases_equal_stage_chain():
    """With biases the layer equals the per-op chain with torch's fp16 adds in between
    (moe_experts.py:565-575,654-655)."""
    import torch
    r = np.random.default_rng(25)
    d = layer_inputs(r, T=6, E=4, k=2)
    E, N13 = d["w13"].shape[:2]
    b1 = r.standard_normal((E, N13)).astype(np.float16)
    b2 = r.standard_normal((E, d["w2"].shape[1])).astype(np.float16)
    T, k = d["ids"].shape
    bm = 8
    sti, eid, ntp = O.moe_align(d["ids"], bm, 4)
    row_e = np.repeat(np.maximum(eid, 0), bm)[:sti.size]
    x16 = d["x"].astype(np.float16)
    o1, valid = O.grouped_gemm_padded(x16, d["w13"], d["s13"], d["z13"], sti, eid, ntp, k, bm)
    o1 = (torch.from_numpy(np.nan_to_num(o1)) + torch.from_numpy(b1[row_e])).numpy()
    I = o1.shape[1] // 2
    h = O.silu_and_mul(o1[:, :I], o1[:, I:])
    P = sti.size
    ident = np.where(valid, np.arange(P), P).astype(np.int32)
    o2, _ = O.grouped_gemm_padded(h, d["w2"], d["s2"], d["z2"], ident, eid, ntp, 1, bm)
    o2 = (torch.from_numpy(np.nan_to_num(o2)) + torch.from_numpy(b2[row_e])).numpy()
    chain = O.gather_reduce(o2, sti, d["tw"].reshape(-1), ntp, k)
    lay = O.moe_layer(d["x"], d["w13"], d["s13"], d["z13"], d["w2"], d["s2"], d["z2"],
                      d["tw"], d["ids"], w1_bias=b1, w2_bias=b2)
    assert np.array_equal(chain, lay)


def test_layer_expert_map_equals_local_subset():
    """Global ids 0..7 with experts 4..7 local (as 0..3): the layer equals the same layer on
    the local weights with the non-local slots' router weights set to zero."""
    r = np.random.default_rng(26)
    d = layer_inputs(r, T=7, E=4, k=3)
    ids_g = r.integers(0, 8, (7, 3)).astype(np.int32)
    emap = np.array([-1, -1, -1, -1, 0, 1, 2, 3], np.int32)
    got = O.moe_layer(d["x"], d["w13"], d["s13"], d["z13"], d["w2"], d["s2"], d["z2"],
                      d["tw"], ids_g, expert_map=emap)
    local = np.where(ids_g >= 4, ids_g - 4, 0)
    tw0 = np.where(ids_g >= 4, d["tw"], 0).astype(np.float32)
    ref = O.moe_layer(d["x"], d["w13"], d["s13"], d["z13"], d["w2"], d["s2"], d["z2"],
                      tw0, local)
    assert np.array_equal(got, ref)
