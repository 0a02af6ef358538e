"""Pin the oracle's numeric primitives against libraries and closed forms (CPU)."""
import os

import numpy as np
import pytest
import torch

import oracle as O

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def torch_e4m3(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(
        torch.float8_e4m3fn).view(torch.uint8).numpy()


def test_e4m3_encode_exhaustive_fp16_inputs():
    # every fp16 bit pattern (subnormals, ties, overflow, inf, nan)
    h = np.arange(65536, dtype=np.uint16).view(np.float16).astype(np.float32)
    assert np.array_equal(O.e4m3_encode(h), torch_e4m3(h))


def test_e4m3_encode_random_fp32():
    r = np.random.default_rng(7)
    x = (r.standard_normal(1 << 20) * np.exp2(r.integers(-16, 12, 1 << 20))).astype(np.float32)
    assert np.array_equal(O.e4m3_encode(x), torch_e4m3(x))


def test_e4m3_encode_ties_round_to_even():
    # midpoints between adjacent e4m3 values round to the even mantissa
    vals = O.E4M3_TO_F64[:0x7E].copy()
    vals = np.unique(vals[np.isfinite(vals) & (vals >= 0)])
    mids = ((vals[:-1] + vals[1:]) / 2).astype(np.float32)
    got = O.e4m3_decode(O.e4m3_encode(mids))
    codes_lo = O.e4m3_encode(vals[:-1].astype(np.float32))
    codes_hi = O.e4m3_encode(vals[1:].astype(np.float32))
    even = np.where(codes_lo % 2 == 0, vals[:-1], vals[1:])
    assert np.array_equal(got, even.astype(np.float32))
    assert np.array_equal(O.e4m3_encode(mids), torch_e4m3(mids))
    del codes_hi


def test_e4m3_decode_all_codes():
    codes = np.arange(256, dtype=np.uint8)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    assert np.array_equal(O.e4m3_decode(codes), ref, equal_nan=True)


def test_dequant_table_exhaustive():
    # all 16 nibbles x 16 zero-points: e4m3 byte of (n - z) == torch cast, exact in e4m3
    for z in range(16):
        t = O.dequant_table(z)
        n = np.arange(16)
        assert np.array_equal(t, torch_e4m3((n - z).astype(np.float32)))
        assert np.array_equal(O.e4m3_decode(t), (n - z).astype(np.float32))


def test_dequant_table_e2m1_is_exact():
    t = O.dequant_table(0, e2m1=True)
    assert np.array_equal(O.e4m3_decode(t), O.E2M1_LUT)
    assert t[8] == 0x80  # -0.0 keeps its sign


def test_dequant_codes_matches_unpack():
    r = np.random.default_rng(1)
    E, N, K, g = 2, 16, 256, 128
    nib = r.integers(0, 16, (E, N, K))
    zp = r.integers(0, 16, (E, N, K // g))
    w = O.pack_nibbles(nib)
    z = O.pack_zeros(zp)
    assert np.array_equal(O.unpack_nibbles(w), nib)
    assert np.array_equal(O.unpack_zeros(z, N), zp)
    codes = O.dequant_codes(w, z, g)
    expect = nib - np.repeat(zp, g, axis=-1)
    assert np.array_equal(O.e4m3_decode(codes), expect.astype(np.float32))
    sym = O.dequant_codes(w, None, g)
    assert np.array_equal(O.e4m3_decode(sym), (nib - 8).astype(np.float32))


def test_unpack_nibble_order_low_first():
    w = np.array([[0x76543210]], dtype=np.uint32).view(np.int32)
    assert O.unpack_nibbles(w).tolist() == [[0, 1, 2, 3, 4, 5, 6, 7]]
    z = np.array([[[0x76543210]]], dtype=np.uint32).view(np.int32)   # (1, N/8=1, G=1)
    assert O.unpack_zeros(z, 8)[0, :, 0].tolist() == list(range(8))


def test_act_quant_matches_torch_reciprocal_form():
    r = np.random.default_rng(3)
    x = (r.standard_normal((64, 512)) * np.exp2(r.integers(-6, 6, (64, 1)))).astype(np.float16)
    x[0] = 0                      # all-zero row -> scale floor
    x[1, :] = np.float16(1e-4)    # tiny row
    x[2, 5] = np.float16(60000)   # large outlier
    q, s = O.act_quant(x)
    xt = torch.from_numpy(x).float()
    amax = xt.abs().amax(1)
    st = torch.clamp(amax / 448.0, min=1e-8)
    qt = (xt * (1.0 / st)[:, None]).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(s, st.numpy())
    assert np.array_equal(q, qt)
    assert s[0] == np.float32(1e-8) and np.all(q[0] == 0)


def test_act_quant_invariants():
    r = np.random.default_rng(4)
    x = r.standard_normal((32, 256)).astype(np.float16)
    q, s = O.act_quant(x)
    deq = O.e4m3_decode(q) * s[:, None]
    xf = x.astype(np.float32)
    # the absmax element maps to +-448 exactly; every element within half an e4m3 ulp
    assert np.all(np.abs(O.e4m3_decode(q)).max(1) == 448.0)
    assert np.all(np.abs(deq - xf) <= np.abs(xf) * 2.0 ** -4 + s[:, None] * 2.0 ** -10)


def test_silu_and_mul_against_torch():
    r = np.random.default_rng(5)
    g = (r.standard_normal(4096) * 4).astype(np.float16)
    u = (r.standard_normal(4096) * 2).astype(np.float16)
    got = O.silu_and_mul(g, u).astype(np.float64)
    silu = torch.nn.functional.silu(torch.from_numpy(g).double()).numpy()
    ref = silu * u.astype(np.float64)
    # two fp16 roundings: |err| <= 2^-10 |ref| + fp16 subnormal step
    assert np.all(np.abs(got - ref) <= np.abs(ref) * 2.0 ** -10 * 1.01 + 2.0 ** -24 * 4)


def test_silu_exhaustive_table_against_oracle():
    """tests/golden/silu_fp16_exhaustive.npy holds fp16(g / (1 + expf(-g))) for every fp16 g,
    evaluated on the GPU with the device expf and an IEEE division (make_silu_exhaustive.py).
    Against the oracle's numpy form it agrees everywhere (NaN bits included) except where
    expf and numpy's exp round differently and the fp32 quotient sits next to an fp16 rounding
    midpoint: three inputs, one fp16 ulp each. The GPU suite holds every SiLU in the library
    to this table."""
    table = np.load(os.path.join(GOLDEN, "silu_fp16_exhaustive.npy"))
    assert table.dtype == np.uint16 and table.shape == (65536,)
    g = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16)
    with np.errstate(over="ignore", invalid="ignore"):
        ref = O.silu_and_mul(g, np.ones_like(g)).view(np.uint16)
    diff = np.nonzero(table != ref)[0]
    assert len(diff) <= 3
    assert np.all(np.abs(table[diff].astype(np.int32) - ref[diff].astype(np.int32)) == 1)
    # SiLU(+0) = +0, SiLU(-0) = -0, SiLU(+inf) = +inf, SiLU(-inf) = NaN
    assert table[0x0000] == 0x0000 and table[0x8000] == 0x8000
    assert table[0x7C00] == 0x7C00 and np.isnan(table[0xFC00:0xFC01].view(np.float16))[0]


def test_topk_softmax_bruteforce_and_ties():
    r = np.random.default_rng(6)
    lg = r.standard_normal((50, 64)).astype(np.float32)
    lg[0, :] = 0.5                   # all tied -> lowest ids
    w, ids = O.topk_softmax(lg, 8)
    assert ids[0].tolist() == list(range(8))
    for t in range(50):
        order = sorted(range(64), key=lambda e: (-float(lg[t, e]), e))[:8]
        assert ids[t].tolist() == order
        p = np.exp(lg[t].astype(np.float64) - lg[t].max())
        sel = p[order] / p[order].sum()
        np.testing.assert_allclose(w[t], sel, rtol=1e-6)
    assert np.allclose(w.sum(1), 1.0, atol=1e-6)


def test_gather_reduce_closed_form():
    # 2 tokens, top_k 2, P = 4 rows; slot 3 missing
    out2 = np.array([[1, 2], [3, 4], [5, 6], [7, 8]], dtype=np.float16)
    sti = np.array([2, 0, 1, 4], dtype=np.int32)   # row 3 is padding (sentinel 4)
    tw = np.array([0.5, 0.25, 2.0, 1.0], dtype=np.float32)
    out = O.gather_reduce(out2, sti, tw, np.array([4], np.int32), 2)
    # token 0: slot0 row1 (3,4)*0.5 + slot1 row2 (5,6)*0.25 ; token 1: slot2 row0 (1,2)*2
    assert np.allclose(out, [[3 * .5 + 5 * .25, 4 * .5 + 6 * .25], [2.0, 4.0]])


def test_fma32_is_single_rounding():
    a = np.float32(1 + 2 ** -23)
    b = np.float32(1 - 2 ** -23)
    c = np.float32(-1.0)
    # exact a*b - 1 = -2^-46, representable; a separate multiply would round to 0
    assert O.fma32(a, b, c) == np.float32(-(2.0 ** -46))


@pytest.mark.parametrize("bits", [0x3F800000, 0x3F808000, 0x3F818000, 0x7F7FFFFF])
def test_bf16_rounding(bits):
    x = np.array([bits], np.uint32).view(np.float32)
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(O.f32_to_bf16_bits(x), ref)


@pytest.mark.parametrize("E,N,K,zp", [(1, 16, 128, True), (2, 32, 256, False), (3, 48, 384, True)])
def test_repack_fragments_bruteforce(E, N, K, zp):
    """Every nibble of row n, column k sits in block (n // 16, k // 128) of its tile, lane
    n % 16 + 16 * ((k % 128) // 32), nibble (k % 32) of that lane's 16 bytes (low nibble
    first): the fp8 MFMA B operand layout (lane l -> column l % 16, k = 32 (l // 16) + i).
    Row n's scale and zero-point for group g are metadata word (n % 16) G + g after tile
    n // 16's blocks (scale bits low, zero-point in bits 16..19, 8 without zero-points)."""
    r = np.random.default_rng(E * 1000 + N + K)
    G = K // 128
    nib = r.integers(0, 16, (E, N, K))
    w = O.pack_nibbles(nib)
    sc = r.uniform(0.005, 0.02, (E, N, G)).astype(np.float16)
    zz = r.integers(0, 16, (E, N, G))
    z = O.pack_zeros(zz) if zp else None
    f = O.repack_fragments(w, sc, z)
    assert f.shape == (E, N // 16, 17, 16 * G) and f.dtype == np.int32
    f = f.reshape(E, N // 16, 272 * G)
    blocks = f[:, :, :256 * G].reshape(E, N // 16, G, 64, 4)
    lane_nib = O.unpack_nibbles(blocks)            # (E, N/16, G, 64, 32)
    meta = f[:, :, 256 * G:].view(np.uint32)
    for e in range(E):
        for n in range(N):
            for k in range(K):
                lane = n % 16 + 16 * ((k % 128) // 32)
                assert lane_nib[e, n // 16, k // 128, lane, k % 32] == nib[e, n, k]
            for g in range(G):
                m = int(meta[e, n // 16, (n % 16) * G + g])
                assert m & 0xFFFF == int(sc[e, n, g].view(np.uint16))
                assert (m >> 16) == (int(zz[e, n, g]) if zp else 8)
    w2, sc2, zp2 = O.unrepack_fragments(f.reshape(E, N // 16, 17, 16 * G))
    assert np.array_equal(w2, w) and np.array_equal(sc2.view(np.uint16), sc.view(np.uint16))
    assert np.array_equal(zp2, zz if zp else np.full_like(zz, 8))


def test_repack_fragments_is_a_permutation_of_words():
    r = np.random.default_rng(7)
    w = r.integers(-2**31, 2**31, (4, 64, 512 // 8), dtype=np.int64).astype(np.int32)
    sc = np.ones((4, 64, 4), np.float16)
    f = O.repack_fragments(w, sc).reshape(4, 4, 272 * 4)
    G = 4
    assert np.array_equal(np.sort(f[:, :, :256 * G].ravel()), np.sort(w.ravel()))
    # a planted transposition of lane halves is caught by the inverse
    bad = f.copy()
    blk = bad[:, :, :256 * G].reshape(4, 4, G, 64, 4)
    blk[..., [0, 16], :] = blk[..., [16, 0], :]
    bad[:, :, :256 * G] = blk.reshape(4, 4, 256 * G)
    assert not np.array_equal(O.unrepack_fragments(bad.reshape(4, 4, 17, 64))[0], w)


def _swigluoai_f64(x16, alpha=1.702, limit=7.0):
    x = np.asarray(x16, np.float16).astype(np.float64)
    gate, up = x[..., 0::2], x[..., 1::2]
    g = np.minimum(gate, limit)
    u = np.clip(up, -limit, limit)
    return (u + 1.0) * g / (1.0 + np.exp(-alpha * g))


def test_swigluoai_against_float64_closed_form():
    """Within half an fp16 ulp (plus the fp32 intermediates' few ulps) of the float64 closed
    form, over values that cross both clamps."""
    r = np.random.default_rng(21)
    x = (r.standard_normal((64, 512)) * 6).astype(np.float16)
    got = O.swigluoai_and_mul(x).astype(np.float64)
    ref = _swigluoai_f64(x)
    ulp = np.spacing(np.abs(ref).astype(np.float16)).astype(np.float64)
    assert np.all(np.abs(got - ref) <= 0.5 * ulp + 1e-6 * np.abs(ref) + 1e-12)


def test_swigluoai_cases_and_planted_mistakes():
    # clamps: gate above 7 -> 7; up beyond +-7 -> +-7; up = -1 -> 0; gate = 0 -> 0
    x = np.array([[100, 0, 100, 100, 100, -100, 0, 5, 3, -1]], np.float16)
    got = O.swigluoai_and_mul(x).astype(np.float64)[0]
    s7 = 7.0 / (1.0 + np.exp(-1.702 * 7.0))
    exp = np.array([s7 * 1.0, s7 * 8.0, s7 * -6.0, 0.0, 0.0])
    assert np.allclose(got, exp, rtol=1e-3, atol=0)
    # mistakes the definition rules out: [gate | up] halves instead of interleaved pairs,
    # no clamp, the +1 dropped
    r = np.random.default_rng(22)
    x = (r.standard_normal((16, 256)) * 6).astype(np.float16)
    good = O.swigluoai_and_mul(x).astype(np.float64)
    halves = np.concatenate([x[:, :128], x[:, 128:]], axis=1)
    inter = np.empty_like(x)
    inter[:, 0::2], inter[:, 1::2] = x[:, :128], x[:, 128:]
    assert np.abs(O.swigluoai_and_mul(inter).astype(np.float64) - good).max() > 1e-1
    xf = x.astype(np.float64)
    no_clamp = (xf[:, 1::2] + 1) * xf[:, 0::2] / (1 + np.exp(-1.702 * xf[:, 0::2]))
    assert np.abs(no_clamp - good).max() > 1e-1
    no_plus1 = _swigluoai_f64(x) - np.minimum(xf[:, 0::2], 7.0) / (1 + np.exp(-1.702 * np.minimum(xf[:, 0::2], 7.0)))
    assert np.abs(no_plus1 - good).max() > 1e-1
    del halves


def test_e8m0_to_fp16_all_codes():
    """2^(s - 127): exact in fp16 for exponents -24..15, 0 below (2^-25 ties to even), +inf
    above and for the NaN code 255."""
    import math
    got = O.e8m0_to_fp16(np.arange(256)).astype(np.float64)
    for s_ in range(256):
        e = s_ - 127
        if e > 15:
            assert np.isinf(got[s_]) and got[s_] > 0
        elif e >= -24:
            assert got[s_] == math.ldexp(1.0, e), s_
        else:
            assert got[s_] == 0.0, s_


def test_convert_mxfp4_nibble_order_bruteforce():
    """Code k of row n is the low nibble of byte k / 2 for even k, the high one for odd k,
    and lands at nibble k % 8 of word k / 8."""
    r = np.random.default_rng(23)
    wp = r.integers(0, 256, (2, 4, 32), dtype=np.uint8)
    wp_s = r.integers(100, 140, (2, 4, 2), dtype=np.uint8)
    w, sc = O.convert_mxfp4(wp, wp_s)
    wu = w.view(np.uint32)
    for e in range(2):
        for n in range(4):
            for k in range(64):
                code = (int(wp[e, n, k // 2]) >> (4 * (k % 2))) & 0xF
                assert (int(wu[e, n, k // 8]) >> (4 * (k % 8))) & 0xF == code
    assert np.array_equal(sc, O.e8m0_to_fp16(wp_s))