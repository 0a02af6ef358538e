"""GPU parity of the individual gfx950 kernels against the CPU oracle, through the C ABI.

Bars: bit-exact for act-quant bytes/scales, dequant bytes, align indices and router ids;
max|out - ref| / max|ref| <= 1e-2 for fp32-accumulated GEMM outputs.
"""
import os

import numpy as np
import pytest
import torch

import oracle as O
import w4a8_fp8_wmma as W

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


def rng(seed):
    return np.random.default_rng(seed)


# --------------------------------------------------------------------------- #
# act-quant / dequant / silu
# --------------------------------------------------------------------------- #
@pytest.mark.parametrize("k8", [False, True])
@pytest.mark.parametrize("K", [128, 512, 2048, 4096])
def test_act_quant_bit_exact(k8, K):
    r = rng(K)
    x = (r.standard_normal((67, K)) * np.exp2(r.integers(-8, 8, (67, 1)))).astype(np.float16)
    x[0] = 0
    x[1] = np.float16(6e-8)
    x[2, ::7] = np.float16(-65504)
    q, s = W.act_quant_fp8(torch.from_numpy(x).to(DEV), k8_interleave=k8)
    qo, so = O.act_quant(x)
    if k8:   # byte p of each 8-block holds k = {0,2,4,6,1,3,5,7}[p]
        perm = np.array([0, 2, 4, 6, 1, 3, 5, 7])
        qo = qo.reshape(67, K // 8, 8)[:, :, perm].reshape(67, K)
    assert np.array_equal(s.cpu().numpy(), so)
    assert np.array_equal(q.cpu().numpy(), qo)


@pytest.mark.parametrize("K", [512, 2048, 4096])
def test_act_quant_nan_and_inf_rows(K):
    """The absmax skips NaNs (fmaxf, as the reference kernel) and takes infinities: rows with
    NaNs get the scale of their finite values and the same bytes as the oracle at every
    non-NaN position; a row holding an infinity gets an infinite scale. (The kernels find
    the maximum on the magnitude bits and take an exact pass only for a row with a NaN.)"""
    r = rng(K + 7)
    x = (r.standard_normal((6, K)) * 5).astype(np.float16)
    x[0, 3] = np.nan
    x[1, K - 1] = np.nan
    x[1, :K // 2] *= 40
    x[2, ::5] = np.nan
    x[3, 9] = np.inf
    x[4, K // 3] = -np.inf
    q, s = W.act_quant_fp8(torch.from_numpy(x).to(DEV), k8_interleave=False)
    q, s = q.cpu().numpy(), s.cpu().numpy()
    xf = x.astype(np.float32)
    amax = np.nanmax(np.abs(xf), axis=1)
    s_ref = np.maximum(amax / np.float32(448.0), np.float32(1e-8)).astype(np.float32)
    assert np.array_equal(s, s_ref)
    for row in range(3):   # NaN rows: finite scale, oracle bytes where the input is a number
        finite = ~np.isnan(xf[row])
        inv = np.float32(1.0) / s_ref[row]
        ref = O.e4m3_encode((xf[row] * inv).astype(np.float32))
        assert np.array_equal(q[row][finite], ref[finite])
    assert np.isinf(s[3]) and np.isinf(s[4]) and np.isfinite(s[5])
    qo, so = O.act_quant(x[5:6])
    assert np.array_equal(q[5:6], qo) and np.array_equal(s[5:6], so)


@pytest.mark.parametrize("K", [512, 2048])
def test_act_quant_misaligned_rows_bit_exact(K):
    """Rows whose start is not 16-byte aligned take the element-wise loads: same bytes."""
    r = rng(K + 1)
    x = (r.standard_normal((9, K)) * 3).astype(np.float16)
    buf = torch.zeros(9 * K + 4, dtype=torch.float16, device=DEV)
    buf[4:].copy_(torch.from_numpy(x.reshape(-1)).to(DEV))
    xv = buf[4:].view(9, K)                     # data pointer 8 bytes past an aligned start
    assert xv.data_ptr() % 16 == 8
    q, s = W.act_quant_fp8(xv, k8_interleave=False)
    qo, so = O.act_quant(x)
    assert np.array_equal(s.cpu().numpy(), so)
    assert np.array_equal(q.cpu().numpy(), qo)


@pytest.mark.parametrize("asym", [True, False])
def test_dequant_bit_exact_all_zero_points(asym):
    r = rng(5)
    E, N, K, g = 3, 64, 1024, 128
    w = r.integers(-2**31, 2**31, (E, N, K // 8), dtype=np.int64).astype(np.int32)
    z = r.integers(-2**31, 2**31, (E, N // 8, K // g), dtype=np.int64).astype(np.int32) if asym else None
    got = W.dequant_fp8(torch.from_numpy(w).to(DEV), g,
                        None if z is None else torch.from_numpy(z).to(DEV))
    ref = O.dequant_codes(w, z, g)
    assert np.array_equal(got.cpu().numpy(), ref)
    # every (nibble, zp) pair occurs
    nib = O.unpack_nibbles(w)
    if asym:
        zp = np.repeat(O.unpack_zeros(z, N), g, -1)
        assert np.unique(nib.astype(np.int64) * 16 + zp).size == 256


def test_dequant_e2m1_bit_exact():
    r = rng(6)
    w = r.integers(-2**31, 2**31, (2, 16, 32), dtype=np.int64).astype(np.int32)
    got = W.dequant_fp8(torch.from_numpy(w).to(DEV), 32, None, weight_is_e2m1=True)
    assert np.array_equal(got.cpu().numpy(), O.dequant_codes(w, None, 32, e2m1=True))


def test_silu_every_fp16_input_bit_exact_to_exact_form():
    """SiLU(gate) * 1 for all 65536 fp16 gates == the exact form's table bit for bit
    (tests/golden/silu_fp16_exhaustive.npy: fp16(g / (1 + expf(-g))), device expf, IEEE
    division). The library evaluates SiLU with the hardware exp2 and reciprocal and falls back
    to the exact form only for results below the fp16 normal range and non-finite inputs, so
    this covers every input of every SiLU epilogue (they share silu_mul_h)."""
    table = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                                 "silu_fp16_exhaustive.npy"))
    gate = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16).reshape(256, 256)
    out = torch.empty((256, 256), dtype=torch.float16, device=DEV)
    W.silu_and_mul(out, torch.from_numpy(np.concatenate([gate, np.ones_like(gate)], 1)).to(DEV))
    got = out.cpu().numpy().view(np.uint16).reshape(-1)
    bad = np.nonzero(got != table)[0]
    assert len(bad) == 0, f"{len(bad)} inputs differ, first gates {gate.reshape(-1)[bad[:8]]}"
    # the up factor multiplies the fp16 SiLU once more (hmul): up = -2 negates and doubles
    W.silu_and_mul(out, torch.from_numpy(np.concatenate(
        [gate, np.full_like(gate, -2.0)], 1)).to(DEV))
    ref = (table.view(np.float16).astype(np.float32) * np.float32(-2.0)).astype(np.float16)
    got2 = out.cpu().numpy().reshape(-1)
    num = ~np.isnan(ref)
    assert np.array_equal(got2[num].view(np.uint16), ref[num].view(np.uint16))
    assert np.all(np.isnan(got2[~num]))


def test_silu_and_mul_close():
    r = rng(7)
    x = (r.standard_normal((33, 2 * 256)) * 3).astype(np.float16)
    out = torch.empty((33, 256), dtype=torch.float16, device=DEV)
    W.silu_and_mul(out, torch.from_numpy(x).to(DEV))
    ref = O.silu_and_mul(x[:, :256], x[:, 256:])
    diff = np.abs(out.cpu().numpy().astype(np.float32) - ref.astype(np.float32))
    # expf may differ from numpy exp by an ulp -> at most one fp16 ulp of difference
    assert np.all(diff <= np.abs(ref.astype(np.float32)) * 2.0 ** -10 * 2.01 + 2.0 ** -24 * 4)


# --------------------------------------------------------------------------- #
# router and align
# --------------------------------------------------------------------------- #
@pytest.mark.parametrize("T,E,k", [(1, 256, 8), (32, 256, 8), (1000, 128, 8), (7, 64, 1)])
def test_topk_softmax(T, E, k):
    r = rng(T + E)
    lg = r.standard_normal((T, E)).astype(np.float32)
    lg[0, :] = 0.25   # ties resolve to the lowest ids
    w, ids = W.fused_topk(None, torch.from_numpy(lg).to(DEV), k, True)
    wo, io = O.topk_softmax(lg, k)
    assert np.array_equal(ids.cpu().numpy(), io)
    np.testing.assert_allclose(w.cpu().numpy(), wo, rtol=2e-5, atol=1e-7)


@pytest.mark.parametrize("T,k,E,bm", [(1, 8, 256, 16), (32, 8, 256, 16), (32, 8, 256, 8),
                                      (128, 8, 256, 64), (4096, 8, 256, 64), (2048, 8, 128, 64),
                                      (200, 4, 1024, 32), (1, 1, 1, 1),
                                      (4096, 8, 1024, 64)])   # chunk counts beyond one LDS
def test_align_bit_exact(T, k, E, bm):
    r = rng(T * 7 + E)
    ids = np.stack([r.permutation(E)[:k] for _ in range(T)]).astype(np.int32)
    sti, eid, ntp = W.moe_align_block_size(torch.from_numpy(ids).to(DEV), bm, E)
    so, eo, no = O.moe_align(ids, bm, E)
    assert int(ntp.item()) == int(no[0])
    assert np.array_equal(sti.cpu().numpy(), so)
    assert np.array_equal(eid.cpu().numpy(), eo)


def test_align_zipf_skew_and_expert_map():
    r = rng(8)
    T, k, E, bm = 4096, 8, 256, 64
    p = 1.0 / np.arange(1, E + 1) ** 1.1
    lg = np.log(p / p.sum())[r.permutation(E)] + r.gumbel(size=(T, E))
    ids = np.argsort(-lg, axis=1)[:, :k].astype(np.int32)
    emap = np.where(np.arange(E) % 3 == 0, np.arange(E) // 3, -1).astype(np.int32)
    for em in (None, emap):
        tm = None if em is None else torch.from_numpy(em).to(DEV)
        sti, eid, ntp = W.moe_align_block_size(torch.from_numpy(ids).to(DEV), bm, E, tm)
        so, eo, no = O.moe_align(ids, bm, E, expert_map=em)
        assert int(ntp.item()) == int(no[0])
        assert np.array_equal(sti.cpu().numpy(), so) and np.array_equal(eid.cpu().numpy(), eo)


@pytest.mark.parametrize("numel", [512, 1024, 32768, 65536 + 37])
def test_align_degenerate_ids(numel):
    """Every slot on one expert (one wave holds 64 equal ids), repeated ids inside a token,
    and ids outside [0, E) (dropped): the per-wave ballot ranks against the oracle."""
    r = rng(numel)
    E, k, bm = 256, 8, 64
    cases = [np.full(numel, 17, np.int32),
             r.integers(0, 3, numel).astype(np.int32),
             np.where(r.random(numel) < 0.1, -1,
                      np.where(r.random(numel) < 0.05, E + 5, r.integers(0, E, numel))).astype(np.int32)]
    for ids in cases:
        ids2 = ids.reshape(-1, 1) if numel % k else ids.reshape(-1, k)
        sti, eid, ntp = W.moe_align_block_size(torch.from_numpy(ids2).to(DEV), bm, E)
        so, eo, no = O.moe_align(ids2, bm, E)
        assert int(ntp.item()) == int(no[0])
        assert np.array_equal(sti.cpu().numpy(), so)
        assert np.array_equal(eid.cpu().numpy(), eo)


# --------------------------------------------------------------------------- #
# grouped GEMMs
# --------------------------------------------------------------------------- #
def make_case(seed, T, E, N, K, k, g, asym=True):
    r = rng(seed)
    nib = r.integers(0, 16, (E, N, K))
    zp = r.integers(0, 16, (E, N, K // g))
    w = O.pack_nibbles(nib)
    z = O.pack_zeros(zp) if asym else None
    sc = r.uniform(0.005, 0.02, (E, N, K // g)).astype(np.float16)
    x = r.standard_normal((T, K)).astype(np.float16)
    ids = np.stack([r.permutation(E)[:k] for _ in range(T)]).astype(np.int32)
    tw = r.random((T, k)).astype(np.float32)
    return x, w, z, sc, ids, tw


def to_dev(*arrs):
    return [None if a is None else torch.from_numpy(np.ascontiguousarray(a)).to(DEV) for a in arrs]


GEMM_CASES = [
    # (T, E, N, K, top_k, block_m, g)   reference sweep shapes (test_moe_correctness.py:149-156)
    (64, 8, 128, 256, 2, 16, 128),
    (32, 4, 256, 512, 2, 32, 128),
    (128, 8, 512, 1024, 2, 64, 128),
    (1, 8, 512, 1024, 2, 16, 128),
    (16, 16, 256, 256, 4, 16, 32),
    (64, 8, 128, 256, 2, 16, 32),
    (40, 8, 256, 2048, 8, 128, 128),
    # K % 512 != 0 keeps these on the streamed-K tiles: 128-row (block_m 128) and 64-row tiles
    (96, 8, 256, 768, 2, 128, 128),
    (200, 4, 384, 1280, 4, 64, 128),
    # K / 128 = 36 is past both streamed-K tables: the general tiles (and gemv falls back)
    (24, 4, 256, 4608, 2, 64, 128),
]


@pytest.mark.parametrize("kernel", ["scalar", "wmma", "gemv"])
@pytest.mark.parametrize("asym", [True, False])
@pytest.mark.parametrize("case", GEMM_CASES)
def test_moe_gemm_vs_oracle(kernel, asym, case):
    T, E, N, K, k, bm, g = case
    if kernel == "gemv" and bm > 64:
        pytest.skip("gemv block_m <= 64 (reference contract)")
    x, w, z, sc, ids, _ = make_case(hash(case) % 1000, T, E, N, K, k, g, asym)
    sti, eid, ntp = O.moe_align(ids, bm, E)
    xd, wd, zd, scd, stid, eidd, ntpd = to_dev(x, w, z, sc, sti, eid, ntp)
    out = W.mmq_fp8_moe_gemm(xd, wd, scd, stid, eidd, ntpd, k, bm, kernel=kernel, w_zeros=zd)
    ref, valid = O.grouped_gemm_padded(x, w, sc, z, sti, eid, ntp, k, bm)
    got = out.cpu().numpy()[valid]
    assert maxrel(got, ref[valid]) <= REL_TOL


@pytest.mark.parametrize("kernel", ["scalar", "wmma", "gemv"])
def test_raw_nibble_zero_point_arithmetic_exact(kernel):
    """Every (nibble, zero-point) pair through the GEMM kernels' own int4 arithmetic (raw
    nibbles as e4m3 n * 2^-9 with the z * sum(a) term deferred, or the scalar kernel's table),
    where the sums are exact: token t is one-hot at k = 8 t (e4m3 448 after act-quant),
    column c = 16 z + o has zero-point z and nibble (t + o) % 16 at that k, and the scales
    are powers of two, so out[t, c] = e4m3(n - z) * s[c, t // 16] (the dequant table,
    pinned exhaustively) exactly in fp16. A swapped nibble order, a wrong zero-point or a
    scale from the wrong group changes at least one of the 16 x 16 pairs."""
    r = rng(77)
    T, N, K, g = 64, 256, 512, 128
    t = np.arange(T)
    c = np.arange(N)
    z_of, o_of = c // 16, c % 16
    nib = r.integers(0, 16, (1, N, K))
    nib[0][:, 8 * t] = (t[None, :] + o_of[:, None]) % 16
    zp = np.repeat(z_of[:, None], K // g, axis=1)[None]
    sc = np.exp2(r.integers(-8, -1, (1, N, K // g))).astype(np.float16)
    x = np.zeros((T, K), np.float16)
    x[t, 8 * t] = 1.0
    w, z = O.pack_nibbles(nib), O.pack_zeros(zp)
    ids = np.zeros((T, 1), np.int32)
    sti, eid, ntp = O.moe_align(ids, 16, 1)
    xd, wd, zd, scd, stid, eidd, ntpd = to_dev(x, w, z, sc, sti, eid, ntp)
    out = W.mmq_fp8_moe_gemm(xd, wd, scd, stid, eidd, ntpd, 1, 16, kernel=kernel, w_zeros=zd)
    got = out.cpu().numpy()
    rows = np.empty(T, np.int64)
    rows[sti[:T]] = np.arange(T)           # padded row of token t (all of them are real here)
    nv = nib[0][:, 8 * t].T                 # (T, N) nibble at the token's k
    want = np.empty((T, N), np.float32)
    for zz in range(16):
        tab = O.e4m3_decode(O.dequant_table(zz)).astype(np.float32)
        cols = z_of == zz
        want[:, cols] = tab[nv[:, cols]] * sc[0][cols][:, t // 16].T.astype(np.float32)
    assert np.array_equal(got[rows].astype(np.float32), want.astype(np.float16).astype(np.float32))


E2M1_CASES = [
    # (T, E, N, K, top_k, block_m, g): mxfp4's block of 32, 64 and 128-wide groups
    (64, 8, 128, 256, 2, 16, 32),
    (40, 8, 256, 1024, 4, 64, 32),
    (32, 4, 256, 512, 2, 32, 64),
    (128, 8, 512, 1024, 2, 128, 128),
]


@pytest.mark.parametrize("case", E2M1_CASES)
def test_e2m1_fp4_tiles_equal_scalar(case):
    """E2M1 weights on the matrix-core tiles take fp4 MFMA operands (the f8f6f4 MFMA decodes
    the raw codes; one MFMA per K group of 32, 64 or 128, each folded with its scale). Both
    the tiles and the scalar golden kernel match the oracle's E2M1 codebook GEMM
    (tile_config.h:59-71), and each other to fp32 summation order: e4m3 x e2m1 products
    span more than fp32's 24 bits, so the MFMA's internal sum and the scalar fmaf chain may
    round differently, within 2e-3 of the output's range."""
    T, E, N, K, k, bm, g = case
    r = rng(sum(case) + 7)
    codes = r.integers(0, 16, (E, N, K))
    w = O.pack_nibbles(codes)
    sc = r.uniform(0.005, 0.02, (E, N, K // g)).astype(np.float16)
    x = r.standard_normal((T, K)).astype(np.float16)
    ids = np.stack([r.permutation(E)[:k] for _ in range(T)]).astype(np.int32)
    sti, eid, ntp = O.moe_align(ids, bm, E)
    xd, wd, scd, stid, eidd, ntpd = to_dev(x, w, sc, sti, eid, ntp)
    outs = {kern: W.mmq_fp8_moe_gemm(xd, wd, scd, stid, eidd, ntpd, k, bm, kernel=kern,
                                     weight_is_e2m1=True) for kern in ("scalar", "wmma")}
    ref, valid = O.grouped_gemm_padded(x, w, sc, None, sti, eid, ntp, k, bm, e2m1=True)
    got = outs["wmma"].cpu().numpy()[valid]
    assert maxrel(outs["scalar"].cpu().numpy()[valid], ref[valid]) <= REL_TOL
    assert maxrel(got, ref[valid]) <= REL_TOL
    assert maxrel(got, outs["scalar"].cpu().numpy()[valid]) <= 2e-3


@pytest.mark.parametrize("case", [(32, 8, 512, 2048, 8, 16, 128), (24, 16, 256, 512, 4, 16, 128),
                                  (9, 8, 384, 1024, 2, 32, 128), (40, 8, 256, 1536, 2, 64, 128),
                                  (8, 8, 256, 4096, 2, 16, 128), (33, 16, 512, 4096, 8, 64, 128)])
def test_gemv_in_kernel_quant_matches_prequant(case):
    """With no workspace the decode GEMV quantises its rows in registers; that path must give
    the bytes act_quant gives, so both calls agree bit for bit (K = 4096: eight groups a
    wave, the second weight chunk issued after the conversion)."""
    from w4a8_fp8_wmma._lib import lib as L
    from w4a8_fp8_wmma._ops import _ptr, _stream, _workspace
    T, E, N, K, k, bm, g = case
    x, w, z, sc, ids, _ = make_case(sum(case), T, E, N, K, k, g)
    sti, eid, ntp = O.moe_align(ids, bm, E)
    xd, wd, zd, scd, stid, eidd, ntpd = to_dev(x, w, z, sc, sti, eid, ntp)
    P = sti.size
    outs = []
    for with_ws in (True, False):
        out = torch.full((P, N), float("nan"), dtype=torch.float16, device=DEV)
        ws = _workspace(L.w4a8_moe_gemm_workspace_size(T, K), xd.device)
        rc = L.w4a8_mmq_fp8_moe_gemm(
            _ptr(xd), T, K, _ptr(wd), _ptr(scd), _ptr(zd), E, N, g, _ptr(stid), P, _ptr(eidd),
            _ptr(ntpd), k, bm, 7, 0, _ptr(out), ws.data_ptr() if with_ws else None,
            ws.numel() if with_ws else 0, _stream(xd))
        assert rc == 0, L.w4a8_last_error()
        outs.append(out)
    torch.cuda.synchronize()
    valid = torch.from_numpy((np.arange(P) < ntp[0]) & (sti < T * k)).to(DEV)
    assert torch.equal(outs[0][valid], outs[1][valid])
    ref, vmask = O.grouped_gemm_padded(x, w, sc, z, sti, eid, ntp, k, bm)
    assert maxrel(outs[1].cpu().numpy()[vmask], ref[vmask]) <= REL_TOL


@pytest.mark.parametrize("case", [(64, 8, 256, 256, 2, 16, 128), (128, 8, 512, 512, 2, 64, 128),
                                  (256, 4, 1024, 2048, 2, 128, 128), (16, 16, 256, 256, 4, 16, 32),
                                  (512, 16, 1024, 2048, 8, 64, 128), (200, 8, 768, 1536, 4, 64, 128)])
def test_gemm1_silu_fused_bit_exact_to_unfused(case):
    """Fused gemm1+SiLU == gemm1 fp16 store + silu_and_mul, bit for bit
    (test_moe_experts.py:283-315). Shapes with K % 512 == 0, K <= 2048, block_m % 64 == 0
    run the activation-resident prefill tiles (the whole layer's gemm1), the others the
    streamed-K and small tiles."""
    T, E, N, K, k, bm, g = case
    x, w, z, sc, ids, _ = make_case(sum(case), T, E, N, K, k, g)
    sti, eid, ntp = O.moe_align(ids, bm, E)
    xd, wd, zd, scd, stid, eidd, ntpd = to_dev(x, w, z, sc, sti, eid, ntp)
    out1 = W.mmq_fp8_moe_gemm(xd, wd, scd, stid, eidd, ntpd, k, bm, kernel="wmma", w_zeros=zd)
    unf = torch.empty((out1.shape[0], N // 2), dtype=torch.float16, device=DEV)
    W.silu_and_mul(unf, out1)
    fused = W.mmq_fp8_moe_gemm1_silu(xd, wd, scd, stid, eidd, ntpd, k, bm, kernel="wmma",
                                      w_zeros=zd)
    valid = torch.from_numpy(
        (np.arange(sti.size) < ntp[0]) & (sti < T * k)).to(DEV)
    assert torch.equal(fused[valid], unf[valid])
    # and close to the oracle
    ref, vmask = O.grouped_gemm_padded(x, w, sc, z, sti, eid, ntp, k, bm)
    h = O.silu_and_mul(ref[:, :N // 2], ref[:, N // 2:])
    assert maxrel(fused.cpu().numpy()[vmask], h[vmask]) <= REL_TOL


@pytest.mark.parametrize("kernel", ["scalar", "wmma", "gemv"])
def test_scatter_vs_oracle(kernel):
    T, E, N, K, k, bm, g = 24, 8, 256, 512, 4, 16, 128
    x, w, z, sc, ids, tw = make_case(41, T, E, N, K, k, g)
    sti, eid, ntp = O.moe_align(ids, bm, E)
    P = sti.size
    h = rng(42).standard_normal((P, K)).astype(np.float16)
    out = torch.zeros((T, N), dtype=torch.float32, device=DEV)
    hd, wd, zd, scd, stid, eidd, ntpd, twd = to_dev(h, w, z, sc, sti, eid, ntp, tw.reshape(-1))
    W.mmq_fp8_moe_gemm_scatter(hd, wd, scd, stid, eidd, ntpd, twd, out, k, bm, kernel=kernel,
                               w_zeros=zd)
    ref = O.gemm_scatter(h, w, sc, z, sti, eid, ntp, tw.reshape(-1), np.zeros((T, N), np.float32),
                         k, bm)
    assert maxrel(out.cpu().numpy(), ref) <= REL_TOL


def test_gather_reduce_bit_exact():
    r = rng(50)
    T, k, E, bm, N = 33, 8, 64, 16, 384
    ids = np.stack([r.permutation(E)[:k] for _ in range(T)]).astype(np.int32)
    sti, eid, ntp = O.moe_align(ids, bm, E)
    out2 = r.standard_normal((sti.size, N)).astype(np.float16)
    tw = r.random(T * k).astype(np.float32)
    o2d, stid, twd, ntpd = to_dev(out2, sti, tw, ntp)
    got = W.mmq_fp8_moe_gather_reduce(o2d, stid, twd, ntpd, k)
    ref = O.gather_reduce(out2, sti, tw, ntp, k)
    assert np.array_equal(got.cpu().numpy(), ref)


@pytest.mark.parametrize("kernel", ["reference_scalar", "prefill_wmma", "decode_gemv",
                                    "prefill_wmma_ashuffle"])
def test_dense_config1(kernel):
    """Config 1: dense M=16, N=1024, K=2048 AWQ g128 with zero-points."""
    r = rng(1001)
    M, N, K, g = 16, 1024, 2048, 128
    x = torch.randn(M, K, generator=torch.Generator().manual_seed(1001)).to(torch.bfloat16)
    x16 = x.to(torch.float16).numpy()
    nib = r.integers(0, 16, (N, K))
    zp = r.integers(0, 16, (N, K // g))
    w = O.pack_nibbles(nib)
    z = O.pack_zeros(zp)
    sc = r.uniform(0.005, 0.02, (N, K // g)).astype(np.float16)
    xd, wd, zd, scd = to_dev(x16, w, z, sc)
    out = W.mmq_fp8_gemm(xd, wd, scd, kernel=kernel, w_zeros=zd)
    ref = O.dense_gemm(x16, w, sc, z)
    assert maxrel(out.cpu().numpy(), ref) <= REL_TOL
