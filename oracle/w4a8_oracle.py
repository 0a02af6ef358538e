"""numpy restatement of the reference W4A8 MoE arithmetic (TEST INFRASTRUCTURE ONLY).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import this module, and only as the checker. The product never calls it.

All citations are into patcarter883/rdna4-vllm:
  * ``moe_kernel.hip``      = w4a8_fp8_wmma/moe_kernel.hip
  * ``tile_config.h``       = w4a8_fp8_wmma/tile_config.h
  * ``moe_gemm_tiled.h``    = w4a8_fp8_wmma/moe_gemm_tiled.h
  * ``moe_experts.py``      = w4a8_fp8_wmma/w4a8_fp8_wmma/moe_experts.py
  * ``test_moe_experts.py`` = w4a8_fp8_wmma/test_moe_experts.py
  * ``test_moe_correctness.py`` / ``test_correctness.py`` likewise under w4a8_fp8_wmma/
  * ``moe_wna16.py``        = patches/moe_wna16.py
  * ``dense_kernel.hip``    = w4a8_fp8_wmma/w4a8_fp8_wmma_kernel.hip

Rounding points follow the kernels: fp32 per-group partial sums (exact here: fp8 x int4
products summed in float64 are exact, then rounded once to fp32), a sequential fp32
fused multiply-add over groups, fp16 stores, fp32 reduce with ``j`` ascending.
"""
from __future__ import annotations

import numpy as np

E4M3_MAX = np.float32(448.0)
ACT_SCALE_FLOOR = np.float32(1e-8)   # moe_kernel.hip:117-118 (`if (s < 1e-8f) s = 1e-8f`)
PACK_FACTOR = 8

# How every function below is pinned (see tests/test_oracle_*.py).
PINNING = {
    "e4m3_encode": "exhaustive over all 65536 fp16 bit patterns + 2^20 random fp32 vs "
                   "torch.float8_e4m3fn (library cast); RNE ties and subnormals",
    "e4m3_decode": "all 256 codes vs torch.float8_e4m3fn -> float32",
    "dequant_codes": "exhaustive 16 nibbles x 16 zero-points vs torch cast of (n - z); "
                     "E2M1 table vs the OCP codebook",
    "act_quant": "closed form with torch ops (reciprocal multiply + torch cast) on random "
                 "and edge rows; invariants |q*s - x| <= half-ulp bound",
    "moe_align": "brute-force pure-Python restatement on tiny inputs + invariants "
                 "(permutation, single-expert blocks, sentinel padding, ntp formula)",
    "grouped_run / grouped_gemm_padded": "float64 dense matmul of dequantised weights "
                                        "(independent formulation) + planted-mistake checks",
    "silu_and_mul": "torch.nn.functional.silu in float64 within fp16 half-ulp",
    "gather_reduce": "closed form on hand-built inputs",
    "topk_softmax": "brute force sort + float64 softmax; tie-break on equal logits",
    "awq_to_op_layout / convert_awq_tensor / wna16_to_op_layout": "dequant equality "
        "against the unpacked ground truth (reference test property) + round trips",
    "moe_layer": "float64 un-quantised MoE within the fp8 quantisation error bound; "
                 "composition equals the per-stage oracle chain; biases: closed form on a "
                 "zero-weight layer and the per-stage chain with torch fp16 adds; "
                 "swigluoai with biases: float64 un-quantised layer (moe_layer_f64) within "
                 "the fp8 error, planted bias / gate-up-layout mistakes caught",
    "expert_weights_f64": "equals the e4m3 byte round trip E4M3_TO_F64[dequant_codes] on "
                           "random weights, sym and asym (exhaustive table test covers all "
                           "256 nibble/zero-point pairs)",
    "swigluoai_and_mul": "float64 closed form within fp16 half-ulp; the clamp and interleave "
                         "cases by hand; planted mistakes (halves instead of interleave, no "
                         "clamp, +1 dropped) must fail",
    "e8m0_to_fp16": "all 256 codes against exact powers of two (math.ldexp) and fp16's "
                    "normal/subnormal/overflow limits",
    "convert_mxfp4": "per-element brute force of the nibble order on random bytes; scales "
                     "through e8m0_to_fp16",
    "repack_fragments": "per-element brute force of the layout definition on tiny shapes "
                        "(nibble of row n, k lands in lane n % 16 + 16 * ((k % 128) // 32); "
                        "scale and zero-point of (n, g) in metadata word (n % 16) G + g of "
                        "tile n / 16); inverse restores the op layout exactly",
}

# --------------------------------------------------------------------------- #
# fp8 e4m3 (OCP e4m3fn: bias 7, max 448, no inf, 0x7F/0xFF = NaN)
# --------------------------------------------------------------------------- #


def _e4m3_table() -> np.ndarray:
    c = np.arange(256)
    sign = np.where(c & 0x80, -1.0, 1.0)
    exp = (c >> 3) & 0xF
    man = c & 0x7
    val = np.where(exp == 0, man * 2.0 ** -9, (1.0 + man / 8.0) * 2.0 ** (exp - 7.0))
    val = sign * val
    val[(c & 0x7F) == 0x7F] = np.nan
    return val


E4M3_TO_F64 = _e4m3_table()
E4M3_TO_F32 = E4M3_TO_F64.astype(np.float32)


def e4m3_decode(codes) -> np.ndarray:
    """e4m3 byte -> float32 (tile_config.h:39-41 `__builtin_amdgcn_cvt_f32_fp8`)."""
    return E4M3_TO_F32[np.asarray(codes, dtype=np.uint8)]


def e4m3_encode(x) -> np.ndarray:
    """float32 -> e4m3 byte, round-to-nearest-even, NaN (0x7F|sign) at |x| >= 480 or
    after rounding past 448 (tile_config.h:35-38 `__builtin_amdgcn_cvt_pk_fp8_f32`)."""
    x = np.asarray(x, dtype=np.float32)
    bits = x.view(np.uint32)
    sign = ((bits >> 31) & 1).astype(np.uint8) << 7
    a = np.abs(x).astype(np.float64)
    out = np.zeros(x.shape, dtype=np.int64)
    bad = ~np.isfinite(a) | (a >= 480.0)
    sub = (a < 2.0 ** -6) & ~bad
    out[sub] = np.rint(a[sub] * 512.0).astype(np.int64)        # m * 2^-9, m in 0..8
    nrm = ~sub & ~bad
    f, ex = np.frexp(a[nrm])                                    # a = f * 2^ex, f in [0.5,1)
    ms = np.rint(f * 16.0).astype(np.int64)                     # 1.mmm * 8 in [8,16]
    carry = ms == 16
    ms[carry] = 8
    ex = ex + carry
    code = ((ex - 1 + 7) << 3) | (ms - 8)
    code[(ex - 1 + 7) > 15] = 0x7F
    out[nrm] = code
    out[bad] = 0x7F
    out = np.minimum(out, 0x7F)
    return (out.astype(np.uint8) | sign).astype(np.uint8)


# --------------------------------------------------------------------------- #
# fp16 / bf16 helpers
# --------------------------------------------------------------------------- #


def f32_to_bf16_bits(x) -> np.ndarray:
    """float32 -> bfloat16 bit pattern, round-to-nearest-even (torch's `.to(bfloat16)`)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    b = x.view(np.uint32).astype(np.uint64)
    rounded = (b + 0x7FFF + ((b >> 16) & 1)) >> 16
    nan = np.isnan(x)
    rounded[nan] = (b[nan] >> 16) | 0x40
    return rounded.astype(np.uint16)


def bf16_bits_to_f32(b) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint32) << 16).view(np.float32)


def fma32(a, b, c) -> np.ndarray:
    """fp32 fused multiply-add: the kernels' `x += p * s` contracts to v_fma_f32."""
    return (np.asarray(a, np.float64) * np.asarray(b, np.float64)
            + np.asarray(c, np.float64)).astype(np.float32)


# --------------------------------------------------------------------------- #
# int4 unpack and int4 -> fp8 dequant
# --------------------------------------------------------------------------- #

# OCP E2M1 codebook (tile_config.h:59-63; moe_kernel.hip:73-77)
E2M1_LUT = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0,
                     -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0], dtype=np.float32)


def unpack_nibbles(w_packed) -> np.ndarray:
    """(..., K/8) int32 -> (..., K) uint8; nibble j of word w is k = 8w + j, low nibble
    first (moe_kernel.hip:181-182 `(word >> ((k % 8) * 4)) & 0xF`)."""
    w = np.asarray(w_packed).astype(np.int64) & 0xFFFFFFFF
    shifts = np.arange(8, dtype=np.int64) * 4
    nib = (w[..., None] >> shifts) & 0xF
    return nib.reshape(*w.shape[:-1], w.shape[-1] * 8).astype(np.uint8)


def pack_nibbles(nib) -> np.ndarray:
    """(..., K) ints in 0..15 -> (..., K/8) int32 (inverse of unpack_nibbles;
    test_moe_correctness.py:27-33 `pack_uint4`)."""
    nib = np.asarray(nib).astype(np.int64) & 0xF
    K = nib.shape[-1]
    nib = nib.reshape(*nib.shape[:-1], K // 8, 8)
    w = np.zeros(nib.shape[:-1], dtype=np.int64)
    for j in range(8):
        w |= nib[..., j] << (4 * j)
    return w.astype(np.uint32).view(np.int32)


FRAG_TILE_WORDS_PER_GROUP = 272    # per 16-row tile and K group: 256 fragment + 16 metadata words


def repack_fragments(w_packed, scales, w_zeros=None) -> np.ndarray:
    """Op layout (E, N, K/8) int32, scales (E, N, K/128) fp16 and zero-points
    (E, N/8, K/128) int32 or None -> fragment layout (E, N/16, 17, 16 K/128) int32 (tile t:
    [..., :16, :] its weight blocks, [..., 16, :] its metadata).

    Not a reference function: the gfx950 kernels' load-time layout. 16-row tile t of expert e
    is G = K/128 blocks of 1 KB, then its metadata, G * 16 words. Block (e, t, g) lane l
    (16 bytes = 4 words) holds row n = 16t + l % 16, words 16g + 4 (l // 16) .. +3, i.e.
    k in [128g + 32 (l // 16), +32): the raw-nibble fp8 MFMA B operand of lane l. Metadata
    word r * G + g of the tile is row 16t + r, group g: its fp16 scale's bits in bits 0..15
    and its zero-point (8 when there are none) in bits 16..19."""
    w = np.asarray(w_packed)
    E, N, K8 = w.shape
    G = K8 // 16
    assert N % 16 == 0 and K8 % 16 == 0
    # (E, t, c, g, q, word) -> (E, t, g, q, c, word); lane = 16 q + c
    v = w.reshape(E, N // 16, 16, G, 4, 4).transpose(0, 1, 3, 4, 2, 5).reshape(E, N // 16, G * 256)
    sb = np.asarray(scales, dtype=np.float16).view(np.uint16).astype(np.uint32)
    assert sb.shape == (E, N, G)
    z = np.full((E, N, G), 8, np.uint32) if w_zeros is None else \
        unpack_zeros(w_zeros, N).astype(np.uint32)
    meta = (sb | (z << 16)).reshape(E, N // 16, 16 * G)
    f = np.concatenate([v.astype(np.int32), meta.view(np.int32)], axis=2)
    return np.ascontiguousarray(f).reshape(E, N // 16, 17, 16 * G)


def unrepack_fragments(w_frag):
    """Inverse of repack_fragments: (E, N/16, 17, 16 G) -> (w_packed (E, N, K/8) int32,
    scales (E, N, G) fp16, zero-points (E, N, G) uint8 as integers 0..15)."""
    f = np.asarray(w_frag)
    E, NT = f.shape[:2]
    G = f.shape[3] // 16
    f = f.reshape(E, NT, FRAG_TILE_WORDS_PER_GROUP * G)
    v = f[:, :, :G * 256].reshape(E, NT, G, 4, 16, 4).transpose(0, 1, 4, 2, 3, 5)
    w = np.ascontiguousarray(v).reshape(E, NT * 16, G * 16)
    meta = f[:, :, G * 256:].view(np.uint32).reshape(E, NT * 16, G)
    sc = (meta & 0xFFFF).astype(np.uint16).view(np.float16)
    zp = ((meta >> 16) & 0xF).astype(np.uint8)
    return w, sc, zp


def unpack_zeros(w_zeros, N: int) -> np.ndarray:
    """(..., N/8, G) int32 -> (..., N, G) zero-points; zp(n) = (z[n/8] >> 4(n%8)) & 0xF
    (moe_kernel.hip:172-176). Packing is along N (dim -2)."""
    z = np.asarray(w_zeros).astype(np.int64) & 0xFFFFFFFF
    n = np.arange(N)
    zz = (z[..., n // 8, :] >> ((n % 8) * 4)[:, None]) & 0xF
    return zz.astype(np.uint8)


def pack_zeros(zp) -> np.ndarray:
    """(..., N, G) zero-points -> (..., N/8, G) int32 (test_moe_correctness.py:36-42)."""
    zp = np.asarray(zp).astype(np.int64) & 0xF
    N = zp.shape[-2]
    out = np.zeros(zp.shape[:-2] + (N // 8, zp.shape[-1]), dtype=np.int64)
    for j in range(8):
        out |= zp[..., j::8, :] << (4 * j)
    return out.astype(np.uint32).view(np.int32)


def dequant_table(zp: int, e2m1: bool = False) -> np.ndarray:
    """16-entry nibble -> e4m3 byte table for one zero-point (tile_config.h:42-45,69-71)."""
    n = np.arange(16)
    if e2m1:
        return e4m3_encode(E2M1_LUT)
    return e4m3_encode((n - zp).astype(np.float32))


def dequant_codes(w_packed, w_zeros=None, group_size: int = 128,
                  e2m1: bool = False) -> np.ndarray:
    """Op-layout weights (..., N, K/8) -> e4m3 bytes (..., N, K) of (nibble - zp).

    zp is 8 when ``w_zeros`` is None/empty (symmetric uint4b8, moe_kernel.hip:172),
    ignored for E2M1 (moe_kernel.hip:78-80)."""
    nib = unpack_nibbles(w_packed)
    if e2m1:
        return e4m3_encode(E2M1_LUT)[nib]
    K = nib.shape[-1]
    G = K // group_size
    if w_zeros is None or np.asarray(w_zeros).size == 0:
        zp = np.full(nib.shape[:-1] + (G,), 8, dtype=np.int64)
    else:
        zp = unpack_zeros(w_zeros, nib.shape[-2]).astype(np.int64)
    zk = np.repeat(zp, group_size, axis=-1)
    return e4m3_encode((nib.astype(np.int64) - zk).astype(np.float32))


# --------------------------------------------------------------------------- #
# per-token activation quantisation
# --------------------------------------------------------------------------- #


def act_quant(x16):
    """Per-row fp8 quant (moe_kernel.hip:87-127; dense twin dense_kernel.hip:153-200):
    s = max(fp32 absmax / 448, 1e-8); q = e4m3_RNE(f32(x) * (1/s)), reciprocal in fp32.

    The reference's torch refs divide (test_moe_correctness.py:79-80); the kernel
    multiplies by the fp32 reciprocal, which is what is restated here."""
    xf = np.asarray(x16, dtype=np.float16).astype(np.float32)
    if xf.shape[-1] == 0:
        amax = np.zeros(xf.shape[:-1], np.float32)
    else:
        amax = np.abs(xf).max(axis=-1).astype(np.float32)
    s = (amax / E4M3_MAX).astype(np.float32)
    s = np.maximum(s, ACT_SCALE_FLOOR).astype(np.float32)
    inv = (np.float32(1.0) / s).astype(np.float32)
    q = e4m3_encode((xf * inv[..., None]).astype(np.float32))
    return q, s


# --------------------------------------------------------------------------- #
# router and moe_align_block_size
# --------------------------------------------------------------------------- #


def topk_softmax(logits, top_k: int, renormalize: bool = True):
    """Router softmax -> top-k -> renormalise (vLLM fused_topk; contract from
    BASELINE.json). Selection is on logits, ties to the lower expert id, order
    descending; weights are softmax probabilities (float64 here) of the chosen ids."""
    lg = np.asarray(logits, dtype=np.float32)
    order = np.argsort(-lg.astype(np.float64), axis=-1, kind="stable")[..., :top_k]
    ids = order.astype(np.int32)
    l64 = lg.astype(np.float64)
    p = np.exp(l64 - l64.max(axis=-1, keepdims=True))
    p = p / p.sum(axis=-1, keepdims=True)
    w = np.take_along_axis(p, order, axis=-1)
    if renormalize:
        w = w / w.sum(axis=-1, keepdims=True)
    return w.astype(np.float32), ids


def align_alloc_len(numel: int, num_experts: int, block_m: int) -> int:
    """vLLM `moe_align_block_size(..., pad_sorted_ids=True)` buffer length:
    round_up(T*k + E*(block_m-1), block_m) (moe_experts.py:583-590)."""
    m = numel + num_experts * (block_m - 1)
    return (m + block_m - 1) // block_m * block_m


def moe_align(topk_ids, block_m: int, num_experts: int, expert_map=None):
    """Sort (token, slot) ids `t*k+j` by expert ascending then slot ascending, pad each
    touched expert to a multiple of block_m with the sentinel T*k
    (test_moe_experts.py:136-152, test_moe_correctness.py:49-67; call site
    moe_experts.py:587-589). Entries past ntp hold the sentinel and expert_ids -1.
    With ``expert_map`` ids map to local experts first and -1 slots are dropped."""
    ids = np.asarray(topk_ids).astype(np.int64)
    T, k = ids.shape
    numel = T * k
    flat = ids.reshape(-1)
    if expert_map is not None:
        em = np.asarray(expert_map).astype(np.int64)
        # vLLM passes global_num_experts with a global -> local map of that length
        assert em.size == num_experts, "expert_map must have num_experts (global) entries"
        flat = np.where((flat >= 0) & (flat < em.size), em[np.clip(flat, 0, em.size - 1)], -1)
    P = align_alloc_len(numel, num_experts, block_m)
    sorted_ids = np.full(P, numel, dtype=np.int32)
    expert_ids = np.full(P // block_m, -1, dtype=np.int32)
    valid = (flat >= 0) & (flat < num_experts)
    slots = np.nonzero(valid)[0]
    order = np.lexsort((slots, flat[slots]))          # expert asc, then slot asc
    slots = slots[order]
    exps = flat[slots]
    pos = 0
    for e in np.unique(exps):
        s_e = slots[exps == e]
        n = s_e.size
        npad = (n + block_m - 1) // block_m * block_m
        sorted_ids[pos:pos + n] = s_e
        expert_ids[pos // block_m:(pos + npad) // block_m] = e
        pos += npad
    ntp = np.array([pos], dtype=np.int32)
    return sorted_ids, expert_ids, ntp


# --------------------------------------------------------------------------- #
# grouped GEMM
# --------------------------------------------------------------------------- #


def expert_weights_f64(w_packed_e, w_zeros_e, group_size, e2m1):
    """One expert's weights as the float64 values of their e4m3 codes. For int4 these are
    the integers (nibble - zp) in [-15, 15], which e4m3 holds exactly (the exhaustive table
    test pins decode(encode(n - z)) == n - z for all 256 pairs), so they are formed directly
    instead of through the byte round trip; E2M1 goes through the codebook."""
    if e2m1:
        return E4M3_TO_F64[dequant_codes(w_packed_e, None, group_size, True)]
    nib = unpack_nibbles(w_packed_e).astype(np.int16)
    G = nib.shape[-1] // group_size
    if w_zeros_e is None or np.asarray(w_zeros_e).size == 0:
        zp = np.full(nib.shape[:-1] + (G,), 8, dtype=np.int16)
    else:
        zp = unpack_zeros(w_zeros_e, nib.shape[-2]).astype(np.int16)
    return (nib - np.repeat(zp, group_size, axis=-1)).astype(np.float64)


def grouped_run(a_codes, row_expert, w_packed, scales, w_zeros=None,
                group_size: int = 128, e2m1: bool = False) -> np.ndarray:
    """Per row r: run[r, n] = sum_g fp32(sum_{k in g} a[r,k] * w[e,n,k]) * scale[e,n,g],
    fp32 FMA sequential over g (moe_gemm_tiled.h:144-151; moe_kernel.hip:169-188).
    Returns (R, N) float32 before the activation-scale epilogue. Rows with an
    out-of-range expert are zero."""
    a_codes = np.asarray(a_codes, dtype=np.uint8)
    R, K = a_codes.shape
    wp = np.asarray(w_packed)
    E, N, _ = wp.shape
    G = K // group_size
    sc = np.asarray(scales).astype(np.float32)
    zs = None if w_zeros is None or np.asarray(w_zeros).size == 0 else np.asarray(w_zeros)
    A = E4M3_TO_F64[a_codes]
    run = np.zeros((R, N), dtype=np.float32)
    row_expert = np.asarray(row_expert).astype(np.int64)
    for e in np.unique(row_expert):
        if e < 0 or e >= E:
            continue
        idx = np.nonzero(row_expert == e)[0]
        W = expert_weights_f64(wp[e], None if zs is None else zs[e], group_size, e2m1)
        # every group's partial sums in one batched product: (G, R, gs) @ (G, gs, N); exact
        # in float64 (products of e4m3 and small integers), then one rounding to fp32
        Ag = A[idx].reshape(idx.size, G, group_size).transpose(1, 0, 2)
        Wg = W.reshape(N, G, group_size).transpose(1, 2, 0)
        part = np.matmul(Ag, Wg).astype(np.float32)
        r = np.zeros((idx.size, N), dtype=np.float32)
        for g in range(G):
            r = fma32(part[g], sc[e, :, g][None, :], r)
        run[idx] = r
    return run


def grouped_gemm_padded(x16, w_packed, scales, w_zeros, sorted_ids, expert_ids, ntp,
                        top_k: int, block_m: int, e2m1: bool = False):
    """`mmq_fp8_moe_gemm` semantics in the padded sorted layout
    (moe_kernel.hip:133-196, bindings.cpp:178-228): act-quant x per row, row r with
    slot s = sorted_ids[r] < T*top_k gathers x[s // top_k] and uses expert
    expert_ids[r // block_m]; out[r] = fp16(run * act_scale). Returns (out fp16 with
    NaN in unwritten rows, valid-row mask)."""
    x16 = np.asarray(x16, dtype=np.float16)
    T, K = x16.shape
    E, N, _ = np.asarray(w_packed).shape
    G = np.asarray(scales).shape[-1]
    gs = K // G
    sti = np.asarray(sorted_ids).astype(np.int64)
    P = sti.size
    nv = T * top_k
    ntp_v = int(np.asarray(ntp).reshape(-1)[0])
    rows = np.arange(P)
    valid = (rows < ntp_v) & (sti < nv)
    q, s = act_quant(x16)
    src = np.where(valid, sti // top_k, 0)
    eid = np.asarray(expert_ids).astype(np.int64)[rows // block_m]
    eid = np.where(valid, eid, -1)
    run = grouped_run(q[src], eid, w_packed, scales, w_zeros, gs, e2m1)
    out = np.full((P, N), np.nan, dtype=np.float16)
    y = (run * s[src][:, None]).astype(np.float32)
    out[valid] = y[valid].astype(np.float16)
    return out, valid


def silu_and_mul(gate_h, up_h) -> np.ndarray:
    """fp16(fp16(g / (1 + exp(-g))) * up), g = f32(gate) (moe_kernel.hip:555-561;
    test_moe_experts.py:274-280). fp32 exp here; the kernels use expf."""
    g = np.asarray(gate_h, dtype=np.float16).astype(np.float32)
    silu = (g / (np.float32(1.0) + np.exp(-g))).astype(np.float32).astype(np.float16)
    return (silu.astype(np.float32) * np.asarray(up_h, np.float16).astype(np.float32)
            ).astype(np.float16)


SWIGLUOAI_ALPHA = np.float32(1.702)   # vLLM SwigluOAIAndMul defaults (gpt-oss)
SWIGLUOAI_LIMIT = np.float32(7.0)


def swigluoai_and_mul(x16, alpha=SWIGLUOAI_ALPHA, limit=SWIGLUOAI_LIMIT) -> np.ndarray:
    """vLLM ``swigluoai_and_mul`` (third-party: vLLM 0.22.69, csrc/activation_kernels.cu
    ``swigluoai_and_mul_kernel`` / layers/activation.py ``SwigluOAIAndMul``, not vendored in
    the reference; called through ``apply_moe_activation`` by the reference's mxfp4 hook,
    moe_experts.py:1416-1424): x (..., 2I) fp16 with gate and up interleaved, gate = x[2c],
    up = x[2c + 1]; in fp32 g = min(gate, limit), u = clamp(up, -limit, limit),
    sig = 1 / (1 + exp(-g * alpha)), out = fp16((u + 1) * (g * sig)). fp32 exp here; the
    kernel uses expf."""
    x = np.asarray(x16, dtype=np.float16).astype(np.float32)
    gate, up = x[..., 0::2], x[..., 1::2]
    lim = np.float32(limit)
    with np.errstate(over="ignore", invalid="ignore"):
        g = np.where(gate > lim, lim, gate).astype(np.float32)
        u = np.where(up > lim, lim, np.where(up < -lim, -lim, up)).astype(np.float32)
        sig = (np.float32(1.0) / (np.float32(1.0) + np.exp((-g * np.float32(alpha)).astype(np.float32)))
               ).astype(np.float32)
        glu = (g * sig).astype(np.float32)
        return ((u + np.float32(1.0)) * glu).astype(np.float32).astype(np.float16)


def e8m0_to_fp16(codes) -> np.ndarray:
    """OCP MX E8M0 block scales (uint8, value 2^(s - 127)) -> fp16, the reference's mxfp4
    load step (mxfp4/convert.py:68-98: torch.pow(2, s - 127) in fp32, cast to fp16):
    exact for s - 127 in [-24, 15] (subnormal below -14), 0 below (2^-25 rounds to even),
    +inf above 15, and +inf for the E8M0 NaN code 255 (2^128 overflows fp32)."""
    e = np.asarray(codes, dtype=np.uint8).astype(np.int64) - 127
    with np.errstate(over="ignore"):
        return np.ldexp(np.float64(1.0), e).astype(np.float32).astype(np.float16)


def convert_mxfp4(weight_packed, weight_scale):
    """mxfp4 (compressed-tensors / gpt-oss) expert weights -> the op layout
    (mxfp4/convert.py:100-140): weight_packed (..., N, K/2) uint8, two E2M1 codes a byte, the
    lower K index in the low nibble; weight_scale (..., N, K/32) uint8 E8M0. Returns
    (w_packed (..., N, K/8) int32 with code k at nibble k % 8 of word k / 8, scales fp16
    (..., N, K/32)); the codes are not remapped."""
    wb = np.asarray(weight_packed, dtype=np.uint8)
    codes = np.empty(wb.shape[:-1] + (wb.shape[-1] * 2,), np.uint8)
    codes[..., 0::2] = wb & 0xF
    codes[..., 1::2] = wb >> 4
    return pack_nibbles(codes), e8m0_to_fp16(weight_scale)


def gemm_scatter(xpad16, w_packed, scales, w_zeros, sorted_ids, expert_ids, ntp,
                 topk_weights, output, top_k: int, block_m: int, e2m1: bool = False):
    """`mmq_fp8_moe_gemm_scatter` (moe_kernel.hip:1053-1056, bindings.cpp:293-353):
    identity gather of padded row r, output[s // top_k] += w[s] * run * act_scale[r]
    (no fp16 rounding; accumulation order free). Returns the updated copy."""
    xpad16 = np.asarray(xpad16, dtype=np.float16)
    P, K = xpad16.shape
    G = np.asarray(scales).shape[-1]
    gs = K // G
    out = np.array(output, dtype=np.float32, copy=True)
    M = out.shape[0]
    nv = M * top_k
    sti = np.asarray(sorted_ids).astype(np.int64)
    ntp_v = int(np.asarray(ntp).reshape(-1)[0])
    rows = np.arange(P)
    valid = (rows < ntp_v) & (sti < nv)
    q, s = act_quant(xpad16)
    eid = np.where(valid, np.asarray(expert_ids).astype(np.int64)[rows // block_m], -1)
    run = grouped_run(q, eid, w_packed, scales, w_zeros, gs, e2m1)
    tw = np.asarray(topk_weights, dtype=np.float32).reshape(-1)
    for r in np.nonzero(valid)[0]:
        slot = sti[r]
        out[slot // top_k] += (tw[slot] * (run[r] * s[r])).astype(np.float32)
    return out


def gather_reduce(out2_16, sorted_ids, topk_weights, ntp, top_k: int) -> np.ndarray:
    """`mmq_fp8_moe_gather_reduce` (moe_kernel.hip:1230-1258): slot_to_row[s] = r for
    r < min(P, ntp) with s < M*top_k (later rows win); out[t, n] =
    sum_{j ascending} w[t*k+j] * f32(out2[row, n]), fp32 FMA, missing slots skipped."""
    o2 = np.asarray(out2_16, dtype=np.float16).astype(np.float32)
    P, N = o2.shape
    tw = np.asarray(topk_weights, dtype=np.float32).reshape(-1)
    M = tw.size // top_k
    sti = np.asarray(sorted_ids).astype(np.int64)
    ntp_v = int(np.asarray(ntp).reshape(-1)[0])
    slot_to_row = np.full(M * top_k, -1, dtype=np.int64)
    for r in range(min(P, ntp_v)):
        s = sti[r]
        if 0 <= s < M * top_k:
            slot_to_row[s] = r
    acc = np.zeros((M, N), dtype=np.float32)
    for j in range(top_k):
        rr = slot_to_row[np.arange(M) * top_k + j]
        has = rr >= 0
        vals = np.zeros((M, N), np.float32)
        vals[has] = o2[rr[has]]
        w = np.where(has, tw[np.arange(M) * top_k + j], 0.0).astype(np.float32)
        acc = np.where(has[:, None], fma32(w[:, None], vals, acc), acc)
    return acc


def dense_gemm(x16, w_packed, scales, w_zeros=None, e2m1: bool = False) -> np.ndarray:
    """`mmq_fp8_gemm` reference_scalar (dense_kernel.hip:107-145 + act-quant :153-200):
    the grouped arithmetic with one expert and identity rows. (M,N) fp16."""
    x16 = np.asarray(x16, dtype=np.float16)
    wp = np.asarray(w_packed)[None]
    sc = np.asarray(scales)[None]
    zs = None if w_zeros is None or np.asarray(w_zeros).size == 0 else np.asarray(w_zeros)[None]
    K = x16.shape[1]
    gs = K // sc.shape[-1]
    q, s = act_quant(x16)
    run = grouped_run(q, np.zeros(x16.shape[0], np.int64), wp, sc, zs, gs, e2m1)
    return (run * s[:, None]).astype(np.float32).astype(np.float16)


# --------------------------------------------------------------------------- #
# full layer (the `_run_grouped_moe` composition)
# --------------------------------------------------------------------------- #


def _add_bias_f16(v16, bias, experts):
    """fp16 tensor + per-expert fp16 bias row, as torch adds two fp16 tensors: exact sum of
    the two values rounded once to fp16 (moe_experts.py:565-575, the unfused path's
    ``out + _expand_bias(bias).to(out.dtype)``). Rows with an out-of-range expert use
    expert 0's row, as the reference's ``expert_ids.clamp(min=0)`` does for padding."""
    b = np.asarray(bias, dtype=np.float16)
    e = np.clip(np.asarray(experts).astype(np.int64), 0, b.shape[0] - 1)
    return (np.asarray(v16, np.float16).astype(np.float32)
            + b[e].astype(np.float32)).astype(np.float16)


def moe_layer(x, w13, s13, z13, w2, s2, z2, topk_weights, topk_ids,
              group_size: int = 128, round_y_fp16: bool = True, e2m1: bool = False,
              return_stages: bool = False, w1_bias=None, w2_bias=None, expert_map=None,
              activation: str = "silu"):
    """Whole gated MoE in token order (moe_experts.py:493-665, arithmetic per
    test_moe_experts.py:155-191 with the kernel SiLU moe_kernel.hip:555-561):
      x16 = fp16(x); a1,s1 = act_quant(x16); run1 over w13 per (t, j);
      gate/up = fp16(run1 * s1) (+ fp16 w1_bias[e]); h = silu_and_mul; a2,s2 = act_quant(h);
      y = run2 * s2 (fp16-rounded on the prefill path, moe_gemm_tiled.h:346; not on
      the decode scatter path, moe_kernel.hip:1056; always fp16 with a w2_bias, which is
      added to the fp16 rows, moe_experts.py:654-655);
      out[t] = sum_{j ascending} w[t,j] * y[t,j] in fp32.
    With ``expert_map`` (global id -> local expert or -1) slots without a local expert add
    nothing (moe_experts.py:587-589 aligns with global_num_experts and the map).
    ``activation`` "swigluoai" (gpt-oss) replaces silu_and_mul of the [gate | up] halves by
    swigluoai_and_mul of interleaved gate/up columns.
    ``x`` is float32 (holding bf16 or fp16 values). Returns float32 (T, H)."""
    x16 = np.asarray(x, dtype=np.float32).astype(np.float16)
    T, H = x16.shape
    ids = np.asarray(topk_ids).astype(np.int64)
    if expert_map is not None:
        em = np.asarray(expert_map).astype(np.int64)
        ids = np.where((ids >= 0) & (ids < em.size), em[np.clip(ids, 0, em.size - 1)], -1)
    k = ids.shape[1]
    I2 = np.asarray(w13).shape[1]
    inter = I2 // 2
    a1, sc1 = act_quant(x16)
    tok = np.repeat(np.arange(T), k)
    run1 = grouped_run(a1[tok], ids.reshape(-1), w13, s13, z13, group_size, e2m1)
    g1 = (run1 * sc1[tok][:, None]).astype(np.float32).astype(np.float16)
    if w1_bias is not None:
        g1 = _add_bias_f16(g1, w1_bias, ids.reshape(-1))
    if activation == "swigluoai":
        h = swigluoai_and_mul(g1)
    elif activation == "silu":
        h = silu_and_mul(g1[:, :inter], g1[:, inter:])
    else:
        raise ValueError(f"unknown activation {activation!r}")
    a2, sc2 = act_quant(h)
    run2 = grouped_run(a2, ids.reshape(-1), w2, s2, z2, group_size, e2m1)
    y = (run2 * sc2[:, None]).astype(np.float32)
    if w2_bias is not None:
        y = _add_bias_f16(y.astype(np.float16), w2_bias, ids.reshape(-1)).astype(np.float32)
    elif round_y_fp16:
        y = y.astype(np.float16).astype(np.float32)
    tw = np.asarray(topk_weights, dtype=np.float32).reshape(T, k)
    y = y.reshape(T, k, H)
    acc = np.zeros((T, H), dtype=np.float32)
    for j in range(k):
        acc = fma32(tw[:, j:j + 1], y[:, j], acc)
    if return_stages:
        return acc, dict(a1=a1, s1=sc1, g1=g1, h=h, a2=a2, s2=sc2, y=y)
    return acc


def moe_layer_f64(x, w13, s13, z13, w2, s2, z2, topk_weights, topk_ids,
                  group_size: int = 128, activation: str = "silu", w1_bias=None,
                  w2_bias=None) -> np.ndarray:
    """Un-quantised float64 MoE (dequantised int4 weights, no activation quant):
    the 'ideal' model test_moe_experts.py reports against. ``activation`` "swigluoai" is
    vLLM's gpt-oss activation on interleaved gate/up (alpha 1.702, limit 7); biases are
    per-expert rows added to gemm1's and gemm2's outputs."""
    xf = np.asarray(x, dtype=np.float64)
    T, H = xf.shape
    ids = np.asarray(topk_ids).astype(np.int64)
    tw = np.asarray(topk_weights, dtype=np.float64)
    I2 = np.asarray(w13).shape[1]
    inter = I2 // 2
    out = np.zeros((T, H))
    cache = {}

    def deq(wp, sc, zz, e):
        codes = dequant_codes(wp[e], None if zz is None else zz[e], group_size)
        W = E4M3_TO_F64[codes]
        return W * np.repeat(np.asarray(sc[e], np.float64), group_size, axis=-1)

    for t in range(T):
        for j in range(ids.shape[1]):
            e = ids[t, j]
            if e not in cache:
                cache[e] = (deq(w13, s13, z13, e), deq(w2, s2, z2, e))
            W1, W2 = cache[e]
            g = W1 @ xf[t]
            if w1_bias is not None:
                g = g + np.asarray(w1_bias, np.float64)[e]
            if activation == "swigluoai":
                gt = np.minimum(g[0::2], SWIGLUOAI_LIMIT)
                up = np.clip(g[1::2], -SWIGLUOAI_LIMIT, SWIGLUOAI_LIMIT)
                hh = (up + 1.0) * gt / (1.0 + np.exp(-SWIGLUOAI_ALPHA * gt))
            else:
                hh = g[:inter] / (1.0 + np.exp(-g[:inter])) * g[inter:]
            y = W2 @ hh
            if w2_bias is not None:
                y = y + np.asarray(w2_bias, np.float64)[e]
            out[t] += tw[t, j] * y
    return out


# --------------------------------------------------------------------------- #
# weight-format converters (load-time; the north star's process_weights hook)
# --------------------------------------------------------------------------- #

REVERSE_AWQ_PACK_ORDER = [0, 4, 1, 5, 2, 6, 3, 7]   # moe_experts.py:47


def awq_pack(vals) -> np.ndarray:
    """(E, R, C) nibbles -> (E, R, C/8) int32 in AWQ bit order (test_moe_experts.py:54-61)."""
    v = np.asarray(vals).astype(np.int64) & 0xF
    E, R, C = v.shape
    packed = np.zeros((E, R, C // 8), dtype=np.int64)
    for i in range(8):
        packed |= v[:, :, i::8] << (REVERSE_AWQ_PACK_ORDER[i] * 4)
    return packed.astype(np.uint32).view(np.int32)


def awq_to_op_layout(qweight, scales, qzeros):
    """AWQ MoE (E, K, N/8) int32 packed along output in AWQ order -> op layout
    w (E, N, K/8), scales (E, N, G) fp16, zeros (E, N/8, G) (moe_experts.py:331-396)."""
    qw = np.asarray(qweight).astype(np.int64) & 0xFFFFFFFF
    qz = np.asarray(qzeros).astype(np.int64) & 0xFFFFFFFF
    E, K, Np = qw.shape
    N = Np * 8
    shifts = np.arange(8, dtype=np.int64) * 4
    rev = np.array(REVERSE_AWQ_PACK_ORDER)
    uw = ((qw[..., None] >> shifts) & 0xF)[..., rev].reshape(E, K, N)
    w = pack_nibbles(np.swapaxes(uw, 1, 2))
    uz = ((qz[..., None] >> shifts) & 0xF)[..., rev].reshape(E, qz.shape[1], N)
    z = pack_zeros(np.swapaxes(uz, 1, 2))
    s = np.ascontiguousarray(np.swapaxes(np.asarray(scales), 1, 2)).astype(np.float16)
    return w, s, z


def convert_awq_tensor(tensor, tensor_type: str) -> np.ndarray:
    """vLLM MoeWNA16 loader AWQ -> standard u8 (moe_wna16.py:384-420):
    qweight (K, N/8) int32 -> (N, K/2) u8; qzeros (G, N/8) int32 -> (N/2, G) u8."""
    t = np.ascontiguousarray(tensor, dtype=np.int32)
    size0 = t.shape[0]
    u8 = t.view(np.uint8)
    nib = np.stack([u8 & 0xF, (u8 >> 4) & 0xF], axis=-1)          # (a, 4b, 2)
    nib = nib.reshape(-1, 8)[:, REVERSE_AWQ_PACK_ORDER].reshape(size0, -1)
    nib = np.ascontiguousarray(nib.T)
    if tensor_type == "qweight":
        return (nib[:, 1::2] * 16 + nib[:, ::2]).astype(np.uint8)
    if tensor_type == "qzeros":
        return (nib[1::2, :] * 16 + nib[::2, :]).astype(np.uint8)
    raise ValueError(tensor_type)


def wna16_to_op_layout(qweight_u8, scales, qzeros_u8=None):
    """MoeWNA16 u8 params -> op layout (moe_experts.py:473-482): qweight (E,N,K/2) u8
    viewed as (E,N,K/8) int32; qzeros (E,N/2,G) u8, 4 consecutive N-bytes -> one int32."""
    w = np.ascontiguousarray(qweight_u8, dtype=np.uint8).view(np.int32)
    s = np.asarray(scales).astype(np.float16)
    z = None
    if qzeros_u8 is not None:
        qz = np.ascontiguousarray(qzeros_u8, dtype=np.uint8).astype(np.int64)
        E, Nh, G = qz.shape
        zi = qz.reshape(E, Nh // 4, 4, G)
        z = (zi[:, :, 0] | (zi[:, :, 1] << 8) | (zi[:, :, 2] << 16) | (zi[:, :, 3] << 24))
        z = z.astype(np.uint32).view(np.int32)
    return w, s, z


__all__ = [n for n in dir() if not n.startswith("_")]
