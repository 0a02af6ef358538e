"""torch.ops.w4a8_fp8_wmma.* — the reference's op schemas over the gfx950 C ABI.

Schemas, argument checks and output allocation follow
w4a8_fp8_wmma/bindings.cpp:178-413; kernels run through ``include/w4a8_moe.h``.
Every op enqueues on torch's current stream of the input's device and never
synchronises. Implementations are registered for the CUDA (HIP) key only, like the
reference; fake (meta) impls make the ops traceable (__init__.py:255-297).
"""
from __future__ import annotations

import torch

from ._lib import check, lib

NS = "w4a8_fp8_wmma"
_TAGS = (torch.Tag.pt2_compliant_tag,)
_library = torch.library.Library(NS, "DEF")

_MOE_ARGS = ("Tensor x, Tensor w_packed, Tensor scales, Tensor w_zeros, "
             "Tensor sorted_token_ids, Tensor expert_ids, Tensor num_tokens_post_padded, "
             "int top_k, int block_m, int kernel, bool weight_is_e2m1=False")
SCHEMAS = {
    "mmq_fp8_gemm": "mmq_fp8_gemm(Tensor x, Tensor w_packed, Tensor scales, Tensor w_zeros, "
                    "int kernel, bool weight_is_e2m1=False) -> Tensor",
    "mmq_fp8_moe_gemm": f"mmq_fp8_moe_gemm({_MOE_ARGS}) -> Tensor",
    "mmq_fp8_moe_gemm1_silu": f"mmq_fp8_moe_gemm1_silu({_MOE_ARGS}) -> Tensor",
    "mmq_fp8_moe_gemm_scatter": (
        "mmq_fp8_moe_gemm_scatter(Tensor x, Tensor w_packed, Tensor scales, "
        "Tensor w_zeros, Tensor sorted_token_ids, Tensor expert_ids, "
        "Tensor num_tokens_post_padded, Tensor topk_weights, Tensor(a!) output, "
        "int top_k, int block_m, int kernel, bool weight_is_e2m1=False) -> ()"),
    "mmq_fp8_moe_gather_reduce": (
        "mmq_fp8_moe_gather_reduce(Tensor out2, Tensor sorted_token_ids, "
        "Tensor topk_weights, Tensor num_tokens_post_padded, int top_k) -> Tensor"),
}
for _schema in SCHEMAS.values():
    _library.define(_schema, tags=_TAGS)


def _check(cond: bool, msg: str) -> None:
    if not cond:
        raise RuntimeError(msg)


def _ptr(t: torch.Tensor | None) -> int | None:
    if t is None or t.numel() == 0:
        return None
    return t.data_ptr()


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _workspace(nbytes: int, device) -> torch.Tensor:
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)


def _zeros_or_none(w_zeros: torch.Tensor, N: int, scales: torch.Tensor, e2m1: bool,
                   dims: int) -> torch.Tensor | None:
    if w_zeros is None or w_zeros.numel() == 0:
        return None
    _check(not e2m1, "mxfp4 (E2M1) weights are symmetric; w_zeros must be empty")
    _check(w_zeros.is_cuda and w_zeros.dtype == torch.int32,
           "w_zeros must be CUDA int32 (packed)")
    _check(w_zeros.dim() == dims and w_zeros.size(-2) * 8 == N
           and w_zeros.size(-1) == scales.size(-1),
           f"w_zeros shape mismatch: expected (..., {N // 8}, {scales.size(-1)})")
    _check(w_zeros.is_contiguous(), "w_zeros must be contiguous")
    return w_zeros


def _check_moe_common(x, w_packed, scales, sorted_token_ids, expert_ids,
                      num_tokens_post_padded, block_m, x_rows_name="(T, K)"):
    # bindings.cpp:191-213
    _check(x.is_cuda and w_packed.is_cuda and scales.is_cuda,
           "x, w_packed, scales must be CUDA")
    _check(x.dtype == torch.float16, "x must be fp16")
    _check(w_packed.dtype == torch.int32, "w_packed must be int32")
    _check(scales.dtype == torch.float16, "scales must be fp16")
    _check(x.dim() == 2, f"x must be {x_rows_name}")
    _check(w_packed.dim() == 3 and scales.dim() == 3,
           "w_packed (E,N,K/8) and scales (E,N,K/group) must be 3D")
    _check(sorted_token_ids.dtype == torch.int32 and expert_ids.dtype == torch.int32
           and num_tokens_post_padded.dtype == torch.int32, "routing tensors must be int32")
    _check(sorted_token_ids.is_cuda and expert_ids.is_cuda and num_tokens_post_padded.is_cuda,
           "routing tensors must be CUDA")
    _check(x.is_contiguous() and w_packed.is_contiguous() and scales.is_contiguous(),
           "x, w_packed, scales must be contiguous")
    _check(sorted_token_ids.is_contiguous() and expert_ids.is_contiguous(),
           "routing tensors must be contiguous")
    K = x.size(1)
    E, N = w_packed.size(0), w_packed.size(1)
    P = sorted_token_ids.size(0)
    _check(w_packed.size(2) * 8 == K, f"w_packed last dim must be K/8={K // 8}")
    _check(scales.size(0) == E and scales.size(1) == N, "scales must be (E, N, K/group)")
    _check(scales.size(2) > 0 and K % scales.size(2) == 0, "K not divisible by scales' K dim")
    _check(block_m > 0 and P % block_m == 0, f"P={P} not divisible by block_m={block_m}")
    _check(expert_ids.size(0) == P // block_m,
           f"expert_ids must have P/block_m={P // block_m} entries")
    return K, E, N, P, K // scales.size(2)


# --------------------------------------------------------------------------- #
# CUDA impls
# --------------------------------------------------------------------------- #

def mmq_fp8_moe_gemm_cuda(x, w_packed, scales, w_zeros, sorted_token_ids, expert_ids,
                          num_tokens_post_padded, top_k, block_m, kernel,
                          weight_is_e2m1=False):
    """bindings.cpp:178-228."""
    K, E, N, P, gs = _check_moe_common(x, w_packed, scales, sorted_token_ids, expert_ids,
                                       num_tokens_post_padded, block_m)
    z = _zeros_or_none(w_zeros, N, scales, weight_is_e2m1, 3)
    out = torch.empty((P, N), dtype=torch.float16, device=x.device)
    T = x.size(0)
    ws = _workspace(lib.w4a8_moe_gemm_workspace_size(T, K), x.device)
    check(lib.w4a8_mmq_fp8_moe_gemm(
        _ptr(x), T, K, _ptr(w_packed), _ptr(scales), _ptr(z), E, N, gs,
        _ptr(sorted_token_ids), P, _ptr(expert_ids), _ptr(num_tokens_post_padded),
        int(top_k), int(block_m), int(kernel), int(bool(weight_is_e2m1)), _ptr(out),
        ws.data_ptr(), ws.numel(), _stream(x)), "mmq_fp8_moe_gemm")
    return out


def mmq_fp8_moe_gemm1_silu_cuda(x, w_packed, scales, w_zeros, sorted_token_ids, expert_ids,
                                num_tokens_post_padded, top_k, block_m, kernel,
                                weight_is_e2m1=False):
    """bindings.cpp:235-287."""
    K, E, N, P, gs = _check_moe_common(x, w_packed, scales, sorted_token_ids, expert_ids,
                                       num_tokens_post_padded, block_m)
    _check(int(kernel) == 6, f"fused gemm1+silu needs the 'wmma' kernel; got id {kernel}")
    _check(N % 2 == 0, f"w13 N must be 2*inter (even); got {N}")
    z = _zeros_or_none(w_zeros, N, scales, weight_is_e2m1, 3)
    out = torch.empty((P, N // 2), dtype=torch.float16, device=x.device)
    T = x.size(0)
    ws = _workspace(lib.w4a8_moe_gemm_workspace_size(T, K), x.device)
    check(lib.w4a8_mmq_fp8_moe_gemm1_silu(
        _ptr(x), T, K, _ptr(w_packed), _ptr(scales), _ptr(z), E, N, gs,
        _ptr(sorted_token_ids), P, _ptr(expert_ids), _ptr(num_tokens_post_padded),
        int(top_k), int(block_m), int(kernel), int(bool(weight_is_e2m1)), _ptr(out),
        ws.data_ptr(), ws.numel(), _stream(x)), "mmq_fp8_moe_gemm1_silu")
    return out


def mmq_fp8_moe_gemm_scatter_cuda(x, w_packed, scales, w_zeros, sorted_token_ids,
                                  expert_ids, num_tokens_post_padded, topk_weights, output,
                                  top_k, block_m, kernel, weight_is_e2m1=False):
    """bindings.cpp:293-353 (in-place accumulate into the pre-zeroed `output`)."""
    K, E, N, P, gs = _check_moe_common(x, w_packed, scales, sorted_token_ids, expert_ids,
                                       num_tokens_post_padded, block_m, "(P, K)")
    _check(topk_weights.dtype == torch.float32 and output.dtype == torch.float32,
           "topk_weights and output must be fp32")
    _check(topk_weights.is_contiguous() and output.is_contiguous(),
           "x, w_packed, scales, topk_weights, output must be contiguous")
    _check(output.dim() == 2 and output.size(1) == N, f"output must be (M, N) with N={N}")
    M = output.size(0)
    _check(topk_weights.numel() == M * top_k, f"topk_weights must have M*top_k={M * top_k} entries")
    _check(x.size(0) >= P, "x must have one row per padded row (P, K)")
    z = _zeros_or_none(w_zeros, N, scales, weight_is_e2m1, 3)
    ws = _workspace(lib.w4a8_moe_gemm_workspace_size(x.size(0), K), x.device)
    check(lib.w4a8_mmq_fp8_moe_gemm_scatter(
        _ptr(x), x.size(0), K, _ptr(w_packed), _ptr(scales), _ptr(z), E, N, gs,
        _ptr(sorted_token_ids), P, _ptr(expert_ids), _ptr(num_tokens_post_padded),
        _ptr(topk_weights), _ptr(output), M, int(top_k), int(block_m), int(kernel),
        int(bool(weight_is_e2m1)), ws.data_ptr(), ws.numel(), _stream(x)),
        "mmq_fp8_moe_gemm_scatter")


def mmq_fp8_moe_gather_reduce_cuda(out2, sorted_token_ids, topk_weights,
                                   num_tokens_post_padded, top_k):
    """bindings.cpp:357-380."""
    _check(out2.is_cuda and out2.dtype == torch.float16 and out2.dim() == 2,
           "out2 must be (P,N) fp16 CUDA")
    _check(sorted_token_ids.dtype == torch.int32 and num_tokens_post_padded.dtype == torch.int32,
           "sorted_token_ids / num_tokens_post_padded must be int32")
    _check(topk_weights.dtype == torch.float32, "topk_weights must be fp32")
    _check(out2.is_contiguous() and topk_weights.is_contiguous(),
           "out2 and topk_weights must be contiguous")
    _check(top_k > 0 and topk_weights.numel() % top_k == 0,
           "topk_weights.numel() must be M*top_k")
    P, N = out2.shape
    M = topk_weights.numel() // top_k
    out = torch.zeros((M, N), dtype=torch.float32, device=out2.device)
    ws = _workspace(lib.w4a8_gather_reduce_workspace_size(M * top_k), out2.device)
    check(lib.w4a8_mmq_fp8_moe_gather_reduce(
        _ptr(out2), P, N, _ptr(sorted_token_ids), _ptr(topk_weights), M * top_k,
        _ptr(num_tokens_post_padded), int(top_k), _ptr(out), ws.data_ptr(), ws.numel(),
        _stream(out2)), "mmq_fp8_moe_gather_reduce")
    return out


def mmq_fp8_gemm_cuda(x, w_packed, scales, w_zeros, kernel, weight_is_e2m1=False):
    """bindings.cpp:98-146."""
    _check(x.is_cuda and w_packed.is_cuda and scales.is_cuda, "x, w_packed, scales must be CUDA")
    _check(x.dtype == torch.float16, "x must be fp16")
    _check(w_packed.dtype == torch.int32, "w_packed must be int32")
    _check(scales.dtype == torch.float16, "scales must be fp16")
    _check(x.dim() == 2 and w_packed.dim() == 2 and scales.dim() == 2, "all inputs must be 2D")
    _check(x.is_contiguous() and w_packed.is_contiguous() and scales.is_contiguous(),
           "all inputs must be contiguous")
    M, K = x.shape
    N = w_packed.size(0)
    _check(w_packed.size(1) * 8 == K,
           f"w_packed last dim mismatch: expected K/8 = {K // 8} got {w_packed.size(1)}")
    _check(scales.size(0) == N, f"scales.size(0) must equal N={N}")
    _check(scales.size(1) > 0 and K % scales.size(1) == 0, "K not divisible by scales' K dim")
    gs = K // scales.size(1)
    z = _zeros_or_none(w_zeros, N, scales, weight_is_e2m1, 2)
    out = torch.empty((M, N), dtype=torch.float16, device=x.device)
    ws = _workspace(lib.w4a8_moe_gemm_workspace_size(M, K), x.device)
    check(lib.w4a8_mmq_fp8_gemm(
        _ptr(x), M, K, _ptr(w_packed), _ptr(scales), _ptr(z), N, gs, int(kernel),
        int(bool(weight_is_e2m1)), _ptr(out), ws.data_ptr(), ws.numel(), _stream(x)),
        "mmq_fp8_gemm")
    return out


_library.impl("mmq_fp8_gemm", mmq_fp8_gemm_cuda, "CUDA")
_library.impl("mmq_fp8_moe_gemm", mmq_fp8_moe_gemm_cuda, "CUDA")
_library.impl("mmq_fp8_moe_gemm1_silu", mmq_fp8_moe_gemm1_silu_cuda, "CUDA")
_library.impl("mmq_fp8_moe_gemm_scatter", mmq_fp8_moe_gemm_scatter_cuda, "CUDA")
_library.impl("mmq_fp8_moe_gather_reduce", mmq_fp8_moe_gather_reduce_cuda, "CUDA")


# --------------------------------------------------------------------------- #
# fake impls (__init__.py:255-297)
# --------------------------------------------------------------------------- #

@torch.library.register_fake(f"{NS}::mmq_fp8_gemm")
def _fake_mmq_fp8_gemm(x, w_packed, scales, w_zeros, kernel, weight_is_e2m1=False):
    return x.new_empty((x.shape[0], w_packed.shape[0]), dtype=torch.float16)


@torch.library.register_fake(f"{NS}::mmq_fp8_moe_gemm")
def _fake_mmq_fp8_moe_gemm(x, w_packed, scales, w_zeros, sorted_token_ids, expert_ids,
                           num_tokens_post_padded, top_k, block_m, kernel,
                           weight_is_e2m1=False):
    return x.new_empty((sorted_token_ids.shape[0], w_packed.shape[1]), dtype=torch.float16)


@torch.library.register_fake(f"{NS}::mmq_fp8_moe_gemm1_silu")
def _fake_mmq_fp8_moe_gemm1_silu(x, w_packed, scales, w_zeros, sorted_token_ids, expert_ids,
                                 num_tokens_post_padded, top_k, block_m, kernel,
                                 weight_is_e2m1=False):
    return x.new_empty((sorted_token_ids.shape[0], w_packed.shape[1] // 2),
                       dtype=torch.float16)


@torch.library.register_fake(f"{NS}::mmq_fp8_moe_gemm_scatter")
def _fake_mmq_fp8_moe_gemm_scatter(x, w_packed, scales, w_zeros, sorted_token_ids,
                                   expert_ids, num_tokens_post_padded, topk_weights, output,
                                   top_k, block_m, kernel, weight_is_e2m1=False):
    return None


@torch.library.register_fake(f"{NS}::mmq_fp8_moe_gather_reduce")
def _fake_mmq_fp8_moe_gather_reduce(out2, sorted_token_ids, topk_weights,
                                    num_tokens_post_padded, top_k):
    return out2.new_empty((topk_weights.shape[0] // top_k, out2.shape[1]),
                          dtype=torch.float32)


# --------------------------------------------------------------------------- #
# helpers that are not reference torch ops (plain functions over the C ABI)
# --------------------------------------------------------------------------- #

def act_quant_fp8(x: torch.Tensor, k8_interleave: bool = False):
    """Per-row e4m3 quantisation (moe_kernel.hip:87-127) -> (q uint8 (R,K), scales f32 (R,))."""
    _check(x.is_cuda and x.dtype == torch.float16 and x.dim() == 2 and x.is_contiguous(),
           "x must be a contiguous CUDA fp16 (R, K) tensor")
    R, K = x.shape
    q = torch.empty((R, K), dtype=torch.uint8, device=x.device)
    s = torch.empty((R,), dtype=torch.float32, device=x.device)
    check(lib.w4a8_act_quant_fp8(_ptr(x), R, K, _ptr(q), _ptr(s), int(k8_interleave),
                                 _stream(x)), "act_quant_fp8")
    return q, s


def dequant_fp8(w_packed: torch.Tensor, scales_or_group: int, w_zeros=None,
                weight_is_e2m1: bool = False) -> torch.Tensor:
    """Op-layout int4 (E, N, K/8) -> e4m3 bytes (E, N, K) of (nibble - zp), natural order."""
    _check(w_packed.is_cuda and w_packed.dtype == torch.int32 and w_packed.is_contiguous(),
           "w_packed must be contiguous CUDA int32")
    w3 = w_packed if w_packed.dim() == 3 else w_packed.unsqueeze(0)
    E, N, Kw = w3.shape
    K = Kw * 8
    gs = int(scales_or_group)
    z = None
    if w_zeros is not None and w_zeros.numel() > 0:
        z = w_zeros.contiguous()
    out = torch.empty((E, N, K), dtype=torch.uint8, device=w_packed.device)
    check(lib.w4a8_dequant_fp8(_ptr(w3), _ptr(z), E, N, K, gs, int(bool(weight_is_e2m1)),
                               _ptr(out), _stream(w_packed)), "dequant_fp8")
    return out if w_packed.dim() == 3 else out[0]


def moe_align_block_size(topk_ids: torch.Tensor, block_size: int, num_experts: int,
                         expert_map: torch.Tensor | None = None, pad_sorted_ids: bool = True,
                         ignore_invalid_experts: bool = True):
    """vLLM ``moe_align_block_size`` (call site moe_experts.py:587-589) on the gfx950
    align kernels. Always returns the block-padded buffer length
    round_up(numel + E*(block_size-1), block_size) (the pad_sorted_ids=True layout the
    grouped ops require); order is expert ascending, slot ascending."""
    _check(topk_ids.is_cuda and topk_ids.dtype == torch.int32, "topk_ids must be CUDA int32")
    ids = topk_ids.contiguous()
    numel = ids.numel()
    P = lib.w4a8_moe_align_sorted_len(numel, num_experts, block_size)
    dev = ids.device
    sorted_ids = torch.empty((P,), dtype=torch.int32, device=dev)
    expert_ids = torch.empty((P // block_size,), dtype=torch.int32, device=dev)
    ntp = torch.empty((1,), dtype=torch.int32, device=dev)
    emap = None
    if expert_map is not None:
        emap = expert_map.to(device=dev, dtype=torch.int32).contiguous()
    ws = _workspace(lib.w4a8_moe_align_workspace_size(numel, num_experts), dev)
    check(lib.w4a8_moe_align_block_size(
        _ptr(ids), numel, num_experts, block_size, _ptr(emap), _ptr(sorted_ids), P,
        _ptr(expert_ids), _ptr(ntp), ws.data_ptr(), ws.numel(), _stream(ids)),
        "moe_align_block_size")
    return sorted_ids, expert_ids, ntp


def fused_topk(hidden_states: torch.Tensor | None, gating_output: torch.Tensor, topk: int,
               renormalize: bool = True):
    """Router softmax -> top-k -> renormalise (vLLM ``fused_topk``) on gfx950.
    Returns (topk_weights fp32 (T, k), topk_ids int32 (T, k))."""
    g = gating_output.float().contiguous()
    _check(g.is_cuda and g.dim() == 2, "gating_output must be a CUDA (T, E) tensor")
    T, E = g.shape
    w = torch.empty((T, topk), dtype=torch.float32, device=g.device)
    ids = torch.empty((T, topk), dtype=torch.int32, device=g.device)
    check(lib.w4a8_topk_softmax(_ptr(g), T, E, topk, int(bool(renormalize)), _ptr(w), _ptr(ids),
                                _stream(g)), "fused_topk")
    return w, ids


def silu_and_mul(out: torch.Tensor, x: torch.Tensor) -> None:
    """vLLM ``silu_and_mul(out, x)``: (R, 2I) fp16 -> out (R, I) fp16 (moe_kernel.hip:555-561)."""
    _check(x.is_cuda and x.dtype == torch.float16 and x.is_contiguous() and x.dim() == 2,
           "x must be contiguous CUDA fp16 (R, 2I)")
    R, I2 = x.shape
    _check(out.shape == (R, I2 // 2) and out.dtype == torch.float16 and out.is_contiguous(),
           "out must be contiguous fp16 (R, I)")
    check(lib.w4a8_silu_and_mul(_ptr(x), R, I2 // 2, _ptr(out), _stream(x)), "silu_and_mul")


SWIGLUOAI_ALPHA = 1.702     # vLLM SwigluOAIAndMul defaults (gpt-oss)
SWIGLUOAI_LIMIT = 7.0


def swigluoai_and_mul(out: torch.Tensor, x: torch.Tensor, alpha: float = SWIGLUOAI_ALPHA,
                      limit: float = SWIGLUOAI_LIMIT) -> None:
    """vLLM ``swigluoai_and_mul(out, x, alpha, limit)`` (gpt-oss): (R, 2I) fp16 with gate and
    up interleaved (gate = x[:, 0::2], up = x[:, 1::2]) -> out (R, I) fp16,
    (clamp(up, -limit, limit) + 1) * g * sigmoid(alpha * g) with g = min(gate, limit)."""
    _check(x.is_cuda and x.dtype == torch.float16 and x.is_contiguous() and x.dim() == 2,
           "x must be contiguous CUDA fp16 (R, 2I)")
    R, I2 = x.shape
    _check(out.shape == (R, I2 // 2) and out.dtype == torch.float16 and out.is_contiguous(),
           "out must be contiguous fp16 (R, I)")
    check(lib.w4a8_swigluoai_and_mul(_ptr(x), R, I2 // 2, float(alpha), float(limit), _ptr(out),
                                     _stream(x)), "swigluoai_and_mul")


def repack_fragments(w_packed: torch.Tensor, scales: torch.Tensor,
                     w_zeros: torch.Tensor | None = None) -> torch.Tensor:
    """Op-layout int4 weights (E, N, K/8) int32 with their fp16 scales (E, N, K/128) and
    zero-points (E, N/8, K/128) int32 (or None) -> fragment layout (E, N/16, 17, 16 K/128)
    int32. Tile t (rows 16t .. 16t + 15): [..., :16, :] holds K/128 blocks of 1 KB, block g's
    lane l holding row 16t + l % 16 and k in [128g + 32 (l // 16), +32) (the fp8 MFMA B
    operand of lane l); [..., 16, :] holds word r K/128 + g = row 16t + r, group g: fp16 scale
    bits | zero-point << 16 (8 without zero-points). Run once at weight load (the reference's
    process_weights_after_loading, moe_experts.py:1277-1306)."""
    _check(w_packed.is_cuda and w_packed.dtype == torch.int32 and w_packed.dim() == 3,
           "w_packed must be CUDA int32 (E, N, K/8)")
    w = w_packed.contiguous()
    E, N, K8 = w.shape
    K = K8 * 8
    _check(N % 16 == 0 and K % 128 == 0, "fragment layout needs N % 16 == 0 and K % 128 == 0")
    G = K // 128
    _check(scales.dtype == torch.float16 and tuple(scales.shape) == (E, N, G)
           and scales.device == w.device, f"scales must be fp16 (E, N, K/128)=({E},{N},{G})")
    sc = scales.contiguous()
    z = _zeros_of(w_zeros, E, N, G, "zeros")
    if z is not None:
        _check(z.device == w.device, "zeros must be on w_packed's device")
    out = torch.empty((E, N // 16, 17, 16 * G), dtype=torch.int32, device=w.device)
    assert out.numel() == lib.w4a8_fragments_words(E, N, K)
    check(lib.w4a8_repack_int4_fragments(_ptr(w), _ptr(sc), _ptr(z), E, N, K, _ptr(out),
                                         _stream(w)), "repack_fragments")
    return out


def _fail(msg: str):
    raise RuntimeError(msg)


# The per-call checks of the whole-layer entry points test plain conditions first and build
# their messages only on failure (formatting every message cost ~8 us per call).
def _zeros_of(z, E, N, G, name):
    """Optional packed zero-points (E, N/8, G) int32 of one weight, or None."""
    if z is None or z.numel() == 0:
        return None
    if z.dtype != torch.int32:
        _fail(f"{name} must be int32 (packed)")
    if N % 8 != 0 or tuple(z.shape) != (E, N // 8, G):
        _fail(f"{name} must be (E, N/8, K/group)=({E},{N // 8},{G}); got {tuple(z.shape)}")
    return z if z.is_contiguous() else z.contiguous()


def _layer_args(x, w13, w2, w13_s, w2_s, w13_z, w2_z, topk_weights, topk_ids, expert_map,
                global_num_experts, weight_is_e2m1):
    """Validation shared by the whole-layer entry points (the checks bindings.cpp:191-221 and
    _check_moe_common make for the grouped ops, applied to both GEMMs of the layer), so a
    mismatched tensor raises here instead of becoming an out-of-bounds read on the device.
    Shapes are checked before devices. Returns the sizes, the zero-point tensors, the expert
    map and the workspace."""
    if x.dtype not in (torch.float16, torch.bfloat16) or x.dim() != 2:
        _fail("x must be fp16/bf16 (T, H)")
    T, H = x.shape
    frag = w13.dim() == 4
    if w2.dim() != w13.dim():
        _fail("w13 and w2 must share a layout")
    if frag:
        if w13.shape[2] != 17 or w2.shape[2] != 17 or w13.shape[3] % 16 != 0:
            _fail("fragment-layout weights must be (E, N/16, 17, 16 K/128)")
        E, nt13 = w13.shape[:2]
        g13 = w13.shape[3] // 16
        if nt13 % 2 != 0:
            _fail("w13 fragments must hold 2*inter rows")
        inter = nt13 * 8
        if g13 * 128 != H:
            _fail(f"w13 fragments must cover K = H = {H}")
        if tuple(w2.shape) != (E, H // 16, 17, 16 * (inter // 128)):
            _fail(f"w2 fragments must be (E, H/16, 17, 16 inter/128)="
                  f"({E},{H // 16},17,{16 * (inter // 128)})")
        if weight_is_e2m1:
            _fail("fragment layout holds int4 weights only")
    else:
        if w13.dim() != 3:
            _fail("w13 must be (E, 2*inter, H/8) int32")
        E, I2, kw = w13.shape
        if kw * 8 != H or I2 % 2 != 0:
            _fail(f"w13 must be (E, 2*inter, H/8) with H={H}")
        inter = I2 // 2
        if tuple(w2.shape) != (E, H, inter // 8):
            _fail(f"w2 must be (E, H, inter/8)=({E},{H},{inter // 8})")
    if w13.dtype != torch.int32 or w2.dtype != torch.int32:
        _fail("weights must be int32")
    if w13_s.dtype != torch.float16 or w2_s.dtype != torch.float16:
        _fail("scales must be fp16")
    if not (w13_s.dim() == 3 and tuple(w13_s.shape[:2]) == (E, 2 * inter) and w13_s.shape[2] > 0
            and H % w13_s.shape[2] == 0):
        _fail("w13 scales must be (E, 2*inter, H/group)")
    gs = H // w13_s.shape[2]
    if inter % gs != 0 or tuple(w2_s.shape) != (E, H, inter // gs):
        _fail(f"w2 scales must be (E, H, inter/group)=({E},{H},{inter // gs})")
    if not (w13.is_contiguous() and w2.is_contiguous() and w13_s.is_contiguous()
            and w2_s.is_contiguous()):
        _fail("weights/scales must be contiguous")
    z13 = _zeros_of(w13_z, E, 2 * inter, H // gs, "w13 zeros")
    z2 = _zeros_of(w2_z, E, H, inter // gs, "w2 zeros")
    if topk_ids.dim() != 2 or topk_ids.shape[0] != T:
        _fail(f"topk_ids must be (T, top_k) with T={T}")
    top_k = topk_ids.shape[1]
    if topk_weights.numel() != T * top_k:
        _fail(f"topk_weights must have T*top_k={T * top_k} entries")
    emap = None
    if expert_map is not None:
        if expert_map.dim() != 1:
            _fail("expert_map must be 1-d (global_num_experts,)")
        emap = expert_map.to(torch.int32).contiguous()
        n_global = emap.numel() if global_num_experts is None else int(global_num_experts)
        if n_global != emap.numel():
            _fail(f"expert_map must have global_num_experts={n_global} entries")
    else:
        n_global = E if global_num_experts is None else int(global_num_experts)
        if n_global != E:
            _fail("global_num_experts differs from the local expert count; pass expert_map")
    dev = x.device
    for t in (x, w13, w2, w13_s, w2_s, topk_weights, topk_ids, z13, z2, emap):
        if t is not None and (not t.is_cuda or t.device != dev):
            _fail("all tensors must be CUDA tensors on x's device")
    ws = _workspace(lib.w4a8_moe_apply_workspace_size(T, H, inter, E, top_k), dev)
    return T, H, inter, E, gs, top_k, frag, z13, z2, emap, n_global, ws


def moe_apply(x, w13, w2, w13_s, w2_s, w13_z, w2_z, topk_weights, topk_ids, expert_map=None,
              weight_is_e2m1: bool = False, global_num_experts: int | None = None) -> torch.Tensor:
    """Whole gated-SiLU MoE layer in one C-ABI call (the _run_grouped_moe composition,
    moe_experts.py:493-665). x (T, H) fp16/bf16 -> (T, H) same dtype. w13 / w2 are op-layout
    (E, N, K/8) int32, or both fragment layout from repack_fragments (4-d). topk_ids hold
    global expert ids; with expert_map (global_num_experts entries, -1 = not local) they are
    mapped to the E local experts."""
    x = x.contiguous()
    T, H, inter, E, gs, top_k, frag, z13, z2, emap, n_global, ws = _layer_args(
        x, w13, w2, w13_s, w2_s, w13_z, w2_z, topk_weights, topk_ids, expert_map,
        global_num_experts, weight_is_e2m1)
    tw = topk_weights.to(torch.float32).contiguous()
    ids = topk_ids.to(torch.int32).contiguous()
    out = torch.empty_like(x)
    dt = 1 if x.dtype == torch.bfloat16 else 0
    if frag:
        check(lib.w4a8_moe_apply_fragments(
            _ptr(x), dt, T, H, inter, E, top_k, gs, _ptr(w13), _ptr(w13_s), _ptr(z13), _ptr(w2),
            _ptr(w2_s), _ptr(z2), _ptr(tw), _ptr(ids), _ptr(emap), n_global, _ptr(out),
            ws.data_ptr(), ws.numel(), _stream(x)), "moe_apply")
    else:
        check(lib.w4a8_moe_apply(
            _ptr(x), dt, T, H, inter, E, top_k, gs, _ptr(w13), _ptr(w13_s), _ptr(z13), _ptr(w2),
            _ptr(w2_s), _ptr(z2), _ptr(tw), _ptr(ids), _ptr(emap), n_global,
            int(bool(weight_is_e2m1)), _ptr(out), ws.data_ptr(), ws.numel(), _stream(x)),
            "moe_apply")
    return out


def moe_forward(x, router_logits, top_k: int, w13, w2, w13_s, w2_s, w13_z, w2_z,
                renormalize: bool = True, expert_map=None):
    """Router (softmax / top-k / renormalise, the vLLM fused_topk contract) plus the expert
    path in one C-ABI call. router_logits is (T, global experts): E without expert_map, else
    the map's length. Returns (out (T, H) in x.dtype, topk_weights (T, k) fp32, topk_ids
    (T, k) int32)."""
    x = x.contiguous()
    _check(router_logits.dim() == 2 and router_logits.shape[0] == x.shape[0],
           "router_logits must be (T, global experts)")
    T = x.shape[0]
    tw = torch.empty((T, top_k), dtype=torch.float32, device=x.device)
    ids = torch.empty((T, top_k), dtype=torch.int32, device=x.device)
    T, H, inter, E, gs, top_k, frag, z13, z2, emap, n_global, ws = _layer_args(
        x, w13, w2, w13_s, w2_s, w13_z, w2_z, tw, ids, expert_map, router_logits.shape[1], False)
    lg = router_logits.to(torch.float32).contiguous()
    out = torch.empty_like(x)
    check(lib.w4a8_moe_forward(
        _ptr(x), 1 if x.dtype == torch.bfloat16 else 0, T, H, inter, E, top_k, gs, _ptr(lg),
        int(bool(renormalize)), _ptr(w13), _ptr(w13_s), _ptr(z13), _ptr(w2), _ptr(w2_s),
        _ptr(z2), 1 if frag else 0, _ptr(emap), n_global, _ptr(tw), _ptr(ids), _ptr(out),
        ws.data_ptr(), ws.numel(), _stream(x)), "moe_forward")
    return out, tw, ids


def fragments_supported(hidden: int, inter: int, group_size: int) -> bool:
    """Whether moe_apply takes fragment-layout weights of this shape for every batch size
    (what a load hook checks before it repacks)."""
    return bool(lib.w4a8_moe_fragments_supported(int(hidden), int(inter), int(group_size)))


def set_decode_fused(on: bool) -> bool:
    """Runs the decode layer's two GEMVs as one persistent launch (on) or two launches (off,
    the default unless W4A8_DECODE_FUSED=1); returns the previous setting. Process-wide."""
    return bool(lib.w4a8_set_decode_fused(1 if on else 0))


def set_prefill_pair(on: bool) -> bool:
    """Runs gemm1+SiLU and gemm2 of the many-token schedule's activation-resident tiles as one
    launch where both apply (on, the default unless W4A8_PREFILL_PAIR=0) or as two launches
    (off); the results are the same bits. Returns the previous setting. Process-wide."""
    return bool(lib.w4a8_set_prefill_pair(1 if on else 0))


def _decode_fused_test_fault(on: bool) -> None:
    """Test hook: makes the fused decode layer's in-kernel waits give up (its output is then
    NaN), on the current device, until switched off."""
    check(lib.w4a8_decode_fused_test_fault(1 if on else 0), "decode fused test hook")
