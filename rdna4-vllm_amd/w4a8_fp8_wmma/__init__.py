"""W4A8 (int4 weights, fp8-e4m3 activations) MoE expert path for AMD MI355X (gfx950).

Drop-in for the ``w4a8_fp8_wmma`` package of patcarter883/rdna4-vllm: the same public
wrappers (w4a8_fp8_wmma/w4a8_fp8_wmma/__init__.py:60-236), the same torch-op schemas
(w4a8_fp8_wmma/bindings.cpp:388-413) and the same name <-> opaque-kernel-id maps
(:10-22). Kernels are hand-written HIP for CDNA4 behind the C ABI in
``include/w4a8_moe.h``; importing this package loads that library and fails if it is
missing (there is no CPU fallback).

Kernel names: "scalar" runs the scalar golden schedule, "wmma" the fp8-MFMA tiled
grouped GEMM, "gemv" the decode GEMV (fp8 MFMA on compacted token rows).
"""
import torch  # noqa: F401  (torch owns device memory and streams)

from . import _ops  # noqa: F401  registers torch.ops.w4a8_fp8_wmma.*
from ._ops import (  # noqa: F401
    act_quant_fp8,
    dequant_fp8,
    fragments_supported,
    fused_topk,
    moe_align_block_size,
    moe_apply,
    moe_forward,
    repack_fragments,
    set_decode_fused,
    set_prefill_pair,
    silu_and_mul,
)

_MOE_KERNELS = {"scalar": 0, "wmma": 6, "gemv": 7}

_DENSE_KERNELS = {
    "reference_scalar": 0, "rocwmma_v1": 1, "rocwmma_tiled": 2, "rocwmma_pipe": 4,
    "prefill_wmma": 5, "prefill_wmma_b128": 6, "wmma_tiled_tuned": 7, "wmma_dbuf": 8,
    "wmma_dbuf2": 9, "prefill_wmma_ashuffle": 10, "decode_gemv": 11,
    "splitk_smallm": 12, "regdirect_shuffle": 13, "nsplit_smallm": 14,
}


def _resolve_dense_kernel(kernel) -> int:
    """Descriptive dense kernel name -> op id; unknown names / legacy ints raise
    (w4a8_fp8_wmma/__init__.py:25-36)."""
    if isinstance(kernel, str):
        try:
            return _DENSE_KERNELS[kernel]
        except KeyError:
            raise ValueError(
                f"unknown dense kernel {kernel!r}; known: {sorted(_DENSE_KERNELS)}") from None
    raise TypeError(
        f"dense kernel must be a name in {sorted(_DENSE_KERNELS)} (the integer "
        f"'version' was removed); got {kernel!r}")


def _resolve_moe_kernel(kernel) -> int:
    """Descriptive MoE kernel name -> op id (w4a8_fp8_wmma/__init__.py:39-49)."""
    if isinstance(kernel, str):
        try:
            return _MOE_KERNELS[kernel]
        except KeyError:
            raise ValueError(
                f"unknown moe kernel {kernel!r}; known: {sorted(_MOE_KERNELS)}") from None
    raise TypeError(
        f"moe kernel must be a name in {sorted(_MOE_KERNELS)} (the integer 'version' was "
        f"removed); got {kernel!r}")


def _empty_zeros(w_zeros, device):
    if w_zeros is None:
        return torch.empty(0, dtype=torch.int32, device=device)
    return w_zeros


def mmq_fp8_gemm(x, w_packed, scales, kernel="reference_scalar", w_zeros=None,
                 weight_is_e2m1=False):
    """Dense W4A8 GEMM: x (M, K) fp16, w_packed (N, K/8) int32, scales (N, K/g) fp16,
    optional w_zeros (N/8, K/g) int32 -> (M, N) fp16 (__init__.py:60-89)."""
    return torch.ops.w4a8_fp8_wmma.mmq_fp8_gemm(
        x, w_packed, scales, _empty_zeros(w_zeros, x.device), _resolve_dense_kernel(kernel),
        weight_is_e2m1)


def mmq_fp8_moe_gemm(x, w_packed, scales, sorted_token_ids, expert_ids,
                     num_tokens_post_padded, top_k, block_m, kernel="wmma", w_zeros=None,
                     weight_is_e2m1=False):
    """Grouped W4A8 GEMM in the padded sorted layout: out[r] = x[sorted_token_ids[r] //
    top_k] @ W[expert_ids[r // block_m]]^T for real rows r -> (P, N) fp16
    (__init__.py:92-133). Padding rows are not written."""
    return torch.ops.w4a8_fp8_wmma.mmq_fp8_moe_gemm(
        x, w_packed, scales, _empty_zeros(w_zeros, x.device), sorted_token_ids, expert_ids,
        num_tokens_post_padded, top_k, block_m, _resolve_moe_kernel(kernel), weight_is_e2m1)


def mmq_fp8_moe_gemm1_silu(x, w_packed, scales, sorted_token_ids, expert_ids,
                           num_tokens_post_padded, top_k, block_m, kernel="wmma",
                           w_zeros=None, weight_is_e2m1=False):
    """Fused gemm1 (w13 = [gate | up]) + silu_and_mul -> (P, inter) fp16, bit-exact to
    mmq_fp8_moe_gemm + silu_and_mul (__init__.py:136-178)."""
    return torch.ops.w4a8_fp8_wmma.mmq_fp8_moe_gemm1_silu(
        x, w_packed, scales, _empty_zeros(w_zeros, x.device), sorted_token_ids, expert_ids,
        num_tokens_post_padded, top_k, block_m, _resolve_moe_kernel(kernel), weight_is_e2m1)


def mmq_fp8_moe_gemm_scatter(x, w_packed, scales, sorted_token_ids, expert_ids,
                             num_tokens_post_padded, topk_weights, output, top_k, block_m,
                             kernel="wmma", w_zeros=None, weight_is_e2m1=False):
    """Fused gemm2 + top-k weight + atomic scatter into the pre-zeroed fp32 `output`
    (M, N), in place (__init__.py:181-218)."""
    torch.ops.w4a8_fp8_wmma.mmq_fp8_moe_gemm_scatter(
        x, w_packed, scales, _empty_zeros(w_zeros, x.device), sorted_token_ids, expert_ids,
        num_tokens_post_padded, topk_weights, output, top_k, block_m,
        _resolve_moe_kernel(kernel), weight_is_e2m1)


def mmq_fp8_moe_gather_reduce(out2, sorted_token_ids, topk_weights, num_tokens_post_padded,
                              top_k):
    """Deterministic weighted gather-reduce (P, N) fp16 -> (M, N) fp32 (__init__.py:221-236)."""
    return torch.ops.w4a8_fp8_wmma.mmq_fp8_moe_gather_reduce(
        out2, sorted_token_ids, topk_weights, num_tokens_post_padded, top_k)


from . import linear  # noqa: E402,F401  defines torch.ops.vllm.w4a8_dense_apply

__all__ = [
    "mmq_fp8_gemm", "mmq_fp8_moe_gemm", "mmq_fp8_moe_gemm1_silu", "mmq_fp8_moe_gemm_scatter",
    "mmq_fp8_moe_gather_reduce", "act_quant_fp8", "dequant_fp8", "fragments_supported",
    "fused_topk",
    "moe_align_block_size", "moe_apply", "moe_forward", "repack_fragments", "set_decode_fused",
    "set_prefill_pair", "silu_and_mul",
]
