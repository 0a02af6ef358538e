"""MoE composition, weight-layout converters and the vLLM MoeWNA16 hook (gfx950).

Mirrors w4a8_fp8_wmma/w4a8_fp8_wmma/moe_experts.py of patcarter883/rdna4-vllm:
  * ``_run_grouped_moe`` keeps the reference signature and return contract
    (moe_experts.py:493-665): (M, K) output in ``out_dtype``, topk-weighted and reduced;
  * the AWQ / compressed-tensors / MoeWNA16 converters (:331-482) produce the op layout;
  * ``register_moe_wna16`` patches ``MoeWNA16Method`` (:1253-1341) when vLLM is present.

On MI355X the SiLU-gated path is one C-ABI call (``moe_apply``) that schedules
align -> act-quant -> gemm1+SiLU -> act-quant -> gemm2 -> weighted reduce on the GPU.
There is no crossover gate and no stock fallback: every supported batch runs here.
"""
from __future__ import annotations

import logging
import os
from typing import Optional

import torch

from . import _ops
from . import (mmq_fp8_moe_gemm, mmq_fp8_moe_gather_reduce, moe_align_block_size,
               silu_and_mul)

logger = logging.getLogger(__name__)

_REVERSE_AWQ_PACK_ORDER = [0, 4, 1, 5, 2, 6, 3, 7]   # moe_experts.py:47
_VALID_MOE_KERNELS = ("scalar", "wmma", "gemv")      # moe_experts.py:72
GEMV_MAX_M = 96                                      # moe_experts.py:563
APPLY_CHUNK = 4096                                   # moe_experts.py:533


# --------------------------------------------------------------------------- #
# env surface (moe_experts.py:61-122)
# --------------------------------------------------------------------------- #
def _moe_enabled() -> bool:
    if os.environ.get("VLLM_ROCM_USE_W4A8_FP8_WMMA", "1") != "1":
        return False
    return os.environ.get("VLLM_ROCM_W4A8_FP8_WMMA_MOE", "1") == "1"


def _raise_if_removed_moe_env() -> None:
    """Hard-break on the removed numeric kernel override (moe_experts.py:75-86)."""
    if "VLLM_ROCM_W4A8_FP8_WMMA_MOE_VERSION" in os.environ:
        raise RuntimeError(
            "VLLM_ROCM_W4A8_FP8_WMMA_MOE_VERSION is removed; set "
            "VLLM_ROCM_W4A8_FP8_WMMA_MOE_KERNEL=wmma|scalar|gemv instead.")


def _moe_kernel() -> str:
    """Grouped-kernel name from VLLM_ROCM_W4A8_FP8_WMMA_MOE_KERNEL (moe_experts.py:89-100)."""
    _raise_if_removed_moe_env()
    kernel = os.environ.get("VLLM_ROCM_W4A8_FP8_WMMA_MOE_KERNEL", "wmma")
    if kernel not in _VALID_MOE_KERNELS:
        raise RuntimeError(
            f"VLLM_ROCM_W4A8_FP8_WMMA_MOE_KERNEL={kernel!r} invalid; "
            f"use one of {list(_VALID_MOE_KERNELS)}")
    return kernel


def _choose_block_m(M: int, top_k: int, num_experts: int) -> int:
    """moe_align block size for the op-composed path (moe_experts.py:314-325)."""
    env = os.environ.get("VLLM_ROCM_W4A8_FP8_WMMA_MOE_BLOCK_M")
    if env:
        return int(env)
    return 64


def _supported_group_size(gs) -> bool:
    return gs is not None and 16 <= gs <= 128 and gs % 16 == 0   # moe_experts.py:485-486


# --------------------------------------------------------------------------- #
# weight-layout converters
# --------------------------------------------------------------------------- #
def _awq_to_op_layout_single(qw_e, sc_e, qz_e, pf, size_bits, rev, shifts):
    """One expert AWQ (K, N/pf) packed along output, AWQ order -> op layout
    w (N, K/pf) int32, scales (N, G) fp16, zeros (N/pf, G) int32 (moe_experts.py:331-368)."""
    mask = (1 << size_bits) - 1
    K, Np = qw_e.shape
    N = Np * pf
    G = qz_e.shape[0]
    uw = ((qw_e.unsqueeze(-1) >> shifts) & mask)[:, :, rev].reshape(K, N)
    uw = uw.t().contiguous().to(torch.int32)                     # (N, K)
    w = torch.zeros((N, K // pf), dtype=torch.int32, device=qw_e.device)
    for j in range(pf):
        w |= (uw[:, j::pf] & mask) << (j * size_bits)
    s = sc_e.t().contiguous().to(torch.float16)
    uz = ((qz_e.unsqueeze(-1) >> shifts) & mask)[:, :, rev].reshape(G, N)
    uz = uz.t().contiguous().to(torch.int32)                     # (N, G)
    z = torch.zeros((N // pf, G), dtype=torch.int32, device=qw_e.device)
    for j in range(pf):
        z |= (uz[j::pf, :] & mask) << (j * size_bits)
    return w, s, z


def _awq_moe_to_op_layout(qweight, scales, qzeros, group_size, size_bits: int = 4):
    """AWQ MoE (E, K, N/8) -> (w (E,N,K/8), scales (E,N,G) fp16, zeros (E,N/8,G))
    (moe_experts.py:371-396). Looped over experts to bound transient memory."""
    pf = 32 // size_bits
    dev = qweight.device
    rev = torch.tensor(_REVERSE_AWQ_PACK_ORDER[:pf], dtype=torch.long, device=dev)
    shifts = torch.arange(0, 32, size_bits, dtype=torch.int32, device=dev)
    outs = [_awq_to_op_layout_single(qweight[e], scales[e], qzeros[e], pf, size_bits, rev, shifts)
            for e in range(qweight.shape[0])]
    return tuple(torch.stack(t).contiguous() for t in zip(*outs))


def _ct_to_op_layout_single(qw_e, sc_e, pf, size_bits, shifts):
    """compressed-tensors (GPTQ-convention, packed along K) -> op layout
    (moe_experts.py:409-434)."""
    mask = (1 << size_bits) - 1
    Kp, N = qw_e.shape
    K = Kp * pf
    uw = ((qw_e.unsqueeze(1) >> shifts.view(1, pf, 1)) & mask).reshape(K, N)
    w_kn = uw.t().contiguous().to(torch.int32)
    w = torch.zeros((N, K // pf), dtype=torch.int32, device=qw_e.device)
    for j in range(pf):
        w |= (w_kn[:, j::pf] & mask) << (j * size_bits)
    return w, sc_e.t().contiguous().to(torch.float16)


def _ct_moe_to_op_layout(qweight, scales, size_bits: int = 4):
    """(moe_experts.py:437-454); symmetric uint4b8, no zero-points."""
    pf = 32 // size_bits
    shifts = torch.arange(0, 32, size_bits, dtype=torch.int32, device=qweight.device)
    outs = [_ct_to_op_layout_single(qweight[e], scales[e], pf, size_bits, shifts)
            for e in range(qweight.shape[0])]
    return tuple(torch.stack(t).contiguous() for t in zip(*outs))


def _wna16_moe_to_op_layout(qweight_u8, scales, qzeros_u8):
    """MoeWNA16 u8 params -> op layout, zero-copy for the weights (moe_experts.py:473-482):
    (E, N, K/2) u8 .view(int32) -> (E, N, K/8); qzeros (E, N/2, G) u8 -> (E, N/8, G) int32."""
    w = qweight_u8.contiguous().view(torch.int32)
    s = scales if scales.dtype == torch.float16 else scales.to(torch.float16)
    z = None
    if qzeros_u8 is not None:
        E, Nh, G = qzeros_u8.shape
        zi = qzeros_u8.contiguous().to(torch.int32).reshape(E, Nh // 4, 4, G)
        z = (zi[:, :, 0, :] | (zi[:, :, 1, :] << 8) | (zi[:, :, 2, :] << 16)
             | (zi[:, :, 3, :] << 24)).contiguous()
    return w, s, z


# --------------------------------------------------------------------------- #
# composition
# --------------------------------------------------------------------------- #
def _activation_name(activation) -> str:
    v = getattr(activation, "value", activation)
    return str(v).lower().split(".")[-1]


def _run_unfused(x16, w1, w2, w1_s, w2_s, w1_zp, w2_zp, tw_flat, topk_ids, top_k,
                 global_num_experts, expert_map, kernel, weight_is_e2m1, w1_bias, w2_bias):
    """Op-by-op composition (moe_experts.py:587-665): align -> gemm1 -> (+bias) ->
    silu_and_mul -> gemm2 (identity gather) -> (+bias) -> gather-reduce. Used for the
    "scalar" golden kernel and for per-expert biases."""
    block_m = _choose_block_m(x16.size(0), top_k, w1.size(0))
    sorted_ids, expert_ids, ntp = moe_align_block_size(
        topk_ids, block_m, global_num_experts, expert_map)
    P = sorted_ids.size(0)

    def _expand_bias(bias):
        return bias[expert_ids.clamp(min=0).long()].repeat_interleave(block_m, dim=0)[:P]

    out1 = mmq_fp8_moe_gemm(x16, w1, w1_s, sorted_ids, expert_ids, ntp, top_k, block_m,
                            kernel=kernel, w_zeros=w1_zp, weight_is_e2m1=weight_is_e2m1)
    if w1_bias is not None:
        out1 = out1 + _expand_bias(w1_bias).to(out1.dtype)
    buf2 = torch.empty((P, out1.size(1) // 2), dtype=torch.float16, device=x16.device)
    silu_and_mul(buf2, out1.contiguous())
    ident = torch.arange(P, dtype=torch.int32, device=x16.device)
    out2 = mmq_fp8_moe_gemm(buf2, w2, w2_s, ident, expert_ids, ntp, 1, block_m,
                            kernel=kernel, w_zeros=w2_zp, weight_is_e2m1=weight_is_e2m1)
    if w2_bias is not None:
        out2 = out2 + _expand_bias(w2_bias).to(out2.dtype)
    return mmq_fp8_moe_gather_reduce(out2.contiguous(), sorted_ids, tw_flat, ntp, top_k)


def _run_grouped_moe(x, w1, w2, w1_s, w2_s, w1_zp, w2_zp,
                     topk_weights, topk_ids, activation,
                     global_num_experts, expert_map,
                     apply_router_weight_on_input, kernel, out_dtype=None,
                     weight_is_e2m1=False, w1_bias=None, w2_bias=None):
    """Whole gated MoE -> (M, K) in ``out_dtype`` (moe_experts.py:493-665).

    Weights are in op layout: w1 (E, 2*inter, K/8), w2 (E, K, inter/8), scales
    (E, N, K/g), zero-points (E, N/8, K/g) or None (symmetric, zp = 8)."""
    M, K = x.shape
    top_k = topk_ids.size(1)
    if out_dtype is None:
        out_dtype = x.dtype
    if _activation_name(activation) != "silu":
        raise NotImplementedError(
            f"w4a8_fp8_wmma (gfx950) implements the SiLU-gated MoE; got {activation!r}")
    if kernel not in _VALID_MOE_KERNELS:
        raise ValueError(f"unknown moe kernel {kernel!r}; known: {list(_VALID_MOE_KERNELS)}")

    chunk = int(os.environ.get("VLLM_ROCM_W4A8_FP8_WMMA_MOE_APPLY_CHUNK", str(APPLY_CHUNK)))
    if chunk and M > chunk and not apply_router_weight_on_input:
        out = torch.empty((M, K), dtype=out_dtype, device=x.device)
        for lo in range(0, M, chunk):
            hi = min(lo + chunk, M)
            out[lo:hi] = _run_grouped_moe(
                x[lo:hi], w1, w2, w1_s, w2_s, w1_zp, w2_zp, topk_weights[lo:hi],
                topk_ids[lo:hi], activation, global_num_experts, expert_map, False, kernel,
                out_dtype, weight_is_e2m1=weight_is_e2m1, w1_bias=w1_bias, w2_bias=w2_bias)
        return out

    w1_s = w1_s if w1_s.dtype == torch.float16 else w1_s.to(torch.float16)
    w2_s = w2_s if w2_s.dtype == torch.float16 else w2_s.to(torch.float16)
    x_in = x
    if apply_router_weight_on_input:
        assert top_k == 1, "router-weight-on-input requires top_k==1"
        x_in = x_in * topk_weights.reshape(M, 1).to(x_in.dtype)
        tw = torch.ones((M, top_k), dtype=torch.float32, device=x.device)
    else:
        tw = topk_weights.to(torch.float32)
    ids = topk_ids.to(torch.int32)

    has_bias = w1_bias is not None or w2_bias is not None
    if kernel == "scalar" or has_bias:
        x16 = x_in.to(torch.float16).contiguous()
        acc = _run_unfused(x16, w1, w2, w1_s, w2_s, w1_zp, w2_zp, tw.reshape(-1).contiguous(),
                           ids, top_k, global_num_experts, expert_map, kernel, weight_is_e2m1,
                           w1_bias, w2_bias)
        return acc.to(out_dtype)

    if global_num_experts != w1.size(0) and expert_map is None:
        raise ValueError("global_num_experts differs from the local expert count; "
                         "pass expert_map")
    xin = x_in if x_in.dtype in (torch.float16, torch.bfloat16) else x_in.to(torch.float16)
    out = _ops.moe_apply(xin, w1, w2, w1_s, w2_s, w1_zp, w2_zp, tw, ids, expert_map,
                         weight_is_e2m1)
    return out if out.dtype == out_dtype else out.to(out_dtype)


# --------------------------------------------------------------------------- #
# opaque op for torch.compile / graph capture (moe_experts.py:679-733)
# --------------------------------------------------------------------------- #
def _w4a8_moe_apply(x: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor, w1_s: torch.Tensor,
                    w2_s: torch.Tensor, w1_zp: Optional[torch.Tensor],
                    w2_zp: Optional[torch.Tensor], topk_weights: torch.Tensor,
                    topk_ids: torch.Tensor, activation: str, global_num_experts: int,
                    expert_map: Optional[torch.Tensor], apply_router_weight_on_input: bool,
                    kernel: str) -> torch.Tensor:
    return _run_grouped_moe(x, w1, w2, w1_s, w2_s, w1_zp, w2_zp, topk_weights, topk_ids,
                            activation, global_num_experts, expert_map,
                            apply_router_weight_on_input, kernel, out_dtype=x.dtype)


def _w4a8_moe_apply_fake(x, w1, w2, w1_s, w2_s, w1_zp, w2_zp, topk_weights, topk_ids,
                         activation, global_num_experts, expert_map,
                         apply_router_weight_on_input, kernel):
    return torch.empty_like(x)


if not hasattr(torch.ops.vllm, "w4a8_moe_apply"):
    torch.library.custom_op("vllm::w4a8_moe_apply", mutates_args=())(_w4a8_moe_apply)
    torch.library.register_fake("vllm::w4a8_moe_apply")(_w4a8_moe_apply_fake)


# --------------------------------------------------------------------------- #
# vLLM MoeWNA16 hook (moe_experts.py:1253-1341)
# --------------------------------------------------------------------------- #
_MOE_WNA16_REGISTERED = False


def register_moe_wna16(verbose: bool = True) -> bool:
    """Route int4 MoeWNA16 expert layers to the gfx950 path by patching
    ``MoeWNA16Method.process_weights_after_loading`` (zero-copy op-layout views) and
    ``.apply`` (``_run_grouped_moe``). Idempotent; returns False without vLLM or when
    disabled by env. Engages for every batch (no crossover gate)."""
    global _MOE_WNA16_REGISTERED
    if _MOE_WNA16_REGISTERED:
        return True
    _raise_if_removed_moe_env()
    if not _moe_enabled():
        if verbose:
            print("[w4a8_fp8_wmma] WNA16 MoE disabled via env")
        return False
    try:
        from vllm.model_executor.layers.quantization.moe_wna16 import MoeWNA16Method
    except Exception as e:  # noqa: BLE001  (vLLM absent: nothing to patch)
        if verbose:
            print(f"[w4a8_fp8_wmma] WNA16 MoE: vLLM not importable ({type(e).__name__})")
        return False
    install_moe_wna16_hooks(MoeWNA16Method, verbose)
    _MOE_WNA16_REGISTERED = True
    return True


def install_moe_wna16_hooks(method_cls, verbose: bool = False) -> None:
    """Patch ``process_weights_after_loading`` / ``apply`` on a MoeWNA16Method-like class
    (split out so tests can drive it with a stand-in class)."""
    _orig_process = method_cls.process_weights_after_loading
    _orig_apply = method_cls.apply

    def _patched_process(self, layer):
        try:
            eng = (self.quant_config.weight_bits == 4
                   and _supported_group_size(layer.group_size))
        except Exception:  # noqa: BLE001
            eng = False
        self._w4a8_wna16 = eng
        _orig_process(self, layer)
        if not eng:
            return
        has_zp = bool(getattr(self.quant_config, "has_zp", False))
        w13, w13_s, w13_z = _wna16_moe_to_op_layout(
            layer.w13_qweight.data, layer.w13_scales.data,
            layer.w13_qzeros.data if has_zp else None)
        w2, w2_s, w2_z = _wna16_moe_to_op_layout(
            layer.w2_qweight.data, layer.w2_scales.data,
            layer.w2_qzeros.data if has_zp else None)
        layer._w4a8_w13, layer._w4a8_w2 = w13, w2
        layer._w4a8_w13s, layer._w4a8_w2s = w13_s, w2_s
        layer._w4a8_w13z, layer._w4a8_w2z = w13_z, w2_z
        if verbose:
            print(f"[w4a8_fp8_wmma] WNA16 MoE weights ready (int4 g={layer.group_size} "
                  f"has_zp={has_zp}) -> gfx950 grouped fp8 MFMA")

    def _patched_apply(self, layer, x, topk_weights, topk_ids, shared_experts=None,
                       shared_experts_input=None):
        if not getattr(self, "_w4a8_wna16", False):
            return _orig_apply(self, layer, x, topk_weights, topk_ids, shared_experts,
                               shared_experts_input)
        x2 = x.reshape(-1, x.shape[-1])
        out = _run_grouped_moe(
            x2, layer._w4a8_w13, layer._w4a8_w2, layer._w4a8_w13s, layer._w4a8_w2s,
            layer._w4a8_w13z, layer._w4a8_w2z, topk_weights, topk_ids, layer.activation,
            layer.global_num_experts, layer.expert_map, layer.apply_router_weight_on_input,
            _moe_kernel(), out_dtype=x.dtype)
        return out.reshape(x.shape[:-1] + (out.shape[-1],))

    method_cls.process_weights_after_loading = _patched_process
    method_cls.apply = _patched_apply
