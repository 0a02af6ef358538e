"""MoE composition, weight-format conversion and the vLLM MoeWNA16 load/apply hook (gfx950).

Call surface of w4a8_fp8_wmma/w4a8_fp8_wmma/moe_experts.py in patcarter883/rdna4-vllm:
  * ``_run_grouped_moe`` keeps the reference argument list and return contract
    (moe_experts.py:493-665): an (M, K) output in ``out_dtype``, top-k weighted and reduced;
  * ``_awq_moe_to_op_layout`` / ``_ct_moe_to_op_layout`` / ``_wna16_moe_to_op_layout`` turn the
    on-disk formats into the op layout (:331-482);
  * ``register_moe_wna16`` patches ``MoeWNA16Method`` (:1253-1341) when vLLM is present;
  * ``register_moe_mxfp4`` patches ``GptOssMxfp4MoEMethod`` (:1351-1450): E2M1 weights,
    E8M0 scales converted to fp16 at load, biases and the swigluoai activation.

On MI355X the SiLU-gated layer is one C-ABI call (``moe_apply``): align, act-quant,
gemm1+SiLU, act-quant, gemm2 and the weighted reduce all run on the GPU. The WNA16 load hook
repacks the int4 weights once into the fragment layout the gfx950 kernels stream (weights
and each tile's scale / zero-point words), which replaces the u8 parameters' data. There is
no crossover gate and no stock fallback.
"""
from __future__ import annotations

import dataclasses
import logging
import os
from typing import Optional

import torch

from . import _ops
from . import (mmq_fp8_moe_gemm, mmq_fp8_moe_gather_reduce, moe_align_block_size,
               silu_and_mul)

logger = logging.getLogger(__name__)

# Bit position (in nibbles) of logical column c inside an AWQ-packed int32 word: the AWQ
# writer interleaves the eight columns as 0, 2, 4, 6, 1, 3, 5, 7 (moe_experts.py:47 holds the
# inverse list, [0, 4, 1, 5, 2, 6, 3, 7], which reads column c from nibble AWQ_NIBBLE_OF[c]).
AWQ_NIBBLE_OF = (0, 4, 1, 5, 2, 6, 3, 7)
MOE_KERNEL_NAMES = ("scalar", "wmma", "gemv")        # moe_experts.py:72
# gated activations between the GEMMs: SiLU (fused into gemm1 on the whole-layer path) and
# gpt-oss's swigluoai (op by op, as the reference's mxfp4 hook runs it)
GATED_ACTIVATIONS = ("silu", "swigluoai")
GEMV_MAX_M = 96                                      # moe_experts.py:563
APPLY_CHUNK = 4096                                   # moe_experts.py:533
# Transient bytes a converter may hold per chunk of experts (unpacked nibbles are bytes).
_CONVERT_CHUNK_BYTES = 256 << 20


# --------------------------------------------------------------------------- #
# configuration (environment names of moe_experts.py:61-122)
# --------------------------------------------------------------------------- #
@dataclasses.dataclass(frozen=True)
class MoeEnv:
    enabled: bool            # VLLM_ROCM_USE_W4A8_FP8_WMMA and VLLM_ROCM_W4A8_FP8_WMMA_MOE
    kernel: str              # VLLM_ROCM_W4A8_FP8_WMMA_MOE_KERNEL (scalar | wmma | gemv)
    block_m: Optional[int]   # VLLM_ROCM_W4A8_FP8_WMMA_MOE_BLOCK_M (op-by-op composition)
    apply_chunk: int         # VLLM_ROCM_W4A8_FP8_WMMA_MOE_APPLY_CHUNK (tokens per call)

    REMOVED = ("VLLM_ROCM_W4A8_FP8_WMMA_MOE_VERSION",)

    @classmethod
    def read(cls) -> "MoeEnv":
        env = os.environ
        for name in cls.REMOVED:
            if name in env:
                raise RuntimeError(
                    f"{name} is removed; set VLLM_ROCM_W4A8_FP8_WMMA_MOE_KERNEL="
                    f"{'|'.join(MOE_KERNEL_NAMES)} instead.")
        kernel = env.get("VLLM_ROCM_W4A8_FP8_WMMA_MOE_KERNEL", "wmma")
        if kernel not in MOE_KERNEL_NAMES:
            raise RuntimeError(f"VLLM_ROCM_W4A8_FP8_WMMA_MOE_KERNEL={kernel!r} invalid; "
                               f"use one of {list(MOE_KERNEL_NAMES)}")
        bm = env.get("VLLM_ROCM_W4A8_FP8_WMMA_MOE_BLOCK_M")
        return cls(
            enabled=(env.get("VLLM_ROCM_USE_W4A8_FP8_WMMA", "1") == "1"
                     and env.get("VLLM_ROCM_W4A8_FP8_WMMA_MOE", "1") == "1"),
            kernel=kernel,
            block_m=int(bm) if bm else None,
            apply_chunk=int(env.get("VLLM_ROCM_W4A8_FP8_WMMA_MOE_APPLY_CHUNK", str(APPLY_CHUNK))))


def _moe_enabled() -> bool:
    return MoeEnv.read().enabled


def _moe_kernel() -> str:
    """Grouped-kernel name (moe_experts.py:89-100); raises on removed or invalid knobs."""
    return MoeEnv.read().kernel


def _supported_group_size(gs) -> bool:
    """Group sizes the kernels take: multiples of 16 up to 128 (moe_experts.py:485-486)."""
    return gs is not None and gs % 16 == 0 and 16 <= gs <= 128


# --------------------------------------------------------------------------- #
# weight formats -> op layout
#
# Op layout (moe_kernel.hip:7-17): w (E, N, K/8) int32 with nibble j of word w at k = 8w + j,
# which is byte-for-byte vLLM's standard u8 layout (E, N, K/2) (byte b: k = 2b low nibble,
# 2b + 1 high); zero-points (E, N/8, G) int32 with nibble n % 8 of word n / 8, i.e. four
# consecutive bytes along N of the u8 layout (E, N/2, G).
# --------------------------------------------------------------------------- #
def _nibbles(words: torch.Tensor) -> torch.Tensor:
    """(..., W) int32 -> (..., W, 8) uint8: nibble p of each word, p = 0 lowest."""
    b = words.contiguous().view(torch.uint8).reshape(*words.shape, 4)
    return torch.stack((b & 0xF, b >> 4), dim=-1).reshape(*words.shape, 8)


def _pack_bytes_last(nib: torch.Tensor) -> torch.Tensor:
    """(..., L) nibbles (L even) -> (..., L/2) uint8, element 2i low, 2i + 1 high."""
    return nib[..., 0::2] | (nib[..., 1::2] << 4)


def _zero_bytes_to_op(zb: torch.Tensor) -> torch.Tensor:
    """Zero-point bytes grouped by K group, (E, G, N/2) u8 (byte i: n = 2i low, 2i + 1 high)
    -> op layout (E, N/8, G) int32: four consecutive bytes are one little-endian word."""
    E, G, nh = zb.shape
    words = zb.contiguous().view(-1).view(torch.int32).view(E, G, nh // 4)
    return words.transpose(1, 2).contiguous()


def _expert_chunks(E: int, bytes_per_expert: int):
    step = max(1, _CONVERT_CHUNK_BYTES // max(1, bytes_per_expert))
    for lo in range(0, E, step):
        yield lo, min(E, lo + step)


def _awq_moe_to_op_layout(qweight, scales, qzeros, group_size, size_bits: int = 4):
    """AWQ MoE checkpoint tensors -> op layout (moe_experts.py:371-396).

    qweight (E, K, N/8) int32 and qzeros (E, G, N/8) int32 pack eight output columns per word
    in the AWQ interleave; scales (E, G, N). The nibbles are regrouped by column, transposed
    to (N, K) and re-packed as the standard u8 layout, which the op layout views as int32."""
    if size_bits != 4:
        raise NotImplementedError("AWQ MoE conversion supports int4 weights only")
    order = torch.tensor(AWQ_NIBBLE_OF, dtype=torch.long, device=qweight.device)
    E, K, Nw = qweight.shape
    N = Nw * 8
    w = torch.empty((E, N, K // 2), dtype=torch.uint8, device=qweight.device)
    for lo, hi in _expert_chunks(E, K * N):
        cols = _nibbles(qweight[lo:hi]).index_select(-1, order).reshape(hi - lo, K, N)
        w[lo:hi] = _pack_bytes_last(cols.transpose(1, 2))
    zcols = _nibbles(qzeros).index_select(-1, order).reshape(E, qzeros.shape[1], N)
    return (w.view(torch.int32), scales.transpose(1, 2).contiguous().to(torch.float16),
            _zero_bytes_to_op(_pack_bytes_last(zcols)))


def _ct_moe_to_op_layout(qweight, scales, size_bits: int = 4):
    """compressed-tensors / GPTQ MoE (moe_experts.py:437-454): qweight (E, K/8, N) int32 packs
    eight consecutive k per word with nibble j = k % 8, the op layout's own word format, so
    the conversion is a transpose of whole words. Symmetric uint4b8: no zero-points."""
    if size_bits != 4:
        raise NotImplementedError("compressed-tensors MoE conversion supports int4 weights only")
    return (qweight.transpose(1, 2).contiguous(),
            scales.transpose(1, 2).contiguous().to(torch.float16))


def _wna16_moe_to_op_layout(qweight_u8, scales, qzeros_u8):
    """MoeWNA16 parameters (standard u8 layout, moe_experts.py:473-482) -> op layout: the
    weights are a zero-copy int32 view; zero-points regroup four N-bytes per int32."""
    w = qweight_u8.contiguous().view(torch.int32)
    s = scales if scales.dtype == torch.float16 else scales.to(torch.float16)
    z = None if qzeros_u8 is None else _zero_bytes_to_op(qzeros_u8.transpose(1, 2))
    return w, s, z


# mxfp4 (OCP E2M1 codes + E8M0 block scales; gpt-oss through vLLM's GptOssMxfp4MoEMethod)
MXFP4_BLOCK = 32          # one E8M0 scale per 32 weights along K (the MX block)


def e8m0_to_fp16(scale_u8: torch.Tensor) -> torch.Tensor:
    """E8M0 block scales (uint8, value 2^(s - 127)) -> fp16, built from the exponent bits:
    2^e is exact in fp16 for e in [-24, 15] (subnormal below -14); below that it rounds to 0,
    above to +inf (also for the E8M0 NaN code 255), as the reference's fp32 power cast to fp16
    gives (mxfp4/convert.py:68-98). Same device as the input."""
    if scale_u8.dtype != torch.uint8:
        raise TypeError(f"E8M0 scales must be uint8, got {scale_u8.dtype}")
    e = scale_u8.to(torch.int32) - 127
    sub = torch.where(e >= -24, torch.ones_like(e) << (e + 24).clamp(0, 9), torch.zeros_like(e))
    bits = torch.where(e >= -14, (e + 15).clamp(0, 31) << 10, sub)
    bits = torch.where(e > 15, torch.full_like(e, 0x7C00), bits)
    return bits.to(torch.int16).view(torch.float16)


def convert_mxfp4_moe(weight_packed: torch.Tensor, weight_scale: torch.Tensor) -> dict:
    """mxfp4 MoE weights -> the op layout the E2M1 kernels read (mxfp4/convert.py:100-140):
    weight_packed (E, N, K/2) uint8, two E2M1 codes a byte with the lower K index in the low
    nibble, is already the (E, N, K/8) int32 container byte for byte (code k at nibble k % 8 of
    word k / 8), so it is viewed, not copied; weight_scale (E, N, K/32) uint8 E8M0 becomes fp16
    group scales. Symmetric (no zero-points), group size 32. ``scale_info`` reports scales
    fp16 cannot hold (the reference's warning: such layers would need fp32 group scales)."""
    if weight_packed.dtype != torch.uint8 or weight_packed.dim() != 3:
        raise ValueError("mxfp4 weight_packed must be (E, N, K/2) uint8")
    E, N, kh = weight_packed.shape
    K = 2 * kh
    if K % 8 != 0 or tuple(weight_scale.shape) != (E, N, K // MXFP4_BLOCK):
        raise ValueError(f"mxfp4 weight_scale must be (E, N, K/{MXFP4_BLOCK}) for K = {K}")
    w = weight_packed.contiguous().view(torch.int32).view(E, N, K // 8)
    scales = e8m0_to_fp16(weight_scale.contiguous())
    e = weight_scale.to(torch.int32) - 127
    info = dict(exp_min=int(e.min()), exp_max=int(e.max()),
                fp16_overflow_groups=int((e > 15).sum()),
                fp16_subnormal_groups=int(((e < -14) & (e >= -24)).sum()),
                fp16_zero_groups=int((e < -24).sum()),
                e8m0_nan_groups=int((weight_scale == 255).sum()))
    info["fp16_range_ok"] = (info["fp16_overflow_groups"] == 0 and info["e8m0_nan_groups"] == 0
                             and info["fp16_zero_groups"] == 0)
    return dict(w_packed=w, scales=scales, w_zeros=None, group_size=MXFP4_BLOCK, scale_info=info)


def _fragments_to_op_layout(w_frag: torch.Tensor) -> torch.Tensor:
    """Fragment layout (E, N/16, 17, 16 K/128) -> op-layout weights (E, N, K/8): tile t's
    first 16 rows of 16 G words are its G blocks of 64 lanes x 4 words, lane l = 16 q + c of
    block g holding row 16 t + c, words 16 g + 4 q .. + 3 (row 16 is the tile's scale and
    zero-point words, which the op layout keeps in its own tensors)."""
    E, NT = w_frag.shape[:2]
    G = w_frag.shape[3] // 16
    v = w_frag[:, :, :16].reshape(E, NT, G, 4, 16, 4).permute(0, 1, 4, 2, 3, 5)
    return v.reshape(E, NT * 16, G * 16).contiguous()


# --------------------------------------------------------------------------- #
# composition
# --------------------------------------------------------------------------- #
def _activation_name(activation) -> str:
    v = getattr(activation, "value", activation)
    return str(v).lower().split(".")[-1]


def _run_unfused(x16, w1, w2, w1_s, w2_s, w1_zp, w2_zp, tw_flat, topk_ids, top_k,
                 global_num_experts, expert_map, kernel, weight_is_e2m1, w1_bias, w2_bias,
                 block_m, activation="silu"):
    """Op-by-op composition (moe_experts.py:587-665): align, gemm1, + bias, the gated
    activation (silu_and_mul on [gate | up] halves, or gpt-oss swigluoai_and_mul on
    interleaved gate/up), gemm2 on the padded rows, + bias, gather-reduce. Runs the "scalar"
    golden kernel, layers with per-expert biases and non-SiLU activations."""
    sorted_ids, expert_ids, ntp = moe_align_block_size(
        topk_ids, block_m, global_num_experts, expert_map)
    P = sorted_ids.size(0)
    # per-padded-row expert of every block, for the (E, N) bias tables
    row_expert = expert_ids.clamp(min=0).long().repeat_interleave(block_m)[:P]

    out1 = mmq_fp8_moe_gemm(x16, w1, w1_s, sorted_ids, expert_ids, ntp, top_k, block_m,
                            kernel=kernel, w_zeros=w1_zp, weight_is_e2m1=weight_is_e2m1)
    if w1_bias is not None:
        out1 = out1 + w1_bias.to(out1.dtype).index_select(0, row_expert)
    h = torch.empty((P, out1.size(1) // 2), dtype=torch.float16, device=x16.device)
    if activation == "swigluoai":
        _ops.swigluoai_and_mul(h, out1.contiguous())
    else:
        silu_and_mul(h, out1.contiguous())
    rows = torch.arange(P, dtype=torch.int32, device=x16.device)   # gemm2 gathers by row
    out2 = mmq_fp8_moe_gemm(h, w2, w2_s, rows, expert_ids, ntp, 1, block_m,
                            kernel=kernel, w_zeros=w2_zp, weight_is_e2m1=weight_is_e2m1)
    if w2_bias is not None:
        out2 = out2 + w2_bias.to(out2.dtype).index_select(0, row_expert)
    return mmq_fp8_moe_gather_reduce(out2.contiguous(), sorted_ids, tw_flat, ntp, top_k)


def _run_grouped_moe(x, w1, w2, w1_s, w2_s, w1_zp, w2_zp,
                     topk_weights, topk_ids, activation,
                     global_num_experts, expert_map,
                     apply_router_weight_on_input, kernel, out_dtype=None,
                     weight_is_e2m1=False, w1_bias=None, w2_bias=None):
    """Whole gated MoE -> (M, K) in ``out_dtype`` (moe_experts.py:493-665).

    w1 (E, 2*inter, K/8) / w2 (E, K, inter/8) int32 in the op layout, or both in the fragment
    layout (4-d, ``repack_fragments``); scales (E, N, K/g); zero-points (E, N/8, K/g) or None
    (symmetric, zp = 8). topk_ids are global expert ids; ``expert_map`` maps them to the E
    local experts."""
    M, K = x.shape
    top_k = topk_ids.size(1)
    out_dtype = x.dtype if out_dtype is None else out_dtype
    act = _activation_name(activation)
    if act not in GATED_ACTIVATIONS:
        raise NotImplementedError(
            f"w4a8_fp8_wmma (gfx950) implements the gated activations {GATED_ACTIVATIONS}; "
            f"got {activation!r}")
    if kernel not in MOE_KERNEL_NAMES:
        raise ValueError(f"unknown moe kernel {kernel!r}; known: {list(MOE_KERNEL_NAMES)}")
    env = MoeEnv.read()

    if env.apply_chunk and M > env.apply_chunk and not apply_router_weight_on_input:
        # bounded intermediates: the layer is token-separable, so chunks are independent
        out = torch.empty((M, K), dtype=out_dtype, device=x.device)
        for lo in range(0, M, env.apply_chunk):
            hi = min(lo + env.apply_chunk, M)
            out[lo:hi] = _run_grouped_moe(
                x[lo:hi], w1, w2, w1_s, w2_s, w1_zp, w2_zp, topk_weights[lo:hi],
                topk_ids[lo:hi], activation, global_num_experts, expert_map, False, kernel,
                out_dtype, weight_is_e2m1=weight_is_e2m1, w1_bias=w1_bias, w2_bias=w2_bias)
        return out

    w1_s = w1_s.to(torch.float16)
    w2_s = w2_s.to(torch.float16)
    if apply_router_weight_on_input:
        if top_k != 1:
            raise ValueError("router-weight-on-input requires top_k == 1")
        x = x * topk_weights.reshape(M, 1).to(x.dtype)
        tw = torch.ones((M, top_k), dtype=torch.float32, device=x.device)
    else:
        tw = topk_weights.to(torch.float32)
    ids = topk_ids.to(torch.int32)

    if kernel == "scalar" or w1_bias is not None or w2_bias is not None or act != "silu":
        if w1.dim() == 4:   # the op-by-op kernels read the op layout
            w1, w2 = _fragments_to_op_layout(w1), _fragments_to_op_layout(w2)
        acc = _run_unfused(x.to(torch.float16).contiguous(), w1, w2, w1_s, w2_s, w1_zp, w2_zp,
                           tw.reshape(-1).contiguous(), ids, top_k, global_num_experts,
                           expert_map, kernel, weight_is_e2m1, w1_bias, w2_bias,
                           env.block_m or 64, act)
        return acc.to(out_dtype)

    if x.dtype not in (torch.float16, torch.bfloat16):
        x = x.to(torch.float16)
    out = _ops.moe_apply(x, w1, w2, w1_s, w2_s, w1_zp, w2_zp, tw, ids, expert_map,
                         weight_is_e2m1, global_num_experts=global_num_experts)
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
class MoeWNA16Hook:
    """Load and apply hooks for a ``MoeWNA16Method``-like class.

    Load (``process_weights_after_loading``): after the stock step, an int4 layer with a
    supported group size gets op-layout scales and zero-points, and its weights are repacked
    once into the gfx950 fragment layout (weights plus each tile's scale / zero-point words,
    17/16 of the u8 bytes), which replaces the weight parameters' data, one weight at a time,
    so the u8 bytes are freed as each fragment tensor is made. Shapes the fragment kernels
    do not take, and the "scalar" golden kernel, keep zero-copy op-layout views.
    Apply: every batch of an engaged layer runs ``_run_grouped_moe``; other layers keep the
    stock apply."""

    ATTR = "_w4a8_wna16"

    def __init__(self, method_cls, verbose: bool = False):
        self.method_cls = method_cls
        self.verbose = verbose
        self.stock_process = method_cls.process_weights_after_loading
        self.stock_apply = method_cls.apply

    @staticmethod
    def engages(method, layer) -> bool:
        try:
            return (method.quant_config.weight_bits == 4
                    and _supported_group_size(layer.group_size))
        except AttributeError:
            return False

    @staticmethod
    def prepare(layer, has_zp: bool, kernel: str) -> str:
        """Builds the layer's ``_w4a8`` weight record; returns the weight layout used."""
        views = {}
        for name in ("w13", "w2"):
            views[name] = _wna16_moe_to_op_layout(
                getattr(layer, f"{name}_qweight").data, getattr(layer, f"{name}_scales").data,
                getattr(layer, f"{name}_qzeros").data if has_zp else None)
        w13, s13, z13 = views["w13"]
        w2, s2, z2 = views["w2"]
        E, N13, kw = w13.shape
        hidden, inter = kw * 8, N13 // 2
        group = hidden // s13.shape[2]
        layout = "op"
        if kernel != "scalar" and _ops.fragments_supported(hidden, inter, group):
            layout = "fragments"
            for name in ("w13", "w2"):
                w, s, z = views[name]
                frag = _ops.repack_fragments(w, s, z)
                del w
                views[name] = (frag, s, z)
                getattr(layer, f"{name}_qweight").data = frag   # the u8 bytes are released
            w13, w2 = views["w13"][0], views["w2"][0]
        layer._w4a8 = dict(w13=w13, w2=w2, s13=s13, s2=s2, z13=z13, z2=z2, layout=layout)
        return layout

    def process(self, method, layer):
        engaged = self.engages(method, layer)
        setattr(method, self.ATTR, engaged)
        self.stock_process(method, layer)
        if not engaged:
            return
        has_zp = bool(getattr(method.quant_config, "has_zp", False))
        layout = self.prepare(layer, has_zp, _moe_kernel())
        if self.verbose:
            print(f"[w4a8_fp8_wmma] WNA16 MoE weights ready (int4 g={layer.group_size} "
                  f"has_zp={has_zp}, {layout} layout) -> gfx950 grouped fp8 MFMA")

    def apply(self, method, layer, x, topk_weights, topk_ids, shared_experts=None,
              shared_experts_input=None):
        if not getattr(method, self.ATTR, False):
            return self.stock_apply(method, layer, x, topk_weights, topk_ids, shared_experts,
                                    shared_experts_input)
        w = layer._w4a8
        flat = x.reshape(-1, x.shape[-1])
        out = _run_grouped_moe(
            flat, w["w13"], w["w2"], w["s13"], w["s2"], w["z13"], w["z2"], topk_weights,
            topk_ids, layer.activation, layer.global_num_experts, layer.expert_map,
            layer.apply_router_weight_on_input, _moe_kernel(), out_dtype=x.dtype)
        return out.reshape(*x.shape[:-1], out.shape[-1])

    def install(self) -> None:
        hook = self

        def process_weights_after_loading(self, layer):
            hook.process(self, layer)

        def apply(self, layer, x, topk_weights, topk_ids, shared_experts=None,
                  shared_experts_input=None):
            return hook.apply(self, layer, x, topk_weights, topk_ids, shared_experts,
                              shared_experts_input)

        self.method_cls.process_weights_after_loading = process_weights_after_loading
        self.method_cls.apply = apply


_MOE_WNA16_REGISTERED = False


def install_moe_wna16_hooks(method_cls, verbose: bool = False) -> MoeWNA16Hook:
    """Patch a MoeWNA16Method-like class (split out so tests can use a stand-in class)."""
    hook = MoeWNA16Hook(method_cls, verbose)
    hook.install()
    return hook


def register_moe_wna16(verbose: bool = True) -> bool:
    """Route int4 MoeWNA16 expert layers to the gfx950 path. Idempotent; False without vLLM
    or when disabled by the environment. Engages for every batch (no crossover gate)."""
    global _MOE_WNA16_REGISTERED
    if _MOE_WNA16_REGISTERED:
        return True
    env = MoeEnv.read()   # raises on removed knobs at boot
    if not env.enabled:
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


# --------------------------------------------------------------------------- #
# vLLM mxfp4 (gpt-oss) hook (moe_experts.py:1351-1450)
# --------------------------------------------------------------------------- #
class MoeMxfp4Hook:
    """Load and apply hooks for a ``GptOssMxfp4MoEMethod``-like class.

    Load: the layer's E2M1 weights (``w13_weight`` / ``w2_weight``, (E, N, K/2) uint8) and
    E8M0 scales (``w*_weight_scale``, (E, N, K/32) uint8) become the op layout on their own
    device (``convert_mxfp4_moe``: the weight bytes are viewed, the scales become fp16); the
    per-expert biases are kept; the source scale parameters are emptied. Apply: every batch
    runs ``_run_grouped_moe`` with ``weight_is_e2m1`` (fp4-operand matrix-core tiles), the
    layer's activation (swigluoai for gpt-oss) and both biases. A layer whose tensors are not
    in that layout keeps the stock path."""

    ATTR = "_w4a8_mxfp4"

    def __init__(self, method_cls, verbose: bool = False):
        self.method_cls = method_cls
        self.verbose = verbose
        self.stock_process = method_cls.process_weights_after_loading
        self.stock_apply = method_cls.apply

    @staticmethod
    def prepare(layer) -> dict:
        c13 = convert_mxfp4_moe(layer.w13_weight.data, layer.w13_weight_scale.data)
        c2 = convert_mxfp4_moe(layer.w2_weight.data, layer.w2_weight_scale.data)
        b13 = getattr(layer, "w13_bias", None)
        b2 = getattr(layer, "w2_bias", None)
        rec = dict(w13=c13["w_packed"], w2=c2["w_packed"], s13=c13["scales"], s2=c2["scales"],
                   b13=None if b13 is None else b13.data, b2=None if b2 is None else b2.data,
                   scale_info=(c13["scale_info"], c2["scale_info"]))
        layer._w4a8_mx = rec
        # the fp16 scales replace the E8M0 bytes; the weight parameters keep their storage
        # (the op-layout weights are views of it)
        for name in ("w13_weight_scale", "w2_weight_scale"):
            prm = getattr(layer, name, None)
            if prm is not None and hasattr(prm, "data"):
                prm.data = torch.empty(0, dtype=prm.dtype, device=prm.device)
        return rec

    def process(self, method, layer):
        try:
            rec = self.prepare(layer)
        except (AttributeError, ValueError, TypeError) as e:   # not the E2M1/E8M0 layout
            setattr(method, self.ATTR, False)
            if self.verbose:
                print(f"[w4a8_fp8_wmma] mxfp4 MoE: stock path ({e})")
            return self.stock_process(method, layer)
        setattr(method, self.ATTR, True)
        if not all(i["fp16_range_ok"] for i in rec["scale_info"]):
            logger.warning("mxfp4 MoE: E8M0 scales outside the fp16 group-scale range; "
                           "results may be wrong (%s)", rec["scale_info"])
        if self.verbose:
            print("[w4a8_fp8_wmma] mxfp4 MoE weights ready (E2M1, E8M0 -> fp16, group 32) "
                  "-> gfx950 fp4-operand MFMA")

    def apply(self, method, layer, x, topk_weights, topk_ids, shared_experts=None,
              shared_experts_input=None, **kw):
        if not getattr(method, self.ATTR, False):
            return self.stock_apply(method, layer, x, topk_weights, topk_ids, shared_experts,
                                    shared_experts_input, **kw)
        w = layer._w4a8_mx
        flat = x.reshape(-1, x.shape[-1])
        out = _run_grouped_moe(
            flat, w["w13"], w["w2"], w["s13"], w["s2"], None, None, topk_weights, topk_ids,
            layer.activation, layer.global_num_experts, layer.expert_map,
            layer.apply_router_weight_on_input, _moe_kernel(), out_dtype=x.dtype,
            weight_is_e2m1=True, w1_bias=w["b13"], w2_bias=w["b2"])
        return out.reshape(*x.shape[:-1], out.shape[-1])

    def install(self) -> None:
        hook = self

        def process_weights_after_loading(self, layer):
            hook.process(self, layer)

        def apply(self, layer, x, topk_weights, topk_ids, shared_experts=None,
                  shared_experts_input=None, **kw):
            return hook.apply(self, layer, x, topk_weights, topk_ids, shared_experts,
                              shared_experts_input, **kw)

        self.method_cls.process_weights_after_loading = process_weights_after_loading
        self.method_cls.apply = apply


_MOE_MXFP4_REGISTERED = False


def install_moe_mxfp4_hooks(method_cls, verbose: bool = False) -> MoeMxfp4Hook:
    """Patch a GptOssMxfp4MoEMethod-like class (split out so tests can use a stand-in)."""
    hook = MoeMxfp4Hook(method_cls, verbose)
    hook.install()
    return hook


def register_moe_mxfp4(verbose: bool = True) -> bool:
    """Route gpt-oss mxfp4 expert layers to the gfx950 path (moe_experts.py:1351-1450).
    Idempotent; False without vLLM or when disabled by the environment."""
    global _MOE_MXFP4_REGISTERED
    if _MOE_MXFP4_REGISTERED:
        return True
    env = MoeEnv.read()
    if not env.enabled:
        if verbose:
            print("[w4a8_fp8_wmma] mxfp4 MoE disabled via env")
        return False
    try:
        from vllm.model_executor.layers.quantization.mxfp4 import GptOssMxfp4MoEMethod
    except Exception as e:  # noqa: BLE001  (vLLM absent: nothing to patch)
        if verbose:
            print(f"[w4a8_fp8_wmma] mxfp4 MoE: vLLM not importable ({type(e).__name__})")
        return False
    install_moe_mxfp4_hooks(GptOssMxfp4MoEMethod, verbose)
    _MOE_MXFP4_REGISTERED = True
    return True
