"""Dense W4A8 linear layers on gfx950: the reference's ``vllm::w4a8_dense_apply`` op and its
``MPLinearKernel`` adapter (w4a8_fp8_wmma/w4a8_fp8_wmma/vllm_adapter.py:265-593).

``w4a8_dense_apply`` keeps the reference op's thirteen arguments and its return contract
(vllm_adapter.py:265-354): 2-D activations of any float dtype are cast to fp16, the result
is (M, N) fp16. The kernel for a batch of M rows is picked by name:

  * ``"decode_gemv"`` for M <= ``VLLM_ROCM_W4A8_DECODE_MAX_M`` at group 128, and (with the
    variable unset) up to 2048 rows while the MFMA tile grid would hold fewer than 128
    tiles (a K outside the GEMV's split-K table runs the MFMA tiles instead);
  * ``"prefill_wmma_ashuffle"`` otherwise (``"prefill_wmma"`` for group sizes other than 32 and
    128, the reference's rule). On gfx950 both names run the fp8-MFMA tiles.

There is no Triton W4A16 fallback on this build: the Triton-layout arguments (``tri_bq``,
``tri_s``, ``tri_zp``) and the measured crossover ``cached_min_m`` are accepted for the call
surface and unused, and every M runs the native kernels. ``VLLM_ROCM_W4A8_FORCE=off`` (stock
path only) therefore raises instead of silently running the native kernels.

Weights arrive in the op layout: ``w_q`` (N, K/8) int32 (nibble j of word k8 is k = 8 k8 + j),
``w_s`` (N, K/group) fp16, optional AWQ zero points (N/8, K/group) int32. AutoGPTQ checkpoints
store the transpose (K/8, N) packed along K; ``gptq_to_op_layout`` converts them.
"""
from __future__ import annotations

import logging
import os
from typing import Optional

import torch

from . import mmq_fp8_gemm

logger = logging.getLogger(__name__)

#: Rows up to which the decode GEMV runs when VLLM_ROCM_W4A8_DECODE_MAX_M is unset. Measured
#: on MI355X (HIP-graph replay) against the MFMA tiles for (N, K) = (1024, 2048), (4096, 4096),
#: (12288, 4096), (4096, 12288): the GEMV leads through M = 128 on every shape.
DECODE_MAX_M_DEFAULT = 128
#: Past that (env unset) the GEMV still runs while the MFMA tile grid, ceil(N / 256) x
#: ceil(M / 64) work-groups, holds fewer than half as many tiles as MI355X has CUs: such a grid
#: leaves most CUs idle, and the GEMV measured faster on every shape above (e.g. (4096, 4096)
#: at M = 256: 37.7 against 61.2 us; (1024, 2048) at M = 512: 14.3 against 38.0 us).
DENSE_GEMV_MAX_M = 2048
DENSE_TILE_ROWS, DENSE_TILE_COLS, DENSE_MIN_TILES = 64, 256, 128
#: Symmetric int4 (vLLM ``uint4b8``) stores w + 8; the kernels' implicit zero point.
UINT4B8_BIAS = 8


def _force_mode() -> str:
    """VLLM_ROCM_W4A8_FORCE (vllm_adapter.py:35-50): auto | on | off."""
    v = os.environ.get("VLLM_ROCM_W4A8_FORCE", "auto").strip().lower()
    if v in ("on", "1", "true"):
        return "on"
    if v in ("off", "0", "false"):
        return "off"
    return "auto"


def decode_max_m() -> int:
    return int(os.environ.get("VLLM_ROCM_W4A8_DECODE_MAX_M", str(DECODE_MAX_M_DEFAULT)))


def dense_kernel_for(M: int, N: int, K: int, group_size: int) -> str:
    """The dense kernel name for an (M, N, K) GEMM with this group size (the ladder of
    vllm_adapter.py:296-324 without its Triton band). A K outside the GEMV's split-K table
    runs the MFMA tiles under either name (the C ABI's own fallback)."""
    if group_size == 128 and K % group_size == 0:
        if M <= decode_max_m():
            return "decode_gemv"
        tiles = -(-N // DENSE_TILE_COLS) * -(-M // DENSE_TILE_ROWS)
        if ("VLLM_ROCM_W4A8_DECODE_MAX_M" not in os.environ and M <= DENSE_GEMV_MAX_M
                and tiles < DENSE_MIN_TILES):
            return "decode_gemv"
    return "prefill_wmma_ashuffle" if group_size in (32, 128) else "prefill_wmma"


def w4a8_dense_apply(x2d: torch.Tensor, w_q: torch.Tensor, w_s: torch.Tensor,
                     w_zp: Optional[torch.Tensor], tri_bq: Optional[torch.Tensor],
                     tri_s: Optional[torch.Tensor], tri_zp: Optional[torch.Tensor],
                     N: int, K: int, group_size: int, zero_points: bool,
                     weight_type_bias: int, cached_min_m: int) -> torch.Tensor:
    """One dense W4A8 linear: x2d (M, K) -> (M, N) fp16 (vllm_adapter.py:265-354)."""
    del tri_bq, tri_s, tri_zp, cached_min_m   # Triton fallback inputs: no Triton here
    if _force_mode() == "off":
        raise RuntimeError("VLLM_ROCM_W4A8_FORCE=off selects the stock Triton path, which "
                           "this build does not ship; disable the plugin instead")
    if x2d.dim() != 2 or x2d.shape[1] != K:
        raise ValueError(f"x must be (M, K={K}), got {tuple(x2d.shape)}")
    if tuple(w_q.shape) != (N, K // 8):
        raise ValueError(f"w_q must be (N, K/8)=({N}, {K // 8}), got {tuple(w_q.shape)}")
    use_zp = bool(zero_points) and w_zp is not None
    if not use_zp and int(weight_type_bias) != UINT4B8_BIAS:
        raise ValueError("weights without zero points must be uint4b8 (bias 8), "
                         f"got bias {weight_type_bias}")
    if x2d.dtype != torch.float16:
        x2d = x2d.to(torch.float16)
    x2d = x2d.contiguous()
    kernel = dense_kernel_for(x2d.shape[0], N, K, group_size)
    return mmq_fp8_gemm(x2d, w_q, w_s, kernel=kernel, w_zeros=w_zp if use_zp else None)


def _w4a8_dense_apply_fake(x2d, w_q, w_s, w_zp, tri_bq, tri_s, tri_zp, N, K, group_size,
                           zero_points, weight_type_bias, cached_min_m):
    return x2d.new_empty((x2d.shape[0], N), dtype=torch.float16)


_SCHEMA = ("w4a8_dense_apply(Tensor x2d, Tensor w_q, Tensor w_s, Tensor? w_zp, Tensor? tri_bq, "
           "Tensor? tri_s, Tensor? tri_zp, SymInt N, SymInt K, SymInt group_size, "
           "bool zero_points, SymInt weight_type_bias, SymInt cached_min_m) -> Tensor")
_vllm_lib = None


def register_dense_op() -> None:
    """Define ``torch.ops.vllm.w4a8_dense_apply`` (CUDA kernel + fake) unless it exists, as
    the reference's direct_register_custom_op call does (vllm_adapter.py:376-386)."""
    global _vllm_lib
    if _vllm_lib is not None or hasattr(torch.ops.vllm, "w4a8_dense_apply"):
        return
    lib = torch.library.Library("vllm", "FRAGMENT")
    lib.define(_SCHEMA)
    lib.impl("w4a8_dense_apply", w4a8_dense_apply, "CUDA")
    torch.library.register_fake("vllm::w4a8_dense_apply", _w4a8_dense_apply_fake, lib=lib)
    _vllm_lib = lib


def gptq_to_op_layout(qweight: torch.Tensor, scales: torch.Tensor,
                      K: int, N: int) -> tuple[torch.Tensor, torch.Tensor]:
    """AutoGPTQ (K/8, N) int32 packed along K and (K/group, N) scales -> the op layout
    (N, K/8) and (N, K/group) fp16 (vllm_adapter.py:427-445). Both formats put k = 8 k8 + j
    in nibble j of word k8, so the words themselves carry over and only their matrix is
    transposed."""
    if tuple(qweight.shape) != (K // 8, N):
        raise ValueError(f"GPTQ qweight must be (K/8, N)=({K // 8}, {N}), "
                         f"got {tuple(qweight.shape)}")
    if scales.dim() != 2 or scales.shape[1] != N:
        raise ValueError(f"GPTQ scales must be (K/group, N), got {tuple(scales.shape)}")
    return (qweight.t().contiguous(),
            scales.t().to(torch.float16).contiguous())


def _on_gfx950() -> bool:
    try:
        return torch.cuda.get_device_properties(0).gcnArchName.split(":")[0] == "gfx950"
    except Exception:  # noqa: BLE001  (no device)
        return False


def make_linear_kernel(base, scalar_types, is_rocm):
    """Build the vLLM linear kernel class on ``base`` (vLLM's MPLinearKernel): the adapter
    of vllm_adapter.py:390-593 over ``w4a8_dense_apply``. Weights are normalised once at
    load to the op layout; there is no second (Triton-layout) copy and no crossover table."""
    supported = [scalar_types.uint4b8, scalar_types.uint4]

    class RocmW4A8Fp8WmmaLinearKernel(base):
        """fp8-MFMA (gfx950) kernel for int4 weights with per-group fp16 scales."""
        SUPPORTED_QUANT_TYPES = supported

        @classmethod
        def get_min_capability(cls) -> int:
            return 0

        @classmethod
        def can_implement(cls, c) -> tuple[bool, Optional[str]]:
            if not is_rocm():
                return False, "ROCm only"
            if not _on_gfx950():
                return False, "requires gfx950 (MI355X)"
            if c.weight_type not in supported:
                return False, f"unsupported weight_type {c.weight_type}"
            if c.act_type not in (torch.float16, torch.bfloat16):
                return False, f"act_type must be fp16/bf16, got {c.act_type}"
            if c.has_g_idx:
                return False, "act reordering (g_idx) not supported"
            K = c.partition_weight_shape[0]
            if c.group_size != 128:
                return False, ("group_size must be 128 (other group sizes run only the "
                               f"scalar kernel here), got {c.group_size}")
            if K % 128 != 0:
                return False, f"K={K} not divisible by group_size=128"
            return True, None

        def process_weights_after_loading(self, layer: torch.nn.Module) -> None:
            c = self.config
            K, N = c.partition_weight_shape
            w_q, w_s, w_zp, _ = self._get_weight_params(layer)
            if tuple(w_q.shape) == (K // 8, N) and (K // 8, N) != (N, K // 8):
                wq, ws = gptq_to_op_layout(w_q.data, w_s.data, K, N)
                self._transform_param(layer, self.w_q_name, lambda _p: wq)
            elif tuple(w_q.shape) == (N, K // 8):
                ws = w_s.data
                if not w_q.is_contiguous():
                    self._transform_param(layer, self.w_q_name, lambda p: p.contiguous())
            else:
                raise RuntimeError(f"unexpected w_q shape {tuple(w_q.shape)}; expected "
                                   f"(N, K/8)={(N, K // 8)} or GPTQ (K/8, N)={(K // 8, N)}")
            layer._w4a8_fp8_w_s = ws.to(torch.float16).contiguous()
            if w_zp is not None and not w_zp.is_contiguous():
                self._transform_param(layer, self.w_zp_name, lambda p: p.contiguous())

        def apply_weights(self, layer: torch.nn.Module, x: torch.Tensor,
                          bias: Optional[torch.Tensor] = None) -> torch.Tensor:
            c = self.config
            K, N = c.partition_weight_shape
            w_q, _, w_zp, _ = self._get_weight_params(layer)
            x2d = x.reshape(-1, x.shape[-1])
            bias_w = c.weight_type.bias if c.weight_type.has_bias() else 0
            out = torch.ops.vllm.w4a8_dense_apply(
                x2d, w_q, layer._w4a8_fp8_w_s,
                w_zp if (c.zero_points and w_zp is not None) else None,
                None, None, None, N, K, c.group_size, bool(c.zero_points), int(bias_w), 0)
            if out.dtype != x.dtype:
                out = out.to(x.dtype)
            if bias is not None:
                out = out + bias
            return out.reshape(x.shape[:-1] + (N,))

    return RocmW4A8Fp8WmmaLinearKernel


_DENSE_REGISTERED = False


def register_dense_linear(verbose: bool = True) -> bool:
    """Prepend the kernel class to vLLM's ROCm linear-kernel list (register.py:42-83).
    False without vLLM."""
    global _DENSE_REGISTERED
    if _DENSE_REGISTERED:
        return True
    try:
        from vllm.model_executor.kernels.linear import _POSSIBLE_KERNELS
        from vllm.model_executor.kernels.linear.mixed_precision.MPLinearKernel import (
            MPLinearKernel)
        from vllm.platforms import PlatformEnum, current_platform
        from vllm.scalar_type import scalar_types
    except Exception as e:  # noqa: BLE001  (vLLM absent: nothing to register)
        if verbose:
            print(f"[w4a8_fp8_wmma] dense linear: vLLM not importable ({type(e).__name__})")
        return False
    register_dense_op()
    cls = make_linear_kernel(MPLinearKernel, scalar_types, current_platform.is_rocm)
    lst = _POSSIBLE_KERNELS.setdefault(PlatformEnum.ROCM, [])
    if not any(k.__name__ == cls.__name__ for k in lst):
        lst.insert(0, cls)
    _DENSE_REGISTERED = True
    if verbose:
        print("[w4a8_fp8_wmma] dense linear kernel registered at _POSSIBLE_KERNELS[ROCM][0]")
    return True


register_dense_op()
