"""vLLM general-plugin entry point (w4a8_fp8_wmma/w4a8_fp8_wmma/register.py:42-175).

``register()`` prepends the dense W4A8 linear kernel to vLLM's ROCm linear-kernel list and
installs the MoeWNA16 and the mxfp4 (gpt-oss) MoE hooks, each best-effort so one failing
leaves the others in place. The reference's other hooks (mxfp4 dense registry,
compressed-tensors MoE) are outside this package's scope. Removed env knobs raise at boot, like the reference
(register.py:29-39).
"""
from __future__ import annotations

import os

_REMOVED_ENV = ("VLLM_ROCM_W4A8_FP8_WMMA_VERSION", "VLLM_ROCM_W4A8_FP8_WMMA_MOE_VERSION")


def _check_removed_w4a8_env() -> None:
    for name in _REMOVED_ENV:
        if name in os.environ:
            raise RuntimeError(f"{name} is removed; use the descriptive kernel-name env vars")


def register() -> None:
    if os.environ.get("VLLM_ROCM_USE_W4A8_FP8_WMMA", "1") != "1":
        print("[w4a8_fp8_wmma] disabled via VLLM_ROCM_USE_W4A8_FP8_WMMA")
        return
    _check_removed_w4a8_env()
    from .linear import register_dense_linear
    try:
        register_dense_linear()
    except ImportError as e:
        print(f"[w4a8_fp8_wmma] dense linear kernel not registered: {e}")
    from .moe_experts import register_moe_mxfp4, register_moe_wna16
    for hook in (register_moe_wna16, register_moe_mxfp4):
        try:
            hook()
        except ImportError as e:
            print(f"[w4a8_fp8_wmma] MoE hook {hook.__name__} not installed: {e}")
