"""ctypes binding of the gfx950 C ABI (``include/w4a8_moe.h``).

Loading fails loudly: there is no CPU or Python fallback for any kernel.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libw4a8moe.so"

_c_void_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_int = ctypes.c_int
_size = ctypes.c_size_t

# name -> (restype, argtypes); must match include/w4a8_moe.h exactly.
SIGNATURES = {
    "w4a8_abi_version": (_int, []),
    "w4a8_last_error": (ctypes.c_char_p, []),
    "w4a8_act_quant_fp8": (_int, [_c_void_p, _i64, _i64, _c_void_p, _c_void_p, _int, _c_void_p]),
    "w4a8_dequant_fp8": (_int, [_c_void_p, _c_void_p, _i64, _i64, _i64, _i64, _int, _c_void_p,
                                _c_void_p]),
    "w4a8_topk_softmax": (_int, [_c_void_p, _i64, _i64, _i64, _int, _c_void_p, _c_void_p,
                                 _c_void_p]),
    "w4a8_moe_align_sorted_len": (_i64, [_i64, _i64, _i64]),
    "w4a8_moe_align_workspace_size": (_size, [_i64, _i64]),
    "w4a8_moe_align_block_size": (_int, [_c_void_p, _i64, _i64, _i64, _c_void_p, _c_void_p, _i64,
                                         _c_void_p, _c_void_p, _c_void_p, _size, _c_void_p]),
    "w4a8_moe_gemm_workspace_size": (_size, [_i64, _i64]),
    "w4a8_mmq_fp8_moe_gemm": (_int, [_c_void_p, _i64, _i64, _c_void_p, _c_void_p, _c_void_p,
                                     _i64, _i64, _i64, _c_void_p, _i64, _c_void_p, _c_void_p,
                                     _i64, _i64, _i64, _int, _c_void_p, _c_void_p, _size,
                                     _c_void_p]),
    "w4a8_mmq_fp8_moe_gemm1_silu": (_int, [_c_void_p, _i64, _i64, _c_void_p, _c_void_p,
                                           _c_void_p, _i64, _i64, _i64, _c_void_p, _i64,
                                           _c_void_p, _c_void_p, _i64, _i64, _i64, _int,
                                           _c_void_p, _c_void_p, _size, _c_void_p]),
    "w4a8_mmq_fp8_moe_gemm_scatter": (_int, [_c_void_p, _i64, _i64, _c_void_p, _c_void_p,
                                             _c_void_p, _i64, _i64, _i64, _c_void_p, _i64,
                                             _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64,
                                             _i64, _i64, _i64, _int, _c_void_p, _size,
                                             _c_void_p]),
    "w4a8_gather_reduce_workspace_size": (_size, [_i64]),
    "w4a8_mmq_fp8_moe_gather_reduce": (_int, [_c_void_p, _i64, _i64, _c_void_p, _c_void_p, _i64,
                                              _c_void_p, _i64, _c_void_p, _c_void_p, _size,
                                              _c_void_p]),
    "w4a8_silu_and_mul": (_int, [_c_void_p, _i64, _i64, _c_void_p, _c_void_p]),
    "w4a8_swigluoai_and_mul": (_int, [_c_void_p, _i64, _i64, ctypes.c_float, ctypes.c_float,
                                      _c_void_p, _c_void_p]),
    "w4a8_mmq_fp8_gemm": (_int, [_c_void_p, _i64, _i64, _c_void_p, _c_void_p, _c_void_p, _i64,
                                 _i64, _i64, _int, _c_void_p, _c_void_p, _size, _c_void_p]),
    "w4a8_moe_apply_workspace_size": (_size, [_i64, _i64, _i64, _i64, _i64]),
    "w4a8_moe_apply_set_stage_events": (_int, [ctypes.POINTER(_c_void_p), _int]),
    "w4a8_moe_apply": (_int, [_c_void_p, _int, _i64, _i64, _i64, _i64, _i64, _i64, _c_void_p,
                              _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                              _c_void_p, _c_void_p, _i64, _int, _c_void_p, _c_void_p, _size,
                              _c_void_p]),
    "w4a8_repack_int4_fragments": (_int, [_c_void_p, _c_void_p, _c_void_p, _i64, _i64, _i64,
                                          _c_void_p, _c_void_p]),
    "w4a8_fragments_words": (_i64, [_i64, _i64, _i64]),
    "w4a8_moe_forward": (_int, [_c_void_p, _int, _i64, _i64, _i64, _i64, _i64, _i64, _c_void_p,
                                _int, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                                _c_void_p, _int, _c_void_p, _i64, _c_void_p, _c_void_p,
                                _c_void_p, _c_void_p, _size, _c_void_p]),
    "w4a8_moe_apply_fragments": (_int, [_c_void_p, _int, _i64, _i64, _i64, _i64, _i64, _i64,
                                        _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                                        _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64,
                                        _c_void_p, _c_void_p, _size, _c_void_p]),
    "w4a8_moe_fragments_supported": (_int, [_i64, _i64, _i64]),
    "w4a8_moe_forward_noalloc": (_int, [_c_void_p, _int, _i64, _i64, _i64, _i64, _i64, _i64,
                                        _c_void_p, _int, _c_void_p, _c_void_p, _c_void_p,
                                        _c_void_p, _c_void_p, _c_void_p, _int, _c_void_p, _i64,
                                        _c_void_p, _c_void_p, _c_void_p, _c_void_p]),
    "w4a8_set_decode_fused": (_int, [_int]),
    "w4a8_set_prefill_pair": (_int, [_int]),
    "w4a8_decode_fused_test_fault": (_int, [_int]),
}

ABI_VERSION = 3


class W4A8LibraryError(RuntimeError):
    pass


def _load() -> ctypes.CDLL:
    path = os.environ.get("W4A8_MOE_LIB", str(LIB_PATH))
    if not Path(path).exists():
        raise ImportError(
            f"w4a8_fp8_wmma: HIP library not built ({path}); run "
            "`python rdna4-vllm_amd/build.py` (there is no CPU fallback)")
    lib = ctypes.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if lib.w4a8_abi_version() != ABI_VERSION:
        raise ImportError(f"w4a8_fp8_wmma: ABI version mismatch in {path}")
    return lib


lib = _load()


def check(rc: int, what: str) -> None:
    """Raise RuntimeError (the reference's TORCH_CHECK surface) on a non-zero status."""
    if rc != 0:
        msg = (lib.w4a8_last_error() or b"").decode(errors="replace")
        raise RuntimeError(f"{what}: {msg} (status {rc})")
