"""Build the gfx950 C-ABI library ``w4a8_fp8_wmma/libw4a8moe.so`` in-tree.

Every ``csrc/*.hip`` file is compiled with hipcc for gfx950 only, then linked into one
shared library whose exported symbols are exactly the ``extern "C"`` entry points of
``include/w4a8_moe.h``. Usage: ``python rdna4-vllm_amd/build.py [-j N]``.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
OUT_DIR = HERE / "w4a8_fp8_wmma"
LIB_NAME = "libw4a8moe.so"
BUILD_DIR = HERE / "_build"
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    # code object v5 loads on every ROCm 6.x/7.x runtime (torch bundles its own)
    "-mcode-object-version=5",
    "-fvisibility=hidden",
    # keep fp32 arithmetic unpacked (no v_pk_*_f32)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def hipcc() -> str:
    cand = os.environ.get("HIPCC") or shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(cand).exists():
        raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")
    return cand


# Per-file extras: the prefill tiles keep MFMA results in VGPRs (the fp32 scale fold reads
# every result once; from AGPRs each read would cost an extra v_accvgpr_read).
EXTRA_FLAGS = {
    "prefill_gemm.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
    "prefill_ares.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
}


def _compile(src: Path, obj: Path) -> None:
    cmd = [hipcc(), *HIPCC_FLAGS, *EXTRA_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{r.stdout}\n{r.stderr}")
    # hipcc's host pass warns that it does not know the packed-fp32 feature; drop that noise
    noise = "packed-fp32-ops"
    msgs = [ln for ln in (r.stderr or "").splitlines() if noise not in ln and ln.strip()]
    if msgs:
        print("\n".join(msgs), file=sys.stderr)


def build(jobs: int | None = None, verbose: bool = True) -> Path:
    BUILD_DIR.mkdir(exist_ok=True)
    srcs = sorted(CSRC.glob("*.hip"))
    objs = [BUILD_DIR / (s.stem + ".o") for s in srcs]
    jobs = jobs or min(8, os.cpu_count() or 1, len(srcs))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(lambda so: _compile(*so), zip(srcs, objs)))
    lib = OUT_DIR / LIB_NAME
    tmp = OUT_DIR / (LIB_NAME + ".tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, lib)
    if verbose:
        print(f"built {lib} ({lib.stat().st_size // 1024} KiB)")
    return lib


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("-j", type=int, default=None)
    a = ap.parse_args()
    build(a.j)
