"""Write tests/golden/silu_fp16_exhaustive.npy: SiLU of every fp16 input, as fp16 bits.

SiLU(gate) * up in vLLM's silu_and_mul (and in the reference's fused gemm1 epilogue,
moe_kernel.hip:549-561) rounds g / (1 + expf(-g)) in fp32 to fp16, g being an fp16 value, so
the whole function is a table of 65536 entries. This script evaluates that table on the GPU
with the exact form (the device expf and an IEEE fp32 division) through the library's
``silu_and_mul`` with up = 1 (the product by 1 is exact), and stores the bits. The tests hold
every SiLU in the library to this table, so a faster evaluation of the same function has to
reproduce the exact form's bits on all inputs, and check the table against the numpy oracle
(expf and numpy's exp may differ in an fp32 ulp; the table may then differ by one fp16 ulp).

Run on a GPU box with a library whose SiLU is the exact form:

    python tests/golden/make_silu_exhaustive.py
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "..", "..", "rdna4-vllm_amd"))


def main() -> None:
    import torch
    import w4a8_fp8_wmma as W

    gate = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16).reshape(256, 256)
    x = np.concatenate([gate, np.ones_like(gate)], axis=1)
    out = torch.empty((256, 256), dtype=torch.float16, device="cuda")
    W.silu_and_mul(out, torch.from_numpy(x).cuda())
    torch.cuda.synchronize()
    bits = out.cpu().numpy().view(np.uint16).reshape(-1)
    path = os.path.join(HERE, "silu_fp16_exhaustive.npy")
    np.save(path, bits)
    print(f"wrote {path}: {bits.size} entries")


if __name__ == "__main__":
    main()
