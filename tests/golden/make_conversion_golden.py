"""Write tests/golden/conversion_ref.npz: AWQ and GPTQ/compressed-tensors conversion vectors
produced by the reference's OWN numpy test modules.

The nibble order of the AWQ format (which bit position holds which output column) is the
one fact of the weight conversion that a round trip through our own packer cannot pin: a
packer and an unpacker that share a wrong order still agree. The reference ships two
torch-free modules that define the order independently of this repository:

  * w4a8_fp8_wmma/test_moe_conversion_numpy.py     (``awq_pack``, ``awq_to_op_layout``)
  * w4a8_fp8_wmma/test_moe_conversion_ct_numpy.py  (``gptq_pack``, ``ct_to_op``)

This script imports them from /root/reference (in the build container only; the reference
never travels), runs them on seeded inputs and stores inputs and outputs as data. The
tests check our torch converters and the oracle against these vectors.

    python tests/golden/make_conversion_golden.py
"""
from __future__ import annotations

import importlib.util
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REF = "/root/reference/w4a8_fp8_wmma"


def _load(name):
    spec = importlib.util.spec_from_file_location(name, os.path.join(REF, name + ".py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def main():
    awq = _load("test_moe_conversion_numpy")
    ct = _load("test_moe_conversion_ct_numpy")
    rng = np.random.default_rng(0)
    out = {}
    # (E, K, N, group): AWQ with zero-points; the same nibbles GPTQ-packed along K
    for i, (E, K, N, g) in enumerate([(2, 256, 64, 32), (3, 128, 32, 128), (1, 512, 16, 64)]):
        G = K // g
        qvals = rng.integers(0, 16, (E, K, N)).astype(np.int32)
        zeros = rng.integers(0, 16, (E, G, N)).astype(np.int32)
        scales = (rng.random((E, G, N)) * 0.015 + 0.005).astype(np.float16)
        qweight = awq.awq_pack(qvals)
        qzeros = awq.awq_pack(zeros)
        w_op, s_op, z_op = awq.awq_to_op_layout(qweight, scales, qzeros, g)
        gq = ct.gptq_pack(qvals)
        cw_op, cs_op = ct.ct_to_op(gq, scales)
        out.update({
            f"c{i}_qvals": qvals.astype(np.uint8), f"c{i}_zeros": zeros.astype(np.uint8),
            f"c{i}_scales": scales, f"c{i}_group": np.int32(g),
            f"c{i}_awq_qweight": qweight, f"c{i}_awq_qzeros": qzeros,
            f"c{i}_awq_w_op": w_op.astype(np.int32), f"c{i}_awq_s_op": s_op.astype(np.float16),
            f"c{i}_awq_z_op": z_op.astype(np.int32),
            f"c{i}_gptq_qweight": gq, f"c{i}_ct_w_op": cw_op.astype(np.int32),
        })
    path = os.path.join(HERE, "conversion_ref.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path} ({os.path.getsize(path)} bytes)")


if __name__ == "__main__":
    main()
