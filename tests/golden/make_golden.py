"""Write the golden fixtures under tests/golden/ from the CPU oracle.

The reference ships no golden tensors (its tests draw fresh random data each run), so
these fixtures are the oracle's outputs on small, seeded, hand-shaped inputs: they lock
the pinned oracle against regressions and give the GPU tests fixed known answers that
do not depend on numpy's generator streams. Inputs and outputs are stored together.

    python tests/golden/make_golden.py          # rewrite every fixture
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
import oracle as O  # noqa: E402


def dequant_fixture():
    """Every (nibble, zero-point) pair and the E2M1 codebook -> e4m3 bytes."""
    tables = np.stack([O.dequant_table(z) for z in range(16)]).astype(np.uint8)
    return dict(tables=tables, e2m1=O.dequant_table(0, e2m1=True).astype(np.uint8))


def act_quant_fixture():
    r = np.random.default_rng(101)
    x = (r.standard_normal((8, 256)) * np.exp2(r.integers(-6, 6, (8, 1)))).astype(np.float16)
    x[0] = 0                                   # all-zero row: scale floor 1e-8
    x[1] = np.float16(6e-8)                    # sub-floor magnitudes
    x[2, ::5] = np.float16(-65504)             # fp16 extremes
    x[3] = np.float16(448.0) * (np.arange(256) % 3 - 1)   # exact e4m3 grid points
    x[4, 7] = np.float16(0)
    q, s = O.act_quant(x)
    return dict(x_bits=x.view(np.uint16), q=q.astype(np.uint8), scales=s)


def routing_fixture():
    r = np.random.default_rng(102)
    lg = r.standard_normal((9, 16)).astype(np.float32)
    lg[0] = 0.5                                # full tie -> lowest ids
    lg[1, [3, 9, 12]] = 4.0                    # partial tie among the winners
    lg[2] = -np.arange(16, dtype=np.float32)   # strictly ordered
    w, ids = O.topk_softmax(lg, 4, renormalize=True)
    return dict(logits=lg, top_k=np.int32(4), weights=w, ids=ids)


def align_fixture():
    r = np.random.default_rng(103)
    cases = {}
    # (name, T, k, E, block_m, expert_map?)
    ids_a = np.stack([r.permutation(16)[:4] for _ in range(7)]).astype(np.int32)
    ids_b = np.minimum(r.zipf(1.6, size=(40, 8)) - 1, 31).astype(np.int32)   # skewed, repeats
    ids_c = np.stack([r.permutation(12)[:3] for _ in range(10)]).astype(np.int32)
    emap_c = np.where(np.arange(12) % 2 == 0, np.arange(12) // 2, -1).astype(np.int32)
    ids_d = np.zeros((0, 8), dtype=np.int32)
    for name, ids, E, bm, em in (("a", ids_a, 16, 8, None), ("b", ids_b, 32, 16, None),
                                 ("c", ids_c, 12, 4, emap_c), ("d", ids_d, 8, 16, None)):
        so, eo, no = O.moe_align(ids, bm, E, expert_map=em)
        cases.update({f"{name}_ids": ids, f"{name}_E": np.int32(E), f"{name}_bm": np.int32(bm),
                      f"{name}_emap": em if em is not None else np.zeros(0, np.int32),
                      f"{name}_sorted": so, f"{name}_experts": eo, f"{name}_ntp": no})
    return cases


def layer_fixture():
    """Tiny asymmetric AWQ-g128 MoE layer: T=5, H=256, I=128, E=4, top-2."""
    r = np.random.default_rng(104)
    T, H, I, E, k, g = 5, 256, 128, 4, 2, 128
    x = r.standard_normal((T, H)).astype(np.float32)
    xb = O.f32_to_bf16_bits(x)
    xf = O.bf16_bits_to_f32(xb)
    w13 = O.pack_nibbles(r.integers(0, 16, (E, 2 * I, H)))
    z13 = O.pack_zeros(r.integers(0, 16, (E, 2 * I, H // g)))
    s13 = r.uniform(0.005, 0.02, (E, 2 * I, H // g)).astype(np.float16)
    w2 = O.pack_nibbles(r.integers(0, 16, (E, H, I)))
    z2 = O.pack_zeros(r.integers(0, 16, (E, H, I // g)))
    s2 = r.uniform(0.005, 0.02, (E, H, I // g)).astype(np.float16)
    tw, ids = O.topk_softmax(r.standard_normal((T, E)).astype(np.float32), k)
    out = O.moe_layer(xf, w13, s13, z13, w2, s2, z2, tw, ids, g, round_y_fp16=False)
    return dict(x_bf16_bits=xb, w13=w13, z13=z13, s13_bits=s13.view(np.uint16), w2=w2, z2=z2,
                s2_bits=s2.view(np.uint16), topk_weights=tw, topk_ids=ids,
                group_size=np.int32(g), out=out)


FIXTURES = {
    "dequant_tables.npz": dequant_fixture,
    "act_quant.npz": act_quant_fixture,
    "routing.npz": routing_fixture,
    "align.npz": align_fixture,
    "layer_tiny.npz": layer_fixture,
}


def main() -> None:
    for name, fn in FIXTURES.items():
        path = os.path.join(HERE, name)
        np.savez_compressed(path, **fn())
        print(f"wrote {path} ({os.path.getsize(path)} bytes)")


if __name__ == "__main__":
    main()
