"""The torch-CPU port (oracle/cpu_port.py, the bench's CPU baseline) equals the pinned numpy
oracle: act-quant bit for bit, the grouped run bit for bit, the whole layer to fp32
rounding of the exp in SiLU (torch and numpy evaluate exp with different libm code)."""
import numpy as np
import pytest
import torch

import oracle as O
from oracle import cpu_port as P


def test_act_quant_bit_exact():
    r = np.random.default_rng(60)
    x = (r.standard_normal((16, 512)) * np.exp2(r.integers(-8, 8, (16, 1)))).astype(np.float16)
    x[0] = 0
    q, s = O.act_quant(x)
    qt, st = P.act_quant(torch.from_numpy(x))
    assert np.array_equal(st.numpy(), s)
    assert np.array_equal(qt.numpy(), O.E4M3_TO_F64[q])


@pytest.mark.parametrize("asym", [True, False])
def test_grouped_run_bit_exact(asym):
    r = np.random.default_rng(61)
    E, N, K = 3, 64, 512
    w = r.integers(-2**31, 2**31 - 1, (E, N, K // 8)).astype(np.int32)
    z = r.integers(-2**31, 2**31 - 1, (E, N // 8, K // 128)).astype(np.int32) if asym else None
    sc = (r.random((E, N, K // 128)) * 0.015 + 0.005).astype(np.float16)
    x = r.standard_normal((20, K)).astype(np.float16)
    rows = r.integers(0, E, 20)
    q, _ = O.act_quant(x)
    ref = O.grouped_run(q, rows, w, sc, z, 128)
    got = P.grouped_run(torch.from_numpy(O.E4M3_TO_F64[q]), torch.from_numpy(rows),
                        torch.from_numpy(w), torch.from_numpy(sc),
                        None if z is None else torch.from_numpy(z), 128)
    assert np.array_equal(got.numpy(), ref)


def test_layer_matches_oracle():
    r = np.random.default_rng(62)
    E, H, I, T, k = 8, 256, 128, 9, 2
    w13 = r.integers(-2**31, 2**31 - 1, (E, 2 * I, H // 8)).astype(np.int32)
    w2 = r.integers(-2**31, 2**31 - 1, (E, H, I // 8)).astype(np.int32)
    z13 = r.integers(-2**31, 2**31 - 1, (E, 2 * I // 8, H // 128)).astype(np.int32)
    z2 = r.integers(-2**31, 2**31 - 1, (E, H // 8, I // 128)).astype(np.int32)
    s13 = (r.random((E, 2 * I, H // 128)) * 0.015 + 0.005).astype(np.float16)
    s2 = (r.random((E, H, I // 128)) * 0.015 + 0.005).astype(np.float16)
    x = r.standard_normal((T, H)).astype(np.float32)
    tw, ids = O.topk_softmax(r.standard_normal((T, E)).astype(np.float32), k)
    ref = O.moe_layer(x, w13, s13, z13, w2, s2, z2, tw, ids, 128, round_y_fp16=False)
    t = lambda a: torch.from_numpy(a)  # noqa: E731
    got = P.moe_layer(t(x), t(w13), t(s13), t(z13), t(w2), t(s2), t(z2), t(tw), t(ids), 128)
    rel = np.abs(got.numpy() - ref).max() / np.abs(ref).max()
    assert rel <= 1e-3, rel
    assert np.mean(got.numpy() == ref) > 0.9
