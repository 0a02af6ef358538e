"""GPU parity of the dense linear path: ``torch.ops.vllm.w4a8_dense_apply`` (the reference's op,
vllm_adapter.py:265-386) and the MPLinearKernel adapter built on a stand-in base class
(vllm_adapter.py:390-593), against the oracle's dense GEMM (the reference_scalar arithmetic
of dense_kernel.hip:107-200) at the layer tolerance. Batches cover both sides of the
decode-GEMV / MFMA-tile ladder, symmetric (uint4b8) and AWQ zero-point weights, bf16 and
fp16 activations, and AutoGPTQ-layout checkpoints."""
import numpy as np
import pytest
import torch

import oracle as O
from w4a8_fp8_wmma import linear

pytestmark = pytest.mark.gpu
DEV = "cuda"
REL_TOL = 1e-2


def maxrel(got, ref):
    return float(np.abs(np.asarray(got, np.float64) - ref).max() / max(np.abs(ref).max(), 1e-30))


def make_weights(r, N, K, g, asym):
    nib = r.integers(0, 16, (N, K))
    zp = r.integers(0, 16, (N, K // g)) if asym else None
    sc = r.uniform(0.005, 0.02, (N, K // g)).astype(np.float16)
    return nib, zp, sc


@pytest.mark.parametrize("M", [1, 2, 5, 16, 17, 64, 300])
@pytest.mark.parametrize("asym", [True, False])
def test_dense_apply_vs_oracle(M, asym):
    r = np.random.default_rng(7000 + M + 1000 * asym)
    N, K, g = 1024, 2048, 128
    nib, zp, sc = make_weights(r, N, K, g, asym)
    w = O.pack_nibbles(nib)
    z = O.pack_zeros(zp) if asym else None
    x = torch.randn(M, K, generator=torch.Generator().manual_seed(M)).to(torch.bfloat16)
    x16 = x.to(torch.float16).numpy()
    wd = torch.from_numpy(w).to(DEV)
    sd = torch.from_numpy(sc).to(DEV)
    zd = torch.from_numpy(z).to(DEV) if asym else None
    out = torch.ops.vllm.w4a8_dense_apply(x.to(DEV), wd, sd, zd, None, None, None, N, K, g,
                                          asym, 0 if asym else 8, 0)
    assert out.dtype == torch.float16 and tuple(out.shape) == (M, N)
    ref = O.dense_gemm(x16, w, sc, z)
    assert maxrel(out.cpu().numpy(), ref) <= REL_TOL
    # fp16 activations give the same bits (the op casts bf16 to fp16 first)
    out16 = linear.w4a8_dense_apply(torch.from_numpy(x16).to(DEV), wd, sd, zd, None, None, None,
                                    N, K, g, asym, 0 if asym else 8, 0)
    assert torch.equal(out, out16)


@pytest.mark.parametrize("M", [1, 40])
def test_dense_long_k_vs_oracle(M):
    """K = 6144 (48 groups): past the GEMV and streamed-K tables, so both names run the
    general MFMA tiles."""
    r = np.random.default_rng(7050 + M)
    N, K, g = 384, 6144, 128
    nib, zp, sc = make_weights(r, N, K, g, True)
    w, z = O.pack_nibbles(nib), O.pack_zeros(zp)
    x = torch.randn(M, K, generator=torch.Generator().manual_seed(M)).to(torch.float16)
    out = linear.w4a8_dense_apply(x.to(DEV), torch.from_numpy(w).to(DEV), torch.from_numpy(sc).to(DEV),
                                  torch.from_numpy(z).to(DEV), None, None, None, N, K, g, True, 0, 0)
    assert maxrel(out.cpu().numpy(), O.dense_gemm(x.numpy(), w, sc, z)) <= REL_TOL


@pytest.mark.parametrize("M", [1, 8, 16, 300, 1000])
def test_dense_gemv_equals_tiles(M):
    """Both sides of the ladder compute the same arithmetic: the decode GEMV and the MFMA tiles
    agree to within one fp16 rounding of each other (different fp32 summation order)."""
    r = np.random.default_rng(7100 + M)
    N, K, g = 2048, 4096, 128
    nib, zp, sc = make_weights(r, N, K, g, True)
    wd = torch.from_numpy(O.pack_nibbles(nib)).to(DEV)
    sd = torch.from_numpy(sc).to(DEV)
    zd = torch.from_numpy(O.pack_zeros(zp)).to(DEV)
    x = torch.randn(M, K, generator=torch.Generator().manual_seed(M)).to(torch.float16).to(DEV)
    from w4a8_fp8_wmma import mmq_fp8_gemm
    a = mmq_fp8_gemm(x, wd, sd, kernel="decode_gemv", w_zeros=zd).float()
    b = mmq_fp8_gemm(x, wd, sd, kernel="prefill_wmma_ashuffle", w_zeros=zd).float()
    assert float((a - b).abs().max() / b.abs().max()) <= 2e-3


@pytest.mark.parametrize("M,N,K,asym", [(1, 16, 1024, True), (3, 384, 3072, True), (16, 1024, 1024, False),
                                         (1, 4096, 4096, False), (7, 2048, 4096, True)])
def test_dense_few_rows_vs_oracle(M, N, K, asym):
    """1 <= M <= 16 rows take the dense GEMV (rows quantised in the kernel, K split over eight
    waves): every split (one to four groups a wave), one column tile, symmetric and AWQ
    weights, against the oracle and the MFMA tiles."""
    r = np.random.default_rng(7200 + M + N + K)
    g = 128
    nib, zp, sc = make_weights(r, N, K, g, asym)
    w = O.pack_nibbles(nib)
    z = O.pack_zeros(zp) if asym else None
    x = torch.randn(M, K, generator=torch.Generator().manual_seed(M + K)).to(torch.float16)
    wd, sd = torch.from_numpy(w).to(DEV), torch.from_numpy(sc).to(DEV)
    zd = torch.from_numpy(z).to(DEV) if asym else None
    out = linear.w4a8_dense_apply(x.to(DEV), wd, sd, zd, None, None, None, N, K, g, asym,
                                  0 if asym else 8, 0)
    assert tuple(out.shape) == (M, N) and torch.isfinite(out.float()).all()
    assert maxrel(out.cpu().numpy(), O.dense_gemm(x.numpy(), w, sc, z)) <= REL_TOL
    from w4a8_fp8_wmma import mmq_fp8_gemm
    b = mmq_fp8_gemm(x.to(DEV), wd, sd, kernel="prefill_wmma_ashuffle", w_zeros=zd).float()
    assert float((out.float() - b).abs().max() / b.abs().max()) <= 2e-3


def gptq_pack(nib):
    """(N, K) nibbles -> AutoGPTQ qweight (K/8, N): word [k8, n] holds k = 8 k8 + j of column
    n in nibble j (packed along K)."""
    N, K = nib.shape
    return O.pack_nibbles(nib.T.reshape(K // 8, 8, N).transpose(0, 2, 1))[..., 0]


# --- the MPLinearKernel adapter on a stand-in base (vLLM is not installed) -------------------
class _ScalarType:
    def __init__(self, name, bias):
        self.name, self.bias = name, bias

    def has_bias(self):
        return self.bias != 0


class _ScalarTypes:
    uint4b8 = _ScalarType("uint4b8", 8)
    uint4 = _ScalarType("uint4", 0)


class _Config:
    def __init__(self, K, N, g, weight_type, zero_points, act_type=torch.bfloat16):
        self.partition_weight_shape = (K, N)
        self.group_size = g
        self.weight_type = weight_type
        self.zero_points = zero_points
        self.act_type = act_type
        self.has_g_idx = False


class _MPLinearKernelStandIn:
    """The parts of vLLM's MPLinearKernel the adapter uses: the config, the parameter names
    and _get_weight_params / _transform_param."""
    w_q_name, w_s_name, w_zp_name = "weight_packed", "weight_scale", "weight_zero_point"

    def __init__(self, c):
        self.config = c

    def _get_weight_params(self, layer):
        return (getattr(layer, self.w_q_name), getattr(layer, self.w_s_name),
                getattr(layer, self.w_zp_name, None), None)

    def _transform_param(self, layer, name, fn):
        old = getattr(layer, name)
        setattr(layer, name, torch.nn.Parameter(fn(old.data), requires_grad=False))


@pytest.mark.parametrize("layout,asym,M", [("ct", True, 3), ("ct", False, 40),
                                           ("gptq", False, 1), ("gptq", False, 130)])
def test_linear_kernel_adapter(layout, asym, M):
    """process_weights_after_loading + apply_weights through the adapter, with a bias, for
    compressed-tensors (N, K/8) and AutoGPTQ (K/8, N) checkpoints."""
    Cls = linear.make_linear_kernel(_MPLinearKernelStandIn, _ScalarTypes, lambda: True)
    r = np.random.default_rng(7200 + M)
    N, K, g = 768, 1024, 128
    nib, zp, sc = make_weights(r, N, K, g, asym)
    w = O.pack_nibbles(nib)
    wt = _ScalarTypes.uint4 if asym else _ScalarTypes.uint4b8
    cfg = _Config(K, N, g, wt, asym)
    ok, why = Cls.can_implement(cfg)
    assert ok, why
    layer = torch.nn.Module()
    P = lambda a: torch.nn.Parameter(torch.from_numpy(np.ascontiguousarray(a)).to(DEV),  # noqa: E731
                                     requires_grad=False)
    if layout == "gptq":
        layer.weight_packed = P(gptq_pack(nib))
        layer.weight_scale = P(sc.T.astype(np.float32))
    else:
        layer.weight_packed = P(w)
        layer.weight_scale = P(sc)
    if asym:
        layer.weight_zero_point = P(O.pack_zeros(zp))
    kern = Cls(cfg)
    kern.process_weights_after_loading(layer)
    assert tuple(layer.weight_packed.shape) == (N, K // 8)
    x = torch.randn(2, M, K, generator=torch.Generator().manual_seed(M)).to(torch.bfloat16)
    bias = torch.randn(N, generator=torch.Generator().manual_seed(1)).to(torch.bfloat16)
    out = kern.apply_weights(layer, x.to(DEV), bias.to(DEV))
    assert out.dtype == torch.bfloat16 and tuple(out.shape) == (2, M, N)
    ref = O.dense_gemm(x.reshape(-1, K).to(torch.float16).numpy(), w, sc,
                       O.pack_zeros(zp) if asym else None)
    ref = (torch.from_numpy(ref).to(torch.bfloat16) + bias).float().numpy()
    assert maxrel(out.reshape(-1, N).float().cpu().numpy(), ref) <= REL_TOL
