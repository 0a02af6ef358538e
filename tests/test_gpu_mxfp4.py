"""gpt-oss (mxfp4) MoE layers on the GPU: E2M1 codes and E8M0 block scales converted at
load (convert_mxfp4_moe), per-expert biases, and the swigluoai activation between the
GEMMs (moe_experts.py:1351-1450 in the reference), through ``_run_grouped_moe`` and through
the patched GptOssMxfp4MoEMethod apply, against the CPU oracle.

gpt-oss shapes: hidden = intermediate = 2880 (22.5 K steps of 128: the fp4 tiles' last K
step is partial), top-4, mxfp4 block 32. The fp4 matrix core rounds a group's product sum
itself (see test_gpu_layer.test_e2m1_layer), so the layer is pinned in two steps, as there:
gemm1 on the same tiles against the oracle's gemm1 (2e-3), then the layer against the
oracle's second half (bias, swigluoai, act-quant, gemm2, bias, reduce) run from the
kernel's own gemm1 bits at the usual 1e-2; end to end the oracle is held to 3e-2."""
import numpy as np
import pytest
import torch

import oracle as O
from oracle.w4a8_oracle import _add_bias_f16
import w4a8_fp8_wmma as W
from w4a8_fp8_wmma import _ops, moe_experts

pytestmark = pytest.mark.gpu
DEV = "cuda"
REL_TOL = 1e-2


def maxrel(got, ref):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.abs(got - ref).max() / max(np.abs(ref).max(), 1e-30))


def test_swigluoai_kernel_vs_oracle():
    """Interleaved gate/up, both clamps crossed; expf may differ from numpy's exp by an ulp,
    so at most one fp16 ulp of difference."""
    r = np.random.default_rng(31)
    x = (r.standard_normal((37, 2 * 320)) * 6).astype(np.float16)
    out = torch.empty((37, 320), dtype=torch.float16, device=DEV)
    _ops.swigluoai_and_mul(out, torch.from_numpy(x).to(DEV))
    ref = O.swigluoai_and_mul(x).astype(np.float32)
    got = out.cpu().numpy().astype(np.float32)
    assert np.all(np.abs(got - ref) <= np.abs(ref) * 2.0 ** -10 * 2.01 + 2.0 ** -24 * 4)
    # alpha / limit reach the kernel
    out2 = torch.empty_like(out)
    _ops.swigluoai_and_mul(out2, torch.from_numpy(x).to(DEV), alpha=1.0, limit=3.0)
    ref2 = O.swigluoai_and_mul(x, alpha=1.0, limit=3.0).astype(np.float32)
    assert np.all(np.abs(out2.cpu().numpy().astype(np.float32) - ref2)
                  <= np.abs(ref2) * 2.0 ** -10 * 2.01 + 2.0 ** -24 * 4)


def mxfp4_layer(seed, E, H, I, T, k):
    """Random E2M1 codes, E8M0 scales near gpt-oss's (2^-9 .. 2^-4), fp16 biases."""
    r = np.random.default_rng(seed)
    raw = dict(w13=r.integers(0, 256, (E, 2 * I, H // 2), dtype=np.uint8),
               s13=r.integers(118, 124, (E, 2 * I, H // 32), dtype=np.uint8),
               w2=r.integers(0, 256, (E, H, I // 2), dtype=np.uint8),
               s2=r.integers(118, 124, (E, H, I // 32), dtype=np.uint8))
    b13 = (r.standard_normal((E, 2 * I)) * 0.1).astype(np.float16)
    b2 = (r.standard_normal((E, H)) * 0.1).astype(np.float16)
    x = torch.from_numpy(r.standard_normal((T, H)).astype(np.float32)).to(torch.bfloat16).to(DEV)
    logits = torch.from_numpy(r.standard_normal((T, E)).astype(np.float32)).to(DEV)
    tw, ids = W.fused_topk(None, logits, k, True)
    return raw, b13, b2, x, tw, ids


def oracle_after_gemm1(g1_slots, ids, tw, w2, s2, b13, b2):
    """The oracle layer's second half from gemm1's fp16 rows (slot order): + w13 bias,
    swigluoai, act-quant, gemm2 over the E2M1 codebook, + w2 bias (fp16 rows), weighted sum."""
    T, k = ids.shape
    e = ids.reshape(-1)
    g1 = _add_bias_f16(g1_slots, b13, e)
    h = O.swigluoai_and_mul(g1)
    a2, sc2 = O.act_quant(h)
    y = (O.grouped_run(a2, e, w2, s2, None, 32, True) * sc2[:, None]).astype(np.float32)
    y = _add_bias_f16(y.astype(np.float16), b2, e).astype(np.float32).reshape(T, k, -1)
    acc = np.zeros((T, y.shape[2]), np.float32)
    for j in range(k):
        acc = O.fma32(tw[:, j:j + 1].astype(np.float32), y[:, j], acc)
    return acc


@pytest.mark.parametrize("H,I,T", [(2880, 2880, 6), (2880, 2880, 100), (2048, 1024, 40)])
def test_gpt_oss_layer(H, I, T):
    E, k = 8, 4
    raw, b13, b2, x, tw, ids = mxfp4_layer(3100 + T + H, E, H, I, T, k)
    c13 = moe_experts.convert_mxfp4_moe(torch.from_numpy(raw["w13"]).to(DEV),
                                        torch.from_numpy(raw["s13"]).to(DEV))
    c2 = moe_experts.convert_mxfp4_moe(torch.from_numpy(raw["w2"]).to(DEV),
                                       torch.from_numpy(raw["s2"]).to(DEV))
    assert c13["scale_info"]["fp16_range_ok"] and c2["scale_info"]["fp16_range_ok"]
    out = moe_experts._run_grouped_moe(
        x, c13["w_packed"], c2["w_packed"], c13["scales"], c2["scales"], None, None, tw, ids,
        "swigluoai", E, None, False, "wmma", weight_is_e2m1=True,
        w1_bias=torch.from_numpy(b13).to(DEV), w2_bias=torch.from_numpy(b2).to(DEV))
    assert out.dtype == x.dtype and torch.isfinite(out.float()).all()
    w13, s13 = O.convert_mxfp4(raw["w13"], raw["s13"])
    w2, s2 = O.convert_mxfp4(raw["w2"], raw["s2"])
    ids_np, tw_np = ids.cpu().numpy(), tw.cpu().numpy()
    ref, st = O.moe_layer(x.float().cpu().numpy(), w13, s13, None, w2, s2, None, tw_np, ids_np,
                          32, e2m1=True, w1_bias=b13, w2_bias=b2, activation="swigluoai",
                          return_stages=True)
    # gemm1 on the same fp4 tiles (the unfused path's first op), rows back in slot order
    bm = 64
    sti, eid, ntp = O.moe_align(ids_np.astype(np.int32), bm, E)
    n = int(ntp[0])
    g1 = W.mmq_fp8_moe_gemm(x.half(), c13["w_packed"], c13["scales"],
                            *[torch.from_numpy(a).to(DEV) for a in (sti, eid, ntp)], k, bm,
                            kernel="wmma", weight_is_e2m1=True).cpu().numpy()
    real = np.nonzero(sti[:n] < T * k)[0]
    g1_slots = np.empty((T * k, g1.shape[1]), np.float16)
    g1_slots[sti[real]] = g1[real]
    a1, sc1 = st["a1"], st["s1"]
    tok = np.repeat(np.arange(T), k)
    run1 = O.grouped_run(a1[tok], ids_np.reshape(-1), w13, s13, None, 32, True)
    g1_ref = (run1 * sc1[tok][:, None]).astype(np.float32).astype(np.float16)
    assert maxrel(g1_slots, g1_ref) <= 2e-3
    got = out.float().cpu().numpy()
    assert maxrel(got, oracle_after_gemm1(g1_slots, ids_np, tw_np, w2, s2, b13, b2)) <= REL_TOL
    assert maxrel(got, ref) <= 3e-2


def test_mxfp4_hook_apply_on_gpu():
    """The patched GptOssMxfp4MoEMethod (a stand-in class here; vLLM is absent) loads a layer
    and its apply equals _run_grouped_moe on the converted weights, bit for bit."""
    class Method:
        def process_weights_after_loading(self, layer):
            raise AssertionError("stock process must not run for an mxfp4 layer")

        def apply(self, *a, **kw):
            raise AssertionError("stock apply must not run for an mxfp4 layer")

    moe_experts.install_moe_mxfp4_hooks(Method)
    E, H, I, T, k = 8, 2880, 2880, 12, 4
    raw, b13, b2, x, tw, ids = mxfp4_layer(3200, E, H, I, T, k)

    def prm(a):
        return torch.nn.Parameter(torch.from_numpy(a).to(DEV), requires_grad=False)

    class Layer:
        w13_weight = prm(raw["w13"])
        w13_weight_scale = prm(raw["s13"])
        w2_weight = prm(raw["w2"])
        w2_weight_scale = prm(raw["s2"])
        w13_bias = prm(b13)
        w2_bias = prm(b2)
        activation = "swigluoai"
        global_num_experts = E
        expert_map = None
        apply_router_weight_on_input = False

    m, layer = Method(), Layer()
    m.process_weights_after_loading(layer)
    got = m.apply(layer, x.reshape(2, T // 2, H), tw, ids)
    assert got.shape == (2, T // 2, H) and got.dtype == x.dtype
    c13 = moe_experts.convert_mxfp4_moe(torch.from_numpy(raw["w13"]).to(DEV),
                                        torch.from_numpy(raw["s13"]).to(DEV))
    c2 = moe_experts.convert_mxfp4_moe(torch.from_numpy(raw["w2"]).to(DEV),
                                       torch.from_numpy(raw["s2"]).to(DEV))
    ref = moe_experts._run_grouped_moe(
        x, c13["w_packed"], c2["w_packed"], c13["scales"], c2["scales"], None, None, tw, ids,
        "swigluoai", E, None, False, moe_experts._moe_kernel(), weight_is_e2m1=True,
        w1_bias=torch.from_numpy(b13).to(DEV), w2_bias=torch.from_numpy(b2).to(DEV))
    assert torch.equal(got.reshape(T, H), ref)
