"""GPU parity through the reference's drop-in boundary: the patched MoeWNA16Method
process_weights_after_loading + apply (moe_experts.py:1277-1332), driven with a stand-in
method class and a layer holding MoeWNA16-format u8 parameters, as
test_wna16_moe_layer.py:19-84 builds them. The u8 tensors come from AWQ-packed nibbles
through the vLLM loader's AWQ -> standard conversion (moe_wna16.py:384-420, restated by
oracle.convert_awq_tensor); the oracle computes the layer from the unpacked nibbles."""
import numpy as np
import pytest
import torch

import oracle as O
from w4a8_fp8_wmma import moe_experts

pytestmark = pytest.mark.gpu
DEV = "cuda"
REL_TOL = 1e-2


def maxrel(got, ref):
    return float(np.abs(np.asarray(got, np.float64) - ref).max() / max(np.abs(ref).max(), 1e-30))


class _QC:
    weight_bits = 4

    def __init__(self, has_zp):
        self.has_zp = has_zp


def _stand_in_method():
    class Method:
        def __init__(self, has_zp):
            self.quant_config = _QC(has_zp)

        def process_weights_after_loading(self, layer):
            pass

        def apply(self, layer, x, topk_weights, topk_ids, shared_experts=None,
                  shared_experts_input=None):
            raise AssertionError("stock apply must not run for an engaged layer")

    moe_experts.install_moe_wna16_hooks(Method)
    return Method


def _awq_to_u8(packed):      # (E, R, C/8) AWQ int32 -> loader's standard u8, per expert
    kind = "qweight"
    return np.stack([O.convert_awq_tensor(packed[e], kind) for e in range(packed.shape[0])])


def _awq_zeros_to_u8(packed):
    return np.stack([O.convert_awq_tensor(packed[e], "qzeros") for e in range(packed.shape[0])])


def make_layer(r, E, H, I, g, has_zp):
    """MoeWNA16 layer parameters and the ground-truth op-layout arrays for the oracle."""
    G13, G2 = H // g, I // g
    nib13 = r.integers(0, 16, (E, H, 2 * I))          # AWQ orientation (K, N)
    nib2 = r.integers(0, 16, (E, I, H))
    zp13 = r.integers(0, 16, (E, G13, 2 * I)) if has_zp else None
    zp2 = r.integers(0, 16, (E, G2, H)) if has_zp else None
    s13 = (r.random((E, 2 * I, G13)) * 0.015 + 0.005).astype(np.float16)
    s2 = (r.random((E, H, G2)) * 0.015 + 0.005).astype(np.float16)

    class Layer:
        pass

    layer = Layer()
    layer.group_size = g
    layer.activation = "silu"
    layer.global_num_experts = E
    layer.expert_map = None
    layer.apply_router_weight_on_input = False
    P = lambda a: torch.nn.Parameter(torch.from_numpy(np.ascontiguousarray(a)).to(DEV), False)  # noqa: E731
    layer.w13_qweight = P(_awq_to_u8(O.awq_pack(nib13)))
    layer.w2_qweight = P(_awq_to_u8(O.awq_pack(nib2)))
    layer.w13_scales, layer.w2_scales = P(s13), P(s2)
    if has_zp:
        layer.w13_qzeros = P(_awq_zeros_to_u8(O.awq_pack(zp13)))
        layer.w2_qzeros = P(_awq_zeros_to_u8(O.awq_pack(zp2)))
    truth = dict(
        w13=O.pack_nibbles(np.swapaxes(nib13, 1, 2)), w2=O.pack_nibbles(np.swapaxes(nib2, 1, 2)),
        s13=s13, s2=s2,
        z13=O.pack_zeros(np.swapaxes(zp13, 1, 2)) if has_zp else None,
        z2=O.pack_zeros(np.swapaxes(zp2, 1, 2)) if has_zp else None)
    return layer, truth


# (E, hidden, inter, top_k, group, T, has_zp): test_wna16_moe_layer.py:63-65 shapes at the
# gfx950 group sizes, plus the c3 decode shape (Qwen3.x-35B-A3B experts)
CASES = [(8, 256, 128, 2, 128, 64, True), (16, 512, 256, 4, 128, 32, True),
         (4, 256, 128, 2, 128, 1, True), (8, 256, 128, 2, 128, 32, False),
         (8, 256, 128, 2, 64, 40, True), (16, 512, 256, 4, 128, 200, True),
         (256, 2048, 512, 8, 128, 32, True)]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "E{}_H{}_I{}_k{}_g{}_T{}_zp{}".format(*c))
def test_patched_moe_wna16_layer(case):
    E, H, I, k, g, T, has_zp = case
    r = np.random.default_rng(E * 7 + H + T)
    Method = _stand_in_method()
    method = Method(has_zp)
    layer, truth = make_layer(r, E, H, I, g, has_zp)
    u8_ptr = layer.w13_qweight.data.data_ptr()
    method.process_weights_after_loading(layer)
    rec = layer._w4a8
    want = "fragments" if g == 128 else "op"
    assert rec["layout"] == want
    # the parameter holds what the kernels read: the fragments, or the zero-copy op view
    assert rec["w13"].data_ptr() == layer.w13_qweight.data.data_ptr()
    if want == "fragments":
        assert rec["w13"].shape == (E, 2 * I // 16, 17, 16 * (H // 128))
        w, sc, zp = O.unrepack_fragments(rec["w13"].cpu().numpy())
        assert np.array_equal(w, truth["w13"]) and np.array_equal(sc, truth["s13"])
        want_zp = O.unpack_zeros(truth["z13"], 2 * I) if has_zp else np.full(sc.shape, 8)
        assert np.array_equal(zp, want_zp)
        assert np.array_equal(moe_experts._fragments_to_op_layout(rec["w13"]).cpu().numpy(),
                              truth["w13"])
    else:
        assert rec["w13"].data_ptr() == u8_ptr

    x = torch.from_numpy(r.standard_normal((T, H)).astype(np.float32)).to(DEV).to(torch.bfloat16)
    logits = r.standard_normal((T, E)).astype(np.float32)
    tw_np, ids_np = O.topk_softmax(logits, k)
    out = method.apply(layer, x.reshape(1, T, H), torch.from_numpy(tw_np).to(DEV),
                       torch.from_numpy(ids_np).to(DEV))
    assert out.shape == (1, T, H) and out.dtype == torch.bfloat16
    ref = O.moe_layer(x.float().cpu().numpy(), truth["w13"], truth["s13"], truth["z13"],
                      truth["w2"], truth["s2"], truth["z2"], tw_np, ids_np, g,
                      round_y_fp16=T > 96)
    rel = maxrel(out.reshape(T, H).float().cpu().numpy(), ref)
    print(f"  {want} layout, max_rel_err={rel:.3e}")
    assert rel <= REL_TOL
