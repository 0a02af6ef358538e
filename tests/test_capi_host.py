"""C-ABI library exports, argument validation and host-side API logic (CPU only).

No kernel is launched here: every C call below fails validation before touching HIP.
"""
import ctypes
import os
import re
import subprocess

import numpy as np
import pytest
import torch

import oracle as O
import w4a8_fp8_wmma as W
from w4a8_fp8_wmma import _lib, moe_experts

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "w4a8_moe.h")


def header_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"W4A8_API\s+[\w\s\*]+?\b(w4a8_\w+)\s*\(", text)))


def test_library_exports_exactly_the_header():
    syms = header_symbols()
    assert len(syms) >= 18
    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)],
                         capture_output=True, text=True, check=True).stdout
    exported = sorted(l.split()[-1] for l in out.splitlines() if " T " in l and "w4a8_" in l)
    assert exported == syms
    assert sorted(_lib.SIGNATURES) == syms
    cdll = ctypes.CDLL(str(_lib.LIB_PATH))
    for s in syms:
        assert getattr(cdll, s) is not None


def test_abi_version_and_sizes():
    L = _lib.lib
    assert L.w4a8_abi_version() == 3
    assert L.w4a8_fragments_words(2, 32, 256) == 2 * 2 * 272 * 2     # 16-row tiles of 272 G words
    assert L.w4a8_moe_align_sorted_len(256, 256, 16) == O.align_alloc_len(256, 256, 16)
    assert L.w4a8_moe_align_sorted_len(32768, 256, 64) == 48896      # c4: T k + E (64 - 1)
    assert L.w4a8_moe_align_sorted_len(8, 256, 8) == 1800            # C2 with block_m 8
    assert L.w4a8_moe_align_workspace_size(256, 256) == 0            # one-chunk path
    assert L.w4a8_moe_align_workspace_size(32768, 256) > 0
    assert L.w4a8_moe_gemm_workspace_size(32, 2048) >= 32 * 2048 + 32 * 4
    assert L.w4a8_moe_apply_workspace_size(32, 2048, 512, 256, 8) > 0


def _err():
    return _lib.lib.w4a8_last_error().decode()


def test_validation_errors_are_reported_without_gpu():
    L = _lib.lib
    # K not a multiple of 8
    rc = L.w4a8_mmq_fp8_moe_gemm(1, 4, 12, 1, 1, None, 2, 16, 16, 1, 16, 1, 1, 1, 16, 6, 0,
                                 1, 1, 1 << 20, None)
    assert rc == 1 and "multiple of 8" in _err()
    # bad kernel id
    rc = L.w4a8_mmq_fp8_moe_gemm(1, 4, 256, 1, 1, None, 2, 16, 128, 1, 16, 1, 1, 1, 16, 5, 0,
                                 1, 1, 1 << 20, None)
    assert rc == 1 and "kernel id" in _err()
    # gemv block_m cap
    rc = L.w4a8_mmq_fp8_moe_gemm(1, 4, 256, 1, 1, None, 2, 16, 128, 1, 128, 1, 1, 1, 128, 7, 0,
                                 1, 1, 1 << 20, None)
    assert rc == 1 and "gemv" in _err()
    # fused silu needs wmma
    rc = L.w4a8_mmq_fp8_moe_gemm1_silu(1, 4, 256, 1, 1, None, 2, 32, 128, 1, 16, 1, 1, 1, 16,
                                       7, 0, 1, 1, 1 << 20, None)
    assert rc == 1 and "wmma" in _err()
    # e2m1 with zero-points
    rc = L.w4a8_dequant_fp8(1, 1, 1, 8, 128, 128, 1, 1, None)
    assert rc == 1 and "symmetric" in _err()
    # align: wrong sorted_len
    rc = L.w4a8_moe_align_block_size(1, 16, 8, 4, None, 1, 17, 1, 1, None, 0, None)
    assert rc == 1 and "sorted_len" in _err()
    # dense: retired v3 id
    rc = L.w4a8_mmq_fp8_gemm(1, 16, 256, 1, 1, None, 64, 128, 3, 0, 1, 1, 1 << 20, None)
    assert rc == 1 and "dense kernel" in _err()
    # group size > 128
    rc = L.w4a8_mmq_fp8_gemm(1, 16, 512, 1, 1, None, 64, 256, 0, 0, 1, 1, 1 << 20, None)
    assert rc == 1 and "group_size" in _err()
    # moe_apply bad dtype
    rc = L.w4a8_moe_apply(1, 7, 4, 256, 128, 8, 2, 128, 1, 1, None, 1, 1, None, 1, 1, None, 0,
                          0, 1, 1, 1 << 20, None)
    assert rc == 1 and "dtype" in _err()
    # global expert count without a map
    rc = L.w4a8_moe_apply(1, 0, 4, 256, 128, 8, 2, 128, 1, 1, None, 1, 1, None, 1, 1, None, 16,
                          0, 1, 1, 1 << 20, None)
    assert rc == 1 and "expert_map" in _err()
    # fragment layout: decode needs a GEMV split for K/128 (5 is not one), prefill K <= 4096
    rc = L.w4a8_moe_apply_fragments(1, 0, 4, 640, 128, 8, 2, 128, 1, 1, None, 1, 1, None, 1, 1,
                                    None, 0, 1, 1, 1 << 20, None)
    assert rc == 1 and "fragment" in _err()
    rc = L.w4a8_moe_apply_fragments(1, 0, 200, 8192, 128, 8, 2, 128, 1, 1, None, 1, 1, None, 1,
                                    1, None, 0, 1, 1, 1 << 20, None)
    assert rc == 1 and "fragment" in _err()
    # the router covers at most 1024 experts
    rc = L.w4a8_moe_forward(1, 0, 4, 256, 128, 8, 2, 128, 1, 1, 1, 1, None, 1, 1, None, 0, 1,
                            2048, 1, 1, 1, 1, 1 << 20, None)
    assert rc == 1 and "1024" in _err()
    assert L.w4a8_moe_fragments_supported(2048, 512, 128) == 1     # c2-c4 shape
    assert L.w4a8_moe_fragments_supported(4096, 1536, 128) == 1    # c5 shape (K/128 = 32, 12)
    assert L.w4a8_moe_fragments_supported(640, 512, 128) == 0      # K/128 = 5: no GEMV split
    assert L.w4a8_moe_fragments_supported(2048, 512, 64) == 0      # g64: op layout only
    with pytest.raises(RuntimeError, match="multiple of 8"):
        _lib.check(L.w4a8_act_quant_fp8(1, 4, 12, 1, 1, 0, None), "act_quant")


def test_kernel_name_maps():
    assert W._resolve_moe_kernel("scalar") == 0
    assert W._resolve_moe_kernel("wmma") == 6
    assert W._resolve_moe_kernel("gemv") == 7
    assert W._resolve_dense_kernel("decode_gemv") == 11
    with pytest.raises(ValueError):
        W._resolve_moe_kernel("v5")
    with pytest.raises(TypeError):
        W._resolve_moe_kernel(6)
    with pytest.raises(ValueError):
        W._resolve_dense_kernel("nope")
    with pytest.raises(TypeError):
        W._resolve_dense_kernel(5)


def test_op_schemas_match_reference():
    s = torch.ops.w4a8_fp8_wmma.mmq_fp8_moe_gemm_scatter.default._schema
    assert "Tensor(a!) output" in str(s)
    for name in ("mmq_fp8_gemm", "mmq_fp8_moe_gemm", "mmq_fp8_moe_gemm1_silu",
                 "mmq_fp8_moe_gemm_scatter", "mmq_fp8_moe_gather_reduce"):
        op = getattr(torch.ops.w4a8_fp8_wmma, name).default
        assert torch.Tag.pt2_compliant_tag in op.tags


def test_fake_impls_shapes():
    from torch._subclasses.fake_tensor import FakeTensorMode
    with FakeTensorMode():
        x = torch.empty(8, 256, dtype=torch.float16)
        w = torch.empty(4, 64, 32, dtype=torch.int32)
        s = torch.empty(4, 64, 2, dtype=torch.float16)
        z = torch.empty(0, dtype=torch.int32)
        sti = torch.empty(128, dtype=torch.int32)
        eid = torch.empty(8, dtype=torch.int32)
        ntp = torch.empty(1, dtype=torch.int32)
        o = torch.ops.w4a8_fp8_wmma.mmq_fp8_moe_gemm(x, w, s, z, sti, eid, ntp, 2, 16, 6)
        assert o.shape == (128, 64) and o.dtype == torch.float16
        o = torch.ops.w4a8_fp8_wmma.mmq_fp8_moe_gemm1_silu(x, w, s, z, sti, eid, ntp, 2, 16, 6)
        assert o.shape == (128, 32)
        tw = torch.empty(16, dtype=torch.float32)
        g = torch.ops.w4a8_fp8_wmma.mmq_fp8_moe_gather_reduce(o, sti, tw, ntp, 2)
        assert g.shape == (8, 32) and g.dtype == torch.float32
        d = torch.ops.w4a8_fp8_wmma.mmq_fp8_gemm(x, w[0], s[0], z, 0)
        assert d.shape == (8, 64)
        out = torch.ops.vllm.w4a8_moe_apply(x, w, w, s, s, None, None, tw.view(8, 2),
                                             sti[:16].view(8, 2), "silu", 4, None, False, "wmma")
        assert out.shape == x.shape


def test_ops_reject_cpu_tensors():
    x = torch.zeros(4, 256, dtype=torch.float16)
    w = torch.zeros(2, 16, 32, dtype=torch.int32)
    s = torch.zeros(2, 16, 2, dtype=torch.float16)
    sti = torch.zeros(16, dtype=torch.int32)
    with pytest.raises((RuntimeError, NotImplementedError)):
        W.mmq_fp8_moe_gemm(x, w, s, sti, sti[:1], sti[:1], 2, 16)


def test_torch_converters_match_oracle():
    r = np.random.default_rng(30)
    E, K, N, g = 3, 256, 64, 32
    q = r.integers(0, 16, (E, K, N))
    zz = r.integers(0, 16, (E, K // g, N))
    s = r.uniform(0.005, 0.02, (E, K // g, N)).astype(np.float16)
    qw, qz = O.awq_pack(q), O.awq_pack(zz)
    w, sc, z = moe_experts._awq_moe_to_op_layout(torch.from_numpy(qw), torch.from_numpy(s),
                                                 torch.from_numpy(qz), g)
    wo, so, zo = O.awq_to_op_layout(qw, s, qz)
    assert np.array_equal(w.numpy(), wo) and np.array_equal(z.numpy(), zo)
    assert np.array_equal(sc.numpy(), so)
    # MoeWNA16 zero-copy view
    u8w = np.stack([O.convert_awq_tensor(qw[e], "qweight") for e in range(E)])
    u8z = np.stack([O.convert_awq_tensor(qz[e], "qzeros") for e in range(E)])
    tw_, ts_, tz_ = moe_experts._wna16_moe_to_op_layout(
        torch.from_numpy(u8w), torch.from_numpy(np.swapaxes(s, 1, 2).copy()), torch.from_numpy(u8z))
    assert np.array_equal(tw_.numpy(), wo) and np.array_equal(tz_.numpy(), zo)
    # compressed-tensors (GPTQ-packed along K, symmetric)
    ct = np.zeros((E, K // 8, N), np.int64)
    for j in range(8):
        ct |= (q[:, j::8, :] & 0xF) << (4 * j)
    cw, cs = moe_experts._ct_moe_to_op_layout(torch.from_numpy(ct.astype(np.uint32).view(np.int32)),
                                              torch.from_numpy(s))
    assert np.array_equal(O.unpack_nibbles(cw.numpy()), np.swapaxes(q, 1, 2))


def test_run_grouped_moe_rejects_unknown_activations():
    x = torch.zeros(2, 256, dtype=torch.bfloat16)
    with pytest.raises(NotImplementedError):
        moe_experts._run_grouped_moe(x, None, None, None, None, None, None, None,
                                     torch.zeros(2, 2, dtype=torch.int32), "gelu", 4, None,
                                     False, "wmma")


def test_mxfp4_converter_matches_oracle():
    """convert_mxfp4_moe: the E2M1 bytes are viewed as the op layout (no copy) and the E8M0
    scales become the oracle's fp16 values, every code included."""
    r = np.random.default_rng(11)
    E, N, K = 3, 16, 256
    wp = r.integers(0, 256, (E, N, K // 2), dtype=np.uint8)
    ws = r.integers(0, 256, (E, N, K // 32), dtype=np.uint8)
    ws.reshape(-1)[:256] = np.arange(256)                      # all 256 E8M0 codes
    c = moe_experts.convert_mxfp4_moe(torch.from_numpy(wp), torch.from_numpy(ws))
    ow, osc = O.convert_mxfp4(wp, ws)
    assert c["w_packed"].dtype == torch.int32 and c["w_packed"].shape == (E, N, K // 8)
    assert np.array_equal(c["w_packed"].numpy(), ow)
    assert np.array_equal(c["scales"].numpy().view(np.uint16), osc.view(np.uint16))
    assert c["w_zeros"] is None and c["group_size"] == 32
    info = c["scale_info"]
    assert info["e8m0_nan_groups"] >= 1 and not info["fp16_range_ok"]
    with pytest.raises(ValueError):
        moe_experts.convert_mxfp4_moe(torch.from_numpy(wp), torch.from_numpy(ws[..., :-1]))


def test_mxfp4_hook_with_stand_in_class():
    """Drive the patched mxfp4 process with a stand-in GptOssMxfp4MoEMethod (no vLLM): the
    layer gets op-layout views of its E2M1 bytes, fp16 scales and its biases; a layer in
    another layout keeps the stock path."""
    calls = {}

    class Method:
        def process_weights_after_loading(self, layer):
            calls["process"] = True

        def apply(self, layer, x, topk_weights, topk_ids, shared_experts=None,
                  shared_experts_input=None, **kw):
            return "stock"

    moe_experts.install_moe_mxfp4_hooks(Method)
    E, H, I = 2, 64, 32
    r = np.random.default_rng(12)

    def u8(*shape):
        return torch.nn.Parameter(torch.from_numpy(r.integers(0, 256, shape, dtype=np.uint8)), False)

    class Layer:
        w13_weight = u8(E, 2 * I, H // 2)
        w13_weight_scale = u8(E, 2 * I, H // 32)
        w2_weight = u8(E, H, I // 2)
        w2_weight_scale = u8(E, H, I // 32)
        w13_bias = torch.nn.Parameter(torch.zeros(E, 2 * I), False)
        w2_bias = torch.nn.Parameter(torch.zeros(E, H), False)

    layer = Layer()
    s13 = layer.w13_weight_scale.data.clone()
    m = Method()
    m.process_weights_after_loading(layer)
    assert "process" not in calls and m._w4a8_mxfp4
    rec = layer._w4a8_mx
    assert rec["w13"].shape == (E, 2 * I, H // 8) and rec["w13"].dtype == torch.int32
    assert rec["w13"].data_ptr() == layer.w13_weight.data.data_ptr()      # zero-copy view
    assert np.array_equal(rec["s13"].numpy().view(np.uint16), O.e8m0_to_fp16(s13.numpy()).view(np.uint16))
    assert rec["b13"].data_ptr() == layer.w13_bias.data_ptr() and layer.w13_weight_scale.numel() == 0

    class Other:       # a layout the converter refuses: the stock path stays
        w13_weight = torch.nn.Parameter(torch.zeros(E, 2 * I, H // 2), False)

    m2 = Method()
    m2.process_weights_after_loading(Other())
    assert calls.get("process") and not m2._w4a8_mxfp4
    assert m2.apply(Other(), None, None, None) == "stock"


def test_env_hard_break_and_kernel_env(monkeypatch):
    monkeypatch.setenv("VLLM_ROCM_W4A8_FP8_WMMA_MOE_VERSION", "6")
    with pytest.raises(RuntimeError, match="removed"):
        moe_experts._moe_kernel()
    monkeypatch.delenv("VLLM_ROCM_W4A8_FP8_WMMA_MOE_VERSION")
    monkeypatch.setenv("VLLM_ROCM_W4A8_FP8_WMMA_MOE_KERNEL", "bogus")
    with pytest.raises(RuntimeError, match="invalid"):
        moe_experts._moe_kernel()
    monkeypatch.setenv("VLLM_ROCM_W4A8_FP8_WMMA_MOE_KERNEL", "gemv")
    assert moe_experts._moe_kernel() == "gemv"


def test_wna16_hook_with_stand_in_class(monkeypatch):
    """Drive the patched process/apply with a stand-in MoeWNA16Method (no vLLM)."""
    calls = {}

    class QC:
        weight_bits = 4
        has_zp = True

    class Method:
        def __init__(self):
            self.quant_config = QC()

        def process_weights_after_loading(self, layer):
            calls["process"] = True

        def apply(self, layer, x, topk_weights, topk_ids, shared_experts, shared_experts_input):
            calls["orig_apply"] = True
            return "stock"

    moe_experts.install_moe_wna16_hooks(Method)
    E, N, K, g = 2, 16, 256, 128

    class Layer:
        group_size = g
        w13_qweight = torch.nn.Parameter(torch.zeros(E, N, K // 2, dtype=torch.uint8), False)
        w2_qweight = torch.nn.Parameter(torch.zeros(E, K, N // 4, dtype=torch.uint8), False)
        w13_scales = torch.nn.Parameter(torch.ones(E, N, K // g), False)
        w2_scales = torch.nn.Parameter(torch.ones(E, K, 1), False)
        w13_qzeros = torch.nn.Parameter(torch.zeros(E, N // 2, K // g, dtype=torch.uint8), False)
        w2_qzeros = torch.nn.Parameter(torch.zeros(E, K // 2, 1, dtype=torch.uint8), False)

    m, layer = Method(), Layer()
    m.process_weights_after_loading(layer)
    assert calls["process"] and m._w4a8_wna16
    rec = layer._w4a8
    # inter = 8 is no multiple of 128: the fragment kernels do not take it, op-layout views stay
    assert rec["layout"] == "op"
    assert rec["w13"].shape == (E, N, K // 8) and rec["w13"].dtype == torch.int32
    assert rec["w13"].data_ptr() == layer.w13_qweight.data.data_ptr()      # zero-copy view
    assert rec["z13"].shape == (E, N // 8, K // g)
    assert rec["s13"].dtype == torch.float16
    # unsupported group size keeps the stock apply
    layer2 = Layer()
    layer2.group_size = 256
    m2 = Method()
    m2.process_weights_after_loading(layer2)
    assert m2.apply(layer2, None, None, None) == "stock"


def test_fragments_to_op_layout_inverts_the_repack():
    r = np.random.default_rng(31)
    w = r.integers(-2**31, 2**31 - 1, (3, 48, 384 // 8), dtype=np.int64).astype(np.int32)
    sc = r.standard_normal((3, 48, 3)).astype(np.float16)
    f = O.repack_fragments(w, sc, O.pack_zeros(r.integers(0, 16, (3, 48, 3))))
    back = moe_experts._fragments_to_op_layout(torch.from_numpy(f))
    assert np.array_equal(back.numpy(), w)


def _layer_tensors(T=4, E=4, H=256, I=128, k=2, g=128):
    i32 = torch.int32
    return dict(
        x=torch.zeros(T, H, dtype=torch.bfloat16), w13=torch.zeros(E, 2 * I, H // 8, dtype=i32),
        w2=torch.zeros(E, H, I // 8, dtype=i32),
        w13_s=torch.zeros(E, 2 * I, H // g, dtype=torch.float16),
        w2_s=torch.zeros(E, H, I // g, dtype=torch.float16),
        w13_z=torch.zeros(E, 2 * I // 8, H // g, dtype=i32), w2_z=torch.zeros(E, H // 8, I // g, dtype=i32),
        topk_weights=torch.zeros(T, k), topk_ids=torch.zeros(T, k, dtype=i32))


@pytest.mark.parametrize("bad,match", [
    (dict(w2=torch.zeros(4, 256, 8, dtype=torch.int32)), "w2 must be"),
    (dict(w13_s=torch.zeros(4, 256, 3, dtype=torch.float16)), "w13 scales"),
    (dict(w2_s=torch.zeros(4, 256, 2, dtype=torch.float16)), "w2 scales"),
    (dict(w13_z=torch.zeros(4, 16, 2, dtype=torch.int32)), "w13 zeros"),
    (dict(w2_z=torch.zeros(4, 32, 2, dtype=torch.int32)), "w2 zeros"),
    (dict(topk_ids=torch.zeros(5, 2, dtype=torch.int32)), "topk_ids"),
    (dict(topk_weights=torch.zeros(4, 3)), "topk_weights"),
    (dict(expert_map=torch.zeros(8, dtype=torch.int32), global_num_experts=6), "expert_map"),
    (dict(global_num_experts=8), "pass expert_map"),
    ({}, "CUDA"),                 # shapes all fine: the device check is last
])
def test_layer_args_rejections(bad, match):
    """Every shape the whole-layer kernels index by is checked on the host (no device read
    can run past a tensor)."""
    t = _layer_tensors()
    extra = {k: bad.pop(k) for k in ("expert_map", "global_num_experts") if k in bad}
    t.update(bad)
    with pytest.raises(RuntimeError, match=match):
        W.moe_apply(t["x"], t["w13"], t["w2"], t["w13_s"], t["w2_s"], t["w13_z"], t["w2_z"],
                    t["topk_weights"], t["topk_ids"], extra.get("expert_map"),
                    global_num_experts=extra.get("global_num_experts"))


# --- dense linear (vllm::w4a8_dense_apply and its adapter) ---------------------------------
def test_dense_ladder_and_env(monkeypatch):
    from w4a8_fp8_wmma import linear
    monkeypatch.delenv("VLLM_ROCM_W4A8_DECODE_MAX_M", raising=False)
    d = linear.DECODE_MAX_M_DEFAULT
    big = 12288                       # N: 48 tile columns, so M = d + 1 fills >= 128 tiles
    assert linear.dense_kernel_for(1, big, 2048, 128) == "decode_gemv"
    assert linear.dense_kernel_for(d, big, 2048, 128) == "decode_gemv"
    assert linear.dense_kernel_for(d + 1, big, 2048, 128) == "prefill_wmma_ashuffle"
    assert linear.dense_kernel_for(1, big, 2048, 64) == "prefill_wmma"
    assert linear.dense_kernel_for(1, big, 2048, 32) == "prefill_wmma_ashuffle"
    # an under-filled tile grid stays on the GEMV: ceil(4096/256) * ceil(M/64) < 128
    assert linear.dense_kernel_for(256, 4096, 4096, 128) == "decode_gemv"       # 64 tiles
    assert linear.dense_kernel_for(512, 4096, 4096, 128) == "prefill_wmma_ashuffle"   # 128
    assert linear.dense_kernel_for(512, 1024, 2048, 128) == "decode_gemv"       # 32 tiles
    assert linear.dense_kernel_for(4096, 256, 2048, 128) == "prefill_wmma_ashuffle"   # M cap
    monkeypatch.setenv("VLLM_ROCM_W4A8_DECODE_MAX_M", "2")
    assert linear.dense_kernel_for(3, big, 2048, 128) == "prefill_wmma_ashuffle"
    assert linear.dense_kernel_for(3, 256, 2048, 128) == "prefill_wmma_ashuffle"  # env is strict
    for name in ("decode_gemv", "prefill_wmma_ashuffle", "prefill_wmma"):
        assert name in W._DENSE_KERNELS


def test_gptq_to_op_layout_from_the_format_definition():
    """AutoGPTQ qweight (K/8, N): word [k8, n] holds k = 8 k8 + j of column n in nibble j.
    Built element by element here, then converted and compared with the oracle's op-layout
    pack of the same matrix."""
    from w4a8_fp8_wmma import linear
    r = np.random.default_rng(5)
    N, K, g = 24, 64, 32
    nib = r.integers(0, 16, (N, K))
    gq = np.zeros((K // 8, N), np.int64)
    for k in range(K):
        for n in range(N):
            gq[k // 8, n] |= int(nib[n, k]) << (4 * (k % 8))
    gq = gq.astype(np.uint32).view(np.int32)
    sc = r.uniform(0.005, 0.02, (K // g, N)).astype(np.float32)
    wq, ws = linear.gptq_to_op_layout(torch.from_numpy(gq), torch.from_numpy(sc), K, N)
    assert np.array_equal(wq.numpy(), O.pack_nibbles(nib))
    assert ws.dtype == torch.float16 and np.array_equal(ws.numpy(), sc.T.astype(np.float16))
    with pytest.raises(ValueError, match="GPTQ qweight"):
        linear.gptq_to_op_layout(torch.from_numpy(gq).t(), torch.from_numpy(sc), K, N)


def test_dense_apply_rejections(monkeypatch):
    from w4a8_fp8_wmma import linear
    x = torch.zeros(2, 256, dtype=torch.bfloat16)
    wq = torch.zeros(64, 32, dtype=torch.int32)
    ws = torch.zeros(64, 2, dtype=torch.float16)
    args = (None, None, None, None, 64, 256, 128)
    with pytest.raises(ValueError, match="bias 8"):
        linear.w4a8_dense_apply(x, wq, ws, *args, False, 0, 0)
    with pytest.raises(ValueError, match="w_q must be"):
        linear.w4a8_dense_apply(x, wq[:, :16], ws, *args, False, 8, 0)
    with pytest.raises(ValueError, match="x must be"):
        linear.w4a8_dense_apply(x[:, :128], wq, ws, *args, False, 8, 0)
    monkeypatch.setenv("VLLM_ROCM_W4A8_FORCE", "off")
    with pytest.raises(RuntimeError, match="Triton"):
        linear.w4a8_dense_apply(x, wq, ws, *args, False, 8, 0)


def test_dense_apply_op_registered_with_fake():
    from torch._subclasses.fake_tensor import FakeTensorMode
    from w4a8_fp8_wmma import linear  # noqa: F401  (defines torch.ops.vllm.w4a8_dense_apply)
    with FakeTensorMode():
        x = torch.empty(5, 256, dtype=torch.bfloat16)
        wq = torch.empty(64, 32, dtype=torch.int32)
        ws = torch.empty(64, 2, dtype=torch.float16)
        o = torch.ops.vllm.w4a8_dense_apply(x, wq, ws, None, None, None, None, 64, 256, 128,
                                            False, 8, 0)
        assert o.shape == (5, 64) and o.dtype == torch.float16


def test_linear_kernel_can_implement():
    from w4a8_fp8_wmma import linear

    class Base:
        def __init__(self, c):
            self.config = c

    class T:
        uint4b8, uint4 = object(), object()

    class C:
        partition_weight_shape = (2048, 1024)
        group_size = 128
        weight_type = T.uint4
        act_type = torch.bfloat16
        has_g_idx = False

    Cls = linear.make_linear_kernel(Base, T, lambda: True)
    ok, why = Cls.can_implement(C)
    assert not ok and "gfx950" in why          # no device in this container
    ok, why = linear.make_linear_kernel(Base, T, lambda: False).can_implement(C)
    assert not ok and why == "ROCm only"
    assert linear.register_dense_linear(verbose=False) is False   # vLLM absent
