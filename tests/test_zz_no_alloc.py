"""w4a8_moe_forward_noalloc (the entry point that allocates nothing) against
w4a8_moe_forward with a caller workspace, through the C ABI: bit-identical outputs,
top-k weights and ids on two calls in a row, the second smaller than the first (so it runs
over the scratch contents the first call left), on both weight layouts; and the refusal of a
shape whose workspace exceeds the library's static scratch."""
import ctypes

import pytest
import torch

import bench
import w4a8_fp8_wmma as W
from w4a8_fp8_wmma import _lib

pytestmark = pytest.mark.gpu
DEV = "cuda"
L = _lib.lib
W4A8_ERR_WORKSPACE = 3
DTYPE_CODE = {torch.float16: 0, torch.bfloat16: 1}


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    assert torch.cuda.is_available(), "GPU tests need a visible MI355X"


def _p(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _weights(H, I, E, seed, layout):
    cfg = dict(T=1, H=H, E=E, k=1, I=I, g=128, routing="uniform")
    ws = bench.make_weights(cfg, seed, DEV)
    if layout == 1:
        ws["w13"] = W.repack_fragments(ws["w13"], ws["s13"], ws["z13"])
        ws["w2"] = W.repack_fragments(ws["w2"], ws["s2"], ws["z2"])
    return ws


def _call_pair(ws, T, H, I, E, k, seed, layout, dtype):
    """(regular outputs, no-alloc outputs) for one shape; every tensor is allocated before
    either call."""
    cfg = dict(T=T, H=H, E=E, k=k, I=I, g=128, routing="uniform")
    x, logits = bench.make_inputs(cfg, seed, DEV)
    x = x.to(dtype).contiguous()
    logits = logits.float().contiguous()
    nbytes = int(L.w4a8_moe_apply_workspace_size(T, H, I, E, k))
    assert nbytes <= 32 << 20, "test shape must fit the static scratch"
    workspace = torch.empty(nbytes, dtype=torch.uint8, device=DEV)
    outs = []
    for _ in range(2):
        outs.append((torch.empty_like(x),
                     torch.empty((T, k), dtype=torch.float32, device=DEV),
                     torch.empty((T, k), dtype=torch.int32, device=DEV)))
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    def args(o):
        return [_p(x), DTYPE_CODE[dtype], T, H, I, E, k, 128, _p(logits), 1, _p(ws["w13"]),
                _p(ws["s13"]), _p(ws["z13"]), _p(ws["w2"]), _p(ws["s2"]), _p(ws["z2"]), layout,
                None, E, _p(o[1]), _p(o[2]), _p(o[0])]

    torch.cuda.synchronize()
    _lib.check(L.w4a8_moe_forward(*args(outs[0]), _p(workspace), nbytes, stream), "moe_forward")
    _lib.check(L.w4a8_moe_forward_noalloc(*args(outs[1]), stream), "moe_forward_noalloc")
    torch.cuda.synchronize()
    return outs


@pytest.mark.parametrize("layout,shapes", [
    (1, [(32, 8), (5, 4)]),          # fragments, decode schedule (T <= 96)
    (0, [(160, 4), (100, 2)]),       # op layout, prefill schedule (T > 96)
])
def test_noalloc_matches_forward_two_calls(layout, shapes):
    H, I, E = 1024, 256, 32
    print(f"noalloc layout={layout} H={H} I={I} E={E} calls={shapes}", flush=True)
    ws = _weights(H, I, E, 900 + layout, layout)
    for call, (T, k) in enumerate(shapes):
        (ref, tw_ref, ids_ref), (got, tw, ids) = _call_pair(
            ws, T, H, I, E, k, 910 + 10 * layout + call, layout, torch.bfloat16)
        assert torch.equal(ids, ids_ref), f"call {call}: topk ids differ"
        assert torch.equal(tw, tw_ref), f"call {call}: topk weights differ"
        assert torch.equal(got, ref), f"call {call}: layer output differs"
        assert torch.isfinite(got.float()).all()


def test_noalloc_refuses_shapes_beyond_the_scratch():
    T, H, I, E, k = 4096, 2048, 768, 128, 8
    need = int(L.w4a8_moe_apply_workspace_size(T, H, I, E, k))
    assert need > 32 << 20
    rc = L.w4a8_moe_forward_noalloc(None, 1, T, H, I, E, k, 128, None, 1, None, None, None,
                                    None, None, None, 0, None, E, None, None, None, None)
    assert rc == W4A8_ERR_WORKSPACE
    msg = L.w4a8_last_error().decode()
    assert "static scratch" in msg and str(need) in msg
