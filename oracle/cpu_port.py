"""torch-CPU restatement of the reference W4A8 MoE layer (TEST / BASELINE INFRASTRUCTURE ONLY).

Only ``tests/`` and ``bench.py``'s ``cpu_baseline`` leg may import this module: it is the
CPU baseline the bench times beside the GPU (run on all host cores) and never part of the
product. It computes what ``w4a8_oracle.moe_layer`` computes, vectorised per expert with
torch tensor ops instead of numpy, keeping the kernels' rounding points (the arithmetic of
``fp8_ref_moe``, w4a8_fp8_wmma/test_moe_experts.py:155-191, with the kernel SiLU of
moe_kernel.hip:555-561 and the per-token act-quant of moe_kernel.hip:87-127):

  * x16 = fp16(x); per-row s = max(absmax / 448, 1e-8); a = e4m3(x16 * (1/s));
  * per expert, per 128-wide K group, the partial sums of e4m3 values times the integers
    (nibble - zero-point) in float64 (exact), rounded once to fp32; run += part * scale
    sequentially over groups (moe_gemm_tiled.h:144-151);
  * gate/up = fp16(run * s); h = fp16(fp16(g / (1 + exp(-g))) * up);
  * the same for gemm2 on the act-quantised h; y = run2 * s2 in fp32 (fp16-rounded with
    ``round_y_fp16``, the prefill path);
  * out[t] = sum over j ascending of w[t, j] * y[t, j] in fp32.

Pinned by tests/test_cpu_port.py against the numpy oracle.
"""
from __future__ import annotations

import torch

E4M3_MAX = 448.0
ACT_SCALE_FLOOR = 1e-8


def act_quant(x16: torch.Tensor):
    """(R, K) fp16 -> (e4m3 values as float64 (R, K), scales fp32 (R,))."""
    xf = x16.float()
    amax = xf.abs().amax(dim=-1) if xf.shape[-1] else torch.zeros(xf.shape[0])
    s = torch.clamp(amax / E4M3_MAX, min=ACT_SCALE_FLOOR)
    inv = 1.0 / s
    q = (xf * inv[:, None]).to(torch.float8_e4m3fn)
    return q.to(torch.float64), s


def _nibbles(words: torch.Tensor) -> torch.Tensor:
    """(..., W) int32 -> (..., 8 W) int16, nibble j of word w at position 8 w + j."""
    w = words.to(torch.int64) & 0xFFFFFFFF
    shifts = torch.arange(0, 32, 4, dtype=torch.int64)
    return ((w[..., None] >> shifts) & 0xF).reshape(*words.shape[:-1], -1).to(torch.int16)


def expert_weights(w_e: torch.Tensor, z_e, group: int) -> torch.Tensor:
    """One expert's op-layout weights (N, K/8) -> float64 (N, K) of (nibble - zero-point)."""
    nib = _nibbles(w_e)
    N, K = nib.shape
    if z_e is None:
        zp = torch.full((N, K // group), 8, dtype=torch.int16)
    else:
        zw = z_e.to(torch.int64) & 0xFFFFFFFF                      # (N/8, G)
        n = torch.arange(N)
        zp = ((zw[n // 8] >> ((n % 8) * 4)[:, None]) & 0xF).to(torch.int16)
    return (nib - zp.repeat_interleave(group, dim=1)).to(torch.float64)


def grouped_run(a: torch.Tensor, slot_expert: torch.Tensor, w, scales, zeros, group: int):
    """run[r, n] for rows r (e4m3 values a, float64) of the experts in slot_expert."""
    R, K = a.shape
    E, N, _ = w.shape
    G = K // group
    run = torch.zeros((R, N), dtype=torch.float32)
    for e in torch.unique(slot_expert).tolist():
        if e < 0 or e >= E:
            continue
        idx = torch.nonzero(slot_expert == e).flatten()
        W = expert_weights(w[e], None if zeros is None else zeros[e], group)
        part = torch.matmul(a[idx].reshape(-1, G, group).transpose(0, 1),
                            W.reshape(N, G, group).permute(1, 2, 0)).to(torch.float32)
        sc = scales[e].to(torch.float64)                           # (N, G)
        r = torch.zeros((idx.numel(), N), dtype=torch.float32)
        for g in range(G):      # fp32 fused multiply-add, sequential over groups
            r = (part[g].to(torch.float64) * sc[:, g] + r.to(torch.float64)).to(torch.float32)
        run[idx] = r
    return run


def moe_layer(x, w13, s13, z13, w2, s2, z2, topk_weights, topk_ids, group: int = 128,
              round_y_fp16: bool = False) -> torch.Tensor:
    """Whole layer on CPU tensors (op-layout weights). x (T, H) float -> (T, H) float32."""
    x16 = x.to(torch.float16)
    T, H = x16.shape
    ids = topk_ids.to(torch.int64)
    k = ids.shape[1]
    inter = w13.shape[1] // 2
    a1, sc1 = act_quant(x16)
    tok = torch.arange(T).repeat_interleave(k)
    flat = ids.reshape(-1)
    run1 = grouped_run(a1[tok], flat, w13, s13, z13, group)
    g1 = (run1 * sc1[tok][:, None]).to(torch.float16)
    g = g1[:, :inter].float()
    silu = (g / (1.0 + torch.exp(-g))).to(torch.float16)
    h = (silu.float() * g1[:, inter:].float()).to(torch.float16)
    a2, sc2 = act_quant(h)
    y = grouped_run(a2, flat, w2, s2, z2, group) * sc2[:, None]
    if round_y_fp16:
        y = y.to(torch.float16).float()
    y = y.reshape(T, k, H)
    tw = topk_weights.to(torch.float32).reshape(T, k)
    acc = torch.zeros((T, H), dtype=torch.float32)
    for j in range(k):
        acc = (tw[:, j:j + 1].to(torch.float64) * y[:, j].to(torch.float64)
               + acc.to(torch.float64)).to(torch.float32)
    return acc
