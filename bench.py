#!/usr/bin/env python3
"""Benchmark of the MI355X W4A8 MoE expert path (one MoE layer = one step).

A step is: router softmax/top-k on the logits, then the whole expert path
(align -> fp8 act-quant -> gemm1+SiLU -> act-quant -> gemm2 -> top-k weighted reduce)
on one batch of synthetic tokens whose weights are already resident in HBM. Weights
rotate over several independent sets so the 256 MB Infinity Cache cannot hold them.

Prints ONE JSON line: MoE-layer tokens/s (HIP-graph replays of the step), the dominant
kernel's roofline fraction (kernel-exact HIP events on the kernels' own stream) beside the
layer's own fraction, the host cost of eager calls, and the torch-CPU port of the reference
layer timed on a bounded sample of the same workload on the host cores. The default (c3,
decode) line also carries a ``prefill`` object: the c4 layer (T = 4096, Zipf routing)
measured the same way, with its MFMA fractions, an expert-stratified parity sample and the
CPU port's time on it. ``--gpus N`` with N > 1 exits: this build runs on one GPU.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "rdna4-vllm_amd"))

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
FP8_PEAK_TFLOPS = 5000.0       # MI355X dense fp8 MFMA

# BASELINE.json configs (index 1..5). c1 is the dense CPU-reference case.
CONFIGS = {
    "c1": dict(kind="dense", M=16, N=1024, K=2048, g=128),
    "c2": dict(kind="moe", T=1, H=2048, E=256, k=8, I=512, g=128, routing="uniform"),
    "c3": dict(kind="moe", T=32, H=2048, E=256, k=8, I=512, g=128, routing="uniform"),
    "c4": dict(kind="moe", T=4096, H=2048, E=256, k=8, I=512, g=128, routing="zipf"),
    "c5": dict(kind="moe", T=2048, H=4096, E=128, k=8, I=1536, g=128, routing="uniform"),
}
DEFAULT_CONFIG = "c3"     # the headline decode shape BASELINE.json's metric is quoted on


def expert_bytes(H, I, g):
    """int4 weights + fp16 scales + packed int4 zero-points of w13 and w2 per expert."""
    w13 = 2 * I * H // 2 + 2 * I * (H // g) * 2 + (2 * I // 8) * (H // g) * 4
    w2 = H * I // 2 + H * (I // g) * 2 + (H // 8) * (I // g) * 4
    return w13, w2


def make_weights(cfg, seed, device):
    """Uniform nibbles and zero-points (random int32 words), fp16 scales ~ U(0.005, 0.02)."""
    import torch
    E, H, I, g = cfg["E"], cfg["H"], cfg["I"], cfg["g"]
    gen = torch.Generator(device=device).manual_seed(seed)

    def words(*shape):
        return torch.randint(-2**31, 2**31 - 1, shape, generator=gen, device=device,
                             dtype=torch.int64).to(torch.int32)

    def scales(*shape):
        return (torch.rand(shape, generator=gen, device=device) * 0.015 + 0.005).to(torch.float16)

    return dict(w13=words(E, 2 * I, H // 8), s13=scales(E, 2 * I, H // g),
                z13=words(E, 2 * I // 8, H // g),
                w2=words(E, H, I // 8), s2=scales(E, H, I // g), z2=words(E, H // 8, I // g))


def make_inputs(cfg, seed, device):
    """bf16 hidden ~ N(0,1); router logits N(0,1) (uniform routing) or
    log p_zipf(rank) + Gumbel (Zipf(s) routing without replacement, shuffled ranks)."""
    import torch
    T, H, E = cfg["T"], cfg["H"], cfg["E"]
    gen = torch.Generator(device=device).manual_seed(seed)
    x = torch.randn((T, H), generator=gen, device=device).to(torch.bfloat16)
    if cfg["routing"] == "zipf":
        s = cfg.get("s", 1.1)
        p = 1.0 / torch.arange(1, E + 1, device=device, dtype=torch.float64) ** s
        p = p / p.sum()
        perm = torch.randperm(E, generator=gen, device=device)
        u = torch.rand((T, E), generator=gen, device=device, dtype=torch.float64).clamp_(1e-12, 1 - 1e-12)
        logits = (torch.log(p)[perm][None, :] - torch.log(-torch.log(u))).to(torch.float32)
    else:
        logits = torch.randn((T, E), generator=gen, device=device)
    return x, logits


class HipEvents:
    """Raw hipEvent_t handles from the HIP runtime torch already loaded."""

    def __init__(self, n):
        import torch  # noqa: F401  (ensures torch's libamdhip64 is the loaded runtime)
        self.hip = ctypes.CDLL("libamdhip64.so.7")
        self.hip.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        self.hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float),
                                                 ctypes.c_void_p, ctypes.c_void_p]
        self.hip.hipEventSynchronize.argtypes = [ctypes.c_void_p]
        self.hip.hipEventDestroy.argtypes = [ctypes.c_void_p]
        self.ev = []
        for _ in range(n):
            e = ctypes.c_void_p()
            assert self.hip.hipEventCreate(ctypes.byref(e)) == 0
            self.ev.append(e)

    def elapsed(self, a, b):
        ms = ctypes.c_float()
        assert self.hip.hipEventSynchronize(self.ev[b]) == 0
        assert self.hip.hipEventElapsedTime(ctypes.byref(ms), self.ev[a], self.ev[b]) == 0
        return ms.value

    def elapsed_if_recorded(self, a, b):
        """Interval between two events, or None when they were never recorded."""
        ms = ctypes.c_float()
        if self.hip.hipEventElapsedTime(ctypes.byref(ms), self.ev[a], self.ev[b]) != 0:
            self.hip.hipGetLastError()   # the failed query is not the next launch's error
            return None
        return ms.value

    def close(self):
        for e in self.ev:
            self.hip.hipEventDestroy(e)


STAGES = ["align", "act_quant_x", "reserved", "gemm1_silu", "act_quant_h", "gemm2",
          "reduce_cast"]


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def cpu_baseline(cfg, ws, x, tw, ids, out_gpu, budget_s, sample=None):
    """The torch-CPU port of the reference layer (oracle/cpu_port.py, vectorised per expert)
    on all host cores: the sample S (the first S tokens) doubles until one pass takes about a
    fifth of the budget, then three timed passes give the median. The same pass checks the
    GPU output on those tokens. With `sample` (token indices), that token set is the sample:
    one timed pass, then two more while they fit in the budget."""
    import numpy as np
    import torch
    import oracle as O
    from oracle import cpu_port
    # every core the process may use (its affinity set), within the host's thread budget
    # for one GPU (OMP_NUM_THREADS on the GPU boxes)
    cores = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    if os.environ.get("OMP_NUM_THREADS", "").isdigit():
        cores = min(cores, int(os.environ["OMP_NUM_THREADS"]))
    cores = max(1, cores)
    torch.set_num_threads(cores)
    host = {k: (None if v is None else v.cpu()) for k, v in ws.items()}
    for k in ("w13", "w2"):   # the port reads the op layout
        if host[k].dim() == 4:
            host[k] = torch.from_numpy(O.unrepack_fragments(host[k].numpy())[0])
    xc, twc, idc = x.float().cpu(), tw.cpu(), ids.cpu()
    T = xc.shape[0]
    round_y = T > 96

    def run(sel):
        t0 = time.perf_counter()
        ref = cpu_port.moe_layer(xc[sel], host["w13"], host["s13"], host["z13"], host["w2"],
                                 host["s2"], host["z2"], twc[sel], idc[sel], cfg["g"],
                                 round_y_fp16=round_y)
        return time.perf_counter() - t0, ref

    if sample is not None:
        sel = torch.from_numpy(np.asarray(sample, np.int64))
        S = int(sel.numel())
        dt, ref = run(sel)
        times = [dt]
        while len(times) < 3 and sum(times) + dt < budget_s:
            times.append(run(sel)[0])
        what = f"an expert-stratified set of {S} of {T} tokens (first and last slot of every " \
               f"touched expert, the hottest expert's last 64-row tile)"
    else:
        S, spent = min(T, 8), 0.0
        while True:
            dt, ref = run(slice(0, S))
            spent += dt
            if S >= T or dt * 5 > budget_s or spent + 2 * dt > budget_s / 2:
                break
            S = min(T, S * 2)
        sel = slice(0, S)
        times = [run(sel)[0] for _ in range(3)]        # the sizing passes warmed the caches
        what = f"first {S} of {T} tokens"
    med = sorted(times)[(len(times) - 1) // 2]
    got = out_gpu[sel].float().cpu().numpy()
    refn = ref.numpy()
    maxrel = float(np.abs(got - refn).max() / max(np.abs(refn).max(), 1e-30))
    return dict(value=S / med, unit="tokens/s", cores=int(cores), kind="port",
                sample=f"{what} through the torch-CPU port of the reference layer "
                       f"(oracle/cpu_port.py, float64 group sums, per-expert batches); "
                       f"median of {len(times)} passes {med:.3f} s "
                       f"({', '.join(f'{t:.3f}' for t in times)}); "
                       f"torch threads={torch.get_num_threads()}; cpu='{cpu_model()}' "
                       f"os.cpu_count={os.cpu_count()}"), maxrel, S


def gemm1_kernel_name(cfg, decode, layout, fused=False):
    frag = "true" if layout == "fragments" else "false"
    H = cfg["H"]
    if decode and layout == "fragments" and fused:
        # both decode GEMVs in one persistent launch (decode_gemv.hip launch_layer_e)
        split = {(16, 4): "4, 4, 4, 1", (32, 12): "8, 4, 3, 4", (4, 2): "4, 1, 2, 1",
                 (2, 1): "2, 1, 1, 1", (16, 16): "4, 4, 4, 4", (8, 4): "2, 4, 4, 1"}[
            (H // 128, cfg["I"] // 128)]
        return f"decode_layer_kernel<{split}, true>"
    if decode and layout == "fragments":
        # persistent decode kernel (decode_gemv.hip dec_split): groups per wave, split-K
        split = {1: "1, 1", 2: "2, 1", 3: "3, 1", 4: "4, 1", 8: "2, 4", 12: "3, 4", 16: "4, 4",
                 32: "8, 4"}[H // 128]
        # the bench's activations are bf16. After a router launch (T > 4) gemm1 reads the
        # rows the router quantised (ABF16 false, PREQ true); with T <= 4 tokens it routes
        # them itself and quantises the bf16 rows in registers (ABF16 true, PREQ false)
        if cfg["T"] > 4:
            return f"decode_gemv_kernel<(w4a8::Epi)1, {split}, false, true>"
        return f"decode_gemv_kernel<(w4a8::Epi)1, {split}, true, false>"
    if decode:
        split = {1: "1, 1", 2: "2, 1", 3: "3, 1", 4: "4, 1", 8: "4, 2", 12: "3, 4", 16: "4, 4",
                 32: "8, 4"}[H // 128]
        return f"grouped_gemv_kernel<kSiluHalf, {split}, false, {frag}>"
    # activation-resident tiles: 64 rows up to K = 2048, 32 rows up to K = 4096; gemm1 takes
    # prequantised rows (the last template argument, SQ, is false). fused: gemm1+SiLU and the
    # self-quantising gemm2 of each tile in one launch (prefill_ares.hip, the pair kernel)
    if fused:
        return f"prefill_ares_pair_kernel<{frag}>"
    if H % 512 == 0 and H <= 2048:
        return f"prefill_ares_kernel<kSiluHalf, {frag}, 64, false>"
    if H % 512 == 0 and H <= 4096:
        return f"prefill_ares_kernel<kSiluHalf, {frag}, 32, false>"
    return f"prefill_mfma_kernel<kSiluHalf, 4, {frag}>"


def stratified_tokens(ids, block_m=64):
    """Tokens covering the first and last slot of every touched expert and the hottest
    expert's last prefill tile (slots of an expert in ascending order, as the align orders
    them): every expert's weights and the last live row of every partial tile are checked."""
    import numpy as np
    T, k = ids.shape
    flat = ids.reshape(-1)
    toks, hot, hot_n = set(), -1, -1
    for e in np.unique(flat):
        slots = np.nonzero(flat == e)[0]
        toks.update((int(slots[0] // k), int(slots[-1] // k)))
        if slots.size > hot_n:
            hot, hot_n = e, slots.size
    slots = np.nonzero(flat == hot)[0]
    toks.update(int(s_ // k) for s_ in slots[(slots.size - 1) // block_m * block_m:])
    return np.array(sorted(toks))


def measure(name, args, steps, warmup, cpu_budget, tokens=0, eager=False, stratified=False):
    """One workload: graph-replayed layer steps (the value), kernel-exact GEMM times, the
    roofline pieces, optionally eager-call host overhead and the CPU port beside it."""
    import torch
    import w4a8_fp8_wmma as W
    from w4a8_fp8_wmma import _lib

    cfg = dict(CONFIGS[name])
    if tokens > 0:
        cfg["T"] = tokens
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    cfgno = int(name[1:])
    T, H, E, k, I, g = cfg["T"], cfg["H"], cfg["E"], cfg["k"], cfg["I"], cfg["g"]
    b13, b2 = expert_bytes(H, I, g)
    per_set = E * (b13 + b2)
    R = args.rotate or max(4, math.ceil(1.0e9 / per_set))
    sets = [make_weights(cfg, 1000 + cfgno * 17 + r, dev) for r in range(R)]
    if args.layout == "fragments":
        # load-time repack (the process_weights_after_loading step); op-layout copies freed
        for ws in sets:
            ws["w13"] = W.repack_fragments(ws["w13"], ws["s13"], ws["z13"])
            ws["w2"] = W.repack_fragments(ws["w2"], ws["s2"], ws["z2"])
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
    x, logits = make_inputs(cfg, 1000 + cfgno, dev)
    torch.cuda.synchronize()

    def step(i):
        # router (softmax / top-8 / renormalise) + the whole expert path, one C-ABI call
        ws = sets[i % R]
        return W.moe_forward(x, logits, k, ws["w13"], ws["w2"], ws["s13"], ws["s2"], ws["z13"],
                             ws["z2"])

    out0, tw0, ids0 = step(0)
    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()

    graphs = None
    L = 0
    if not args.no_graph:
        graphs = []
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            for r in range(R):
                step(r)
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        # One graph holds L consecutive layer steps (the weight sets in turn, L a multiple of
        # R near 40), as a serving engine captures a model's layers back to back in one graph
        # (a 30B-A3B-class model has ~48 MoE layers); a second graph holds the first K % L
        # steps when K is not a multiple of L. Replays then carry no per-layer graph launch
        # gap, and the timed region still runs exactly K steps.
        L = min(steps, R * max(1, round(40 / R)))
        def capture(n):
            gph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(gph):
                for r in range(n):
                    step(r)
            return gph
        graphs = [capture(L)]
        if steps % L:
            graphs.append(capture(steps % L))
        for gph in graphs:
            gph.replay()
        torch.cuda.synchronize()

    # ---- timed region: exactly K steps ----
    ev = HipEvents(2 + 12)
    stream = torch.cuda.current_stream().cuda_stream
    hip = ev.hip
    hip.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    torch.cuda.synchronize()
    t_wall = time.perf_counter()
    hip.hipEventRecord(ev.ev[0], stream)
    if graphs is not None:
        for _ in range(steps // L):
            graphs[0].replay()
        if steps % L:
            graphs[1].replay()
    else:
        for i in range(steps):
            step(i)
    hip.hipEventRecord(ev.ev[1], stream)
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t_wall) * 1e3
    total_ms = ev.elapsed(0, 1)
    ms_per_step = total_ms / steps

    # ---- eager calls: host cost of one moe_forward call (Python checks, workspace, ctypes),
    # the calls issued back to back with no synchronisation between them ----
    eager_info = None
    if eager:
        n_eager = max(20, min(200, steps))
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(n_eager):
            step(i)
        t_issue = time.perf_counter() - t0
        torch.cuda.synchronize()
        t_all = time.perf_counter() - t0
        eager_info = {
            "calls": n_eager,
            "host_issue_us_per_call": round(t_issue / n_eager * 1e6, 2),
            "wall_us_per_call": round(t_all / n_eager * 1e6, 2),
            "graph_us_per_step": round(ms_per_step * 1e3, 2),
            "host_overhead_us_per_call": round(t_all / n_eager * 1e6 - ms_per_step * 1e3, 2),
            "note": "eager moe_forward calls back to back (no sync between them); overhead = "
                    "eager wall per call minus the graph-replayed GPU time per step",
        }

    # ---- per-stage and per-kernel timing (eager layer calls; events recorded by the C ABI
    # on the kernels' own stream). events[8..11] are stamped by hipExtLaunchKernel at the
    # start and end of the gemm1 and gemm2 kernels themselves: their interval is the
    # kernel's duration, the figure a rocprofv3 kernel trace reports for it. ----
    stage_ev = (ctypes.c_void_p * 12)(*[e.value for e in ev.ev[2:14]])
    _lib.check(_lib.lib.w4a8_moe_apply_set_stage_events(stage_ev, 12), "stage events")
    n_stage = max(10, min(50, steps))
    acc = [0.0] * 7
    k1 = k2 = 0.0
    fused = False   # the layer's two GEMMs ran as one kernel (stamped as gemm1)
    for i in range(n_stage):
        step(i)
        torch.cuda.synchronize()
        for j in range(7):
            acc[j] += ev.elapsed(2 + j, 3 + j)
        k1 += ev.elapsed(10, 11)
        e2 = ev.elapsed_if_recorded(12, 13)
        fused = e2 is None
        k2 += 0.0 if fused else e2
    _lib.check(_lib.lib.w4a8_moe_apply_set_stage_events(None, 0), "stage events off")
    stage_ms = {STAGES[j]: acc[j] / n_stage for j in range(7)}
    g1_ms, g2_ms = k1 / n_stage, k2 / n_stage

    # ---- algorithmic work ----
    distinct = int(torch.unique(ids0).numel())
    layer_bytes = distinct * (b13 + b2) + T * H * 2 * 2
    layer_flops = 2 * T * k * (H * 2 * I + I * H)
    decode = T <= 96
    g1_bytes = distinct * b13 + T * H + T * k * I * 2        # weights + fp8 x in + fp16 h out
    g2_bytes = distinct * b2 + T * k * I * 2 + T * k * H * (4 if decode else 2)
    g1_flops = 2 * T * k * H * 2 * I
    g2_flops = 2 * T * k * I * H
    layer_s = ms_per_step * 1e-3
    kname = gemm1_kernel_name(cfg, decode, args.layout, fused)
    if decode:
        # the fused kernel runs both GEMVs: its bytes are both GEMMs' (h stays in HBM/L2
        # between them and is counted as written and read, as for two launches)
        k_bytes = g1_bytes + g2_bytes if fused else g1_bytes
        achieved = k_bytes / (g1_ms * 1e-3) / 1e9
        roof = dict(bound="hbm", achieved=round(achieved, 1), peak=HBM_PEAK_GBS, unit="GB/s",
                    frac=round(achieved / HBM_PEAK_GBS, 4), traffic=None, kernel=kname,
                    algorithmic_bytes=k_bytes, avg_ms=round(g1_ms, 5))
        lay_ach = layer_bytes / layer_s / 1e9
        roof["layer"] = dict(bound="hbm", achieved=round(lay_ach, 1), unit="GB/s",
                             frac=round(lay_ach / HBM_PEAK_GBS, 4),
                             algorithmic_bytes=layer_bytes, ms=round(ms_per_step, 5),
                             target_frac=0.70)
        if not fused:
            roof["gemm2"] = dict(achieved=round(g2_bytes / (g2_ms * 1e-3) / 1e9, 1), unit="GB/s",
                                 frac=round(g2_bytes / (g2_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                                 algorithmic_bytes=g2_bytes, avg_ms=round(g2_ms, 5))
    else:
        # the pair kernel runs both GEMMs of every tile: its FLOPs are both GEMMs'
        k_flops = g1_flops + g2_flops if fused else g1_flops
        achieved = k_flops / (g1_ms * 1e-3) / 1e12
        roof = dict(bound="mfma", achieved=round(achieved, 1), peak=FP8_PEAK_TFLOPS,
                    unit="TFLOP/s", frac=round(achieved / FP8_PEAK_TFLOPS, 4), traffic=None,
                    kernel=kname, algorithmic_flops=k_flops, avg_ms=round(g1_ms, 5))
        lay_ach = layer_flops / layer_s / 1e12
        roof["layer"] = dict(bound="mfma", achieved=round(lay_ach, 1), unit="TFLOP/s",
                             frac=round(lay_ach / FP8_PEAK_TFLOPS, 4), flops=layer_flops,
                             ms=round(ms_per_step, 5), target_frac=0.50,
                             hbm_frac=round(layer_bytes / layer_s / 1e9 / HBM_PEAK_GBS, 4))
        if not fused:
            roof["gemm2"] = dict(achieved=round(g2_flops / (g2_ms * 1e-3) / 1e12, 1),
                                 unit="TFLOP/s",
                                 frac=round(g2_flops / (g2_ms * 1e-3) / 1e12 / FP8_PEAK_TFLOPS, 4),
                                 algorithmic_flops=g2_flops, avg_ms=round(g2_ms, 5))
    roof["timing"] = (f"kernel-exact HIP events (hipExtLaunchKernel start/stop of the kernel "
                      f"itself) over {n_stage} eager layer calls on the launch stream")
    # HBM bytes per launch of that kernel, from rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE runs
    # of this workload and weight layout (profiles/roofline_traffic.json); null otherwise
    tr_file = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "roofline_traffic.json")
    if os.path.exists(tr_file) and tokens == 0:
        tr = json.load(open(tr_file)).get(f"{name}/{args.layout}")
        if tr is not None and tr.get("kernel") == kname:
            roof["traffic"] = tr["traffic_bytes"]
            roof["traffic_source"] = "profiles/roofline_traffic.json (" + tr["kernel"] + ")"

    res = dict(cfg=cfg, T=T, R=R, ms_per_step=ms_per_step, wall_ms=wall_ms, roof=roof,
               graphs=graphs is not None, graph_steps=L, distinct=distinct, layer_bytes=layer_bytes,
               layer_flops=layer_flops, stage_ms=stage_ms, g1_ms=g1_ms, g2_ms=g2_ms,
               fused=fused, eager=eager_info)
    if cpu_budget > 0:
        sample = stratified_tokens(ids0.cpu().numpy()) if stratified else None
        cb, maxrel, S = cpu_baseline(cfg, sets[0], x, tw0, ids0, out0, cpu_budget, sample)
        res["cpu_baseline"] = cb
        res["parity_sample"] = {"tokens": S, "max_rel_err": maxrel, "bar": 1e-2,
                                "selection": "expert-stratified" if stratified else "first S"}
    ev.close()
    del sets, graphs
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", default=DEFAULT_CONFIG, choices=[c for c in CONFIGS if c != "c1"])
    ap.add_argument("--rotate", type=int, default=0, help="weight sets (0 = auto, >= 1 GiB)")
    ap.add_argument("--no-graph", action="store_true", help="time eager launches")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=20.0)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--tokens", type=int, default=0,
                    help="override the config's token count (shape studies, not a headline line)")
    ap.add_argument("--layout", choices=["fragments", "op"], default="fragments",
                    help="weights as stored after loading: the gfx950 fragment layout "
                         "(repacked once per weight set, outside the timed region) or the "
                         "reference op layout")
    ap.add_argument("--no-prefill", action="store_true",
                    help="skip the c4 prefill object the default (c3) line carries")
    ap.add_argument("--prefill-steps", type=int, default=40)
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build runs the MoE expert path on ONE GPU; multi-GPU (EP/TP) "
              "sharding is a design note only. Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    budget = 0.0 if args.no_cpu_baseline else args.cpu_budget
    m = measure(args.config, args, args.steps, args.warmup, budget, tokens=args.tokens,
                eager=True, stratified=args.config in ("c4", "c5") and args.tokens == 0)
    cfg, T = m["cfg"], m["T"]
    layer_s = m["ms_per_step"] * 1e-3
    line = {
        "metric": "MoE-layer tokens/s; % HBM BW at decode, % FP8 MFMA peak at prefill",
        "value": round(T / layer_s, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(m["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8e4m3 x int4 (fp32 accumulate)",
        "data": "synthetic (seeded; random int4 weights/zero-points, fp16 scales, bf16 N(0,1) "
                "hidden, router logits)",
        "config": {"workload": f"{args.config}{' (tokens override)' if args.tokens > 0 else ''}: "
                               f"MoE layer T={T} H={cfg['H']} E={cfg['E']} top{cfg['k']} "
                               f"I={cfg['I']} AWQ-int4 g{cfg['g']} zp, {cfg['routing']} routing",
                   "T": T, "H": cfg["H"], "E": cfg["E"], "top_k": cfg["k"], "I": cfg["I"],
                   "group": cfg["g"], "routing": cfg["routing"],
                   "weight_sets_rotated": m["R"],
                   "timing": "hip-graph replay" if m["graphs"] else "eager",
                   "layer_steps_per_graph": m["graph_steps"],
                   "weight_layout": args.layout,
                   "parallelism": "1 GPU"},
        "roofline": m["roof"],
        "layer": {"distinct_experts": m["distinct"], "algorithmic_bytes": m["layer_bytes"],
                  "hbm_frac": round(m["layer_bytes"] / layer_s / 1e9 / HBM_PEAK_GBS, 4),
                  "flops": m["layer_flops"],
                  "mfma_frac": round(m["layer_flops"] / layer_s / 1e12 / FP8_PEAK_TFLOPS, 4),
                  "stage_ms_eager": {k_: round(v, 5) for k_, v in m["stage_ms"].items()},
                  "kernel_ms": ({"gemm1_gemm2_fused": round(m["g1_ms"], 5)} if m["fused"] else
                                {"gemm1": round(m["g1_ms"], 5), "gemm2": round(m["g2_ms"], 5)}),
                  "wall_ms_timed_region": round(m["wall_ms"], 3)},
        "eager": m["eager"],
        "cpu_baseline": m.get("cpu_baseline"),
    }
    if "parity_sample" in m:
        line["parity_sample"] = m["parity_sample"]
    # the prefill half of the metric: the c4 layer (T = 4096, Zipf routing) measured the same
    # way, beside the decode headline
    if args.config == "c3" and args.tokens == 0 and not args.no_prefill:
        p = measure("c4", args, args.prefill_steps, min(args.warmup, 10),
                    0.0 if args.no_cpu_baseline else min(args.cpu_budget, 15.0),
                    stratified=True)
        pl = p["ms_per_step"] * 1e-3
        pr = p["roof"]
        line["prefill"] = {
            "workload": f"c4: MoE layer T={p['T']} H={p['cfg']['H']} E={p['cfg']['E']} "
                        f"top{p['cfg']['k']} I={p['cfg']['I']} AWQ-int4 g128 zp, Zipf(1.1) routing",
            "steps": args.prefill_steps, "weight_sets_rotated": p["R"],
            "timing": "hip-graph replay" if p["graphs"] else "eager",
            "layer_ms": round(p["ms_per_step"], 5),
            "tokens_per_s": round(p["T"] / pl, 1),
            "layer_mfma_frac": pr["layer"]["frac"],
            "layer_hbm_frac": pr["layer"]["hbm_frac"],
            "target_mfma_frac": 0.50,
            **({"gemm1_gemm2": {"kernel": pr["kernel"], "ms": pr["avg_ms"],
                                "tflops": pr["achieved"], "mfma_frac": pr["frac"]}}
               if "gemm2" not in pr else
               {"gemm1": {"kernel": pr["kernel"], "ms": pr["avg_ms"], "tflops": pr["achieved"],
                          "mfma_frac": pr["frac"]},
                "gemm2": {"ms": pr["gemm2"]["avg_ms"], "tflops": pr["gemm2"]["achieved"],
                          "mfma_frac": pr["gemm2"]["frac"]}}),
            "stage_ms_eager": {k_: round(v, 5) for k_, v in p["stage_ms"].items()},
            "distinct_experts": p["distinct"], "flops": p["layer_flops"],
            "algorithmic_bytes": p["layer_bytes"],
            "cpu_port": p.get("cpu_baseline"),
            "parity_sample": p.get("parity_sample"),
        }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
