// Router top-k softmax and deterministic moe_align_block_size (gfx950).
//
// Align contract (test_moe_experts.py:136-152; vLLM call at moe_experts.py:587-589):
// slots t*top_k+j are grouped by expert ascending and, within an expert, by slot
// ascending; each expert's run is padded to a multiple of block_m with the sentinel
// numel; expert_ids[b] names the expert of block b; ntp = total padded rows. Entries past
// ntp keep the sentinel and expert id -1.
//
// Schedule: slots are cut into chunks of kChunk. Per chunk, a work-group builds a
// per-expert histogram and the stable in-chunk rank of every slot (bucket the slots with
// LDS atomics, then rank each slot by counting smaller slot ids in its bucket, so the
// result never depends on atomic order). A single work-group scans the chunk histograms
// into expert offsets. Small inputs (one chunk) run all three phases in one launch.
#include "w4a8_common.h"
#include "w4a8_internal.h"
#include "act_quant.h"

namespace w4a8 {
namespace {

constexpr int kChunk = 1024;       // slots per chunk (one per thread)
constexpr int kAlignThreads = 1024;
constexpr int kMaxExperts = 1024;  // experts handled by the align kernels

struct ChunkScratch {
    int hist[kMaxExperts];
    int boff[kMaxExperts];    // bucket start (exclusive scan of hist)
    int fill[kMaxExperts];
    int16_t bucket[kChunk];   // in-chunk slot indices grouped by expert
    int warp_tot[kAlignThreads / 64];
};

__device__ __forceinline__ int map_expert(const int32_t* __restrict__ ids, int64_t i,
                                          const int32_t* __restrict__ emap, int E) {
    int e = ids[i];
    if (emap != nullptr) e = (e >= 0 && e < E) ? emap[e] : -1;
    return (e >= 0 && e < E) ? e : -1;
}

// Block-wide exclusive scan of one int per thread (1024 threads, wave64).
__device__ int block_exclusive_scan(int v, int* warp_tot, int& total) {
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    int x = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_up(x, o, 64);
        if (lane >= o) x += y;
    }
    if (lane == 63) warp_tot[wid] = x;
    __syncthreads();
    if (wid == 0) {
        int t = (lane < kAlignThreads / 64) ? warp_tot[lane] : 0;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int y = __shfl_up(t, o, 64);
            if (lane >= o) t += y;
        }
        if (lane < kAlignThreads / 64) warp_tot[lane] = t;
    }
    __syncthreads();
    const int before = (wid > 0) ? warp_tot[wid - 1] : 0;
    total = warp_tot[kAlignThreads / 64 - 1];
    __syncthreads();
    return before + x - v;
}

// Phase A for one chunk: histogram, buckets and the stable rank of this thread's slot.
// Returns the expert (or -1) of slot `base + threadIdx.x`, writes its rank.
__device__ int chunk_rank(const int32_t* __restrict__ ids, int64_t numel, int64_t base,
                          const int32_t* __restrict__ emap, int E, ChunkScratch& s,
                          int& rank) {
    const int tid = threadIdx.x;
    for (int e = tid; e < E; e += kAlignThreads) { s.hist[e] = 0; s.fill[e] = 0; }
    __syncthreads();
    const int64_t i = base + tid;
    const int e = (i < numel) ? map_expert(ids, i, emap, E) : -1;
    if (e >= 0) atomicAdd(&s.hist[e], 1);
    __syncthreads();
    // bucket offsets: scan hist over experts (E <= 1024 -> one element per thread)
    int total;
    const int h = (tid < E) ? s.hist[tid] : 0;
    const int off = block_exclusive_scan(h, s.warp_tot, total);
    if (tid < E) s.boff[tid] = off;
    __syncthreads();
    if (e >= 0) {
        const int p = atomicAdd(&s.fill[e], 1);
        s.bucket[s.boff[e] + p] = (int16_t)tid;
    }
    __syncthreads();
    rank = 0;
    if (e >= 0) {
        const int b0 = s.boff[e], n = s.hist[e];
        for (int q = 0; q < n; ++q) rank += (s.bucket[b0 + q] < tid) ? 1 : 0;
    }
    return e;
}

// Writes expert_ids, the padding sentinels and ntp from per-expert totals `cnt` and
// padded offsets `eoff` (both in LDS). One thread per expert.
__device__ void write_layout(const int* cnt, const int* eoff, int E, int64_t block_m,
                             int64_t numel, int total_padded, int32_t* __restrict__ sorted_ids,
                             int64_t sorted_len, int32_t* __restrict__ expert_ids,
                             int32_t* __restrict__ ntp) {
    const int tid = threadIdx.x;
    for (int e = tid; e < E; e += kAlignThreads) {
        const int c = cnt[e];
        if (c == 0) continue;
        const int o = eoff[e];
        const int padded = (int)((c + block_m - 1) / block_m * block_m);
        for (int r = o + c; r < o + padded; ++r) sorted_ids[r] = (int32_t)numel;
        for (int b = (int)(o / block_m); b < (int)((o + padded) / block_m); ++b)
            expert_ids[b] = e;
    }
    for (int64_t r = total_padded + tid; r < sorted_len; r += kAlignThreads)
        sorted_ids[r] = (int32_t)numel;
    for (int64_t b = total_padded / block_m + tid; b < sorted_len / block_m; b += kAlignThreads)
        expert_ids[b] = -1;
    if (tid == 0) ntp[0] = total_padded;
}

// Single launch for numel <= kChunk.
// Whole align for numel <= kChunk inside one work-group of kAlignThreads threads.
__device__ __forceinline__ void align_small_body(
    const int32_t* __restrict__ ids, int64_t numel, int E, int64_t block_m,
    const int32_t* __restrict__ emap, int32_t* __restrict__ sorted_ids, int64_t sorted_len,
    int32_t* __restrict__ expert_ids, int32_t* __restrict__ ntp,
    int32_t* __restrict__ slot_to_row) {
    __shared__ ChunkScratch s;
    __shared__ int eoff[kMaxExperts];
    int rank;
    const int e = chunk_rank(ids, numel, 0, emap, E, s, rank);
    const int tid = threadIdx.x;
    int total;
    const int padded = (tid < E) ? (int)((s.hist[tid] + block_m - 1) / block_m * block_m) : 0;
    const int off = block_exclusive_scan(padded, s.warp_tot, total);
    if (tid < E) eoff[tid] = off;
    __syncthreads();
    if (e >= 0) sorted_ids[eoff[e] + rank] = tid;
    if (slot_to_row != nullptr && tid < numel) slot_to_row[tid] = e >= 0 ? eoff[e] + rank : -1;
    write_layout(s.hist, eoff, E, block_m, numel, total, sorted_ids, sorted_len, expert_ids,
                 ntp);
}

__global__ void __launch_bounds__(kAlignThreads) align_small_kernel(
    const int32_t* __restrict__ ids, int64_t numel, int E, int64_t block_m,
    const int32_t* __restrict__ emap, int32_t* __restrict__ sorted_ids, int64_t sorted_len,
    int32_t* __restrict__ expert_ids, int32_t* __restrict__ ntp,
    int32_t* __restrict__ slot_to_row) {
    align_small_body(ids, numel, E, block_m, emap, sorted_ids, sorted_len, expert_ids, ntp,
                     slot_to_row);
}

// Multi-chunk phase 1: per-chunk histograms -> counts[chunk][E].
__global__ void __launch_bounds__(kAlignThreads) align_count_kernel(
    const int32_t* __restrict__ ids, int64_t numel, int E, const int32_t* __restrict__ emap,
    int32_t* __restrict__ counts) {
    __shared__ int hist[kMaxExperts];
    const int tid = threadIdx.x;
    for (int e = tid; e < E; e += kAlignThreads) hist[e] = 0;
    __syncthreads();
    const int64_t i = (int64_t)blockIdx.x * kChunk + tid;
    const int e = (i < numel) ? map_expert(ids, i, emap, E) : -1;
    if (e >= 0) atomicAdd(&hist[e], 1);
    __syncthreads();
    for (int x = tid; x < E; x += kAlignThreads) counts[(int64_t)blockIdx.x * E + x] = hist[x];
}

// Multi-chunk phase 2 (one work-group): counts -> per-chunk expert bases (in place),
// padded expert offsets, layout.
__global__ void __launch_bounds__(kAlignThreads) align_scan_kernel(
    int32_t* __restrict__ counts, int nchunks, int E, int64_t block_m, int64_t numel,
    int32_t* __restrict__ eoff_out, int32_t* __restrict__ sorted_ids, int64_t sorted_len,
    int32_t* __restrict__ expert_ids, int32_t* __restrict__ ntp) {
    __shared__ int cnt[kMaxExperts];
    __shared__ int eoff[kMaxExperts];
    __shared__ int warp_tot[kAlignThreads / 64];
    const int tid = threadIdx.x;
    if (tid < E) {
        // exclusive prefix over the chunks, 16 chunk counts requested at a time
        constexpr int kBatch = 16;
        int run = 0;
        for (int c0 = 0; c0 < nchunks; c0 += kBatch) {
            int v[kBatch];
#pragma unroll
            for (int u = 0; u < kBatch; ++u)
                v[u] = c0 + u < nchunks ? counts[(int64_t)(c0 + u) * E + tid] : 0;
#pragma unroll
            for (int u = 0; u < kBatch; ++u) {
                if (c0 + u < nchunks) counts[(int64_t)(c0 + u) * E + tid] = run;
                run += v[u];
            }
        }
        cnt[tid] = run;
    }
    __syncthreads();
    int total;
    const int padded = (tid < E) ? (int)((cnt[tid] + block_m - 1) / block_m * block_m) : 0;
    const int off = block_exclusive_scan(padded, warp_tot, total);
    if (tid < E) { eoff[tid] = off; eoff_out[tid] = off; }
    __syncthreads();
    write_layout(cnt, eoff, E, block_m, numel, total, sorted_ids, sorted_len, expert_ids, ntp);
}

// Multi-chunk phases 2 + 3 in one launch when the chunk histograms fit LDS: every
// work-group reads all of them (one batch of loads), derives the per-expert totals, padded
// expert offsets and its own chunk's bases, and places its chunk; work-group 0 also writes
// the layout (sentinels, expert_ids, ntp).
constexpr int kScanPlaceMaxCounts = 16384;   // nchunks * E held in LDS
__global__ void __launch_bounds__(kAlignThreads) align_scan_place_kernel(
    const int32_t* __restrict__ ids, int64_t numel, int E, int64_t block_m,
    const int32_t* __restrict__ emap, const int32_t* __restrict__ counts, int nchunks,
    int32_t* __restrict__ sorted_ids, int64_t sorted_len, int32_t* __restrict__ expert_ids,
    int32_t* __restrict__ ntp, int32_t* __restrict__ slot_to_row) {
    __shared__ ChunkScratch s;
    __shared__ int lc[kScanPlaceMaxCounts];
    __shared__ int cnt[kMaxExperts];
    __shared__ int eoff[kMaxExperts];
    __shared__ int base[kMaxExperts];
    const int tid = threadIdx.x;
    const int b = blockIdx.x;
    const int ncount = nchunks * E;
    constexpr int kPer = kScanPlaceMaxCounts / kAlignThreads;
    int v[kPer];
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
        const int i = u * kAlignThreads + tid;
        v[u] = i < ncount ? counts[i] : 0;
    }
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
        const int i = u * kAlignThreads + tid;
        if (i < ncount) lc[i] = v[u];
    }
    int rank;
    const int e = chunk_rank(ids, numel, (int64_t)b * kChunk, emap, E, s, rank);   // syncs
    for (int x = tid; x < E; x += kAlignThreads) {
        int run = 0, mine = 0;
        for (int c = 0; c < nchunks; ++c) {
            if (c == b) mine = run;
            run += lc[c * E + x];
        }
        cnt[x] = run;
        base[x] = mine;
    }
    __syncthreads();
    int total;
    const int padded = (tid < E) ? (int)((cnt[tid] + block_m - 1) / block_m * block_m) : 0;
    const int off = block_exclusive_scan(padded, s.warp_tot, total);
    if (tid < E) eoff[tid] = off;
    __syncthreads();
    const int64_t slot = (int64_t)b * kChunk + tid;
    const int row = e >= 0 ? eoff[e] + base[e] + rank : -1;
    if (e >= 0) sorted_ids[row] = (int32_t)slot;
    if (slot_to_row != nullptr && slot < numel) slot_to_row[slot] = row;
    if (b == 0)
        write_layout(cnt, eoff, E, block_m, numel, total, sorted_ids, sorted_len, expert_ids, ntp);
}

// Multi-chunk phase 3: stable placement.
__global__ void __launch_bounds__(kAlignThreads) align_place_kernel(
    const int32_t* __restrict__ ids, int64_t numel, int E, const int32_t* __restrict__ emap,
    const int32_t* __restrict__ chunk_base, const int32_t* __restrict__ eoff,
    int32_t* __restrict__ sorted_ids, int32_t* __restrict__ slot_to_row) {
    __shared__ ChunkScratch s;
    int rank;
    const int64_t base = (int64_t)blockIdx.x * kChunk;
    const int e = chunk_rank(ids, numel, base, emap, E, s, rank);
    const int64_t slot = base + threadIdx.x;
    const int row = e >= 0 ? eoff[e] + chunk_base[(int64_t)blockIdx.x * E + e] + rank : -1;
    if (e >= 0) sorted_ids[row] = (int32_t)slot;
    if (slot_to_row != nullptr && slot < numel) slot_to_row[slot] = row;
}

// ---- router: one wave per token ----
constexpr int kRouterMaxPerLane = 16;   // E <= 1024

// NV = logits per lane (E <= 64 * NV). Loads are unconditional (clamped index, the
// out-of-range entries masked to -inf afterwards) so they issue together.
// Selection key: a larger key is a larger logit, equal logits order by the lower expert id
// (the router's tie-break). Entries past E get key 0, below every real entry.
__device__ __forceinline__ uint64_t topk_key(float v, int e) {
    uint32_t b = __float_as_uint(v);
    b = (b & 0x80000000u) ? ~b : (b | 0x80000000u);   // order-preserving float -> uint
    return ((uint64_t)b << 32) | (uint32_t)(0xFFFFFFFFu - (uint32_t)e);
}
__device__ __forceinline__ float topk_key_value(uint64_t key) {
    uint32_t b = (uint32_t)(key >> 32);
    b = (b & 0x80000000u) ? (b & 0x7FFFFFFFu) : ~b;
    return __uint_as_float(b);
}
__device__ __forceinline__ int topk_key_expert(uint64_t key) {
    return (int)(0xFFFFFFFFu - (uint32_t)key);
}
template <int S>
__device__ __forceinline__ uint64_t key_max_dpp(uint64_t k) {
    const uint32_t lo = dpp_step<S>((uint32_t)k), hi = dpp_step<S>((uint32_t)(k >> 32));
    const uint64_t o = ((uint64_t)hi << 32) | lo;
    return o > k ? o : k;
}
// maximum key over the wave, every lane gets it (branch-free compare-selects)
__device__ __forceinline__ uint64_t wave_max_key(uint64_t k) {
    k = key_max_dpp<0>(k);
    k = key_max_dpp<1>(k);
    k = key_max_dpp<2>(k);
    k = key_max_dpp<3>(k);
    {
        const auto lo = __builtin_amdgcn_permlane16_swap((uint32_t)k, (uint32_t)k, false, false);
        const auto hi = __builtin_amdgcn_permlane16_swap((uint32_t)(k >> 32), (uint32_t)(k >> 32), false, false);
        const uint64_t a = ((uint64_t)hi[0] << 32) | lo[0], b = ((uint64_t)hi[1] << 32) | lo[1];
        k = a > b ? a : b;
    }
    {
        const auto lo = __builtin_amdgcn_permlane32_swap((uint32_t)k, (uint32_t)k, false, false);
        const auto hi = __builtin_amdgcn_permlane32_swap((uint32_t)(k >> 32), (uint32_t)(k >> 32), false, false);
        const uint64_t a = ((uint64_t)hi[0] << 32) | lo[0], b = ((uint64_t)hi[1] << 32) | lo[1];
        k = a > b ? a : b;
    }
    return k;
}

// Softmax + top-k of one token's logits row l (E <= 64 * NV) by one wave: lane j < top_k
// writes pick j (weight, expert) to tw[j] / ids[j] and, if ids_lds is given, the expert to
// ids_lds[j] too. Picks are made on the logits (exact ids); the weights are
// exp(l - max) / sum exp(l - max), renormalised over the picks in pick order.
template <int NV>
__device__ __forceinline__ void topk_load(const float* __restrict__ l, int E, int lane, float (&v)[NV]) {
#pragma unroll
    for (int i = 0; i < NV; ++i) v[i] = l[min(lane + 64 * i, E - 1)];
}

// Selection of one token from its logits v (lane l holds entries l + 64 i).
template <int NV>
__device__ __forceinline__ void topk_select(float (&v)[NV], int E, int top_k, bool renorm,
                                            float* __restrict__ tw, int32_t* __restrict__ ids,
                                            int32_t* ids_lds, int lane) {
    float m = -INFINITY;
    uint64_t key[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const bool in = lane + 64 * i < E;
        if (!in) v[i] = -INFINITY;
        m = fmaxf(m, v[i]);
        key[i] = in ? topk_key(v[i], lane + 64 * i) : 0ull;
    }
    m = wave_max(m);
    float ssum = 0.f;
#pragma unroll
    for (int i = 0; i < NV; ++i) ssum += lane + 64 * i < E ? expf(v[i] - m) : 0.f;
    ssum = wave_sum(ssum);
    uint64_t mine = 0;   // lane j < top_k: key of pick j
    for (int j = 0; j < top_k; ++j) {
        uint64_t best = 0;
#pragma unroll
        for (int i = 0; i < NV; ++i) best = key[i] > best ? key[i] : best;
        best = wave_max_key(best);
#pragma unroll
        for (int i = 0; i < NV; ++i) key[i] = key[i] == best ? 0ull : key[i];   // taken
        mine = lane == j ? best : mine;
    }
    const float p = expf(topk_key_value(mine) - m) / ssum;
    float sum_sel = 0.f;   // picks in order, as a sequential sum
    for (int j = 0; j < top_k; ++j)
        sum_sel += __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(p), j));
    if (lane < top_k) {
        const int e = topk_key_expert(mine);
        tw[lane] = renorm ? p / sum_sel : p;
        ids[lane] = e;
        if (ids_lds != nullptr) ids_lds[lane] = e;
    }
}

template <int NV>
__device__ __forceinline__ void topk_one_token(const float* __restrict__ l, int E, int top_k,
                                               bool renorm, float* __restrict__ tw,
                                               int32_t* __restrict__ ids, int32_t* ids_lds,
                                               int lane) {
    float v[NV];
    topk_load<NV>(l, E, lane, v);
    topk_select<NV>(v, E, top_k, renorm, tw, ids, ids_lds, lane);
}

// RowQuant: optional act-quant of the token's activation row by the same wave, after its
// routing (act_quant_kernel's arithmetic; saves a launch for the many-token schedule).
struct RowQuant {
    const void* x = nullptr;   // (T, K) fp16 / bf16, or null: no quantisation
    bool bf16 = false;
    int K = 0;
    uint8_t* xq = nullptr;     // (T, K) k8-interleaved e4m3
    float* xs = nullptr;       // (T,)
    float* gsum = nullptr;     // (T, K / 128) or null
};

template <int NV>
__global__ void __launch_bounds__(256) topk_softmax_kernel(
    const float* __restrict__ logits, int64_t T, int E, int top_k, bool renorm,
    float* __restrict__ tw, int32_t* __restrict__ tids, RowQuant rq) {
    const int lane = threadIdx.x & 63;
    const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= T) return;
    float v[NV];
    topk_load<NV>(logits + t * E, E, lane, v);
    if (rq.x == nullptr) {
        topk_select<NV>(v, E, top_k, renorm, tw + t * top_k, tids + t * top_k, nullptr, lane);
        return;
    }
    // the row's loads go out behind the logits, so the selection runs while they arrive
    RowRegs rr;
    const bool in_regs = row_load(rq.x, t, rq.K, lane, rr);
    topk_select<NV>(v, E, top_k, renorm, tw + t * top_k, tids + t * top_k, nullptr, lane);
    if (!in_regs) {
        if (rq.bf16) quantize_row<true>(rq.x, t, rq.K, rq.xq, rq.xs, true, rq.gsum, lane);
        else quantize_row<false>(rq.x, t, rq.K, rq.xq, rq.xs, true, rq.gsum, lane);
    } else if (rq.bf16) {
        quantize_row_regs<true>(rr, t, rq.K, rq.xq, rq.xs, true, rq.gsum, lane);
    } else {
        quantize_row_regs<false>(rr, t, rq.K, rq.xq, rq.xs, true, rq.gsum, lane);
    }
}

// Decode prologue in one launch: work-group 0 builds the align layout (numel <= kChunk),
// work-groups 1.. quantise 16 activation rows each (one wave per row).
template <bool BF16>
__global__ void __launch_bounds__(kAlignThreads) align_quant_kernel(
    const int32_t* __restrict__ ids, int64_t numel, int E, int64_t block_m,
    const int32_t* __restrict__ emap, int32_t* __restrict__ sorted_ids, int64_t sorted_len,
    int32_t* __restrict__ expert_ids, int32_t* __restrict__ ntp,
    int32_t* __restrict__ slot_to_row, const void* __restrict__ x, int64_t rows, int K,
    uint8_t* __restrict__ xq, float* __restrict__ xs, float* __restrict__ gsum) {
    if (blockIdx.x > 0) {
        const int64_t row = (int64_t)(blockIdx.x - 1) * (kAlignThreads / 64) + (threadIdx.x >> 6);
        if (row < rows) quantize_row<BF16>(x, row, K, xq, xs, true, gsum, threadIdx.x & 63);
        return;
    }
    align_small_body(ids, numel, E, block_m, emap, sorted_ids, sorted_len, expert_ids, ntp,
                     slot_to_row);
}


}  // namespace

size_t align_workspace_bytes(int64_t numel, int64_t num_experts) {
    if (numel <= kChunk) return 0;
    const int64_t nchunks = (numel + kChunk - 1) / kChunk;
    WorkspaceSize s;
    s.take<int32_t>((size_t)(nchunks * num_experts));
    s.take<int32_t>((size_t)num_experts);
    return s.used;
}

int launch_align(const int32_t* ids, int64_t numel, int64_t E, int64_t block_m,
                 const int32_t* emap, int32_t* sorted_ids, int64_t sorted_len,
                 int32_t* expert_ids, int32_t* ntp, void* ws, size_t ws_bytes,
                 hipStream_t stream, int32_t* slot_to_row) {
    if (E > kMaxExperts) {
        set_error("moe_align: num_experts must be <= 1024");
        return W4A8_ERR_INVALID;
    }
    if (numel <= kChunk) {
        align_small_kernel<<<1, kAlignThreads, 0, stream>>>(ids, numel, (int)E, block_m, emap,
                                                           sorted_ids, sorted_len, expert_ids,
                                                           ntp, slot_to_row);
        return check_launch("align_small_kernel");
    }
    const int64_t nchunks = (numel + kChunk - 1) / kChunk;
    Workspace w(ws, ws_bytes);
    int32_t* counts = w.take<int32_t>((size_t)(nchunks * E));
    int32_t* eoff = w.take<int32_t>((size_t)E);
    if (ws == nullptr || !w.ok()) {
        set_error("moe_align: workspace too small");
        return W4A8_ERR_WORKSPACE;
    }
    align_count_kernel<<<(unsigned)nchunks, kAlignThreads, 0, stream>>>(ids, numel, (int)E, emap,
                                                                        counts);
    if (int rc = check_launch("align_count_kernel")) return rc;
    if (nchunks * E <= kScanPlaceMaxCounts) {
        align_scan_place_kernel<<<(unsigned)nchunks, kAlignThreads, 0, stream>>>(
            ids, numel, (int)E, block_m, emap, counts, (int)nchunks, sorted_ids, sorted_len,
            expert_ids, ntp, slot_to_row);
        return check_launch("align_scan_place_kernel");
    }
    align_scan_kernel<<<1, kAlignThreads, 0, stream>>>(counts, (int)nchunks, (int)E, block_m,
                                                       numel, eoff, sorted_ids, sorted_len,
                                                       expert_ids, ntp);
    if (int rc = check_launch("align_scan_kernel")) return rc;
    align_place_kernel<<<(unsigned)nchunks, kAlignThreads, 0, stream>>>(ids, numel, (int)E, emap,
                                                                        counts, eoff,
                                                                        sorted_ids, slot_to_row);
    return check_launch("align_place_kernel");
}

int launch_topk_softmax(const float* logits, int64_t T, int64_t E, int64_t top_k, bool renorm,
                        float* w, int32_t* ids, hipStream_t stream, const void* x, bool x_bf16,
                        int64_t K, uint8_t* xq, float* xs, float* gsum) {
    if (E > 64 * kRouterMaxPerLane || top_k > 64 || top_k > E) {
        set_error("topk_softmax: need E <= 1024 and top_k <= min(64, E)");
        return W4A8_ERR_INVALID;
    }
    if (T == 0) return W4A8_OK;
    RowQuant rq;
    if (x != nullptr) {
        if (K <= 0 || K % 8 != 0 || xq == nullptr || xs == nullptr || (gsum && K % 128 != 0)) {
            set_error("topk_softmax: row quantisation needs K % 8 == 0 (K % 128 with group sums)");
            return W4A8_ERR_INVALID;
        }
        rq.x = x; rq.bf16 = x_bf16; rq.K = (int)K; rq.xq = xq; rq.xs = xs; rq.gsum = gsum;
    }
    const dim3 grid((unsigned)((T + 3) / 4));
    if (E <= 64) topk_softmax_kernel<1><<<grid, 256, 0, stream>>>(logits, T, (int)E, (int)top_k, renorm, w, ids, rq);
    else if (E <= 128) topk_softmax_kernel<2><<<grid, 256, 0, stream>>>(logits, T, (int)E, (int)top_k, renorm, w, ids, rq);
    else if (E <= 256) topk_softmax_kernel<4><<<grid, 256, 0, stream>>>(logits, T, (int)E, (int)top_k, renorm, w, ids, rq);
    else if (E <= 512) topk_softmax_kernel<8><<<grid, 256, 0, stream>>>(logits, T, (int)E, (int)top_k, renorm, w, ids, rq);
    else topk_softmax_kernel<16><<<grid, 256, 0, stream>>>(logits, T, (int)E, (int)top_k, renorm, w, ids, rq);
    return check_launch("topk_softmax_kernel");
}


int launch_align_quant(const int32_t* ids, int64_t numel, int64_t E, int64_t block_m,
                       const int32_t* emap, int32_t* sorted_ids, int64_t sorted_len,
                       int32_t* expert_ids, int32_t* ntp, int32_t* slot_to_row,
                       const void* x, bool x_bf16, int64_t rows, int64_t K, uint8_t* xq,
                       float* xs, float* gsum, hipStream_t stream) {
    if (E > kMaxExperts || numel > kChunk) {
        set_error("align_quant: needs num_experts <= 1024 and numel <= 1024");
        return W4A8_ERR_INVALID;
    }
    const unsigned grid = 1u + (unsigned)((rows + kAlignThreads / 64 - 1) / (kAlignThreads / 64));
    if (x_bf16)
        align_quant_kernel<true><<<grid, kAlignThreads, 0, stream>>>(
            ids, numel, (int)E, block_m, emap, sorted_ids, sorted_len, expert_ids, ntp,
            slot_to_row, x, rows, (int)K, xq, xs, gsum);
    else
        align_quant_kernel<false><<<grid, kAlignThreads, 0, stream>>>(
            ids, numel, (int)E, block_m, emap, sorted_ids, sorted_len, expert_ids, ntp,
            slot_to_row, x, rows, (int)K, xq, xs, gsum);
    return check_launch("align_quant_kernel");
}

}  // namespace w4a8
