// Router top-k softmax and deterministic moe_align_block_size (gfx950).
//
// Align contract (test_moe_experts.py:136-152; vLLM call at moe_experts.py:587-589):
// slots t*top_k+j are grouped by expert ascending and, within an expert, by slot
// ascending; each expert's run is padded to a multiple of block_m with the sentinel
// numel; expert_ids[b] names the expert of block b; ntp = total padded rows. Entries past
// ntp keep the sentinel and expert id -1.
//
// Schedule: slots are cut into chunks of kChunk. Per chunk, a work-group builds a
// per-expert histogram and the stable in-chunk rank of every slot: each wave finds, with
// one ballot per expert-id bit, the lanes that share a lane's expert (its rank in the wave
// is the count of those below it), and an exclusive prefix of the per-wave counts over the
// chunk's waves adds the slots of earlier waves. No atomics, so the result is the same
// every run, and a popular expert costs no more than a rare one. The chunk histograms are
// then scanned into expert offsets and every slot is placed. Small inputs (one chunk) run
// all phases in one launch.
#include "w4a8_common.h"
#include "w4a8_internal.h"
#include "act_quant.h"
#include "router.h"

namespace w4a8 {
namespace {

constexpr int kChunk = 1024;       // slots per chunk (one per thread)
constexpr int kAlignThreads = 1024;
constexpr int kMaxExperts = 1024;  // experts handled by the align kernels

struct ChunkScratch {
    int hist[kMaxExperts];                             // slots of the chunk per expert
    int16_t wpre[kAlignThreads / 64][kMaxExperts];     // per wave: slots, then exclusive prefix
    int warp_tot[kAlignThreads / 64];
};

// Expert of slot i: with an expert map (emap_len entries, indexed by the routed global id)
// the id is mapped to a local expert first; -1 when the slot has no local expert in [0, E).
__device__ __forceinline__ int map_expert(const int32_t* __restrict__ ids, int64_t i,
                                          const int32_t* __restrict__ emap, int emap_len, int E) {
    int e = ids[i];
    if (emap != nullptr) e = (e >= 0 && e < emap_len) ? emap[e] : -1;
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

// Lanes of the wave whose expert equals this lane's (valid lanes only; e < 2^nbits).
__device__ __forceinline__ uint64_t same_expert_lanes(int e, int nbits) {
    uint64_t m = __ballot(e >= 0);
    for (int b = 0; b < nbits; ++b) {
        const bool bit = (e >> b) & 1;
        const uint64_t bb = __ballot(bit);
        m &= bit ? bb : ~bb;
    }
    return m;
}

// Phase A for one chunk: histogram (s.hist) and the stable rank of this thread's slot among
// the chunk's slots of its expert. Returns the expert (or -1) of slot `base + threadIdx.x`.
__device__ int chunk_rank(const int32_t* __restrict__ ids, int64_t numel, int64_t base,
                          const int32_t* __restrict__ emap, int emap_len, int E, ChunkScratch& s,
                          int& rank) {
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int64_t i = base + tid;
    const int e = (i < numel) ? map_expert(ids, i, emap, emap_len, E) : -1;
    int* z = reinterpret_cast<int*>(&s.wpre[0][0]);
    for (int k = tid; k < (kAlignThreads / 64) * kMaxExperts / 2; k += kAlignThreads) z[k] = 0;
    __syncthreads();
    const int nbits = 32 - __clz(E > 1 ? E - 1 : 1);
    const uint64_t same = same_expert_lanes(e, nbits);
    const int rw = __popcll(same & ((1ull << lane) - 1ull));
    if (e >= 0 && rw == 0) s.wpre[w][e] = (int16_t)__popcll(same);
    __syncthreads();
    for (int x = tid; x < E; x += kAlignThreads) {
        int run = 0;
#pragma unroll
        for (int ww = 0; ww < kAlignThreads / 64; ++ww) {
            const int c = s.wpre[ww][x];
            s.wpre[ww][x] = (int16_t)run;
            run += c;
        }
        s.hist[x] = run;
    }
    __syncthreads();
    rank = e >= 0 ? s.wpre[w][e] + rw : 0;
    return e;
}

// Writes expert_ids, the padding sentinels and ntp from per-expert totals `cnt` and
// padded offsets `eoff` (both in LDS), one padded row and one block per thread: the expert of
// padded row r is the largest e with eoff[e] <= r (a binary search over the offsets; an
// expert without slots has the offset of the next one, so it is never the largest), and
// r is a padding row when r - eoff[e] >= cnt[e]. With nwg > 1 work-groups sharing the job,
// work-group wg takes every nwg-th stretch of kAlignThreads rows and blocks.
__device__ void write_layout(const int* cnt, const int* eoff, int E, int64_t block_m,
                             int64_t numel, int total_padded, int32_t* __restrict__ sorted_ids,
                             int64_t sorted_len, int32_t* __restrict__ expert_ids,
                             int32_t* __restrict__ ntp, int wg = 0, int nwg = 1) {
    const int tid = threadIdx.x;
    auto expert_of = [&](int r) {
        int lo = 0, hi = E - 1;             // eoff[0] = 0 <= r
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (eoff[mid] <= r) lo = mid;
            else hi = mid - 1;
        }
        return lo;
    };
    const int64_t step = (int64_t)nwg * kAlignThreads;
    for (int64_t r = (int64_t)wg * kAlignThreads + tid; r < sorted_len; r += step) {
        if (r >= total_padded) {
            sorted_ids[r] = (int32_t)numel;
            continue;
        }
        const int e = expert_of((int)r);
        if (r - eoff[e] >= cnt[e]) sorted_ids[r] = (int32_t)numel;
    }
    const int64_t nblocks = sorted_len / block_m;
    for (int64_t b = (int64_t)wg * kAlignThreads + tid; b < nblocks; b += step)
        expert_ids[b] = b * block_m < total_padded ? expert_of((int)(b * block_m)) : -1;
    if (wg == 0 && tid == 0) ntp[0] = total_padded;
}

// Single launch for numel <= kChunk.
// Whole align for numel <= kChunk inside one work-group of kAlignThreads threads.
__device__ __forceinline__ void align_small_body(
    const int32_t* __restrict__ ids, int64_t numel, int E, int64_t block_m,
    const int32_t* __restrict__ emap, int emap_len, int32_t* __restrict__ sorted_ids,
    int64_t sorted_len, int32_t* __restrict__ expert_ids, int32_t* __restrict__ ntp,
    int32_t* __restrict__ slot_to_row) {
    __shared__ ChunkScratch s;
    __shared__ int eoff[kMaxExperts];
    int rank;
    const int e = chunk_rank(ids, numel, 0, emap, emap_len, E, s, rank);
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
    const int32_t* __restrict__ emap, int emap_len, int32_t* __restrict__ sorted_ids,
    int64_t sorted_len, int32_t* __restrict__ expert_ids, int32_t* __restrict__ ntp,
    int32_t* __restrict__ slot_to_row) {
    align_small_body(ids, numel, E, block_m, emap, emap_len, sorted_ids, sorted_len, expert_ids,
                     ntp, slot_to_row);
}

// Multi-chunk phase 1: per-chunk histograms -> counts[chunk][E], and every slot's expert
// and in-chunk rank as one word: rank << 10 | expert (-1: no expert).
__device__ __forceinline__ int slot_key_pack(int e, int rank) { return e >= 0 ? (rank << 10) | e : -1; }
__global__ void __launch_bounds__(kAlignThreads) align_count_kernel(
    const int32_t* __restrict__ ids, int64_t numel, int E, const int32_t* __restrict__ emap,
    int emap_len, int32_t* __restrict__ counts, int32_t* __restrict__ slot_key) {
    __shared__ ChunkScratch s;
    int rank;
    const int64_t base = (int64_t)blockIdx.x * kChunk;
    const int e = chunk_rank(ids, numel, base, emap, emap_len, E, s, rank);
    if (base + threadIdx.x < numel) slot_key[base + threadIdx.x] = slot_key_pack(e, rank);
    for (int x = threadIdx.x; x < E; x += kAlignThreads) counts[(int64_t)blockIdx.x * E + x] = s.hist[x];
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
// work-group reads all of them together with its chunk's slot keys (one batch of loads),
// derives the per-expert totals, padded expert offsets and its own chunk's bases, and
// places its chunk; work-group 0 also writes the layout (sentinels, expert_ids, ntp).
constexpr int kScanPlaceMaxCounts = 16384;   // nchunks * E held in LDS
__global__ void __launch_bounds__(kAlignThreads) align_scan_place_kernel(
    const int32_t* __restrict__ slot_key, int64_t numel, int E, int64_t block_m,
    const int32_t* __restrict__ counts, int nchunks, int32_t* __restrict__ sorted_ids,
    int64_t sorted_len, int32_t* __restrict__ expert_ids, int32_t* __restrict__ ntp,
    int32_t* __restrict__ slot_to_row) {
    __shared__ int lc[kScanPlaceMaxCounts];
    __shared__ int cnt[kMaxExperts];
    __shared__ int eoff[kMaxExperts];
    __shared__ int base[kMaxExperts];
    __shared__ int warp_tot[kAlignThreads / 64];
    const int tid = threadIdx.x;
    const int b = blockIdx.x;
    const int ncount = nchunks * E;
    const int64_t slot = (int64_t)b * kChunk + tid;
    const int key = slot < numel ? slot_key[slot] : -1;
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
    __syncthreads();
    for (int x = tid; x < E; x += kAlignThreads) {
        int run = 0, mine = 0;
        for (int c0 = 0; c0 < nchunks; c0 += 8) {   // eight independent reads per pass
            int cv[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) cv[u] = c0 + u < nchunks ? lc[(c0 + u) * E + x] : 0;
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                if (c0 + u == b) mine = run;
                run += cv[u];
            }
        }
        cnt[x] = run;
        base[x] = mine;
    }
    __syncthreads();
    int total;
    const int padded = (tid < E) ? (int)((cnt[tid] + block_m - 1) / block_m * block_m) : 0;
    const int off = block_exclusive_scan(padded, warp_tot, total);
    if (tid < E) eoff[tid] = off;
    __syncthreads();
    const int e = key >= 0 ? (key & 1023) : -1;
    const int row = e >= 0 ? eoff[e] + base[e] + (key >> 10) : -1;
    if (e >= 0) sorted_ids[row] = (int32_t)slot;
    if (slot_to_row != nullptr && slot < numel) slot_to_row[slot] = row;
    write_layout(cnt, eoff, E, block_m, numel, total, sorted_ids, sorted_len, expert_ids, ntp, b,
                 nchunks);
}

// Multi-chunk phase 3: stable placement.
__global__ void __launch_bounds__(kAlignThreads) align_place_kernel(
    const int32_t* __restrict__ slot_key, int64_t numel, int E,
    const int32_t* __restrict__ chunk_base, const int32_t* __restrict__ eoff,
    int32_t* __restrict__ sorted_ids, int32_t* __restrict__ slot_to_row) {
    const int64_t slot = (int64_t)blockIdx.x * kChunk + threadIdx.x;
    const int key = slot < numel ? slot_key[slot] : -1;
    const int e = key >= 0 ? (key & 1023) : -1;
    const int row = e >= 0 ? eoff[e] + chunk_base[(int64_t)blockIdx.x * E + e] + (key >> 10) : -1;
    if (e >= 0) sorted_ids[row] = (int32_t)slot;
    if (slot_to_row != nullptr && slot < numel) slot_to_row[slot] = row;
}

// ---- router: one wave per token (selection in router.h) ----

template <int NV>
__device__ __forceinline__ void topk_one_token(const float* __restrict__ l, int E, int top_k,
                                               bool renorm, float* __restrict__ tw,
                                               int32_t* __restrict__ ids, int32_t* ids_lds,
                                               int lane) {
    float v[NV];
    topk_load<NV>(l, E, lane, v);
    topk_select<NV>(v, E, top_k, renorm, tw, ids, ids_lds, lane);
}

// RowQuant: optional act-quant of the tokens' activation rows in the same launch
// (act_quant_kernel's arithmetic; saves a launch), by work-groups of their own beside the
// selecting ones, so a few-token launch ends after the longer of the two chains, not their sum.
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
    const int64_t nsel = (T + 3) / 4;   // work-groups [0, nsel) select, the rest quantise
    if ((int64_t)blockIdx.x >= nsel) {
        const int64_t t = ((int64_t)blockIdx.x - nsel) * 4 + (threadIdx.x >> 6);
        if (t >= T || rq.x == nullptr) return;
        if (rq.bf16) quantize_row<true>(rq.x, t, rq.K, rq.xq, rq.xs, true, rq.gsum, lane);
        else quantize_row<false>(rq.x, t, rq.K, rq.xq, rq.xs, true, rq.gsum, lane);
        return;
    }
    const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= T) return;
    float v[NV];
    topk_load<NV>(logits + t * E, E, lane, v);
    topk_select<NV>(v, E, top_k, renorm, tw + t * top_k, tids + t * top_k, nullptr, lane);
}

// Decode prologue in one launch: work-group 0 builds the align layout (numel <= kChunk),
// work-groups 1.. quantise 16 activation rows each (one wave per row).
template <bool BF16>
__global__ void __launch_bounds__(kAlignThreads) align_quant_kernel(
    const int32_t* __restrict__ ids, int64_t numel, int E, int64_t block_m,
    const int32_t* __restrict__ emap, int emap_len, int32_t* __restrict__ sorted_ids,
    int64_t sorted_len, int32_t* __restrict__ expert_ids, int32_t* __restrict__ ntp,
    int32_t* __restrict__ slot_to_row, const void* __restrict__ x, int64_t rows, int K,
    uint8_t* __restrict__ xq, float* __restrict__ xs, float* __restrict__ gsum) {
    if (blockIdx.x > 0) {
        const int64_t row = (int64_t)(blockIdx.x - 1) * (kAlignThreads / 64) + (threadIdx.x >> 6);
        if (row < rows) quantize_row<BF16>(x, row, K, xq, xs, true, gsum, threadIdx.x & 63);
        return;
    }
    align_small_body(ids, numel, E, block_m, emap, emap_len, sorted_ids, sorted_len, expert_ids,
                     ntp, slot_to_row);
}


}  // namespace

size_t align_workspace_bytes(int64_t numel, int64_t num_experts) {
    if (numel <= kChunk) return 0;
    const int64_t nchunks = (numel + kChunk - 1) / kChunk;
    WorkspaceSize s;
    s.take<int32_t>((size_t)(nchunks * num_experts));
    s.take<int32_t>((size_t)num_experts);
    s.take<int32_t>((size_t)numel);
    return s.used;
}

int launch_align(const int32_t* ids, int64_t numel, int64_t E, int64_t block_m,
                 const int32_t* emap, int64_t emap_len, int32_t* sorted_ids, int64_t sorted_len,
                 int32_t* expert_ids, int32_t* ntp, void* ws, size_t ws_bytes,
                 hipStream_t stream, int32_t* slot_to_row) {
    if (E > kMaxExperts) {
        set_error("moe_align: num_experts must be <= 1024");
        return W4A8_ERR_INVALID;
    }
    if (numel <= kChunk) {
        align_small_kernel<<<1, kAlignThreads, 0, stream>>>(ids, numel, (int)E, block_m, emap,
                                                           (int)emap_len, sorted_ids, sorted_len,
                                                           expert_ids, ntp, slot_to_row);
        return check_launch("align_small_kernel");
    }
    const int64_t nchunks = (numel + kChunk - 1) / kChunk;
    Workspace w(ws, ws_bytes);
    int32_t* counts = w.take<int32_t>((size_t)(nchunks * E));
    int32_t* eoff = w.take<int32_t>((size_t)E);
    int32_t* slot_key = w.take<int32_t>((size_t)numel);
    if (ws == nullptr || !w.ok()) {
        set_error("moe_align: workspace too small");
        return W4A8_ERR_WORKSPACE;
    }
    align_count_kernel<<<(unsigned)nchunks, kAlignThreads, 0, stream>>>(ids, numel, (int)E, emap,
                                                                        (int)emap_len, counts,
                                                                        slot_key);
    if (int rc = check_launch("align_count_kernel")) return rc;
    if (nchunks * E <= kScanPlaceMaxCounts) {
        align_scan_place_kernel<<<(unsigned)nchunks, kAlignThreads, 0, stream>>>(
            slot_key, numel, (int)E, block_m, counts, (int)nchunks, sorted_ids, sorted_len,
            expert_ids, ntp, slot_to_row);
        return check_launch("align_scan_place_kernel");
    }
    align_scan_kernel<<<1, kAlignThreads, 0, stream>>>(counts, (int)nchunks, (int)E, block_m,
                                                       numel, eoff, sorted_ids, sorted_len,
                                                       expert_ids, ntp);
    if (int rc = check_launch("align_scan_kernel")) return rc;
    align_place_kernel<<<(unsigned)nchunks, kAlignThreads, 0, stream>>>(slot_key, numel, (int)E,
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
    const dim3 grid((unsigned)((T + 3) / 4 * (x != nullptr ? 2 : 1)));
    if (E <= 64) topk_softmax_kernel<1><<<grid, 256, 0, stream>>>(logits, T, (int)E, (int)top_k, renorm, w, ids, rq);
    else if (E <= 128) topk_softmax_kernel<2><<<grid, 256, 0, stream>>>(logits, T, (int)E, (int)top_k, renorm, w, ids, rq);
    else if (E <= 256) topk_softmax_kernel<4><<<grid, 256, 0, stream>>>(logits, T, (int)E, (int)top_k, renorm, w, ids, rq);
    else if (E <= 512) topk_softmax_kernel<8><<<grid, 256, 0, stream>>>(logits, T, (int)E, (int)top_k, renorm, w, ids, rq);
    else topk_softmax_kernel<16><<<grid, 256, 0, stream>>>(logits, T, (int)E, (int)top_k, renorm, w, ids, rq);
    return check_launch("topk_softmax_kernel");
}


int launch_align_quant(const int32_t* ids, int64_t numel, int64_t E, int64_t block_m,
                       const int32_t* emap, int64_t emap_len, int32_t* sorted_ids,
                       int64_t sorted_len,
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
            ids, numel, (int)E, block_m, emap, (int)emap_len, sorted_ids, sorted_len, expert_ids,
            ntp, slot_to_row, x, rows, (int)K, xq, xs, gsum);
    else
        align_quant_kernel<false><<<grid, kAlignThreads, 0, stream>>>(
            ids, numel, (int)E, block_m, emap, (int)emap_len, sorted_ids, sorted_len, expert_ids,
            ntp, slot_to_row, x, rows, (int)K, xq, xs, gsum);
    return check_launch("align_quant_kernel");
}

}  // namespace w4a8
