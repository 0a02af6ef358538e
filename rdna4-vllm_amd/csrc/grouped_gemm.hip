// Grouped W4A8 GEMMs over the moe_align padded-sorted layout (gfx950).
//
// Three schedules share one arithmetic contract (see w4a8_common.h):
//   * scalar  (kernel id 0): one thread per (row, column), the golden reference
//                            (moe_kernel.hip:133-196);
//   * mfma    (kernel id 6): block_m x BN tiles, per 128-wide K group the int4 weight slab
//                            is decoded to e4m3 once per work-group into LDS, activations
//                            staged beside it, v_mfma_f32_16x16x128_f8f6f4 per 16x16 tile,
//                            fp32 scale fold per group; double-buffered LDS, one barrier
//                            per group (replaces moe_gemm_tiled.h:192-350);
//   * gemv    (kernel id 7): decode regime, one align block per work-group; the block's
//                            real rows are compacted, each wave streams its weight rows
//                            straight from HBM into MFMA B fragments (no LDS, no barriers)
//                            with several groups of loads in flight (replaces
//                            moe_kernel.hip:884-1062).
// All read prequantised activations: x_fp8 rows in k8-interleaved order + act_scales.
#include "w4a8_common.h"
#include "w4a8_internal.h"

namespace w4a8 {
namespace {

struct Params {
    const uint8_t* xq;          // (x_rows, K) e4m3, k8-interleaved
    const float* asc;           // (x_rows,)
    const int32_t* w;           // (E, N, K/8)
    const __half* scales;       // (E, N, G)
    const int32_t* zeros;       // (E, N/8, G) or null
    const int32_t* sorted_ids;
    const int32_t* expert_ids;
    const int32_t* ntp;
    void* out;
    const float* tw;
    int64_t P;
    int K, N, G, E;
    int top_k, out_top_k, block_m;
    int num_valid;
    int identity;
    int e2m1;
};

// Row resolution shared by all schedules. Returns the activation row (or -1).
__device__ __forceinline__ int resolve_row(const Params& p, int64_t r, int ntp, int& slot) {
    slot = -1;
    if (r >= p.P || r >= ntp) return -1;
    const int s = p.sorted_ids ? p.sorted_ids[r] : (int)r;   // dense: identity rows
    if (s < 0 || s >= p.num_valid) return -1;
    slot = s;
    return p.identity ? (int)r : s / p.top_k;
}

template <Epi EPI>
__device__ __forceinline__ void store_out(const Params& p, int64_t row_pad, int src, int slot,
                                          int col, float run_a, float run_b) {
    const float a = p.asc[src];
    if constexpr (EPI == Epi::kHalf) {
        reinterpret_cast<__half*>(p.out)[row_pad * p.N + col] = __float2half(run_a * a);
    } else if constexpr (EPI == Epi::kSiluHalf) {
        const int inter = p.N / 2;
        reinterpret_cast<__half*>(p.out)[row_pad * inter + col] =
            silu_mul_h(__float2half(run_a * a), __float2half(run_b * a));
    } else if constexpr (EPI == Epi::kScatter) {
        const int64_t tok = slot / p.out_top_k;
        atomicAdd(reinterpret_cast<float*>(p.out) + tok * p.N + col, p.tw[slot] * run_a * a);
    } else {
        reinterpret_cast<float*>(p.out)[(int64_t)slot * p.N + col] = run_a * a;
    }
}

// =====================================================================================
// scalar golden
// =====================================================================================
__device__ __forceinline__ float dot_group_scalar(const uint8_t* __restrict__ arow,
                                                  const int32_t* __restrict__ wrow, uint4 t,
                                                  int g, int gs) {
    float acc = 0.f;
    for (int kw = g * gs / 8; kw < (g + 1) * gs / 8; ++kw) {
        uint32_t lo, hi;
        decode8(static_cast<uint32_t>(wrow[kw]), t, lo, hi);
        const uint32_t a0 = *reinterpret_cast<const uint32_t*>(arow + kw * 8);
        const uint32_t a1 = *reinterpret_cast<const uint32_t*>(arow + kw * 8 + 4);
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            acc = fmaf(e4m3_to_f32((a0 >> (8 * b)) & 0xFF), e4m3_to_f32((lo >> (8 * b)) & 0xFF), acc);
            acc = fmaf(e4m3_to_f32((a1 >> (8 * b)) & 0xFF), e4m3_to_f32((hi >> (8 * b)) & 0xFF), acc);
        }
    }
    return acc;
}

template <Epi EPI>
__global__ void __launch_bounds__(256) grouped_scalar_kernel(Params p) {
    const int64_t r = (int64_t)blockIdx.y * 4 + threadIdx.y;
    const int col = blockIdx.x * 64 + threadIdx.x;
    const int ncols = (EPI == Epi::kSiluHalf) ? p.N / 2 : p.N;
    if (col >= ncols) return;
    int slot;
    const int src = resolve_row(p, r, p.ntp ? p.ntp[0] : (int)p.P, slot);
    if (src < 0) return;
    const int e = p.expert_ids ? p.expert_ids[r / p.block_m] : 0;
    if (e < 0 || e >= p.E) return;
    const int gs = p.K / p.G;
    const int32_t* we = p.w + (int64_t)e * p.N * (p.K / 8);
    const __half* se = p.scales + (int64_t)e * p.N * p.G;
    const int32_t* ze = p.zeros ? p.zeros + (int64_t)e * (p.N / 8) * p.G : nullptr;
    const uint8_t* arow = p.xq + (int64_t)src * p.K;
    float run_a = 0.f, run_b = 0.f;
    const int ncol_b = (EPI == Epi::kSiluHalf) ? col + p.N / 2 : -1;
    for (int g = 0; g < p.G; ++g) {
        const float pa = dot_group_scalar(arow, we + (int64_t)col * (p.K / 8),
                                          load_table(table_index(ze, col, g, p.G, p.e2m1)), g, gs);
        run_a = fmaf(pa, __half2float(se[(int64_t)col * p.G + g]), run_a);
        if constexpr (EPI == Epi::kSiluHalf) {
            const float pb = dot_group_scalar(arow, we + (int64_t)ncol_b * (p.K / 8),
                                              load_table(table_index(ze, ncol_b, g, p.G, p.e2m1)),
                                              g, gs);
            run_b = fmaf(pb, __half2float(se[(int64_t)ncol_b * p.G + g]), run_b);
        }
    }
    store_out<EPI>(p, r, src, slot, col, run_a, run_b);
}

// =====================================================================================
// MFMA helpers
// =====================================================================================
__device__ __forceinline__ v4f mfma_16x16x128(const v8i& a, const v8i& b, const v4f& c) {
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}

// 4 words (32 nibbles, k = 0..31 of a fragment) -> 8 dwords of e4m3 (k8-interleaved).
__device__ __forceinline__ v8i decode_frag(uint4 wv, uint4 t) {
    uint32_t o[8];
    decode8(wv.x, t, o[0], o[1]);
    decode8(wv.y, t, o[2], o[3]);
    decode8(wv.z, t, o[4], o[5]);
    decode8(wv.w, t, o[6], o[7]);
    v8i r;
#pragma unroll
    for (int i = 0; i < 8; ++i) r[i] = (int)o[i];
    return r;
}

// =====================================================================================
// MFMA tiled (prefill) kernel
// =====================================================================================
constexpr int kGroup = 128;          // K per group == K per MFMA
constexpr int kLdsStride = kGroup + 16;

template <Epi EPI, int BM, int BN>
struct TileCfg {
    static constexpr bool kSilu = EPI == Epi::kSiluHalf;
    static constexpr int WM = BM >= 32 ? 2 : 1;   // waves along M
    static constexpr int WN = 4 / WM;             // waves along N
    static constexpr int MW = BM / WM;            // rows per wave
    static constexpr int MT = MW / 16;            // m-tiles per wave
    static constexpr int NWC = BN / WN;           // output columns per wave
    static constexpr int NT = NWC / 16;           // n-tiles per wave (per half for SiLU)
    static constexpr int BROWS = kSilu ? 2 * BN : BN;   // weight rows per group tile
    static constexpr int A_CHUNKS = (BM * 8 + 255) / 256;   // 16-B activation chunks per thread
    static constexpr int B_CHUNKS = BROWS * 4 / 256;    // 16-B weight chunks per thread
    static constexpr int NTT = kSilu ? 2 * NT : NT;     // n-tiles incl. up half
    static constexpr int LDS_A = BM * kLdsStride;
    static constexpr int LDS_B = BROWS * kLdsStride;
    static constexpr int LDS_BYTES = 2 * (LDS_A + LDS_B);
    static_assert(MT >= 1 && NT >= 1 && A_CHUNKS >= 1 && B_CHUNKS >= 1, "tile too small");
};

template <Epi EPI, int BM, int BN>
__global__ void __launch_bounds__(256) grouped_mfma_kernel(Params p) {
    using C = TileCfg<EPI, BM, BN>;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    __shared__ int s_src[BM];
    __shared__ int s_slot[BM];

    const int64_t row0 = (int64_t)blockIdx.y * BM;
    const int ntp = p.ntp ? p.ntp[0] : (int)p.P;
    if (row0 >= ntp || row0 >= p.P) return;
    const int e = p.expert_ids ? p.expert_ids[row0 / p.block_m] : 0;
    if (e < 0 || e >= p.E) return;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave / C::WN;
    const int wn = wave % C::WN;
    const int n0 = blockIdx.x * BN;                  // first output column of this tile
    const int ncols = C::kSilu ? p.N / 2 : p.N;       // output columns
    const int kw_row = p.K / 8;

    if (tid < BM) {
        int slot;
        s_src[tid] = resolve_row(p, row0 + tid, ntp, slot);
        s_slot[tid] = slot;
    }
    __syncthreads();

    const int32_t* we = p.w + (int64_t)e * p.N * kw_row;
    const __half* se = p.scales + (int64_t)e * p.N * p.G;
    const int32_t* ze = p.zeros ? p.zeros + (int64_t)e * (p.N / 8) * p.G : nullptr;

    // ---- staging assignments ----
    // activations: chunk c -> row c/8, 16-byte piece c%8 of the 128-byte group slice
    int a_row[C::A_CHUNKS];
    const uint8_t* a_ptr[C::A_CHUNKS];
#pragma unroll
    for (int i = 0; i < C::A_CHUNKS; ++i) {
        const int c = tid + i * 256;
        a_row[i] = c < BM * 8 ? (c >> 3) : -1;
        const int src = c < BM * 8 ? s_src[c >> 3] : -1;
        a_ptr[i] = src >= 0 ? p.xq + (int64_t)src * p.K + (c & 7) * 16 : nullptr;
    }
    // weights: chunk c -> tile row c/4, 32-nibble piece c%4 of the group
    int b_row[C::B_CHUNKS];
    int b_n[C::B_CHUNKS];   // absolute weight row or -1
#pragma unroll
    for (int i = 0; i < C::B_CHUNKS; ++i) {
        const int c = tid + i * 256;
        const int tr = c >> 2;
        b_row[i] = tr;
        int n;
        if constexpr (C::kSilu) {
            const int col = n0 + (tr < BN ? tr : tr - BN);
            n = col < ncols ? (tr < BN ? col : col + ncols) : -1;
        } else {
            n = n0 + tr;
            if (n >= p.N) n = -1;
        }
        b_n[i] = n;
    }

    uint4 a_reg[C::A_CHUNKS];
    uint4 b_reg[C::B_CHUNKS];
    int b_tab[C::B_CHUNKS];
    auto load_group = [&](int g) {
#pragma unroll
        for (int i = 0; i < C::A_CHUNKS; ++i)
            a_reg[i] = a_ptr[i] ? *reinterpret_cast<const uint4*>(a_ptr[i] + g * kGroup)
                                : make_uint4(0, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < C::B_CHUNKS; ++i) {
            const int n = b_n[i];
            if (n >= 0) {
                b_reg[i] = *reinterpret_cast<const uint4*>(
                    we + (int64_t)n * kw_row + g * (kGroup / 8) + ((tid + i * 256) & 3) * 4);
                b_tab[i] = table_index(ze, n, g, p.G, p.e2m1);
            } else {
                b_reg[i] = make_uint4(0, 0, 0, 0);
                b_tab[i] = -1;
            }
        }
    };
    auto store_group = [&](int buf) {
        uint8_t* A = lds + buf * (C::LDS_A + C::LDS_B);
        uint8_t* B = A + C::LDS_A;
#pragma unroll
        for (int i = 0; i < C::A_CHUNKS; ++i) {
            const int c = tid + i * 256;
            if (a_row[i] >= 0)
                *reinterpret_cast<uint4*>(A + a_row[i] * kLdsStride + (c & 7) * 16) = a_reg[i];
        }
#pragma unroll
        for (int i = 0; i < C::B_CHUNKS; ++i) {
            const int c = tid + i * 256;
            uint8_t* dst = B + b_row[i] * kLdsStride + (c & 3) * 32;
            if (b_tab[i] >= 0) {
                const v8i d = decode_frag(b_reg[i], load_table(b_tab[i]));
                *reinterpret_cast<uint4*>(dst) = make_uint4(d[0], d[1], d[2], d[3]);
                *reinterpret_cast<uint4*>(dst + 16) = make_uint4(d[4], d[5], d[6], d[7]);
            } else {
                *reinterpret_cast<uint4*>(dst) = make_uint4(0, 0, 0, 0);
                *reinterpret_cast<uint4*>(dst + 16) = make_uint4(0, 0, 0, 0);
            }
        }
    };

    // columns of this wave's n-tiles (lane's D column) and their scale rows
    int t_col[C::NTT];
    int t_srow[C::NTT];
#pragma unroll
    for (int j = 0; j < C::NTT; ++j) {
        const int jj = C::kSilu ? (j % C::NT) : j;
        const int col = n0 + wn * C::NWC + jj * 16 + (lane & 15);
        t_col[j] = col;
        const bool up = C::kSilu && j >= C::NT;
        t_srow[j] = col < ncols ? (up ? col + ncols : col) : -1;
    }

    v4f run[C::MT][C::NTT];
#pragma unroll
    for (int i = 0; i < C::MT; ++i)
#pragma unroll
        for (int j = 0; j < C::NTT; ++j) run[i][j] = v4f{0.f, 0.f, 0.f, 0.f};

    load_group(0);
    store_group(0);
    __syncthreads();

    for (int g = 0; g < p.G; ++g) {
        const int buf = g & 1;
        if (g + 1 < p.G) load_group(g + 1);
        float sc[C::NTT];
#pragma unroll
        for (int j = 0; j < C::NTT; ++j)
            sc[j] = t_srow[j] >= 0 ? __half2float(se[(int64_t)t_srow[j] * p.G + g]) : 0.f;

        const uint8_t* A = lds + buf * (C::LDS_A + C::LDS_B);
        const uint8_t* B = A + C::LDS_A;
        v8i bf[C::NTT];
#pragma unroll
        for (int j = 0; j < C::NTT; ++j) {
            const int jj = C::kSilu ? (j % C::NT) : j;
            const int brow = (C::kSilu && j >= C::NT ? BN : 0) + wn * C::NWC + jj * 16 + (lane & 15);
            const uint8_t* src = B + brow * kLdsStride + (lane >> 4) * 32;
            const uint4 lo = *reinterpret_cast<const uint4*>(src);
            const uint4 hi = *reinterpret_cast<const uint4*>(src + 16);
            bf[j] = v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w,
                        (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
        }
#pragma unroll
        for (int i = 0; i < C::MT; ++i) {
            const int arow = wm * C::MW + i * 16 + (lane & 15);
            const uint8_t* src = A + arow * kLdsStride + (lane >> 4) * 32;
            const uint4 lo = *reinterpret_cast<const uint4*>(src);
            const uint4 hi = *reinterpret_cast<const uint4*>(src + 16);
            const v8i af = v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w,
                               (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
#pragma unroll
            for (int j = 0; j < C::NTT; ++j) {
                const v4f acc = mfma_16x16x128(af, bf[j], v4f{0.f, 0.f, 0.f, 0.f});
#pragma unroll
                for (int r = 0; r < 4; ++r) run[i][j][r] = fmaf(acc[r], sc[j], run[i][j][r]);
            }
        }
        if (g + 1 < p.G) store_group(buf ^ 1);
        __syncthreads();
    }

    // ---- epilogue ----
#pragma unroll
    for (int i = 0; i < C::MT; ++i) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int lr = wm * C::MW + i * 16 + (lane >> 4) * 4 + r;
            const int src = s_src[lr];
            if (src < 0) continue;
#pragma unroll
            for (int j = 0; j < C::NT; ++j) {
                const int col = t_col[j];
                if (col >= ncols) continue;
                const float rb = C::kSilu ? run[i][j + (C::kSilu ? C::NT : 0)][r] : 0.f;
                store_out<EPI>(p, row0 + lr, src, s_slot[lr], col, run[i][j][r], rb);
            }
        }
    }
}

// =====================================================================================
// MFMA GEMV (decode) kernel
// =====================================================================================
constexpr int kGemvMaxRows = 64;     // block_m cap (4 m-tiles)
constexpr int kGemvUnroll = 4;       // groups of weight loads in flight per wave

template <Epi EPI, int NT>
__global__ void __launch_bounds__(256) grouped_gemv_kernel(Params p) {
    constexpr bool kSilu = EPI == Epi::kSiluHalf;
    constexpr int NTT = kSilu ? 2 * NT : NT;
    constexpr int MT_MAX = kGemvMaxRows / 16;
    __shared__ int s_src[kGemvMaxRows];
    __shared__ int s_slot[kGemvMaxRows];
    __shared__ int s_pad[kGemvMaxRows];
    __shared__ int s_mreal;

    const int64_t row0 = (int64_t)blockIdx.y * p.block_m;
    const int ntp = p.ntp ? p.ntp[0] : (int)p.P;
    if (row0 >= ntp || row0 >= p.P) return;
    const int e = p.expert_ids ? p.expert_ids[row0 / p.block_m] : 0;
    if (e < 0 || e >= p.E) return;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;

    // compact the block's real rows (wave 0, ballot prefix)
    if (wave == 0) {
        int slot = -1, src = -1;
        if (lane < p.block_m) src = resolve_row(p, row0 + lane, ntp, slot);
        const bool v = src >= 0;
        const uint64_t mask = __ballot(v);
        const int pos = __popcll(mask & ((1ull << lane) - 1ull));
        if (v) { s_src[pos] = src; s_slot[pos] = slot; s_pad[pos] = (int)(row0 + lane); }
        if (lane == 0) s_mreal = __popcll(mask);
    }
    __syncthreads();
    const int mreal = s_mreal;
    if (mreal == 0) return;
    const int mtiles = (mreal + 15) >> 4;

    const int ncols = kSilu ? p.N / 2 : p.N;
    const int kw_row = p.K / 8;
    const int32_t* we = p.w + (int64_t)e * p.N * kw_row;
    const __half* se = p.scales + (int64_t)e * p.N * p.G;
    const int32_t* ze = p.zeros ? p.zeros + (int64_t)e * (p.N / 8) * p.G : nullptr;

    // this wave's tiles: output column tile base, lane's weight row per tile
    const int col0 = (blockIdx.x * 4 + wave) * NT * 16;
    int t_n[NTT];    // weight row feeding this lane's B fragment == scale row of its D column
#pragma unroll
    for (int j = 0; j < NTT; ++j) {
        const int col = col0 + (j % NT) * 16 + (lane & 15);
        const bool up = kSilu && j >= NT;
        t_n[j] = col < ncols ? (up ? col + ncols : col) : -1;
    }
    // activation row pointers for each m-tile (lane's A row)
    const uint8_t* a_ptr[MT_MAX];
#pragma unroll
    for (int i = 0; i < MT_MAX; ++i) {
        const int m = i * 16 + (lane & 15);
        a_ptr[i] = (m < mreal) ? p.xq + (int64_t)s_src[m] * p.K + (lane >> 4) * 32 : nullptr;
    }

    v4f run[MT_MAX][NTT];
#pragma unroll
    for (int i = 0; i < MT_MAX; ++i)
#pragma unroll
        for (int j = 0; j < NTT; ++j) run[i][j] = v4f{0.f, 0.f, 0.f, 0.f};

    for (int g0 = 0; g0 < p.G; g0 += kGemvUnroll) {
        uint4 wv[kGemvUnroll][NTT];
        int tab[kGemvUnroll][NTT];
        float sc[kGemvUnroll][NTT];
#pragma unroll
        for (int u = 0; u < kGemvUnroll; ++u) {
            const int g = g0 + u;
#pragma unroll
            for (int j = 0; j < NTT; ++j) {
                const int n = t_n[j];
                if (g < p.G && n >= 0) {
                    wv[u][j] = *reinterpret_cast<const uint4*>(
                        we + (int64_t)n * kw_row + g * (kGroup / 8) + (lane >> 4) * 4);
                    tab[u][j] = table_index(ze, n, g, p.G, p.e2m1);
                    sc[u][j] = __half2float(se[(int64_t)n * p.G + g]);
                } else {
                    wv[u][j] = make_uint4(0, 0, 0, 0);
                    tab[u][j] = 8;
                    sc[u][j] = 0.f;
                }
            }
        }
#pragma unroll
        for (int u = 0; u < kGemvUnroll; ++u) {
            const int g = g0 + u;
            if (g >= p.G) break;
            v8i bf[NTT];
#pragma unroll
            for (int j = 0; j < NTT; ++j) bf[j] = decode_frag(wv[u][j], load_table(tab[u][j]));
#pragma unroll
            for (int i = 0; i < MT_MAX; ++i) {
                if (i >= mtiles) break;
                v8i af = v8i{0, 0, 0, 0, 0, 0, 0, 0};
                if (a_ptr[i]) {
                    const uint4 lo = *reinterpret_cast<const uint4*>(a_ptr[i] + g * kGroup);
                    const uint4 hi = *reinterpret_cast<const uint4*>(a_ptr[i] + g * kGroup + 16);
                    af = v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w,
                             (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
                }
#pragma unroll
                for (int j = 0; j < NTT; ++j) {
                    const v4f acc = mfma_16x16x128(af, bf[j], v4f{0.f, 0.f, 0.f, 0.f});
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        run[i][j][r] = fmaf(acc[r], sc[u][j], run[i][j][r]);
                }
            }
        }
    }

    // epilogue: D lane holds rows 4*(lane/16)+r of each m-tile, column lane%16
#pragma unroll
    for (int i = 0; i < MT_MAX; ++i) {
        if (i >= mtiles) break;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int m = i * 16 + (lane >> 4) * 4 + r;
            if (m >= mreal) continue;
#pragma unroll
            for (int j = 0; j < NT; ++j) {
                const int col = col0 + j * 16 + (lane & 15);
                if (col >= ncols) continue;
                const float rb = kSilu ? run[i][j + (kSilu ? NT : 0)][r] : 0.f;
                store_out<EPI>(p, s_pad[m], s_src[m], s_slot[m], col, run[i][j][r], rb);
            }
        }
    }
}

Params make_params(const GroupedArgs& a) {
    Params p;
    p.xq = a.x_fp8;
    p.asc = a.act_scales;
    p.w = a.w;
    p.scales = reinterpret_cast<const __half*>(a.scales);
    p.zeros = a.zeros;
    p.sorted_ids = a.sorted_ids;
    p.expert_ids = a.expert_ids;
    p.ntp = a.ntp;
    p.out = a.out;
    p.tw = a.topk_weights;
    p.P = a.P;
    p.K = (int)a.K;
    p.N = (int)a.N;
    p.G = (int)(a.K / a.group_size);
    p.E = (int)a.E;
    p.top_k = (int)a.top_k;
    p.out_top_k = (int)a.out_top_k;
    p.block_m = (int)a.block_m;
    p.num_valid = (int)a.num_valid;
    p.identity = a.identity_gather ? 1 : 0;
    p.e2m1 = a.e2m1 ? 1 : 0;
    return p;
}

template <Epi EPI>
int launch_scalar_t(const Params& p, hipStream_t s) {
    const int ncols = EPI == Epi::kSiluHalf ? p.N / 2 : p.N;
    dim3 grid((unsigned)((ncols + 63) / 64), (unsigned)((p.P + 3) / 4));
    grouped_scalar_kernel<EPI><<<grid, dim3(64, 4), 0, s>>>(p);
    return check_launch("grouped_scalar_kernel");
}

template <Epi EPI, int BM, int BN>
int launch_mfma_t(const Params& p, hipStream_t s) {
    using C = TileCfg<EPI, BM, BN>;
    static bool attr_set = false;   // > 64 KB dynamic LDS needs an explicit opt-in
    if (!attr_set) {
        if (hipFuncSetAttribute(reinterpret_cast<const void*>(&grouped_mfma_kernel<EPI, BM, BN>),
                                hipFuncAttributeMaxDynamicSharedMemorySize,
                                C::LDS_BYTES) != hipSuccess) {
            set_error("grouped_mfma_kernel: cannot reserve dynamic LDS");
            return W4A8_ERR_HIP;
        }
        attr_set = true;
    }
    const int ncols = EPI == Epi::kSiluHalf ? p.N / 2 : p.N;
    dim3 grid((unsigned)((ncols + BN - 1) / BN), (unsigned)((p.P + BM - 1) / BM));
    grouped_mfma_kernel<EPI, BM, BN><<<grid, 256, C::LDS_BYTES, s>>>(p);
    return check_launch("grouped_mfma_kernel");
}

// The work-group tile height must divide block_m so every tile lies in one expert block.
template <Epi EPI>
int launch_mfma_e(const Params& p, hipStream_t s) {
    if (p.block_m % 128 == 0) return launch_mfma_t<EPI, 128, 64>(p, s);
    if (p.block_m % 64 == 0) return launch_mfma_t<EPI, 64, 64>(p, s);
    if (p.block_m % 32 == 0) return launch_mfma_t<EPI, 32, 64>(p, s);
    if (p.block_m % 16 == 0) return launch_mfma_t<EPI, 16, 64>(p, s);
    set_error("wmma grouped GEMM: block_m must be a multiple of 16");
    return W4A8_ERR_INVALID;
}

template <Epi EPI>
int launch_gemv_e(const Params& p, hipStream_t s) {
    constexpr int NT = 1;
    const int ncols = EPI == Epi::kSiluHalf ? p.N / 2 : p.N;
    const int cols_per_block = 4 * NT * 16;
    dim3 grid((unsigned)((ncols + cols_per_block - 1) / cols_per_block),
              (unsigned)((p.P + p.block_m - 1) / p.block_m));
    grouped_gemv_kernel<EPI, NT><<<grid, 256, 0, s>>>(p);
    return check_launch("grouped_gemv_kernel");
}

}  // namespace

bool mfma_supported(int64_t K, int64_t group_size) {
    return group_size == kGroup && K % kGroup == 0;
}

int launch_grouped_scalar(const GroupedArgs& a, hipStream_t s) {
    const Params p = make_params(a);
    if (p.P == 0) return W4A8_OK;
    switch (a.epi) {
        case Epi::kHalf: return launch_scalar_t<Epi::kHalf>(p, s);
        case Epi::kSiluHalf: return launch_scalar_t<Epi::kSiluHalf>(p, s);
        case Epi::kScatter: return launch_scalar_t<Epi::kScatter>(p, s);
        case Epi::kSlotF32: return launch_scalar_t<Epi::kSlotF32>(p, s);
    }
    return W4A8_ERR_INVALID;
}

int launch_grouped_mfma(const GroupedArgs& a, hipStream_t s) {
    const Params p = make_params(a);
    if (p.P == 0) return W4A8_OK;
    switch (a.epi) {
        case Epi::kHalf: return launch_mfma_e<Epi::kHalf>(p, s);
        case Epi::kSiluHalf: return launch_mfma_e<Epi::kSiluHalf>(p, s);
        case Epi::kScatter: return launch_mfma_e<Epi::kScatter>(p, s);
        case Epi::kSlotF32: return launch_mfma_e<Epi::kSlotF32>(p, s);
    }
    return W4A8_ERR_INVALID;
}

int launch_grouped_gemv(const GroupedArgs& a, hipStream_t s) {
    const Params p = make_params(a);
    if (p.P == 0) return W4A8_OK;
    if (p.block_m > kGemvMaxRows) {
        set_error("gemv grouped GEMM: block_m must be <= 64");
        return W4A8_ERR_INVALID;
    }
    switch (a.epi) {
        case Epi::kHalf: return launch_gemv_e<Epi::kHalf>(p, s);
        case Epi::kSiluHalf: return launch_gemv_e<Epi::kSiluHalf>(p, s);
        case Epi::kScatter: return launch_gemv_e<Epi::kScatter>(p, s);
        case Epi::kSlotF32: return launch_gemv_e<Epi::kSlotF32>(p, s);
    }
    return W4A8_ERR_INVALID;
}

}  // namespace w4a8
