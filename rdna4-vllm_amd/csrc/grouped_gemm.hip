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
#include <algorithm>
#include <type_traits>

#include "w4a8_common.h"
#include "w4a8_internal.h"
#include "grouped_params.h"

namespace w4a8 {
namespace {

template <Epi EPI>
__device__ __forceinline__ void store_out(const Params& p, int64_t row_pad, int src, int slot,
                                          int col, float run_a, float run_b) {
    const float a = p.asc[src];
    if constexpr (EPI == Epi::kHalf) {
        reinterpret_cast<__half*>(p.out)[row_pad * p.N + col] = __float2half(as_f32(run_a * a));
    } else if constexpr (EPI == Epi::kSiluHalf) {
        const int inter = p.N / 2;
        reinterpret_cast<__half*>(p.out)[row_pad * inter + col] =
            silu_mul_h(__float2half(as_f32(run_a * a)), __float2half(as_f32(run_b * a)));
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

// FP4: E2M1 weights enter the MFMA as fp4 operands (raw codes, the f8f6f4 MFMA's e2m1
// format decodes them), against activations quantised in natural k order; one MFMA per
// K group of 32, 64 or 128 (the lanes holding other groups' 32-wide K blocks pass zero codes),
// each folded with its own scale, so a group's partial sum is the same exact sum the scalar
// kernel forms. Otherwise int4 / E2M1 words are decoded to e4m3 through the tables
// (k8-interleaved, against k8-interleaved activations).
template <Epi EPI, int BM, int BN, bool FP4>
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
        // padding rows read a real row: their outputs are never stored
        const int src = c < BM * 8 ? s_src[c >> 3] : -1;
        a_ptr[i] = p.xq + (int64_t)(src >= 0 ? src : s_src[0] >= 0 ? s_src[0] : 0) * p.K +
                   (c & 7) * 16;
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
        b_n[i] = n < 0 ? 0 : n;   // edge columns read row 0; they are never stored
    }

    u32x4 a_reg[C::A_CHUNKS];
    u32x4 b_reg[C::B_CHUNKS];
    int b_tab[C::B_CHUNKS];
    // K step g covers k [128 g, 128 g + 128); E2M1 takes K % 128 == 32, 64 or 96 too, and the
    // pieces of its last step past K load as zeros (zero codes against zero activations)
    auto load_group = [&](int g) {
#pragma unroll
        for (int i = 0; i < C::A_CHUNKS; ++i) {
            const bool in = !FP4 || g * kGroup + ((tid + i * 256) & 7) * 16 < p.K;
            a_reg[i] = in ? *reinterpret_cast<const u32x4*>(a_ptr[i] + g * kGroup) : u32x4{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int i = 0; i < C::B_CHUNKS; ++i) {
            const int n = b_n[i];
            const bool in = !FP4 || g * kGroup + ((tid + i * 256) & 3) * 32 < p.K;
            b_reg[i] = in ? *reinterpret_cast<const u32x4*>(
                                we + (int64_t)n * kw_row + g * (kGroup / 8) + ((tid + i * 256) & 3) * 4)
                          : u32x4{0u, 0u, 0u, 0u};
            if constexpr (!FP4) b_tab[i] = table_index(ze, n, g, p.G, p.e2m1);
        }
    };
    auto store_group = [&](int buf) {
        uint8_t* A = lds + buf * (C::LDS_A + C::LDS_B);
        uint8_t* B = A + C::LDS_A;
#pragma unroll
        for (int i = 0; i < C::A_CHUNKS; ++i) {
            const int c = tid + i * 256;
            if (a_row[i] >= 0)
                *reinterpret_cast<u32x4*>(A + a_row[i] * kLdsStride + (c & 7) * 16) = a_reg[i];
        }
#pragma unroll
        for (int i = 0; i < C::B_CHUNKS; ++i) {
            const int c = tid + i * 256;
            uint8_t* dst = B + b_row[i] * kLdsStride + (c & 3) * 32;
            if constexpr (FP4) {
                *reinterpret_cast<u32x4*>(dst) = b_reg[i];   // 32 codes, first half of the slot
            } else {
                const u32x4 w = b_reg[i];
                const v8i d = decode_frag(make_uint4(w.x, w.y, w.z, w.w), load_table(b_tab[i]));
                *reinterpret_cast<uint4*>(dst) = make_uint4(d[0], d[1], d[2], d[3]);
                *reinterpret_cast<uint4*>(dst + 16) = make_uint4(d[4], d[5], d[6], d[7]);
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
        t_srow[j] = col < ncols ? (up ? col + ncols : col) : 0;
    }

    v4f run[C::MT][C::NTT];
#pragma unroll
    for (int i = 0; i < C::MT; ++i)
#pragma unroll
        for (int j = 0; j < C::NTT; ++j) run[i][j] = v4f{0.f, 0.f, 0.f, 0.f};

    // K steps of 128 (FP4: the last may be partial); FP4 takes groups of 32, 64 or 128 (gps
    // groups per full step)
    const int nsteps = (p.K + kGroup - 1) / kGroup;
    const int gps = FP4 ? kGroup / (p.K / p.G) : 1;
    // this lane's 32-wide K block within a step, and the group of the step it belongs to
    const int lane_grp = FP4 ? (lane >> 4) * gps / 4 : 0;

    load_group(0);
    store_group(0);
    __syncthreads();

    for (int g = 0; g < nsteps; ++g) {
        const int buf = g & 1;
        if (g + 1 < nsteps) load_group(g + 1);

        const uint8_t* A = lds + buf * (C::LDS_A + C::LDS_B);
        const uint8_t* B = A + C::LDS_A;
        v8i bf[C::NTT];
#pragma unroll
        for (int j = 0; j < C::NTT; ++j) {
            const int jj = C::kSilu ? (j % C::NT) : j;
            const int brow = (C::kSilu && j >= C::NT ? BN : 0) + wn * C::NWC + jj * 16 + (lane & 15);
            const uint8_t* src = B + brow * kLdsStride + (lane >> 4) * 32;
            const uint4 lo = *reinterpret_cast<const uint4*>(src);
            if constexpr (FP4) {
                bf[j] = v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, 0, 0, 0, 0};
            } else {
                const uint4 hi = *reinterpret_cast<const uint4*>(src + 16);
                bf[j] = v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w,
                            (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
            }
        }
        v8i af[C::MT];
#pragma unroll
        for (int i = 0; i < C::MT; ++i) {
            const int arow = wm * C::MW + i * 16 + (lane & 15);
            // against an fp4 operand (lane kb: k 32kb..32kb+31) an fp8 lane kb holds
            // k 16kb..16kb+15 and 64+16kb..64+16kb+15; fp8 against fp8 pairs element for element
            const uint8_t* src = A + arow * kLdsStride + (lane >> 4) * (FP4 ? 16 : 32);
            const uint4 lo = *reinterpret_cast<const uint4*>(src);
            const uint4 hi = *reinterpret_cast<const uint4*>(src + (FP4 ? 64 : 16));
            af[i] = v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w,
                        (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
        }
        for (int sg = 0; sg < gps; ++sg) {   // gps == 1 without FP4
            const int gi = g * gps + sg;
            if (gi >= p.G) break;               // past K in a partial last step
            float sc[C::NTT];
#pragma unroll
            for (int j = 0; j < C::NTT; ++j) sc[j] = __half2float(se[(int64_t)t_srow[j] * p.G + gi]);
            v8i bm[C::NTT];
#pragma unroll
            for (int j = 0; j < C::NTT; ++j) {
                const bool mine = !FP4 || gps == 1 || lane_grp == sg;
#pragma unroll
                for (int t = 0; t < 8; ++t) bm[j][t] = mine ? bf[j][t] : 0;
            }
#pragma unroll
            for (int i = 0; i < C::MT; ++i) {
#pragma unroll
                for (int j = 0; j < C::NTT; ++j) {
                    v4f acc;
                    if constexpr (FP4)
                        acc = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                            af[i], bm[j], v4f{0.f, 0.f, 0.f, 0.f}, 0, 4, 0, 0, 0, 0);
                    else
                        acc = mfma_16x16x128(af[i], bm[j], v4f{0.f, 0.f, 0.f, 0.f});
#pragma unroll
                    for (int r = 0; r < 4; ++r) run[i][j][r] = fmaf(acc[r], sc[j], run[i][j][r]);
                }
            }
        }
        if (g + 1 < nsteps) store_group(buf ^ 1);
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
// MFMA GEMV (decode) kernel: split-K waves, activations in registers
// =====================================================================================
// Decode blocks hold 1..16 real rows, so the work is a stream of int4 weights. One
// work-group takes one align block and a slice of 16-column tiles (SiLU: 16 gate columns
// plus the matching 16 up columns). The K groups are split over KSPLIT waves, GPW groups
// each; every wave keeps its activation fragments and their group sums in registers for
// the whole slice, so its main loop is weight loads, nibble spreading and MFMA only, with
// the loads of the next chunk in flight behind the current one. The KSPLIT partial sums of
// a tile are added in LDS in a fixed order (deterministic).
//
// Weight nibbles enter the MFMA undecoded. The e4m3 byte with value n (0..15) is exactly
// n * 2^-9 (subnormals 0..7; exponent field 1 for 8..15), so spreading a word's nibbles
// into bytes (two AND, one shift) gives 2^-9 * n in the k8-interleave order. The
// zero-point enters through sum_k a_k (n_k - z) = sum_k a_k n_k - z * sum_k a_k, where the
// row's group sums come from one MFMA against e4m3 1.0 (scaled by 2^-9 in fp32, exact),
// and the 2^9 rides on the activation scale. Every operand is an integer times a power of
// two, so this is the dot product the reference forms with e4m3(n - z) operands
// (tile_config.h:42-45) up to the MFMA's rounding. (Sums against the subnormal 2^-9 byte
// lose accuracy inside the MFMA; against 1.0 they are exact to a few fp32 ulps.) E2M1 weights (a codebook, no
// zero-points) take the matrix-core tiles instead.
constexpr int kGemvMaxRows = 64;                 // block_m cap (16-row passes)
constexpr int kGemvMaxTiles = 8;                 // tiles per team (LDS partials bound)
constexpr uint32_t kOnesE4m3 = 0x38383838u;      // four e4m3 bytes of 1.0

template <Epi EPI, int GPW, int KSPLIT>
struct GemvCfg {
    static constexpr bool kSilu = EPI == Epi::kSiluHalf;
    static constexpr int NF = kSilu ? 2 : 1;      // fragments per column tile
    static constexpr int CT = kSilu ? 1 : 2;      // column tiles per chunk
    static constexpr int FR = NF * CT;            // fragments per chunk and group
    static constexpr int GC = GPW < 4 ? GPW : 4;  // groups per chunk
    static constexpr int NB = GPW / GC;           // chunks per tile set
    static constexpr int TEAMS = 4 / KSPLIT;      // wave teams (independent tile ranges)
    static constexpr bool kPackedScales = GC == 2 || GC == 4;
    // 4-group chunks (one per tile set): the scales and zero-point words of all chunks are
    // loaded once per work-group into LDS instead of alongside every chunk
    static constexpr bool kStagedSZ = GC == 4 && NB == 1;
    static_assert(GPW % GC == 0 && (NB == 1 || NB == 2), "unsupported groups per wave");
    static_assert(KSPLIT == 1 || KSPLIT == 2 || KSPLIT == 4, "KSPLIT divides the 4 waves");
};

// GC consecutive fp16 scales; packed two per word when the vector load is aligned.
template <int GC>
__device__ __forceinline__ void load_scales(const __half* ptr, uint32_t (&s)[GC]) {
    const uint16_t* h = reinterpret_cast<const uint16_t*>(ptr);
    if constexpr (GC == 4) {
        const uint2 v = *reinterpret_cast<const uint2*>(h);
        s[0] = v.x;
        s[1] = v.y;
    } else if constexpr (GC == 2) {
        s[0] = *reinterpret_cast<const uint32_t*>(h);
    } else {
#pragma unroll
        for (int u = 0; u < GC; ++u) s[u] = h[u];
    }
}
template <int GC>
__device__ __forceinline__ float scale_at(const uint32_t (&s)[GC], int u) {
    uint32_t bits;
    if constexpr (GC == 2 || GC == 4) bits = (s[u >> 1] >> (16 * (u & 1))) & 0xFFFFu;
    else bits = s[u] & 0xFFFFu;
    return __half2float(__ushort_as_half(static_cast<unsigned short>(bits)));
}
template <int GC>
__device__ __forceinline__ void load_zero_words(const int32_t* ptr, int32_t (&z)[GC]) {
    if constexpr (GC == 4) {
        const int4 v = *reinterpret_cast<const int4*>(ptr);
        z[0] = v.x; z[1] = v.y; z[2] = v.z; z[3] = v.w;
    } else if constexpr (GC == 2) {
        const int2 v = *reinterpret_cast<const int2*>(ptr);
        z[0] = v.x; z[1] = v.y;
    } else {
#pragma unroll
        for (int u = 0; u < GC; ++u) z[u] = ptr[u];
    }
}

template <bool BF16>
__device__ __forceinline__ float half_bits_to_f32(uint32_t bits) {
    if constexpr (BF16) {
        // bf16 -> fp16 -> f32, the cast the reference applies before quantising (moe_experts.py:596-597)
        const float f = __uint_as_float(bits << 16);
        return __half2float(__float2half(f));
    } else {
        return __half2float(__ushort_as_half(static_cast<unsigned short>(bits)));
    }
}

// fp16 or bf16 bits -> f32 with the input dtype chosen at run time (a single value; loops
// over many values branch on the dtype once and call half_bits_to_f32 instead)
__device__ __forceinline__ float act_bits_to_f32(uint32_t bits, bool bf16) {
    return bf16 ? half_bits_to_f32<true>(bits) : half_bits_to_f32<false>(bits);
}

// Decode GEMV. One work-group per (block of block_m sorted rows, range of column tiles).
// Loads are issued in dependency levels so that no wait drains the weight stream: (1) list
// length, expert id and the block's sorted ids; (2) this pass's activation rows (and, for
// 4-group chunks, every scale and zero-point word the wave will use); (3) the first two
// weight chunks. Waiting for (2) then leaves (3) in flight, and the chunk loop keeps two
// chunks in flight after that. Row compaction (real rows first) is computed by every wave
// from a ballot, so the prologue has no work-group barrier.
// AQ: x is fp16/bf16 and each pass quantises its rows in registers, bit-identical to
// act_quant_kernel (the row absmax is combined across the KSPLIT waves through LDS).
// FRAG: weights in the fragment layout (repack.hip): a fragment-group is one contiguous
// kilobyte, lane l's 16 bytes at offset 16 l.
template <Epi EPI, int GPW, int KSPLIT, bool AQ, bool FRAG>
__global__ void __launch_bounds__(256, 2) grouped_gemv_kernel(Params p, int tpt) {
    using C = GemvCfg<EPI, GPW, KSPLIT>;
    extern __shared__ __attribute__((aligned(16))) uint8_t s_dyn[];   // KSPLIT > 1 partials
    __shared__ float s_amax[4][16];
    __shared__ int s_opad[4][16];
    __shared__ int s_oslot[4][16];
    __shared__ float s_oasc[4][16];
    // staged scales (4 fp16 per row) and zero-point words (4 groups per 8 rows) of every
    // chunk of the wave: [chunk][fragment][column] and [chunk][fragment][column / 8]
    __shared__ uint2 s_sc[4][C::kStagedSZ ? kGemvMaxTiles * C::FR * 16 : 1];
    __shared__ uint4 s_zw[4][C::kStagedSZ ? kGemvMaxTiles * C::FR * 2 : 1];
    v4f* s_part = reinterpret_cast<v4f*>(s_dyn);   // [wave][tile][NF][lane]

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    // wave-uniform (the compiler cannot prove tid >> 6 uniform): keeps the tile range and
    // the chunk loop scalar, so the loop and its wait counts are not per-lane
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int q = lane >> 4;           // k quarter of a group / D row quad of this lane
    const int c16 = lane & 15;         // B column / A row of this lane
    const int64_t row0 = (int64_t)blockIdx.y * p.block_m;

    // ---- level 1: independent metadata loads ----
    const int ntp = p.ntp ? p.ntp[0] : (int)p.P;
    const int e = p.expert_ids ? p.expert_ids[blockIdx.y] : 0;
    const int64_t myrow = row0 + lane;   // lane l resolves padded row row0 + l (block_m <= 64)
    const bool in_blk = lane < p.block_m && myrow < p.P;
    const int sid = in_blk ? (p.sorted_ids ? p.sorted_ids[myrow] : (int)myrow) : -1;
    if (row0 >= ntp || row0 >= p.P) return;
    if (e < 0 || e >= p.E) return;
    int slot = -1, src = -1;
    if (in_blk && myrow < ntp && sid >= 0 && sid < p.num_valid) {
        slot = sid;
        src = p.identity ? (int)myrow : sid / p.top_k;
    }
    const uint64_t vmask = __ballot(src >= 0);
    const int mreal = __popcll(vmask);

    const int team = wave / KSPLIT;
    const int g0 = (wave % KSPLIT) * GPW;
    const int ncols = C::kSilu ? p.N / 2 : p.N;
    const int ntiles = (ncols + 15) / 16;
    const int kw_row = p.K / 8;
    const int t_begin = (blockIdx.x * C::TEAMS + team) * tpt;
    const int t_end = min(ntiles, t_begin + tpt);
    const int nsets = t_end > t_begin ? (t_end - t_begin + C::CT - 1) / C::CT : 0;
    const int nch = nsets * C::NB;
    // fragment layout: 16-row tiles of frag_tile_words(G) words (blocks, then metadata)
    const int32_t* we = p.w + (int64_t)e * (FRAG ? (int64_t)(p.N / 16) * frag_tile_words(p.G)
                                                 : (int64_t)p.N * kw_row);
    const __half* se = p.scales + (int64_t)e * p.N * p.G;
    const int32_t* ze = p.zeros ? p.zeros + (int64_t)e * (p.N / 8) * p.G : nullptr;
    constexpr float wscale = kNibbleScale;

    // weight row of fragment f, column c in the tile set starting at tile t (edge columns
    // read row 0: never stored, and the loads stay unconditional)
    auto row_of_col = [&](int t, int f, int c) -> int {
        const int tt = t + f % C::CT;
        const int col = tt * 16 + c;
        const bool up = C::kSilu && f >= C::CT;
        return (tt < t_end && col < ncols) ? (up ? col + ncols : col) : 0;
    };
    auto row_of = [&](int t, int f) -> int { return row_of_col(t, f, c16); };

    // Issues are unconditional: a chunk past the end (c >= nch) loads the expert's first
    // 16 bytes in every lane instead, so every step of the chunk loop has the same loads in
    // flight and the compiler's wait counts stay exact (a conditional issue makes it wait
    // for everything at the join). Word u * FR + f of a chunk = group u, fragment f,
    // quarter q of this lane's column.
    uint4 wv[2][C::GC * C::FR];
    uint32_t sw[2][C::kStagedSZ ? 1 : C::FR][C::GC];
    int32_t zw[2][C::kStagedSZ ? 1 : C::FR][C::GC];
    auto issue = [&](int c, auto bufc) {
        constexpr int b = decltype(bufc)::value;
        const bool live = c < nch;
        const int t = t_begin + (c / C::NB) * C::CT;
        const int g = live ? g0 + (c % C::NB) * C::GC : g0;
        // byte offsets: a wave-uniform part (group, step) on a scalar base plus a 32-bit lane
        // part (the expert's slice is < 2^31 bytes); past the end every lane reads offset 0
        constexpr uint32_t ustep = FRAG ? 1024u : kGroup / 2;
        const uint8_t* wg = reinterpret_cast<const uint8_t*>(we) + (uint32_t)g * ustep;
#pragma unroll
        for (int f = 0; f < C::FR; ++f) {
            const int n = live ? row_of(t, f) : 0;
            // op layout: row n, bytes 64 (g + u) + 16 q; fragment layout: block (n / 16, g + u)
            const uint32_t woff =
                !live ? 0u
                : FRAG ? (uint32_t)(n >> 4) * (uint32_t)frag_tile_words(p.G) * 4u + (uint32_t)lane * 16u
                       : (uint32_t)n * (uint32_t)(p.K / 2) + (uint32_t)q * 16u;
            // fragment layout: whole 128-byte lines per instruction, streamed (non-temporal,
            // read once per launch); op layout: 64-byte row pieces whose second half the
            // next instruction reads, so they stay cached
#pragma unroll
            for (int u = 0; u < C::GC; ++u) {
                const uint8_t* ptr = wg + (live ? u * ustep : 0u) + opaque_u32(woff);
                wv[b][u * C::FR + f] = FRAG ? load_stream16(ptr) : *reinterpret_cast<const uint4*>(ptr);
            }
            if constexpr (!C::kStagedSZ) {
                load_scales<C::GC>(reinterpret_cast<const __half*>(
                                       reinterpret_cast<const uint8_t*>(se) + (uint32_t)g * 2u +
                                       opaque_u32((uint32_t)n * (uint32_t)p.G * 2u)),
                                   sw[b][f]);
                // symmetric weights load (and ignore) scale words instead: same load count
                load_zero_words<C::GC>(
                    ze ? reinterpret_cast<const int32_t*>(reinterpret_cast<const uint8_t*>(ze) + (uint32_t)g * 4u +
                                                         opaque_u32((uint32_t)(n >> 3) * (uint32_t)p.G * 4u))
                       : reinterpret_cast<const int32_t*>(p.scales),
                    zw[b][f]);
            }
        }
    };
    using B0 = std::integral_constant<int, 0>;
    using B1 = std::integral_constant<int, 1>;

    // ---- level 2a (4-group chunks): every scale / zero-point word of the wave's chunks ----
    constexpr int kScEntries = C::kStagedSZ ? kGemvMaxTiles * C::FR * 16 : 1;
    constexpr int kZwEntries = C::kStagedSZ ? kGemvMaxTiles * C::FR * 2 : 1;
    uint2 sc_reg[(kScEntries + 63) / 64];
    uint4 zw_reg;
    if constexpr (C::kStagedSZ) {
#pragma unroll
        for (int i = 0; i < (kScEntries + 63) / 64; ++i) {
            const int en = i * 64 + lane;
            const int c = en / (C::FR * 16);
            const int f = (en / 16) % C::FR;
            const int n = c < nch ? row_of_col(t_begin + c * C::CT, f, en & 15) : 0;
            sc_reg[i] = *reinterpret_cast<const uint2*>(se + (int64_t)n * p.G + g0);
        }
        {
            const int en = min(lane, kZwEntries - 1);
            const int c = en / (C::FR * 2);
            const int f = (en / 2) % C::FR;
            const int n = c < nch ? row_of_col(t_begin + c * C::CT, f, (en & 1) * 8) : 0;
            zw_reg = *reinterpret_cast<const uint4*>(
                ze ? ze + (int64_t)(n >> 3) * p.G + g0 : reinterpret_cast<const int32_t*>(p.scales));
        }
    }

    for (int m0 = 0; m0 < mreal; m0 += 16) {
        if (m0 > 0) __syncthreads();   // LDS partials / row maxima of the previous pass consumed
        // A row m0 + c16 of this pass (pad rows repeat the last real row)
        const int asrc = __shfl(src, nth_set_bit(vmask, min(m0 + c16, mreal - 1)), 64);

        // ---- level 2: activation rows ----
        v8i af[GPW];
        float my_asc;
        if constexpr (!AQ) {
            const uint8_t* xr = p.xq + (int64_t)asrc * p.K + q * 32;
#pragma unroll
            for (int u = 0; u < GPW; ++u) {
                const uint4 lo = *reinterpret_cast<const uint4*>(xr + (g0 + u) * kGroup);
                const uint4 hi = *reinterpret_cast<const uint4*>(xr + (g0 + u) * kGroup + 16);
                af[u] = v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w,
                            (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
            }
            my_asc = p.asc[asrc];
            // ---- level 3: the first two weight chunks ----
            issue(0, B0{});
            issue(1, B1{});
        } else {
            // the first weight chunks (at eight groups a wave, the first chunk only) go out
            // with the raw rows; the wait for the rows then also covers them, as they were
            // issued just before
            issue(0, B0{});
            if constexpr (GPW <= 4) issue(1, B1{});
            const uint16_t* xr = reinterpret_cast<const uint16_t*>(p.xh) + (int64_t)asrc * p.K + q * 32;
            const bool bf16 = p.xbf16;
            uint4 raw[GPW][4];   // 32 values of group g0 + u: k = 8i .. 8i+7 in raw[u][i]
#pragma unroll
            for (int u = 0; u < GPW; ++u)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    raw[u][i] = reinterpret_cast<const uint4*>(xr + (g0 + u) * kGroup)[i];
            // absmax on the magnitude bits: both conversions are monotone in them, so the
            // max converts to the same value as the max of the converted values (NaNs,
            // which fmaxf skips, count as 0)
            const uint32_t nan_above = bf16 ? 0x7F80u : 0x7C00u;
            uint32_t mbits = 0;
#pragma unroll
            for (int u = 0; u < GPW; ++u)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const uint32_t w[4] = {raw[u][i].x, raw[u][i].y, raw[u][i].z, raw[u][i].w};
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const uint32_t lo = w[j] & 0x7FFFu, hi = (w[j] >> 16) & 0x7FFFu;
                        mbits = max(mbits, lo > nan_above ? 0u : lo);
                        mbits = max(mbits, hi > nan_above ? 0u : hi);
                    }
                }
            float amax = act_bits_to_f32(mbits, bf16);
            {   // the 4 quarter-lanes of each row: lanes l, l ^ 16, l ^ 32, l ^ 48
                const auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(amax), __float_as_uint(amax), false, false);
                amax = fmaxf(__uint_as_float(r16[0]), __uint_as_float(r16[1]));
                const auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(amax), __float_as_uint(amax), false, false);
                amax = fmaxf(__uint_as_float(r32[0]), __uint_as_float(r32[1]));
            }
            if constexpr (KSPLIT > 1) {
                if (q == 0) s_amax[wave][c16] = amax;
                lds_barrier();
#pragma unroll
                for (int j = 0; j < KSPLIT; ++j) amax = fmaxf(amax, s_amax[team * KSPLIT + j][c16]);
            }
            my_asc = act_scale_from_absmax(amax);
            const float inv = 1.0f / my_asc;
            // one branch on the dtype around the whole conversion: a select per value
            // becomes a uniform branch per value, and at eight groups a wave the values
            // live across those joins spill
            auto convert = [&](auto bfc) {
                constexpr bool BF = decltype(bfc)::value;
#pragma unroll
                for (int u = 0; u < GPW; ++u)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {   // k8-interleaved bytes, as act_quant_kernel
                        const uint32_t w[4] = {raw[u][i].x, raw[u][i].y, raw[u][i].z, raw[u][i].w};
                        float f[8];
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            f[2 * j] = half_bits_to_f32<BF>(w[j] & 0xFFFFu) * inv;
                            f[2 * j + 1] = half_bits_to_f32<BF>(w[j] >> 16) * inv;
                        }
                        af[u][2 * i] = (int)pack4_e4m3(f[0], f[2], f[4], f[6]);
                        af[u][2 * i + 1] = (int)pack4_e4m3(f[1], f[3], f[5], f[7]);
                    }
            };
            if (bf16) convert(std::true_type{});
            else convert(std::false_type{});
            // eight groups a wave: 128 VGPRs of rows leave no room for the second chunk
            // until they are converted
            if constexpr (GPW > 4) issue(1, B1{});
        }
        v4f sa[GPW];   // 2^-9 * group sums of rows 4q..4q+3
#pragma unroll
        for (int u = 0; u < GPW; ++u) {
            const int one = (int)kOnesE4m3;
            sa[u] = mfma_16x16x128(af[u], v8i{one, one, one, one, one, one, one, one},
                                   v4f{0.f, 0.f, 0.f, 0.f});
#pragma unroll
            for (int r = 0; r < 4; ++r) sa[u][r] *= 1.0f / kNibbleScale;
        }
        if constexpr (C::kStagedSZ) {
            // the staged words were loaded before the activation rows: in registers by now
            if (m0 == 0) {
#pragma unroll
                for (int i = 0; i < (kScEntries + 63) / 64; ++i) s_sc[wave][i * 64 + lane] = sc_reg[i];
                if (lane < kZwEntries) s_zw[wave][lane] = zw_reg;
            }
        }

        // per-wave table of this pass's 16 output rows (padded row, slot, scale), read back
        // at store time instead of being held in registers across the chunk loop
        if (q == 0) {
            const int j = nth_set_bit(vmask, min(m0 + c16, mreal - 1));
            s_opad[wave][c16] = (int)(row0 + j);
            s_oasc[wave][c16] = my_asc * wscale;
        }
        {
            const int j = nth_set_bit(vmask, min(m0 + c16, mreal - 1));
            const int sl = __shfl(slot, j, 64);   // all lanes active here
            if (q == 0) s_oslot[wave][c16] = sl;
        }
        auto store = [&](int r, int col, float ra, float rb) {
            const int mi = 4 * q + r;
            const int64_t opad = s_opad[wave][mi];
            const int oslot = s_oslot[wave][mi];
            const float a = s_oasc[wave][mi];
            if constexpr (EPI == Epi::kHalf) {
                reinterpret_cast<__half*>(p.out)[opad * p.N + col] = __float2half(as_f32(ra * a));
            } else if constexpr (EPI == Epi::kSiluHalf) {
                reinterpret_cast<__half*>(p.out)[opad * ncols + col] =
                    silu_mul_h(__float2half(as_f32(ra * a)), __float2half(as_f32(rb * a)));
            } else if constexpr (EPI == Epi::kScatter) {
                atomicAdd(reinterpret_cast<float*>(p.out) + (int64_t)(oslot / p.out_top_k) * p.N + col,
                          p.tw[oslot] * ra * a);
            } else {
                reinterpret_cast<float*>(p.out)[(int64_t)oslot * p.N + col] = ra * a;
            }
        };

        v4f run[C::FR];
#pragma unroll
        for (int f = 0; f < C::FR; ++f) run[f] = v4f{0.f, 0.f, 0.f, 0.f};

        auto consume = [&](int c, auto bufc) {
            constexpr int b = decltype(bufc)::value;
            constexpr int gb = C::NB == 2 ? b : 0;   // chunk parity == group batch when NB == 2
            const int t = t_begin + (c / C::NB) * C::CT;
#pragma unroll
            for (int f = 0; f < C::FR; ++f) {
                const int zsh = (row_of(t, f) & 7) * 4;
                uint32_t scw[C::GC];
                int32_t zwd[C::GC];
                if constexpr (C::kStagedSZ) {
                    const uint2 sv = s_sc[wave][(c * C::FR + f) * 16 + c16];
                    const uint4 zv = s_zw[wave][(c * C::FR + f) * 2 + (c16 >> 3)];
                    scw[0] = sv.x;
                    scw[1] = sv.y;
                    zwd[0] = (int32_t)zv.x;
                    zwd[1] = (int32_t)zv.y;
                    zwd[2] = (int32_t)zv.z;
                    zwd[3] = (int32_t)zv.w;
                } else {
#pragma unroll
                    for (int u = 0; u < C::GC; ++u) {
                        scw[u] = sw[b][f][u];
                        zwd[u] = zw[b][f][u];
                    }
                }
#pragma unroll
                for (int u = 0; u < C::GC; ++u) {
                    const int ua = gb * C::GC + u;
                    v4f acc = mfma_16x16x128(af[ua], spread_nibbles(wv[b][u * C::FR + f]),
                                             v4f{0.f, 0.f, 0.f, 0.f});
                    const float z = ze ? (float)((zwd[u] >> zsh) & 0xF) : 8.0f;
#pragma unroll
                    for (int r = 0; r < 4; ++r) acc[r] = fmaf(-z, sa[ua][r], acc[r]);
                    const float s = scale_at<C::GC>(scw, u);
#pragma unroll
                    for (int r = 0; r < 4; ++r) run[f][r] = fmaf(acc[r], s, run[f][r]);
                }
            }
            if (c % C::NB != C::NB - 1) return;
            // tile set complete
#pragma unroll
            for (int ct = 0; ct < C::CT; ++ct) {
                const int tt = t + ct;
                if (tt >= t_end) continue;
                if constexpr (KSPLIT > 1) {
#pragma unroll
                    for (int nf = 0; nf < C::NF; ++nf)
                        s_part[((wave * tpt + (tt - t_begin)) * C::NF + nf) * 64 + lane] =
                            run[nf * C::CT + ct];
                } else {
                    const int col = tt * 16 + c16;
                    if (col < ncols) {
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            if (m0 + 4 * q + r >= mreal) continue;
                            store(r, col, run[ct][r], C::kSilu ? run[C::CT + ct][r] : 0.f);
                        }
                    }
                }
            }
#pragma unroll
            for (int f = 0; f < C::FR; ++f) run[f] = v4f{0.f, 0.f, 0.f, 0.f};
        };

        for (int c = 0; c < nch; c += 2) {
            consume(c, B0{});
            issue(c + 2, B0{});
            if (c + 1 < nch) consume(c + 1, B1{});
            issue(c + 3, B1{});
        }

        if constexpr (KSPLIT > 1) {
            __syncthreads();
            // sum the KSPLIT partials of every (team, tile, lane) in wave order, then store;
            // i & 63 == lane, so the rows and scales are this lane's own
            const int items = C::TEAMS * tpt * 64;
            for (int i = tid; i < items; i += 256) {
                const int tm = i / (tpt * 64);
                const int tl = (i >> 6) % tpt;
                const int tt = (blockIdx.x * C::TEAMS + tm) * tpt + tl;
                const int col = tt * 16 + c16;
                if (tt >= ntiles || col >= ncols) continue;
                v4f sum[C::NF];
#pragma unroll
                for (int nf = 0; nf < C::NF; ++nf) {
                    sum[nf] = s_part[(((tm * KSPLIT) * tpt + tl) * C::NF + nf) * 64 + lane];
#pragma unroll
                    for (int j = 1; j < KSPLIT; ++j) {
                        const v4f v = s_part[(((tm * KSPLIT + j) * tpt + tl) * C::NF + nf) * 64 + lane];
#pragma unroll
                        for (int r = 0; r < 4; ++r) sum[nf][r] += v[r];
                    }
                }
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    if (m0 + 4 * q + r >= mreal) continue;
                    store(r, col, sum[0][r], C::kSilu ? sum[C::NF - 1][r] : 0.f);
                }
            }
        }
    }
}

template <Epi EPI>
int launch_scalar_t(const Params& p, hipStream_t s) {
    const int ncols = EPI == Epi::kSiluHalf ? p.N / 2 : p.N;
    dim3 grid((unsigned)((ncols + 63) / 64), (unsigned)((p.P + 3) / 4));
    grouped_scalar_kernel<EPI><<<grid, dim3(64, 4), 0, s>>>(p);
    return check_launch("grouped_scalar_kernel");
}

template <Epi EPI, int BM, int BN, bool FP4>
int launch_mfma_t(const Params& p, hipStream_t s) {
    using C = TileCfg<EPI, BM, BN>;
    // > 64 KB dynamic LDS needs an explicit opt-in
    if (int rc = reserve_dyn_lds(reinterpret_cast<const void*>(&grouped_mfma_kernel<EPI, BM, BN, FP4>),
                                 C::LDS_BYTES, "grouped_mfma_kernel"))
        return rc;
    const int ncols = EPI == Epi::kSiluHalf ? p.N / 2 : p.N;
    dim3 grid((unsigned)((ncols + BN - 1) / BN), (unsigned)((p.P + BM - 1) / BM));
    grouped_mfma_kernel<EPI, BM, BN, FP4><<<grid, 256, C::LDS_BYTES, s>>>(p);
    return check_launch("grouped_mfma_kernel");
}

// The work-group tile height must divide block_m so every tile lies in one expert block.
template <Epi EPI>
int launch_mfma_b(const Params& p, hipStream_t s) {
    if (p.e2m1) {
        if (p.block_m % 128 == 0) return launch_mfma_t<EPI, 128, 64, true>(p, s);
        if (p.block_m % 64 == 0) return launch_mfma_t<EPI, 64, 64, true>(p, s);
        if (p.block_m % 32 == 0) return launch_mfma_t<EPI, 32, 64, true>(p, s);
        if (p.block_m % 16 == 0) return launch_mfma_t<EPI, 16, 64, true>(p, s);
    } else {
        if (p.block_m % 128 == 0) return launch_mfma_t<EPI, 128, 64, false>(p, s);
        if (p.block_m % 64 == 0) return launch_mfma_t<EPI, 64, 64, false>(p, s);
        if (p.block_m % 32 == 0) return launch_mfma_t<EPI, 32, 64, false>(p, s);
        if (p.block_m % 16 == 0) return launch_mfma_t<EPI, 16, 64, false>(p, s);
    }
    set_error("wmma grouped GEMM: block_m must be a multiple of 16");
    return W4A8_ERR_INVALID;
}
template <Epi EPI>
int launch_mfma_e(const Params& p, hipStream_t s) {
    return launch_mfma_b<EPI>(p, s);
}

// Split of the K groups over waves: G == GPW * KSPLIT for the shapes below; others run
// the matrix-core tiles.
struct GemvSplit {
    int gpw, ksplit;
};
GemvSplit gemv_split(int G) {
    switch (G) {
        case 1: return {1, 1};
        case 2: return {2, 1};
        case 3: return {3, 1};
        case 4: return {4, 1};
        case 6: return {3, 2};
        case 8: return {4, 2};
        case 12: return {3, 4};
        case 16: return {4, 4};
        case 32: return {8, 4};
        default: return {0, 0};
    }
}

// Column tiles per wave team: enough work per work-group to hide the prologue (~64 KB of
// weights per wave), fewer when the grid would otherwise leave CUs idle (two work-groups
// per CU fit; 512 keeps every CU of a 256-CU part busy).
int gemv_default_tpt(const Params& p, int ntiles, int frag_bytes_per_tile_wave, int teams) {
    const int64_t blocks = std::min<int64_t>((p.P + p.block_m - 1) / p.block_m, p.num_valid);
    int tpt = std::max(1, (64 * 1024) / frag_bytes_per_tile_wave);
    tpt = std::min(tpt, kGemvMaxTiles);
    // keep >= ~512 work-groups when the routing touches few blocks (T = 1 decode)
    while (tpt > 1 && blocks * ((ntiles + teams * tpt - 1) / (teams * tpt)) < 512) tpt >>= 1;
    return tpt;
}

template <Epi EPI, int GPW, int KSPLIT, bool AQ, bool FRAG>
int launch_gemv_a(const Params& p, int tpt, dim3 grid, size_t lds, hipStream_t s) {
    using C = GemvCfg<EPI, GPW, KSPLIT>;
    if (int rc = reserve_dyn_lds(reinterpret_cast<const void*>(&grouped_gemv_kernel<EPI, GPW, KSPLIT, AQ, FRAG>),
                                 4 * kGemvMaxTiles * C::NF * 64 * (int)sizeof(v4f),
                                 "grouped_gemv_kernel"))
        return rc;
    launch_kernel(&grouped_gemv_kernel<EPI, GPW, KSPLIT, AQ, FRAG>, grid, dim3(256), lds, s, p, tpt);
    return check_launch("grouped_gemv_kernel");
}

template <Epi EPI, int GPW, int KSPLIT>
int launch_gemv_t(const Params& p, int tpt, hipStream_t s) {
    using C = GemvCfg<EPI, GPW, KSPLIT>;
    const int ncols = C::kSilu ? p.N / 2 : p.N;
    const int ntiles = (ncols + 15) / 16;
    if (tpt <= 0) tpt = gemv_default_tpt(p, ntiles, GPW * C::NF * 1024, C::TEAMS);
    tpt = std::min(tpt, kGemvMaxTiles);
    const size_t lds = KSPLIT > 1 ? (size_t)4 * tpt * C::NF * 64 * sizeof(v4f) : 0;
    const dim3 grid((unsigned)((ntiles + C::TEAMS * tpt - 1) / (C::TEAMS * tpt)),
                    (unsigned)((p.P + p.block_m - 1) / p.block_m));
    if (p.w_frag) {
        // fragment-layout weights come only with prequantised rows (the whole-layer path)
        if (!p.xq) {
            set_error("grouped GEMV: fragment-layout weights need prequantised activations");
            return W4A8_ERR_INVALID;
        }
        return launch_gemv_a<EPI, GPW, KSPLIT, false, true>(p, tpt, grid, lds, s);
    }
    if (p.xq) return launch_gemv_a<EPI, GPW, KSPLIT, false, false>(p, tpt, grid, lds, s);
    return launch_gemv_a<EPI, GPW, KSPLIT, true, false>(p, tpt, grid, lds, s);
}

template <Epi EPI>
int launch_gemv_e(const Params& p, int tpt, hipStream_t s) {
    const GemvSplit sp = gemv_split(p.G);
    switch (sp.gpw * 8 + sp.ksplit) {
        case 1 * 8 + 1: return launch_gemv_t<EPI, 1, 1>(p, tpt, s);
        case 2 * 8 + 1: return launch_gemv_t<EPI, 2, 1>(p, tpt, s);
        case 3 * 8 + 1: return launch_gemv_t<EPI, 3, 1>(p, tpt, s);
        case 3 * 8 + 2: return launch_gemv_t<EPI, 3, 2>(p, tpt, s);
        case 4 * 8 + 1: return launch_gemv_t<EPI, 4, 1>(p, tpt, s);
        case 4 * 8 + 2: return launch_gemv_t<EPI, 4, 2>(p, tpt, s);
        case 3 * 8 + 4: return launch_gemv_t<EPI, 3, 4>(p, tpt, s);
        case 4 * 8 + 4: return launch_gemv_t<EPI, 4, 4>(p, tpt, s);
        case 8 * 8 + 4: return launch_gemv_t<EPI, 8, 4>(p, tpt, s);
    }
    set_error("gemv grouped GEMM: unsupported number of K groups");
    return W4A8_ERR_INVALID;
}

}  // namespace

bool gemv_supported(int64_t K, int64_t group_size) {
    return mfma_supported(K, group_size) && gemv_split((int)(K / group_size)).gpw > 0;
}

bool mfma_supported(int64_t K, int64_t group_size, bool e2m1) {
    // E2M1 runs fp4 operands with one MFMA per group of 32, 64 or 128; K a multiple of the
    // group (the last 128-wide K step may be partial: gpt-oss's 2880)
    if (e2m1) return (group_size == 32 || group_size == 64 || group_size == kGroup) && K % group_size == 0;
    return group_size == kGroup && K % kGroup == 0;
}

int launch_grouped_scalar(const GroupedArgs& a, hipStream_t s) {
    const Params p = make_params(a);
    if (p.P == 0) return W4A8_OK;
    if (a.w_frag) {
        set_error("scalar grouped GEMM reads op-layout weights only");
        return W4A8_ERR_INVALID;
    }
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
    if (a.w_frag) {
        set_error("mfma grouped GEMM reads op-layout weights only");
        return W4A8_ERR_INVALID;
    }
    switch (a.epi) {
        case Epi::kHalf: return launch_mfma_e<Epi::kHalf>(p, s);
        case Epi::kSiluHalf: return launch_mfma_e<Epi::kSiluHalf>(p, s);
        case Epi::kScatter: return launch_mfma_e<Epi::kScatter>(p, s);
        case Epi::kSlotF32: return launch_mfma_e<Epi::kSlotF32>(p, s);
    }
    return W4A8_ERR_INVALID;
}

int launch_grouped_gemv_tpt(const GroupedArgs& a, int tpt, hipStream_t s) {
    const Params p = make_params(a);
    if (p.P == 0) return W4A8_OK;
    if (p.block_m > kGemvMaxRows) {
        set_error("gemv grouped GEMM: block_m must be <= 64");
        return W4A8_ERR_INVALID;
    }
    if (!gemv_supported(a.K, a.group_size)) {
        set_error("gemv grouped GEMM: K / group_size must be one of 1,2,3,4,6,8,12,16,32");
        return W4A8_ERR_INVALID;
    }
    if (a.e2m1) {
        set_error("gemv grouped GEMM: E2M1 weights run on the matrix-core tiles");
        return W4A8_ERR_INVALID;
    }
    if (a.w_frag && (a.N % 16 != 0 || (a.epi == Epi::kSiluHalf && (a.N / 2) % 16 != 0))) {
        set_error("gemv grouped GEMM: fragment-layout weights need 16-row aligned halves");
        return W4A8_ERR_INVALID;
    }
    switch (a.epi) {
        case Epi::kHalf: return launch_gemv_e<Epi::kHalf>(p, tpt, s);
        case Epi::kSiluHalf: return launch_gemv_e<Epi::kSiluHalf>(p, tpt, s);
        case Epi::kScatter: return launch_gemv_e<Epi::kScatter>(p, tpt, s);
        case Epi::kSlotF32: return launch_gemv_e<Epi::kSlotF32>(p, tpt, s);
    }
    return W4A8_ERR_INVALID;
}

int launch_grouped_gemv(const GroupedArgs& a, hipStream_t s) {
    return launch_grouped_gemv_tpt(a, 0, s);
}

}  // namespace w4a8
