// Prefill grouped W4A8 GEMM on the gfx950 fp8 matrix cores.
//
// Replaces the reference's tiled WMMA grouped GEMM (moe_gemm_tiled.h:29-350, dispatched at
// moe_kernel.hip:1110-1155) for the many-token regime. Arithmetic contract as in
// w4a8_common.h; the schedule is this file's own:
//
//   * a work-group owns BM = 16*MT consecutive rows of one align block and 256 weight rows
//     (4 waves x 4 16-column fragments; SiLU: 128 gate + the matching 128 up columns);
//   * per 128-wide K group the block's e4m3 activation rows are staged once in LDS
//     (double-buffered, one barrier per group) and every wave reads its A fragments there;
//   * B never touches LDS: each wave loads its own int4 words straight into registers as
//     MFMA B fragments (next group in flight) and spreads the nibbles into e4m3 bytes
//     n * 2^-9 with two ANDs and a shift (the raw-nibble operand of the decode GEMV);
//   * per group: v_mfma_f32_16x16x128_f8f6f4 per (A, B) fragment pair, then the fp32 scale
//     fold run += acc * scale[n, g] (moe_gemm_tiled.h:144-151);
//   * the zero-point term sum_g s[n,g] z[n,g] sum_k a[m,k] leaves the K loop entirely: after
//     it, two bf16 MFMAs per fragment (16x16x32, K = 16 groups x {hi, lo} halves of the
//     row group sums against hi / lo halves of s*z) form it with ~16-bit operands, and
//     out = act_scale * (512 * run - zero_term);
//   * 16-row fragments past the block's last real row are skipped (the prefill align uses
//     block_m = 128, so the skipped MFMAs are the padding the align adds).
#include <algorithm>
#include <type_traits>

#include "grouped_params.h"

namespace w4a8 {
namespace {

constexpr int kPfWaves = 4;
constexpr int kPfNT = 4;                          // 16-column B fragments per wave
constexpr int kPfBN = kPfWaves * kPfNT * 16;      // 256 weight rows per work-group
constexpr int kPfAStride = kGroup + 16;           // LDS bytes per staged activation row
constexpr int kPfMaxGroups = 32;                  // zero-point term: two 16-group passes

using bf16x8 = __bf16 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ v4f mfma_bf16_16x16x32(const bf16x8& a, const bf16x8& b,
                                                  const v4f& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float half_bits(uint32_t h) {
    return __half2float(__ushort_as_half(static_cast<unsigned short>(h)));
}

// Work-group order: item = n_tile * live_blocks + m_block, so the m-blocks of one expert
// and one weight slice run back to back and share the slice in L2. (Dealing contiguous
// item ranges to each XCD measured slower: empty and full blocks do not balance.)
__device__ __forceinline__ bool prefill_item(int nblocks, int ntiles, int& m_block, int& n_tile) {
    // only blocks below num_tokens_post_padded hold rows
    const int lambda = blockIdx.x;
    if (lambda >= nblocks * ntiles) return false;
    n_tile = lambda / nblocks;
    m_block = lambda % nblocks;
    return true;
}

// Loads take a wave-uniform base plus a 32-bit per-lane byte offset (opaque_u32), so they
// issue in the scalar-base form (one offset register per load, no 64-bit address arithmetic
// per lane).
template <int A_CHUNKS>
__device__ __forceinline__ void pf_load_a(u32x4 (&reg)[A_CHUNKS], const uint8_t* __restrict__ xq,
                                          const uint32_t (&src)[A_CHUNKS], int gg) {
    const uint8_t* base = xq + (uint32_t)gg * kGroup;
#pragma unroll
    for (int i = 0; i < A_CHUNKS; ++i) reg[i] = *reinterpret_cast<const u32x4*>(base + opaque_u32(src[i]));
}
template <int A_CHUNKS>
__device__ __forceinline__ void pf_store_a(const u32x4 (&reg)[A_CHUNKS], uint8_t* dst,
                                           const int (&off)[A_CHUNKS]) {
#pragma unroll
    for (int i = 0; i < A_CHUNKS; ++i) *reinterpret_cast<u32x4*>(dst + off[i]) = reg[i];
}
// B fragments of group gg: weight bytes at wb + gg * gstep + woff[j] (fragment layout:
// lane l's 16 bytes of block (row / 16, group) at ((row / 16) * G + group) * 1 KB + 16 l, so
// gstep = 1 KB; op layout: row * K / 2 + 64 group + 16 q, gstep = 64), the fp16 scale at
// sb + 2 gg + soff[j] (soff = 2 row G).
__device__ __forceinline__ void pf_load_b(uint4 (&w)[kPfNT], uint32_t (&sc)[kPfNT],
                                          const uint8_t* __restrict__ wb, uint32_t gstep,
                                          const uint32_t (&woff)[kPfNT], const uint8_t* __restrict__ sb,
                                          const uint32_t (&soff)[kPfNT], int gg) {
    const uint8_t* wg = wb + (uint32_t)gg * gstep;
    const uint8_t* sg = sb + (uint32_t)gg * 2u;
#pragma unroll
    for (int j = 0; j < kPfNT; ++j) {
        w[j] = *reinterpret_cast<const uint4*>(wg + opaque_u32(woff[j]));
        sc[j] = *reinterpret_cast<const uint16_t*>(sg + opaque_u32(soff[j]));
    }
}

// Dynamic LDS layout (bytes) for a tile of BM rows and Gp = G rounded up to 16 groups.
struct PfLds {
    int a, szh, szl, sah, sal, total;
    __host__ __device__ PfLds(int BM, int Gp) {
        a = 0;                                  // 2 x BM x kPfAStride e4m3 activation tiles
        szh = 2 * BM * kPfAStride;              // kPfBN x Gp bf16: hi half of s[n,g] * z[n,g]
        szl = szh + kPfBN * Gp * 2;             // ... lo half
        sah = szl + kPfBN * Gp * 2;             // BM x Gp bf16: hi half of the row group sums
        sal = sah + BM * Gp * 2;                // ... lo half
        total = sal + BM * Gp * 2;
    }
};

template <Epi EPI, int MT, bool FRAG>
__global__ void __launch_bounds__(256, 1) prefill_mfma_kernel(Params p, int nblocks, int ntiles) {
    constexpr bool kSilu = EPI == Epi::kSiluHalf;
    constexpr int BM = 16 * MT;
    constexpr int A_CHUNKS = (BM * 8 + 255) / 256;   // 16-B pieces of the A tile per thread
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    __shared__ int s_src[BM];
    __shared__ int s_slot[BM];
    __shared__ int s_maxrow;

    const int ntp = p.ntp ? p.ntp[0] : (int)p.P;
    int m_block, n_tile;
    const int live_blocks = min(nblocks, (int)((min((int64_t)ntp, p.P) + BM - 1) / BM));
    if (!prefill_item(live_blocks, ntiles, m_block, n_tile)) return;
    const int64_t row0 = (int64_t)m_block * BM;
    if (row0 >= ntp || row0 >= p.P) return;
    // wave-uniform in a scalar register, so weight addresses are a scalar base + lane offset
    const int e = __builtin_amdgcn_readfirstlane(p.expert_ids ? p.expert_ids[row0 / p.block_m] : 0);
    if (e < 0 || e >= p.E) return;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int q = lane >> 4;
    const int c16 = lane & 15;
    const int ncols = kSilu ? p.N / 2 : p.N;
    const int kw_row = p.K / 8;
    const int G = p.G;
    const int Gp = (G + 15) / 16 * 16;
    const PfLds L(BM, Gp);
    uint8_t* s_a = lds + L.a;
    __bf16* s_szh = reinterpret_cast<__bf16*>(lds + L.szh);
    __bf16* s_szl = reinterpret_cast<__bf16*>(lds + L.szl);
    __bf16* s_sah = reinterpret_cast<__bf16*>(lds + L.sah);
    __bf16* s_sal = reinterpret_cast<__bf16*>(lds + L.sal);

    if (tid == 0) s_maxrow = -1;
    __syncthreads();
    if (tid < BM) {
        int slot;
        const int src = resolve_row(p, row0 + tid, ntp, slot);
        s_src[tid] = src;
        s_slot[tid] = slot;
        if (src >= 0) atomicMax(&s_maxrow, tid);
    }
    __syncthreads();
    const int maxrow = __builtin_amdgcn_readfirstlane(s_maxrow);
    if (maxrow < 0) return;                       // uniform: no real row in this tile
    const int nfl = maxrow / 16 + 1;              // live 16-row fragments
    const int fallback_src = s_src[maxrow];       // a real row: padding rows read it

    // ---- B fragments of this wave ----
    // SiLU: fragments 0,1 = gate columns col0 + {0..15, 16..31}, 2,3 = the same up columns.
    // fragment layout: 16-row tiles of frag_tile_words(G) words (blocks, then metadata)
    const int32_t* we = p.w + (int64_t)e * (FRAG ? (int64_t)(p.N / 16) * frag_tile_words(G)
                                                 : (int64_t)p.N * kw_row);
    const __half* se = p.scales + (int64_t)e * p.N * G;
    const int32_t* ze = p.zeros ? p.zeros + (int64_t)e * (p.N / 8) * G : nullptr;
    auto weight_row = [&](int wv_, int j, int c, int& col) {
        const int col0 = n_tile * (kSilu ? kPfBN / 2 : kPfBN) + wv_ * (kSilu ? 32 : 64);
        col = kSilu ? col0 + 16 * (j & 1) + c : col0 + 16 * j + c;
        const int n = kSilu && j >= 2 ? col + ncols : col;
        return col < ncols ? n : 0;               // edge columns read row 0, never stored
    };
    int wrow[kPfNT];
    int ocol[kPfNT];
#pragma unroll
    for (int j = 0; j < kPfNT; ++j) wrow[j] = weight_row(wave, j, c16, ocol[j]);

    // ---- zero-point operands to LDS (once per work-group) ----
    // All loads of a 16-group pass are issued before any is used (clamped addresses, no
    // branches), so the fill costs one memory latency per pass, not one per group.
    {
        int col_unused;
        const int lr = tid;                       // local weight row 64*wave' + 16*j' + c'
        const int n = weight_row(lr >> 6, (lr >> 4) & 3, lr & 15, col_unused);
        const uint16_t* srow = reinterpret_cast<const uint16_t*>(se) + (int64_t)n * G;
        const int32_t* zrow = ze ? ze + (int64_t)(n >> 3) * G : nullptr;
        const int zsh = (n & 7) * 4;
        for (int g0 = 0; g0 < Gp; g0 += 16) {
            uint32_t sc[16];
            int32_t zw[16];
#pragma unroll
            for (int t = 0; t < 16; ++t) {
                const int g = min(g0 + t, G - 1);
                sc[t] = srow[g];
                zw[t] = zrow ? zrow[g] : 0;
            }
#pragma unroll
            for (int t = 0; t < 16; ++t) {
                const int z = zrow ? (zw[t] >> zsh) & 0xF : 8;
                const float sz = g0 + t < G ? half_bits(sc[t]) * (float)z : 0.f;   // exact
                const __bf16 h = (__bf16)sz;
                s_szh[lr * Gp + g0 + t] = h;
                s_szl[lr * Gp + g0 + t] = (__bf16)(sz - (float)h);
            }
        }
        // row group sums: BM x Gp entries, MT * Gp / 16 per thread
        constexpr int kSaPerThread = BM * kPfMaxGroups / 256;
        float sav[kSaPerThread];
#pragma unroll
        for (int u = 0; u < kSaPerThread; ++u) {
            const int i = tid + u * 256;
            const int r = min(i / Gp, BM - 1), g = min(i % Gp, G - 1);
            const int src = s_src[r] >= 0 ? s_src[r] : fallback_src;
            sav[u] = p.asum[(int64_t)src * G + g];
        }
#pragma unroll
        for (int u = 0; u < kSaPerThread; ++u) {
            const int i = tid + u * 256;
            if (i >= BM * Gp) break;
            const float v = i % Gp < G ? sav[u] : 0.f;
            const __bf16 h = (__bf16)v;
            s_sah[i] = h;
            s_sal[i] = (__bf16)(v - (float)h);
        }
    }

    // ---- A staging: piece c -> row c/8, bytes (c%8)*16 of the group's 128 ----
    // (byte offsets into x_fp8 fit 32 bits: rows * K < 2^31 is checked on the host)
    uint32_t a_src[A_CHUNKS];
    int a_dst[A_CHUNKS];
#pragma unroll
    for (int i = 0; i < A_CHUNKS; ++i) {
        const int c = min(tid + i * 256, BM * 8 - 1);    // BM = 16 keeps threads >= 128 on the last piece
        const int r = c >> 3;
        const int src = s_src[r] >= 0 ? s_src[r] : fallback_src;
        a_src[i] = (uint32_t)src * (uint32_t)p.K + (uint32_t)(c & 7) * 16u;
        a_dst[i] = r * kPfAStride + (c & 7) * 16;
    }

    v4f run[MT][kPfNT];
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < kPfNT; ++j) run[i][j] = v4f{0.f, 0.f, 0.f, 0.f};

    // Two groups in flight: A(g+2) and B(g+2) are requested while group g computes; A(g+1)
    // goes from registers to the LDS ring (3 slots) at the end of group g. Register sets
    // alternate with the group parity (compile-time indices: the loop is unrolled by 2).
    uint4 wv0[kPfNT], wv1[kPfNT];
    uint32_t sv0[kPfNT], sv1[kPfNT];
    // per-lane byte offsets of the B fragments and scales (an expert's slice is < 2^31 bytes)
    const uint8_t* wb = reinterpret_cast<const uint8_t*>(we);
    const uint8_t* sb = reinterpret_cast<const uint8_t*>(se);
    const uint32_t gstep = FRAG ? 1024u : (uint32_t)kGroup / 2;
    uint32_t woff[kPfNT], soff[kPfNT];
#pragma unroll
    for (int j = 0; j < kPfNT; ++j) {
        woff[j] = FRAG ? (uint32_t)(wrow[j] >> 4) * (uint32_t)frag_tile_words(G) * 4u + (uint32_t)lane * 16u
                       : (uint32_t)wrow[j] * (uint32_t)(p.K / 2) + (uint32_t)q * 16u;
        soff[j] = (uint32_t)wrow[j] * (uint32_t)G * 2u;
    }
    // one group of MFMAs on LDS slot g & 1 with spread B fragments bf and scales s
    auto mma = [&](const v8i (&bf)[kPfNT], const float (&s)[kPfNT], int g) {
        const uint8_t* A = s_a + (g & 1) * (BM * kPfAStride) + c16 * kPfAStride + q * 32;
#pragma unroll
        for (int i = 0; i < MT; ++i) {
            if (i >= nfl) break;                   // uniform: past the last real row
            const uint4 lo = *reinterpret_cast<const uint4*>(A + i * 16 * kPfAStride);
            const uint4 hi = *reinterpret_cast<const uint4*>(A + i * 16 * kPfAStride + 16);
            const v8i af = v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w,
                               (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
#pragma unroll
            for (int j = 0; j < kPfNT; ++j) {
                const v4f acc = mfma_16x16x128(af, bf[j], v4f{0.f, 0.f, 0.f, 0.f});
#pragma unroll
                for (int r = 0; r < 4; ++r) run[i][j][r] = fmaf(acc[r], s[j], run[i][j][r]);
            }
        }
    };
    auto slot = [&](int g) { return s_a + (g & 1) * (BM * kPfAStride); };
    const int Gl = G - 1;   // loads past the end re-read the last group (never consumed)

    // B runs two groups ahead in two register sets (alternating with the group parity; the
    // loop is unrolled by 2); A runs one group ahead: A(g+1) is requested at the top of
    // group g and lands in the other LDS slot at its end.
    pf_load_b(wv0, sv0, wb, gstep, woff, sb, soff, 0);
    pf_load_b(wv1, sv1, wb, gstep, woff, sb, soff, min(1, Gl));
    {
        u32x4 a_reg[A_CHUNKS];
        pf_load_a(a_reg, p.xq, a_src, 0);
        pf_store_a(a_reg, slot(0), a_dst);
    }
    __syncthreads();
    for (int g = 0; g < G; g += 2) {
        {
            u32x4 a_reg[A_CHUNKS];
            pf_load_a(a_reg, p.xq, a_src, min(g + 1, Gl));
            v8i bf[kPfNT];
            float sc[kPfNT];
#pragma unroll
            for (int j = 0; j < kPfNT; ++j) { bf[j] = spread_nibbles(wv0[j]); sc[j] = half_bits(sv0[j]); }
            pf_load_b(wv0, sv0, wb, gstep, woff, sb, soff, min(g + 2, Gl));
            mma(bf, sc, g);
            pf_store_a(a_reg, slot(g + 1), a_dst);
            lds_barrier();
        }
        {
            // unconditional (a branch here makes the compiler index the two register sets
            // dynamically through scratch): with odd G the extra half re-reads the last
            // group and folds it with scale 0, which adds exactly nothing to finite sums
            const float live = g + 1 < G ? 1.0f : 0.0f;
            u32x4 a_reg[A_CHUNKS];
            pf_load_a(a_reg, p.xq, a_src, min(g + 2, Gl));
            v8i bf[kPfNT];
            float sc[kPfNT];
#pragma unroll
            for (int j = 0; j < kPfNT; ++j) { bf[j] = spread_nibbles(wv1[j]); sc[j] = half_bits(sv1[j]) * live; }
            pf_load_b(wv1, sv1, wb, gstep, woff, sb, soff, min(g + 3, Gl));
            mma(bf, sc, g + 1);
            pf_store_a(a_reg, slot(g + 2), a_dst);
            lds_barrier();
        }
    }

    // ---- zero-point term and epilogue ----
    // bf16 MFMA operands from LDS, lane (q, c16), K slot 8q + t (t < 8) <-> group
    // 16*pass + 8*(q & 1) + t:
    //   A (rows): hi (q < 2) or lo (q >= 2) bf16 half of the row's group sum;
    //   B (columns): hi (first MFMA) or lo (second) half of s[n,g] * z[n,g], slots 16..31
    //   repeating 0..15, so the two MFMAs add (sa_hi + sa_lo) * (sz_hi + sz_lo).
    const int npass = Gp / 16;
    auto store = [&](int m, int col, float va, float vb) {
        const int64_t row_pad = row0 + m;
        const int slot = s_slot[m];
        if constexpr (EPI == Epi::kHalf) {
            reinterpret_cast<__half*>(p.out)[row_pad * p.N + col] = __float2half(va);
        } else if constexpr (EPI == Epi::kSiluHalf) {
            reinterpret_cast<__half*>(p.out)[row_pad * ncols + col] =
                silu_mul_h(__float2half(va), __float2half(vb));
        } else if constexpr (EPI == Epi::kScatter) {
            atomicAdd(reinterpret_cast<float*>(p.out) + (int64_t)(slot / p.out_top_k) * p.N + col,
                      p.tw[slot] * va);
        } else {
            reinterpret_cast<float*>(p.out)[(int64_t)slot * p.N + col] = va;
        }
    };
    auto lds8 = [](const __bf16* ptr) {
        const uint4 v = *reinterpret_cast<const uint4*>(ptr);
        bf16x8 r;
        __builtin_memcpy(&r, &v, 16);
        return r;
    };

    // fragments are finished in pairs (SiLU: gate j with up j + 2; otherwise j, j + 1)
#pragma unroll
    for (int jp = 0; jp < 2; ++jp) {
        const int ja = kSilu ? jp : 2 * jp;
        const int jb = kSilu ? jp + 2 : 2 * jp + 1;
        const int lra = 64 * wave + 16 * ja + c16, lrb = 64 * wave + 16 * jb + c16;
#pragma unroll
        for (int i = 0; i < MT; ++i) {
            if (i >= nfl) break;
            v4f za = v4f{0.f, 0.f, 0.f, 0.f}, zb = v4f{0.f, 0.f, 0.f, 0.f};
            const __bf16* sa_tab = q < 2 ? s_sah : s_sal;
            for (int ps = 0; ps < npass; ++ps) {
                const int go = 16 * ps + 8 * (q & 1);
                const bf16x8 sa = lds8(sa_tab + (16 * i + c16) * Gp + go);
                za = mfma_bf16_16x16x32(sa, lds8(s_szh + lra * Gp + go), za);
                za = mfma_bf16_16x16x32(sa, lds8(s_szl + lra * Gp + go), za);
                zb = mfma_bf16_16x16x32(sa, lds8(s_szh + lrb * Gp + go), zb);
                zb = mfma_bf16_16x16x32(sa, lds8(s_szl + lrb * Gp + go), zb);
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = 16 * i + 4 * q + r;
                if (m > maxrow) continue;
                const int src = s_src[m];
                if (src < 0) continue;
                const float a = p.asc[src];
                const float va = as_f32(a * (kNibbleScale * run[i][ja][r] - za[r]));
                const float vb = as_f32(a * (kNibbleScale * run[i][jb][r] - zb[r]));
                if constexpr (kSilu) {
                    if (ocol[ja] < ncols) store(m, ocol[ja], va, vb);
                } else {
                    if (ocol[ja] < ncols) store(m, ocol[ja], va, 0.f);
                    if (ocol[jb] < ncols) store(m, ocol[jb], vb, 0.f);
                }
            }
        }
    }
}

template <Epi EPI, int MT, bool FRAG>
int launch_prefill_t(const Params& p, hipStream_t s) {
    constexpr bool kSilu = EPI == Epi::kSiluHalf;
    const int ncols = kSilu ? p.N / 2 : p.N;
    const int per_wg = kSilu ? kPfBN / 2 : kPfBN;
    const int ntiles = (ncols + per_wg - 1) / per_wg;
    const int nblocks = (int)((p.P + 16 * MT - 1) / (16 * MT));
    const int64_t grid = (int64_t)ntiles * nblocks;
    const PfLds L(16 * MT, (p.G + 15) / 16 * 16);
    // > 64 KB of dynamic LDS needs an explicit opt-in
    if (int rc = reserve_dyn_lds(reinterpret_cast<const void*>(&prefill_mfma_kernel<EPI, MT, FRAG>),
                                 PfLds(16 * MT, kPfMaxGroups).total, "prefill_mfma_kernel"))
        return rc;
    launch_kernel(&prefill_mfma_kernel<EPI, MT, FRAG>, dim3((unsigned)grid), dim3(256),
                  (size_t)L.total, s, p, nblocks, ntiles);
    return check_launch("prefill_mfma_kernel");
}

template <Epi EPI, bool FRAG>
int launch_prefill_f(const Params& p, hipStream_t s) {
    // the tile height divides block_m so a tile never spans two experts
    if (p.block_m % 128 == 0) return launch_prefill_t<EPI, 8, FRAG>(p, s);
    if (p.block_m % 64 == 0) return launch_prefill_t<EPI, 4, FRAG>(p, s);
    if (p.block_m % 32 == 0) return launch_prefill_t<EPI, 2, FRAG>(p, s);
    if (p.block_m % 16 == 0) return launch_prefill_t<EPI, 1, FRAG>(p, s);
    set_error("prefill grouped GEMM: block_m must be a multiple of 16");
    return W4A8_ERR_INVALID;
}
template <Epi EPI>
int launch_prefill_e(const Params& p, hipStream_t s) {
    return p.w_frag ? launch_prefill_f<EPI, true>(p, s) : launch_prefill_f<EPI, false>(p, s);
}

}  // namespace

bool prefill_supported(int64_t K, int64_t group_size, bool e2m1) {
    return !e2m1 && group_size == kGroup && K % kGroup == 0 && K / kGroup <= kPfMaxGroups;
}

int launch_grouped_prefill(const GroupedArgs& a, hipStream_t s) {
    const Params p = make_params(a);
    if (p.P == 0) return W4A8_OK;
    if (!prefill_supported(a.K, a.group_size, a.e2m1) || p.xq == nullptr || p.asum == nullptr ||
        a.x_rows * a.K >= ((int64_t)1 << 31) || a.N * a.K / 2 >= ((int64_t)1 << 31)) {
        set_error("prefill grouped GEMM: needs g128 int4 weights, K <= 4096, prequantised rows "
                  "(rows * K < 2^31), their group sums and expert slices below 2 GiB");
        return W4A8_ERR_INVALID;
    }
    if (a.w_frag && (a.N % 16 != 0 || (a.epi == Epi::kSiluHalf && (a.N / 2) % 16 != 0))) {
        set_error("prefill grouped GEMM: fragment-layout weights need 16-row aligned halves");
        return W4A8_ERR_INVALID;
    }
    switch (a.epi) {
        case Epi::kHalf: return launch_prefill_e<Epi::kHalf>(p, s);
        case Epi::kSiluHalf: return launch_prefill_e<Epi::kSiluHalf>(p, s);
        case Epi::kScatter: return launch_prefill_e<Epi::kScatter>(p, s);
        case Epi::kSlotF32: return launch_prefill_e<Epi::kSlotF32>(p, s);
    }
    return W4A8_ERR_INVALID;
}

}  // namespace w4a8
