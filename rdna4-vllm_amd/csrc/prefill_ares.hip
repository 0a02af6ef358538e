// Prefill grouped W4A8 GEMM, activation-resident schedule (gfx950 fp8 MFMA).
//
// Replaces the reference's tiled WMMA grouped GEMM (moe_gemm_tiled.h:29-350, dispatched at
// moe_kernel.hip:1110-1155) for the many-token regime when K <= 4096. Arithmetic contract as
// in w4a8_common.h; the schedule is this file's own:
//
//   * a work-group owns BM consecutive sorted rows (one expert; BM = 64 for K <= 2048, 32 up
//     to K = 4096, so the tile fits LDS) and ALL N columns: its e4m3 activation tile
//     (BM x K bytes) and the rows' per-group sums are loaded into LDS once,
//     then the kernel streams the expert's int4 weights past them, 256 weight rows at a time
//     (a "range": 8 waves, two per SIMD, x 2 16-column fragments; SiLU: 128 gate + the
//     matching 128 up columns);
//   * tiles are taken in an XCD-aware order: work-group b runs sorted tile
//     (b % 8) * ceil(tiles / 8) + b / 8, so each XCD walks a contiguous run of tiles and the
//     tiles of one expert share that XCD's L2 while they stream the same weights;
//   * inside a range each wave keeps the next 4 (range, K group) steps' B fragments in flight
//     (raw int4 words, 16 B per lane per fragment). Load addresses are a wave-uniform step
//     offset plus a fixed per-lane offset, so they cost scalar instructions only; issues are
//     unconditional (steps past the end reload the last range's final groups), so wait
//     counts stay exact;
//   * per step and live 16-row fragment: v_mfma_f32_16x16x128_f8f6f4 on the raw-nibble B
//     (n * 2^-9, two ANDs and a shift) with the operands swapped, so lane (q, c16) holds
//     tile row c16, columns 4q..4q+3; then the fp32 scale fold run += acc * scale[n, g]
//     (moe_gemm_tiled.h:144-151) with the lane's four scales read from a per-wave LDS table
//     one step ahead of the fold that uses them;
//   * the range's scales and zero-points are fetched one range ahead into registers (on
//     fragment weights: the rows' metadata words stored after each 16-row tile's blocks); at
//     a range boundary each wave writes the scale table and s*z (bf16 hi/lo) for its own 32
//     weight rows, so no work-group barrier follows the prologue. The tables hold 16 K
//     groups; for K > 2048 they are rebuilt in the middle of each range, after the first
//     half's zero-point term;
//   * after the last group of a range the zero-point term sum_g sum_k a * z * s is formed by
//     bf16 MFMAs over (row group sums) x (s*z), out = asc * (512 * run - term) is stored
//     (fp16 rows as one 16-byte piece per lane after a lane-row swap; fp16 SiLU(gate) * up,
//     bit-identical to silu_and_mul, as 8-byte pieces) and the accumulators restart;
//   * the two waves of a SIMD take turns at the higher issue priority, one range each, so
//     neither ends a tile far behind the other;
//   * the main loop is instantiated per live 16-row fragment count (1..4), so partial tiles
//     run straight-line code without per-fragment branches;
//   * fp16 rows (gemm2 on h) are quantised by the tile itself in its prologue, four rows per
//     wave at a time, bit-identical to act_quant_kernel; prefill_ares_pair_kernel takes
//     each tile through gemm1+SiLU and then this gemm2 on the h rows it just wrote, both
//     halves routed once.
#include <algorithm>
#include <type_traits>

#include "grouped_params.h"

namespace w4a8 {
namespace {

constexpr int kArBM = 64;                       // rows per work-group (K <= kArMaxK)
constexpr int kArBMWide = 32;                   // rows per work-group for kArMaxK < K <= kArMaxKWide
constexpr int kArWaves = 8;                     // two waves per SIMD
constexpr int kArThreads = kArWaves * 64;
constexpr int kArNT = 2;                        // 16-column B fragments per wave and range
constexpr int kArBN = kArWaves * kArNT * 16;    // 256 weight rows per range
constexpr int kArD = 4;                         // B steps in flight per wave
constexpr int kArMaxK = 2048;                   // 64-row activation tile must fit LDS
constexpr int kArMaxKWide = 4096;               // 32-row activation tile must fit LDS
constexpr int kArMaxKAq = 1536;                 // fp16 rows quantised in the prologue
constexpr int kArGp = 16;                       // group slots of the per-range weight tables
constexpr int kArXcds = 8;                      // work-groups go round-robin to 8 XCDs

template <int BM>
__host__ __device__ constexpr int ar_max_k() { return BM == kArBM ? kArMaxK : kArMaxKWide; }
// group slots of the row-sum table: every K group of the widest K the tile takes
template <int BM>
__host__ __device__ constexpr int ar_gpr() { return ar_max_k<BM>() / kGroup; }

// Activation tile in LDS, group-major: K group g of row m is 128 bytes at g * BM * 128 +
// m * 128, its eight 16-byte chunks stored at chunk ^ (m & 7), so the eight rows a
// ds_read_b128 serves per cycle hit eight different bank quads, and the rows of fragment i
// sit at the fixed offset i * 2 KB.
template <int BM>
__host__ __device__ constexpr int ar_a_group_bytes() { return BM * kGroup; }
template <int BM>
__device__ __forceinline__ int ar_a_off(int m, int g, int chunk) {
    return g * ar_a_group_bytes<BM>() + m * kGroup + ((chunk ^ (m & 7)) << 4);
}
// Dynamic LDS layout (bytes): activation tile; row group sums (hi/lo bf16, every group);
// per range and half of K (16 groups): s*z (hi/lo bf16) of the 256 weight rows, scales
// [wave][group][column / 4][fragment][column % 4] (fp16, the 16 bytes lanes (q, *) read
// per step) and a staging area for the zero-point words. For K = 4096 and 32 rows this is
// 158 KB.
template <int BM>
struct ArLds {
    int a, sah, sal, szh, szl, sc, zst, total;
    __host__ __device__ explicit ArLds(int K) {
        a = 0;
        sah = (K / kGroup) * ar_a_group_bytes<BM>();
        sal = sah + BM * ar_gpr<BM>() * 2;
        szh = sal + BM * ar_gpr<BM>() * 2;
        szl = szh + kArBN * kArGp * 2;
        sc = szl + kArBN * kArGp * 2;
        zst = sc + kArBN * kArGp * 2;
        total = zst + kArBN * 8;
    }
};
template <int BM>
__host__ inline size_t ar_lds_bytes(int K) { return (size_t)ArLds<BM>(K).total + BM * 4; }

// Output columns per range; output column and weight row of fragment j, column c of wave w
// in range r (SiLU: fragment 0 holds gate rows col, fragment 1 the matching up rows
// ncols + col; otherwise the wave's two fragments are 32 adjacent columns).
template <bool kSilu>
__host__ __device__ constexpr int ar_range_cols() { return kSilu ? kArBN / 2 : kArBN; }
template <bool kSilu>
__device__ __forceinline__ int ar_col(int r, int w, int j, int c) {
    return kSilu ? r * (kArBN / 2) + w * 16 + c : r * kArBN + w * 32 + 16 * j + c;
}
template <bool kSilu>
__device__ __forceinline__ int ar_row(int r, int w, int j, int c, int ncols) {
    return ar_col<kSilu>(r, w, j, c) + (kSilu && j == 1 ? ncols : 0);
}


using bf16x8 = __bf16 __attribute__((ext_vector_type(8)));
using lds_void_ptr = __attribute__((address_space(3))) void*;
using global_cvoid_ptr = const __attribute__((address_space(1))) void*;

// s_waitcnt operand waiting for at most n outstanding vector memory operations only
// (gfx9 encoding: vmcnt in bits 3:0 and 15:14, expcnt 6:4 and lgkmcnt 11:8 at their maxima)
constexpr int waitcnt_vm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }

__device__ __forceinline__ v4f mfma_bf16_16x16x32(const bf16x8& a, const bf16x8& b, const v4f& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ bf16x8 lds_bf16x8(const __bf16* ptr) {
    const uint4 v = *reinterpret_cast<const uint4*>(ptr);
    bf16x8 r;
    __builtin_memcpy(&r, &v, 16);
    return r;
}
__device__ __forceinline__ uint32_t pack_bf16x2(__bf16 a, __bf16 b) {
    return (uint32_t)__builtin_bit_cast(uint16_t, a) | ((uint32_t)__builtin_bit_cast(uint16_t, b) << 16);
}

// A tile's expert and, in lane l < BM, the slot of tile row l (-1: padding or past the ntp
// live padded rows). The two GEMMs of a pair kernel's tile share it: both walk the same
// sorted rows.
struct ArRoute {
    int e;
    int slot;
};
template <int BM>
__device__ __forceinline__ ArRoute ar_route(const Params& p, int ntp, int tile) {
    const int64_t row0 = (int64_t)tile * BM;
    ArRoute rt;
    rt.e = p.expert_ids ? p.expert_ids[row0 / p.block_m] : 0;
    // the slot loads do not wait for the expert id (both are in flight together); rows past
    // the live ones load nothing
    int slot = -1;
    if ((threadIdx.x & 63) < BM) resolve_row(p, row0 + (threadIdx.x & 63), ntp, slot);
    rt.slot = rt.e >= 0 && rt.e < p.E ? slot : -1;
    return rt;
}

// One tile (BM sorted rows of one expert, routed by rt) over weight ranges [r_begin, r_end)
// by the whole work-group. SQ: the tile quantises fp16 rows itself (fp16 output,
// K <= kArMaxKAq); otherwise it loads prequantised rows. A compile-time choice: with both
// prologues in one kernel the compiler kept the 16-chunk row staging array in scratch, each
// store waiting for its load.
template <Epi EPI, bool FRAG, int BM, bool SQ>
__device__ __forceinline__ void ar_tile(const Params& p, const ArRoute& rt, int tile, int r_begin,
                                        int r_end) {
    constexpr bool kSilu = EPI == Epi::kSiluHalf;
    static_assert(!(SQ && kSilu), "gemm1 tiles take prequantised rows");
    constexpr int GPR = ar_gpr<BM>();
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int q = lane >> 4;
    const int c16 = lane & 15;
    const int K = p.K;
    const int G = p.G;
    const ArLds<BM> L(K);
    uint8_t* s_a = lds + L.a;                                         // [G][BM][128] e4m3
    __bf16* s_sah = reinterpret_cast<__bf16*>(lds + L.sah);           // [BM][GPR] row sums hi
    __bf16* s_sal = reinterpret_cast<__bf16*>(lds + L.sal);           // ... lo
    __bf16* s_szh = reinterpret_cast<__bf16*>(lds + L.szh);           // [256][16] s*z hi
    __bf16* s_szl = reinterpret_cast<__bf16*>(lds + L.szl);           // ... lo
    uint16_t* s_sc = reinterpret_cast<uint16_t*>(lds + L.sc);         // [8][16][4][2][4] fp16
    uint32_t* s_zst = reinterpret_cast<uint32_t*>(lds + L.zst);       // [8][64] zero words
    float* s_asc = reinterpret_cast<float*>(lds + L.total);           // [BM]

    const int ncols = kSilu ? p.N / 2 : p.N;

    const int64_t row0 = (int64_t)tile * BM;
    const int e = rt.e;
    if (e < 0 || e >= p.E) return;
    // lane l < BM of every wave holds row l's slot; a real row's source is its activation row
    const int src = rt.slot < 0 ? -1 : p.identity ? (int)(row0 + lane) : rt.slot / p.top_k;
    const uint64_t vmask = __ballot(src >= 0);
    if (vmask == 0) return;
    const int maxrow = 63 - __clzll(vmask);
    const int nfl = maxrow / 16 + 1;                   // live 16-row fragments
    const int fallback = __shfl(src, __ffsll((long long)vmask) - 1, 64);
    // source row of tile row r (lane r of every wave resolved it); padding rows read a real
    // row so every load stays in bounds. Every lane must take part (shuffle).
    auto src_of = [&](int r) __attribute__((always_inline)) {
        const int sr = __shfl(src, r, 64);
        return sr >= 0 ? sr : fallback;
    };

    const uint32_t half_k = (uint32_t)K / 2;           // bytes per op-layout weight row
    // fragment layout: 16-row tiles of tile_b bytes (the G weight blocks, then the tile's
    // scales and zero-points)
    const uint32_t tile_b = (uint32_t)frag_tile_words(G) * 4u;
    const uint8_t* we = reinterpret_cast<const uint8_t*>(p.w) +
                        (int64_t)e * (FRAG ? (int64_t)(p.N / 16) * tile_b : (int64_t)p.N * half_k);
    const uint16_t* se = reinterpret_cast<const uint16_t*>(p.scales) + (int64_t)e * p.N * G;
    const int32_t* ze = p.zeros ? p.zeros + (int64_t)e * (p.N / 8) * G : nullptr;

    // ---- B ring. Byte offset of fragment j at step (range r, group g) =
    //      step_off(r, g) + frag_off[j] (wave-uniform) + lane_off ----
    //   fragment layout: 1 KB per (16-row block, group): (row / 16) * tile_b + g * 1024 + lane * 16
    //   op layout: row * K / 2 + g * 64 + q * 16 with row = first row + c16
    const uint32_t g_step = FRAG ? 1024u : 64u;
    const uint32_t r_step = FRAG ? (uint32_t)(ar_range_cols<kSilu>() / 16) * tile_b
                                 : (uint32_t)ar_range_cols<kSilu>() * half_k;
    const uint32_t lane_off = FRAG ? (uint32_t)lane * 16u : (uint32_t)c16 * half_k + q * 16u;
    uint32_t frag_off[kArNT];
#pragma unroll
    for (int j = 0; j < kArNT; ++j) {
        const uint32_t n0 = (uint32_t)ar_row<kSilu>(0, wave, j, 0, ncols);
        frag_off[j] = FRAG ? (n0 / 16) * tile_b : n0 * half_k;
    }
    uint4 bw[kArD][kArNT];
    uint32_t i_off = (uint32_t)r_begin * r_step;   // step_off of the next issue
    int i_g = 0, i_r = r_begin;                     // its group and range
    // Steps past the piece's last range (at most the ring's four, never consumed) reload that
    // range's final four groups, which this wave requested just before and are still in L2:
    // a work-group cannot retire before its loads return, so these must not go to HBM.
    const uint32_t tail_off = (uint32_t)(r_end - 1) * r_step + (uint32_t)(G - kArD) * g_step;
    auto issue = [&](auto slotc) __attribute__((always_inline)) {
        constexpr int sl = decltype(slotc)::value;
        const uint8_t* base = we + i_off;
#pragma unroll
        for (int j = 0; j < kArNT; ++j) {
            const uint8_t* ptr = base + frag_off[j] + lane_off;
            // ordinary (L2-allocating) loads: the tiles of one expert run at the same time
            // on one XCD and read the same weights, so the lines must stay in L2 for the
            // later ones (non-temporal loads cost c5 gemm1 467 against 361 us)
            bw[sl][j] = *reinterpret_cast<const uint4*>(ptr);
        }
        i_off += g_step;
        if (++i_g == G) {
            i_g = 0;
            i_off += r_step - (uint32_t)G * g_step;
            if (++i_r >= r_end) i_off = tail_off;
        }
    };
    using S0 = std::integral_constant<int, 0>;
    using S1 = std::integral_constant<int, 1>;
    using S2 = std::integral_constant<int, 2>;
    using S3 = std::integral_constant<int, 3>;

    // ---- per-range tables, one half of K (16 groups) at a time: half h covers groups
    //      16 h .. 16 h + 15. Lane l of wave w owns weight row lrow = 32 w + (l & 31), i.e.
    //      fragment (l >> 4) & 1, column l & 15, for groups 16 h + 8 (l >> 5) .. + 7: two
    //      8-byte scale loads. Lane l also loads zero-point word 16 h + (l & 15) of the
    //      wave's 8-row group l >> 4; a row's group then reads its 8 words from the staging
    //      area. On the fragment layout the lane's row keeps its scales and zero-points side
    //      by side after its tile's weights: two 16-byte loads, no staging ----
    const int trow = lane & 31, tj = trow >> 4, tc = trow & 15, th = lane >> 5;
    // The range-boundary code (prefetch, build) recomputes its lane-derived indices from an
    // opaque copy of the lane id: hoisted out of the range loop, they stayed live across the
    // main loop and were spilled, and each range start then reloaded them from scratch behind
    // a wait that drained the weight ring.
    auto lane_now = [&]() __attribute__((always_inline)) { int l = lane; asm volatile("" : "+v"(l)); return l; };
    const int lrow = 32 * wave + trow;
    uint2 pf_s[2];
    uint32_t pf_z;
    uint4 pf_m[2];      // fragment layout: metadata words (fp16 scale | zero-point << 16)
    auto prefetch = [&](int r, int h) __attribute__((always_inline)) {
        const int lane = lane_now();
        const int tj = (lane & 31) >> 4, tc = lane & 15, th = lane >> 5;
        const int rr = std::min(r, r_end - 1);
        const int n = ar_row<kSilu>(rr, wave, tj, tc, ncols);
        if constexpr (FRAG) {
            // row n's words for groups 16 h + 8 th .. + 7 (G % 4 == 0: 16-byte aligned)
            const uint8_t* mt = we + (uint32_t)(n >> 4) * tile_b +
                                (uint32_t)frag_meta_word(G, n & 15, 0) * 4u;
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const int qd = std::min(4 * h + 2 * th + u, G / 4 - 1);
                pf_m[u] = *reinterpret_cast<const uint4*>(mt + 16u * (uint32_t)qd);
            }
            return;
        }
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int qd = std::min(4 * h + 2 * th + u, G / 4 - 1);
            pf_s[u] = *reinterpret_cast<const uint2*>(se + (uint32_t)n * G + 4 * qd);
        }
        const int rgl = lane >> 4;                     // the wave's 8-row groups: (fragment, half)
        const int nz = ar_row<kSilu>(rr, wave, rgl >> 1, 8 * (rgl & 1), ncols);
        const int wz = std::min(kArGp * h + (lane & 15), G - 1);
        // symmetric weights read (and ignore) a scale word instead: same load count
        pf_z = ze ? (uint32_t)ze[(uint32_t)(nz >> 3) * G + wz] : *reinterpret_cast<const uint32_t*>(se);
    };
    auto build = [&](int r, int h) __attribute__((always_inline)) {
        const int lane = lane_now();
        const int tj = (lane & 31) >> 4, tc = lane & 15, th = lane >> 5, lrow = 32 * wave + (lane & 31);
        const int n = ar_row<kSilu>(r, wave, tj, tc, ncols);
        uint32_t zw[8];
        if constexpr (FRAG) {
            // scale bits and zero-point of group 8 th + tt, word tt of the two loads
            const uint32_t mw[8] = {pf_m[0].x, pf_m[0].y, pf_m[0].z, pf_m[0].w,
                                    pf_m[1].x, pf_m[1].y, pf_m[1].z, pf_m[1].w};
#pragma unroll
            for (int tt = 0; tt < 8; ++tt) zw[tt] = mw[tt];
        } else {
            s_zst[64 * wave + lane] = pf_z;
            const int rgl = 2 * tj + (tc >> 3);
            const uint4* zr = reinterpret_cast<const uint4*>(s_zst + 64 * wave + 16 * rgl + 8 * th);
            const uint4 z0 = zr[0], z1 = zr[1];
            zw[0] = z0.x; zw[1] = z0.y; zw[2] = z0.z; zw[3] = z0.w;
            zw[4] = z1.x; zw[5] = z1.y; zw[6] = z1.z; zw[7] = z1.w;
        }
        const int zsh = (n & 7) * 4;
        uint32_t szh[4], szl[4];
#pragma unroll
        for (int t = 0; t < 8; t += 2) {
            float sz[2];
#pragma unroll
            for (int v = 0; v < 2; ++v) {
                const int tt = t + v, g = 8 * th + tt;
                uint16_t hb;
                float z;
                if constexpr (FRAG) {
                    hb = (uint16_t)(zw[tt] & 0xFFFF);
                    z = (float)((zw[tt] >> 16) & 0xF);
                } else {
                    const uint2 sp = pf_s[tt / 4];
                    const uint32_t w2 = (tt & 2) ? sp.y : sp.x;
                    hb = (tt & 1) ? (uint16_t)(w2 >> 16) : (uint16_t)(w2 & 0xFFFF);
                    z = ze ? (float)((zw[tt] >> zsh) & 0xF) : 8.0f;
                }
                const float sv = __half2float(__ushort_as_half(hb));
                sz[v] = kArGp * h + g < G ? sv * z : 0.f;   // exact: fp16 scale x integer <= 15
                s_sc[((wave * kArGp + g) * 4 + (tc >> 2)) * 8 + tj * 4 + (tc & 3)] = hb;
            }
            const __bf16 h0 = (__bf16)sz[0], h1 = (__bf16)sz[1];
            szh[t / 2] = pack_bf16x2(h0, h1);
            szl[t / 2] = pack_bf16x2((__bf16)(sz[0] - (float)h0), (__bf16)(sz[1] - (float)h1));
        }
        *reinterpret_cast<uint4*>(s_szh + lrow * kArGp + 8 * th) = make_uint4(szh[0], szh[1], szh[2], szh[3]);
        *reinterpret_cast<uint4*>(s_szl + lrow * kArGp + 8 * th) = make_uint4(szl[0], szl[1], szl[2], szl[3]);
    };

    // ---- prologue. Loads first, in this order: the first range's tables, the activation rows
    //      (self-quantising tiles: fp16 rows into registers; otherwise the row scales and group
    //      sums, then the e4m3 tile straight into LDS), the first four weight steps; the
    //      weights stay in flight behind the table build ----
    // table halves of K: 64-row tiles take K <= 2048 (one half), 32-row tiles 2048 < K <= 4096
    constexpr int GH = BM == kArBM ? 1 : 2;
    prefetch(r_begin, 0);
    constexpr int kRowsPerWave = BM / kArWaves;
    constexpr int kAqPass = kArMaxKAq / 512;
    constexpr bool self_quant = SQ;
    // fp16 rows (self-quantising tiles): wave w takes rows 8 w .. 8 w + 7 in two passes of four
    // rows, sixteen lanes a row; lane c of a row holds its 32 values c * 32 .. c * 32 + 31 of
    // each 512-wide part of K, four 8-value pieces (one 16-byte load each)
    static_assert(!SQ || kRowsPerWave == 8, "self-quantising tiles take 64 rows");
    uint4 raw[SQ ? 2 : 1][SQ ? kAqPass : 1][SQ ? 4 : 1];
    float asv[BM * GPR / kArThreads];                   // row group sums
    // Prequantised rows go straight into the LDS tile (global_load_lds, 16 bytes per lane; no
    // registers, no LDS writes): a wave instruction fills one contiguous KB, rows
    // 8 rb .. 8 rb + 7 of one K group, lane l writing row 8 rb + l / 8 at 16-byte slot l % 8,
    // which holds the row's chunk (l % 8) ^ (row & 7) (the tile's swizzle). Instruction i,
    // issued by wave i % 8, covers group i / (BM / 8), row block i % (BM / 8), so a wave
    // always fills the same row block and each lane's source row and chunk are fixed: one
    // 32-bit offset (x_rows * K < 2^31, checked at launch). The whole tile goes out before
    // the first weight steps. (Loading the first range's later groups behind its first
    // passes was tried: the compiler cannot tell the tile reads from the DMA writes still in
    // flight and waits for all of them, vmcnt(0), before each read, draining the ring.)
    constexpr int kRB = BM / 8;                         // row blocks per K group
    const int act_row = (wave % kRB) * 8 + (lane >> 3);
    const uint32_t act_off = SQ ? 0u : (uint32_t)src_of(act_row) * (uint32_t)K +
                                           ((uint32_t)((lane & 7) ^ (act_row & 7)) << 4);
    uint8_t* const act_dst = s_a + (wave % kRB) * 8 * kGroup;   // + group offset; wave-uniform
    float ascv = 0.f;
    if constexpr (self_quant) {
        // fp16 rows in (the tile owns its rows: each is read by this work-group only);
        // wave w quantises tile rows 8w .. 8w + 7 below
        const int npass = K / 512;                      // 1 to 3 (K <= kArMaxKAq)
        const __half* xh = reinterpret_cast<const __half*>(p.xh);
#pragma unroll
        for (int pp = 0; pp < 2; ++pp) {
            const int sr = src_of(8 * wave + 4 * pp + (lane >> 4));
#pragma unroll
            for (int ps = 0; ps < kAqPass; ++ps)
#pragma unroll
                for (int pc = 0; pc < 4; ++pc)
                    raw[pp][ps][pc] = *reinterpret_cast<const uint4*>(
                        xh + (int64_t)sr * K + std::min(ps, npass - 1) * 512 + c16 * 32 + pc * 8);
        }
    } else {
#pragma unroll
        for (int j = 0; j < BM * GPR / kArThreads; ++j) {   // row sums; groups >= G are 0
            const int i = j * kArThreads + tid;
            const int sr = src_of(i / GPR);
            asv[j] = i % GPR < G ? p.asum[(int64_t)sr * G + i % GPR] : 0.f;
        }
        if (wave == 0 && src >= 0) ascv = p.asc[src];
        for (int i = wave; i < G * kRB; i += kArWaves) {     // instruction i: group i / kRB
            const int g = i / kRB;
            __builtin_amdgcn_global_load_lds((global_cvoid_ptr)(p.xq + act_off + (uint32_t)g * kGroup),
                                             (lds_void_ptr)(act_dst + g * ar_a_group_bytes<BM>()),
                                             16, 0, 0);
        }
    }
    issue(S0{});
    issue(S1{});
    issue(S2{});
    issue(S3{});
    if constexpr (self_quant) {
        // as act_quant_kernel: s = max(absmax / 448, 1e-8), e4m3 RNE of x / s in k8-interleaved
        // order, per-group sums of the e4m3 values; straight into LDS. A row's sixteen lanes
        // reduce its absmax. A group's sixteen 8-value pieces lie in four lanes, four each
        // (piece 4 (c & 3) + pc), so the sum tree of act_quant_kernel (pieces i and i ^ 1,
        // then i ^ 2, i ^ 4, i ^ 8) runs as two adds in the lane and two steps over the four
        // lanes: the same sums in the same order, so the same bits.
        const int npass = K / 512;
        using u16x2 = unsigned short __attribute__((ext_vector_type(2)));
        auto hval = [&](const uint4& w4, int j) __attribute__((always_inline)) {
            const uint32_t wd = j < 2 ? w4.x : j < 4 ? w4.y : j < 6 ? w4.z : w4.w;
            return __half2float(__ushort_as_half((uint16_t)((j & 1) ? wd >> 16 : wd & 0xFFFF)));
        };
#pragma unroll
        for (int pp = 0; pp < 2; ++pp) {
            const int m = 8 * wave + 4 * pp + (lane >> 4);
            // absmax on the magnitude bits, two values per instruction: the conversion to fp32
            // is monotone in them; a NaN (above the infinity pattern), which fmaxf skips,
            // sends the lane to the element-wise form
            u16x2 m2 = {0, 0};
#pragma unroll
            for (int ps = 0; ps < kAqPass; ++ps) {
                if (ps >= npass) break;
#pragma unroll
                for (int pc = 0; pc < 4; ++pc) {
                    const uint4 w4 = raw[pp][ps][pc];
                    const uint32_t wd[4] = {w4.x, w4.y, w4.z, w4.w};
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        m2 = __builtin_elementwise_max(m2, __builtin_bit_cast(u16x2, wd[j] & 0x7FFF7FFFu));
                }
            }
            const uint32_t mbits = max((uint32_t)m2.x, (uint32_t)m2.y);
            float amax;
            if (__builtin_expect(mbits <= 0x7C00u, 1)) {
                amax = __half2float(__ushort_as_half((uint16_t)mbits));
            } else {
                amax = 0.0f;
#pragma unroll
                for (int ps = 0; ps < kAqPass; ++ps) {
                    if (ps >= npass) break;
#pragma unroll
                    for (int pc = 0; pc < 4; ++pc)
#pragma unroll
                        for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fabsf(hval(raw[pp][ps][pc], j)));
                }
            }
            amax = lane_allreduce<4>(amax, MaxOp{});
            const float sc = act_scale_from_absmax(amax);
            if (c16 == 0) s_asc[m] = sc;
            const float inv = 1.0f / sc;
#pragma unroll
            for (int ps = 0; ps < kAqPass; ++ps) {
                if (ps >= npass) break;
                uint32_t lo[4], hi[4];
                float t[4];
#pragma unroll
                for (int pc = 0; pc < 4; ++pc) {
                    float v[8];
#pragma unroll
                    for (int j = 0; j < 8; ++j) v[j] = hval(raw[pp][ps][pc], j) * inv;
                    lo[pc] = pack4_e4m3(v[0], v[2], v[4], v[6]);
                    hi[pc] = pack4_e4m3(v[1], v[3], v[5], v[7]);
                    t[pc] = e4m3_pair_sum(0.f, lo[pc], hi[pc]);
                }
                const int k = ps * 512 + c16 * 32;          // the lane's first value
                const int g = k / kGroup;
                // pieces 0, 1 fill one 16-byte chunk (8 bytes each), pieces 2, 3 the next
#pragma unroll
                for (int h2 = 0; h2 < 2; ++h2)
                    *reinterpret_cast<uint4*>(s_a + ar_a_off<BM>(m, g, (k % kGroup) / 16 + h2)) =
                        make_uint4(lo[2 * h2], hi[2 * h2], lo[2 * h2 + 1], hi[2 * h2 + 1]);
                float gs = (t[0] + t[1]) + (t[2] + t[3]);
                gs = lane_allreduce<2>(gs, SumOp{});
                if ((c16 & 3) == 0) {
                    const __bf16 h = (__bf16)gs;
                    s_sah[m * GPR + g] = h;
                    s_sal[m * GPR + g] = (__bf16)(gs - (float)h);
                }
            }
        }
        for (int i = tid; i < BM * GPR; i += kArThreads) {   // groups >= G are 0
            if (i % GPR >= G) {
                s_sah[i] = (__bf16)0.f;
                s_sal[i] = (__bf16)0.f;
            }
        }
    } else {
#pragma unroll
        for (int j = 0; j < BM * GPR / kArThreads; ++j) {
            const int i = j * kArThreads + tid;
            const __bf16 h = (__bf16)asv[j];
            s_sah[i] = h;
            s_sal[i] = (__bf16)(asv[j] - (float)h);
        }
        if (wave == 0 && lane < BM) s_asc[lane] = ascv;
    }
    build(r_begin, 0);
    // the tables' next (range, half), prefetched right after each build
    auto prefetch_after = [&](int r, int h) __attribute__((always_inline)) {
        if (h + 1 < GH) prefetch(r, h + 1);
        else if (r + 1 < r_end) prefetch(r + 1, 0);
    };
    prefetch_after(r_begin, 0);
    if constexpr (!self_quant) {
        // the tile's DMA done: at most the weight steps issued after it still pending (and
        // the tables' prefetch when issued, so this may wait for a little more)
        __builtin_amdgcn_s_waitcnt(waitcnt_vm(4 * kArNT));
    }
    lds_barrier();

    auto main_loop = [&](auto nflc) __attribute__((always_inline)) {
        constexpr int NF = decltype(nflc)::value;
        // Operands go in swapped (weights first), so the MFMAs produce the transposed block:
        // lane (q, c16) of fragment (i, j) holds tile row 16 i + c16, columns 4 q .. 4 q + 3
        // of fragment j; its four values leave as one 8-byte piece of an output row.
        v4f run[NF][kArNT];
        // Software pipeline: a step first folds the previous step's MFMA results into the
        // accumulators (run += acc * scale, the scale of each of the lane's four columns,
        // read from the table at the step's start), then issues its own MFMAs into the same
        // registers, so every result has a whole step to arrive before it is read. A range's
        // first step has nothing to fold and its second starts the accumulators
        // (run = acc * scale).
        v4f pend[NF][kArNT];
        auto scales_of = [&](int g) __attribute__((always_inline)) {      // fp16 scales [fragment][column 0..3] of group g
            return *reinterpret_cast<const uint4*>(s_sc + ((wave * kArGp + (g & (kArGp - 1))) * 4 + q) * 8);
        };
        auto fold_one = [&](int i, int j, const uint4& sc, auto modec) __attribute__((always_inline)) {
            constexpr int mode = decltype(modec)::value;
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) {
                const uint32_t w = j == 0 ? (rr < 2 ? sc.x : sc.y) : (rr < 2 ? sc.z : sc.w);
                const float f = __half2float(__ushort_as_half((uint16_t)((rr & 1) ? w >> 16 : w & 0xFFFF)));
                if constexpr (mode == 1) run[i][j][rr] = pend[i][j][rr] * f;
                if constexpr (mode == 2) run[i][j][rr] = fmaf(pend[i][j][rr], f, run[i][j][rr]);
            }
        };
        using M0 = std::integral_constant<int, 0>;
        using M1 = std::integral_constant<int, 1>;
        using M2 = std::integral_constant<int, 2>;
        // The scales of group g are read from the table one step ahead of their fold (in step
        // g, folded in step g + 1 or by fold_last): read right before the fold, the LDS
        // round trip stood between the step's MFMAs and its fold every step.
        uint4 scn = make_uint4(0u, 0u, 0u, 0u);
        auto consume = [&](int g, auto slotc, auto modec) __attribute__((always_inline)) {
            constexpr int sl = decltype(slotc)::value;
            constexpr int mode = decltype(modec)::value;
            const uint4 sc = scn;                  // group g - 1 (not read when mode == 0)
            scn = scales_of(g);
            v8i bf[kArNT];
#pragma unroll
            for (int j = 0; j < kArNT; ++j) bf[j] = spread_nibbles(bw[sl][j]);
            // fragment i's rows are 16 i + c16: same swizzle as row c16, offset i * 2 KB
            const uint8_t* A0 = s_a + ar_a_off<BM>(c16, g, 2 * q);
            const uint8_t* A1 = s_a + ar_a_off<BM>(c16, g, 2 * q + 1);
#pragma unroll
            for (int i = 0; i < NF; ++i) {
                const uint4 lo = *reinterpret_cast<const uint4*>(A0 + i * 16 * kGroup);
                const uint4 hi = *reinterpret_cast<const uint4*>(A1 + i * 16 * kGroup);
                const v8i af = v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w,
                                   (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
#pragma unroll
                for (int j = 0; j < kArNT; ++j) {
                    fold_one(i, j, sc, modec);
                    pend[i][j] = mfma_16x16x128(bf[j], af, v4f{0.f, 0.f, 0.f, 0.f});
                }
            }
        };

        // Zero-point term of every (row, column) of a range as bf16 MFMAs over the 16 groups
        // of table half h (lane (q, c16), K slot 8q + t <-> group 16 h + 8 (q & 1) + t: the
        // row operand is the hi (q < 2) or lo (q >= 2) half of the row's group sum; the column
        // operand the hi, then lo, half of s*z with slots 16..31 repeating 0..15, so the two
        // MFMAs add (sa_hi + sa_lo)(sz_hi + sz_lo)); operands swapped as in the main MFMAs. The
        // second half of K adds to the first half's result.
        v4f za[NF], zb[NF];
        auto zterm = [&](int h, auto firstc) __attribute__((always_inline)) {
            constexpr bool first = decltype(firstc)::value;
            const __bf16* sa_tab = q < 2 ? s_sah : s_sal;
            const int go = 8 * (q & 1);
            const int lra = 32 * wave + c16, lrb = lra + 16;
            const bf16x8 zah = lds_bf16x8(s_szh + lra * kArGp + go);
            const bf16x8 zal = lds_bf16x8(s_szl + lra * kArGp + go);
            const bf16x8 zbh = lds_bf16x8(s_szh + lrb * kArGp + go);
            const bf16x8 zbl = lds_bf16x8(s_szl + lrb * kArGp + go);
#pragma unroll
            for (int i = 0; i < NF; ++i) {
                const int m = 16 * i + c16;
                const bf16x8 sa = lds_bf16x8(sa_tab + m * GPR + kArGp * h + go);
                za[i] = mfma_bf16_16x16x32(zah, sa, first ? v4f{0.f, 0.f, 0.f, 0.f} : za[i]);
                za[i] = mfma_bf16_16x16x32(zal, sa, za[i]);
                zb[i] = mfma_bf16_16x16x32(zbh, sa, first ? v4f{0.f, 0.f, 0.f, 0.f} : zb[i]);
                zb[i] = mfma_bf16_16x16x32(zbl, sa, zb[i]);
            }
        };
        // fold of the last step's MFMA results (group g) into the accumulators
        auto fold_last = [&](int g) __attribute__((always_inline)) {
            (void)g;
            const uint4 sc = scn;                  // read by the step of group g
#pragma unroll
            for (int i = 0; i < NF; ++i)
#pragma unroll
                for (int j = 0; j < kArNT; ++j) fold_one(i, j, sc, M2{});
        };
        // Range output: out = asc * (512 * run - zero term), stored.
        auto store_range = [&](int r) __attribute__((always_inline)) {
            const int64_t ldo = kSilu ? ncols : p.N;
            // a wave-uniform base and 32-bit lane offsets recomputed here from an opaque lane
            // id (m * ldo < 2^31): hoisted out of the range loop, the per-fragment 64-bit row
            // addresses stayed live across the main loop
            __half* outb = reinterpret_cast<__half*>(p.out) + row0 * ldo + ar_col<kSilu>(r, wave, 0, 0);
            const int ln = lane_now();
            const int c16n = ln & 15;
            const uint32_t qoff = 4u * (uint32_t)(ln >> 4);
#pragma unroll
            for (int i = 0; i < NF; ++i) {
                const int m = 16 * i + c16n;
                const float av = s_asc[m];
                float va[4], vb[4];
#pragma unroll
                for (int rr = 0; rr < 4; ++rr) {
                    va[rr] = as_f32(av * (kNibbleScale * run[i][0][rr] - za[i][rr]));
                    vb[rr] = as_f32(av * (kNibbleScale * run[i][1][rr] - zb[i][rr]));
                }
                __half* rowp = outb + ((uint32_t)m * (uint32_t)ldo + qoff);
                const bool live = (vmask >> m) & 1;
                if constexpr (kSilu) {
                    __half hv[4];
                    silu_mul_h4(va, vb, hv);
                    const __half2 h01 = __halves2half2(hv[0], hv[1]);
                    const __half2 h23 = __halves2half2(hv[2], hv[3]);
                    if (live)
                        *reinterpret_cast<uint2*>(rowp) = make_uint2(__builtin_bit_cast(uint32_t, h01),
                                                                     __builtin_bit_cast(uint32_t, h23));
                } else {
                    const __half2 a01 = __floats2half2_rn(va[0], va[1]), a23 = __floats2half2_rn(va[2], va[3]);
                    const __half2 b01 = __floats2half2_rn(vb[0], vb[1]), b23 = __floats2half2_rn(vb[2], vb[3]);
                    // one 16-byte piece per lane: rows of 16 lanes pair up (q, q ^ 1); the even
                    // one takes its partner's four fragment-0 columns, the odd one gives its
                    // fragment-0 columns and takes its partner's fragment-1 columns, so lane q
                    // holds columns 4 q + 12 (q & 1) .. + 7 (every lane takes part)
                    const auto s0 = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, a01),
                                                                     __builtin_bit_cast(uint32_t, b01), false, false);
                    const auto s1 = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, a23),
                                                                     __builtin_bit_cast(uint32_t, b23), false, false);
                    if (live)
                        *reinterpret_cast<uint4*>(rowp + 12 * (q & 1)) =
                            make_uint4((uint32_t)s0[0], (uint32_t)s1[0], (uint32_t)s0[1], (uint32_t)s1[1]);
                }
            }
        };

        // The steps of groups [g0, g1): four per pass of the ring (the halves hold multiples of
        // 4 groups, G % 4 == 0), so every pass issues the same loads and the wait counts stay
        // exact; a half's first pass is written out on its own (its first steps fold
        // differently: the range's first step folds nothing and its second starts the
        // accumulators; the second half's first step folds nothing, the middle of the range
        // having folded its predecessor). The scheduling barriers keep each step's MFMAs next
        // to the fold that frees their registers instead of hoisting later steps' MFMAs.
        auto run_steps = [&](int g0, int g1, auto second_mode) __attribute__((always_inline)) {
            consume(g0, S0{}, M0{});
            issue(S0{});
            __builtin_amdgcn_sched_barrier(0);
            consume(g0 + 1, S1{}, second_mode);
            issue(S1{});
            __builtin_amdgcn_sched_barrier(0);
            consume(g0 + 2, S2{}, M2{});
            issue(S2{});
            __builtin_amdgcn_sched_barrier(0);
            consume(g0 + 3, S3{}, M2{});
            issue(S3{});
            __builtin_amdgcn_sched_barrier(0);
            for (int g = g0 + 4; g < g1; g += 4) {
                consume(g, S0{}, M2{});
                issue(S0{});
                __builtin_amdgcn_sched_barrier(0);
                consume(g + 1, S1{}, M2{});
                issue(S1{});
                __builtin_amdgcn_sched_barrier(0);
                consume(g + 2, S2{}, M2{});
                issue(S2{});
                __builtin_amdgcn_sched_barrier(0);
                consume(g + 3, S3{}, M2{});
                issue(S3{});
                __builtin_amdgcn_sched_barrier(0);
            }
        };
        using F0 = std::false_type;
        using F1 = std::true_type;
        for (int r = r_begin; r < r_end; ++r) {
            // Waves w and w + 4 share a SIMD and the issue arbiter favours one of them; the
            // higher priority alternates between the two every range, so neither falls a
            // whole tile behind (the work-group ends with its slowest wave).
            if (((wave >> 2) ^ r) & 1) __builtin_amdgcn_s_setprio(1);
            else __builtin_amdgcn_s_setprio(0);
            if constexpr (GH == 1) {
                run_steps(0, G, M1{});
                fold_last(G - 1);
                zterm(0, F1{});
            } else {
                // K > 2048: the tables hold one half of K; the middle of the range folds the
                // first half's last step, takes its zero-point term and rebuilds the tables
                run_steps(0, kArGp, M1{});
                fold_last(kArGp - 1);
                zterm(0, F1{});
                build(r, 1);
                prefetch_after(r, 1);
                run_steps(kArGp, G, M2{});
                fold_last(G - 1);
                zterm(1, F0{});
            }
            store_range(r);
            if (r + 1 < r_end) {
                build(r + 1, 0);
                prefetch_after(r + 1, 0);
            }
        }
    };
    if constexpr (BM == kArBM) {
        switch (nfl) {
            case 1: main_loop(std::integral_constant<int, 1>{}); break;
            case 2: main_loop(std::integral_constant<int, 2>{}); break;
            case 3: main_loop(std::integral_constant<int, 3>{}); break;
            default: main_loop(std::integral_constant<int, 4>{}); break;
        }
    } else {
        if (nfl == 1) main_loop(std::integral_constant<int, 1>{});
        else main_loop(std::integral_constant<int, 2>{});
    }
}

// Live tiles of a launch, and the XCD-aware order over them: XCD x (work-groups b with
// b % 8 == x) owns a contiguous run of per_xcd tiles and takes its work-groups in the order
// b / 8.
struct ArOrder {
    int ntp, ntiles, per_xcd;
    template <int BM>
    __device__ static ArOrder of(const Params& p) {
        ArOrder o;
        o.ntp = p.ntp ? p.ntp[0] : (int)p.P;
        const int64_t live_rows = std::min<int64_t>((int64_t)o.ntp, p.P);
        o.ntiles = (int)((live_rows + BM - 1) / BM);
        o.per_xcd = (o.ntiles + kArXcds - 1) / kArXcds;
        return o;
    }
};

// One GEMM. Whole tiles fill an XCD's slots in rounds; when the last round would hold at most
// half the slots, its tiles are split into pieces of consecutive ranges instead (each piece
// reloads the tile's rows), so that round ends after a fraction of a tile. The results do not
// depend on the split.
template <Epi EPI, bool FRAG, int BM, bool SQ>
__global__ void __launch_bounds__(kArThreads, 1) prefill_ares_kernel(Params p) {
    constexpr bool kSilu = EPI == Epi::kSiluHalf;
    const int nranges = (kSilu ? p.N / 2 : p.N) / ar_range_cols<kSilu>();
    const ArOrder o = ArOrder::of<BM>(p);
    const int b = blockIdx.x;
    const int t0 = (b % kArXcds) * o.per_xcd;
    const int jx = b / kArXcds;
    const int nx = std::max(0, std::min(o.per_xcd, o.ntiles - t0));
    const int slots = std::max(p.xcd_slots, 1);
    const int tail = nx % slots;
    const int split = tail > 0 && 2 * tail <= slots ? std::min(slots / tail, nranges) : 1;
    const int whole = split > 1 ? nx - tail : nx;
    int tile, r_begin = 0, r_end = nranges;
    if (jx < whole) {
        tile = t0 + jx;
    } else {
        const int i = jx - whole;
        if (split == 1 || i >= tail * split) return;
        tile = t0 + whole + i / split;
        r_begin = (i % split) * nranges / split;
        r_end = (i % split + 1) * nranges / split;
    }
    ar_tile<EPI, FRAG, BM, SQ>(p, ar_route<BM>(p, o.ntp, tile), tile, r_begin, r_end);
}

// gemm1+SiLU and gemm2 of the same 64 sorted rows in one work-group, one tile after the
// other: the tile's h rows (all its intermediate columns) are written by gemm1's epilogues
// and read back, still in this XCD's L2, by gemm2's self-quantising prologue. Whole tiles
// only (a gemm1 piece would leave its h rows to several work-groups).
template <bool FRAG>
__global__ void __launch_bounds__(kArThreads, 1) prefill_ares_pair_kernel(Params p1, Params p2) {
    const ArOrder o = ArOrder::of<kArBM>(p1);
    const int b = blockIdx.x;
    const int jx = b / kArXcds;
    const int tile = (b % kArXcds) * o.per_xcd + jx;
    if (jx >= o.per_xcd || tile >= o.ntiles) return;
    const ArRoute rt = ar_route<kArBM>(p1, o.ntp, tile);
    ar_tile<Epi::kSiluHalf, FRAG, kArBM, false>(p1, rt, tile, 0, (p1.N / 2) / ar_range_cols<true>());
    // every wave's h stores complete (and so visible to the work-group's loads, which share
    // the CU's L1) before any wave reads h rows; also the LDS hand-over between the tiles
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    ar_tile<Epi::kHalf, FRAG, kArBM, true>(p2, rt, tile, 0, p2.N / ar_range_cols<false>());
}

template <Epi EPI, bool FRAG, int BM, bool SQ>
int launch_ares_bm(const Params& p, hipStream_t s) {
    const size_t lds = ar_lds_bytes<BM>(p.K);
    const void* fn = reinterpret_cast<const void*>(&prefill_ares_kernel<EPI, FRAG, BM, SQ>);
    // > 64 KB of dynamic LDS needs an explicit opt-in
    if (int rc = reserve_dyn_lds(fn, (int)ar_lds_bytes<BM>(ar_max_k<BM>()), "prefill_ares_kernel"))
        return rc;
    // work-groups one XCD holds at once (the split of the last round is sized to it)
    const int occ = std::max(1, blocks_per_cu(fn, kArThreads, lds));
    const int ncu = device_cu_count();
    Params q = p;
    q.xcd_slots = std::max(1, ncu * occ / kArXcds);
    // a multiple of 8 work-groups covers every tile under the XCD-aware order, plus one more
    // slot's worth per XCD for the pieces of a split last round
    const int64_t tiles = (p.P + BM - 1) / BM;
    const unsigned grid = (unsigned)(((tiles + kArXcds - 1) / kArXcds + q.xcd_slots) * kArXcds);
    launch_kernel(&prefill_ares_kernel<EPI, FRAG, BM, SQ>, dim3(grid), dim3(kArThreads), lds, s, q);
    return check_launch("prefill_ares_kernel");
}

// 64-row tiles up to K = 2048; 32-row tiles (the activation tile halves) up to K = 4096
template <Epi EPI, bool FRAG>
int launch_ares_t(const Params& p, hipStream_t s) {
    if constexpr (EPI == Epi::kHalf) {
        if (p.xq == nullptr)   // self-quantising tiles: K <= kArMaxKAq, so 64 rows
            return launch_ares_bm<EPI, FRAG, kArBM, true>(p, s);
    }
    return p.K <= kArMaxK ? launch_ares_bm<EPI, FRAG, kArBM, false>(p, s)       // one table half
                          : launch_ares_bm<EPI, FRAG, kArBMWide, false>(p, s);  // two (K <= 4096)
}

template <bool FRAG>
int launch_ares_pair_t(const Params& p1, const Params& p2, hipStream_t s) {
    const size_t lds = std::max(ar_lds_bytes<kArBM>(p1.K), ar_lds_bytes<kArBM>(p2.K));
    const void* fn = reinterpret_cast<const void*>(&prefill_ares_pair_kernel<FRAG>);
    if (int rc = reserve_dyn_lds(fn, (int)ar_lds_bytes<kArBM>(kArMaxK), "prefill_ares_pair_kernel"))
        return rc;
    const int64_t tiles = (p1.P + kArBM - 1) / kArBM;
    const unsigned grid = (unsigned)((tiles + kArXcds - 1) / kArXcds * kArXcds);
    launch_kernel(&prefill_ares_pair_kernel<FRAG>, dim3(grid), dim3(kArThreads), lds, s, p1, p2);
    return check_launch("prefill_ares_pair_kernel");
}

}  // namespace

bool prefill_ares_pair_supported(const GroupedArgs& a1, const GroupedArgs& a2) {
    return a1.epi == Epi::kSiluHalf && a2.epi == Epi::kHalf && a1.w_frag == a2.w_frag &&
           a1.K <= kArMaxK && a2.K <= kArMaxKAq && a2.K == a1.N / 2 &&
           prefill_ares_supported(a1.K, a1.N, a1.group_size, a1.e2m1, a1.block_m, a1.epi) &&
           prefill_ares_supported(a2.K, a2.N, a2.group_size, a2.e2m1, a2.block_m, a2.epi) &&
           a1.x_fp8 != nullptr && a1.act_scales != nullptr && a1.act_group_sums != nullptr &&
           a2.x_fp8 == nullptr && a2.x == a1.out && !a2.x_bf16 && a2.identity_gather &&
           a1.P == a2.P && a1.block_m == a2.block_m && a1.sorted_ids == a2.sorted_ids &&
           a1.expert_ids == a2.expert_ids && a1.ntp == a2.ntp && a1.E == a2.E &&
           a1.num_valid == a2.num_valid &&
           a1.x_rows * a1.K < ((int64_t)1 << 31) && a2.x_rows * a2.K < ((int64_t)1 << 31) &&
           (!a1.w_frag || ((a1.N / 2) % 16 == 0 && a2.N % 16 == 0));
}

int launch_grouped_prefill_ares_pair(const GroupedArgs& a1, const GroupedArgs& a2, hipStream_t s) {
    if (!prefill_ares_pair_supported(a1, a2)) {
        set_error("prefill (activation-resident pair): needs the gemm1+SiLU tile (K <= 2048, "
                  "prequantised rows) and a self-quantising gemm2 tile (K <= 1536) on h, over the "
                  "same sorted rows");
        return W4A8_ERR_INVALID;
    }
    const Params p1 = make_params(a1);
    if (p1.P == 0) return W4A8_OK;
    const Params p2 = make_params(a2);
    return a1.w_frag ? launch_ares_pair_t<true>(p1, p2, s) : launch_ares_pair_t<false>(p1, p2, s);
}

bool prefill_ares_supported(int64_t K, int64_t N, int64_t group_size, bool e2m1, int64_t block_m,
                            Epi epi) {
    if (e2m1 || group_size != kGroup || K % (4 * kGroup) != 0 || K > kArMaxKWide ||
        block_m % (K <= kArMaxK ? kArBM : kArBMWide) != 0)
        return false;
    if (epi == Epi::kSiluHalf) return N % (2 * ar_range_cols<true>()) == 0;
    if (epi == Epi::kHalf) return N % ar_range_cols<false>() == 0;
    return false;
}

bool prefill_ares_quantises_rows(int64_t K, Epi epi) {
    return epi == Epi::kHalf && K <= kArMaxKAq;
}

int launch_grouped_prefill_ares(const GroupedArgs& a, hipStream_t s) {
    const Params p = make_params(a);
    if (p.P == 0) return W4A8_OK;
    // rows come prequantised (x_fp8 with scales and group sums), or, for fp16 output and
    // K <= 1536, as fp16 rows the tile quantises itself
    const bool prequant = p.xq != nullptr && p.asum != nullptr && p.asc != nullptr;
    const bool self_quant = p.xq == nullptr && p.xh != nullptr && !a.x_bf16 &&
                            a.epi == Epi::kHalf && a.K <= kArMaxKAq;
    if (!prefill_ares_supported(a.K, a.N, a.group_size, a.e2m1, a.block_m, a.epi) ||
        !(prequant || self_quant) || a.x_rows * a.K >= ((int64_t)1 << 31)) {
        set_error("prefill (activation-resident): needs g128 int4 weights, K % 512 == 0 and "
                  "K <= 4096, output columns in whole 256-row ranges, block_m % 64 == 0 (32 for "
                  "K > 2048), fp16 out, and prequantised rows with group sums (or fp16 rows, fp16 "
                  "out, K <= 1536)");
        return W4A8_ERR_INVALID;
    }
    if (a.w_frag && (a.N % 16 != 0 || (a.epi == Epi::kSiluHalf && (a.N / 2) % 16 != 0))) {
        set_error("prefill (activation-resident): fragment-layout weights need 16-row aligned halves");
        return W4A8_ERR_INVALID;
    }
    if (a.epi == Epi::kSiluHalf)
        return a.w_frag ? launch_ares_t<Epi::kSiluHalf, true>(p, s) : launch_ares_t<Epi::kSiluHalf, false>(p, s);
    return a.w_frag ? launch_ares_t<Epi::kHalf, true>(p, s) : launch_ares_t<Epi::kHalf, false>(p, s);
}

}  // namespace w4a8
