// Decode expert GEMVs of the whole MoE layer (T <= 96) on fragment-layout weights, without
// an align launch and without act-quant launches (gfx950).
//
// Replaces, for the whole-layer decode schedule, the reference's chain of align
// (moe_experts.py:587-589), per-token act-quant (moe_kernel.hip:87-127) and decode GEMV
// (moe_kernel.hip:884-1062) for each of the two GEMMs. Arithmetic as in w4a8_common.h and
// bit-identical to the grouped GEMV of grouped_gemm.hip (same raw-nibble MFMA operands,
// zero-point term, scale fold order and split-K sum order). The schedule is this file's own:
//
//   * every work-group builds, in LDS, the list of touched experts and each one's slots from
//     topk_ids (the order of slots inside an expert does not matter: every output row
//     depends on its own activation row only);
//   * the layer's work is a list of units (touched expert, column unit: 16 gate + 16 up
//     columns for gemm1+SiLU, 32 columns for gemm2), split exactly evenly over a persistent
//     grid of teams (a team is one wave, or the whole work-group when the K groups are split
//     over its 4 waves), so every CU streams the same number of weight bytes in one round;
//   * a team walks its contiguous unit range expert by expert; per expert (and 16 rows at a
//     time) it loads the activation rows (gemm1: x rows of the slots' tokens, fp16 or bf16;
//     gemm2: the slots' h rows) and quantises them in registers, bit-identical to
//     act_quant_kernel, then streams the units' weights two chunks ahead of the MFMAs;
//   * outputs are per slot: gemm1 writes h (numel, I) fp16 after SiLU*mul, gemm2 writes
//     y (numel, H) fp32, which the slot reduce sums in j order.
#include <algorithm>
#include <type_traits>

#include "grouped_params.h"

namespace w4a8 {
namespace {

constexpr int kDecThreads = 256;
constexpr int kDecMaxSlots = 1024;      // T * top_k
constexpr int kDecMaxExperts = 1024;
constexpr int kDecBatch = 8;            // units per LDS round of split-K partial sums
constexpr uint32_t kDecOnes = 0x38383838u;   // four e4m3 bytes of 1.0
using u16x2 = unsigned short __attribute__((ext_vector_type(2)));

struct DecodeParams {
    const int32_t* ids;      // (numel) routed expert ids
    const int32_t* emap;     // global -> local expert map or null
    int emap_len, numel, top_k, E;
    const void* a;           // activation rows, fp16 / bf16
    int a_bf16;
    int a_per_token;         // 1: slot s reads row s / top_k (x); 0: row s (h)
    const int32_t* w;        // fragment layout (E, N/16, G, 64, 4)
    const __half* scales;    // (E, N, G)
    const int32_t* zeros;    // (E, N/8, G) or null
    void* out;               // kSiluHalf: (numel, N/2) fp16; kSlotF32: (numel, N) fp32
    int K, N, G;
};

struct DecodeLists {
    int n_touched;
    int16_t expert[kDecMaxExperts];        // touched expert r (ascending id)
    int16_t first[kDecMaxExperts + 1];     // its slots are slot[first[r] .. first[r + 1])
    int16_t slot[kDecMaxSlots];
    int cnt[kDecMaxExperts];
    int wtot[2][kDecThreads / 64];
};

// Touched experts and their slot lists (the align's grouping, without padding) in LDS.
__device__ void build_lists(const DecodeParams& p, DecodeLists& L) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    constexpr int kPer = kDecMaxSlots / kDecThreads;
    for (int e = tid; e < p.E; e += kDecThreads) L.cnt[e] = 0;
    int es[kPer];
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
        const int s = tid + kDecThreads * i;
        int e = s < p.numel ? p.ids[s] : -1;
        if (p.emap != nullptr) e = (e >= 0 && e < p.emap_len) ? p.emap[e] : -1;
        es[i] = (e >= 0 && e < p.E) ? e : -1;
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kPer; ++i)
        if (es[i] >= 0) atomicAdd(&L.cnt[es[i]], 1);
    __syncthreads();
    // exclusive scans of (slots, touched) over experts; thread t owns experts 4t .. 4t + 3
    int c[4], tot = 0, tch = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int e = 4 * tid + j;
        c[j] = e < p.E ? L.cnt[e] : 0;
        tot += c[j];
        tch += c[j] > 0 ? 1 : 0;
    }
    int it = tot, ic = tch;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_up(it, o, 64), z = __shfl_up(ic, o, 64);
        if (lane >= o) {
            it += y;
            ic += z;
        }
    }
    if (lane == 63) {
        L.wtot[0][wave] = it;
        L.wtot[1][wave] = ic;
    }
    __syncthreads();
    int off = it - tot, r = ic - tch;
    for (int w = 0; w < wave; ++w) {
        off += L.wtot[0][w];
        r += L.wtot[1][w];
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int e = 4 * tid + j;
        if (c[j] > 0) {
            L.expert[r] = (int16_t)e;
            L.first[r] = (int16_t)off;
            ++r;
        }
        if (e < p.E) L.cnt[e] = off;     // becomes the fill cursor of expert e
        off += c[j];
    }
    if (tid == kDecThreads - 1) {
        L.n_touched = r;
        L.first[r] = (int16_t)off;
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kPer; ++i)
        if (es[i] >= 0) L.slot[atomicAdd(&L.cnt[es[i]], 1)] = (int16_t)(tid + kDecThreads * i);
    __syncthreads();
}

template <Epi EPI, int GPW, int KSPLIT>
struct DecCfg {
    static constexpr bool kSilu = EPI == Epi::kSiluHalf;
    static constexpr int NF = kSilu ? 2 : 1;      // fragments per column tile (gate, up)
    static constexpr int CT = kSilu ? 1 : 2;      // column tiles per unit
    static constexpr int FR = NF * CT;            // fragments per unit and group
    static constexpr int GC = GPW < 4 ? GPW : 4;  // groups per chunk
    static constexpr int NB = GPW / GC;           // chunks per unit
    static constexpr int TEAMS = 4 / KSPLIT;      // teams per work-group
    static constexpr int LDS_BYTES = KSPLIT > 1 ? KSPLIT * kDecBatch * FR * 64 * 16 : 0;
    static_assert(KSPLIT == 1 || KSPLIT == 4, "a team is one wave or the whole work-group");
    static_assert(GPW % GC == 0 && (NB == 1 || NB == 2), "unsupported groups per wave");
};

template <int GC>
__device__ __forceinline__ void dec_load_scales(const __half* ptr, uint32_t (&s)[GC]) {
    const uint16_t* h = reinterpret_cast<const uint16_t*>(ptr);
    if constexpr (GC == 4) {
        const uint2 v = *reinterpret_cast<const uint2*>(h);
        s[0] = v.x & 0xFFFFu; s[1] = v.x >> 16; s[2] = v.y & 0xFFFFu; s[3] = v.y >> 16;
    } else {
#pragma unroll
        for (int u = 0; u < GC; ++u) s[u] = h[u];
    }
}
template <int GC>
__device__ __forceinline__ void dec_load_zeros(const int32_t* ptr, int32_t (&z)[GC]) {
    if constexpr (GC == 4) {
        const int4 v = *reinterpret_cast<const int4*>(ptr);
        z[0] = v.x; z[1] = v.y; z[2] = v.z; z[3] = v.w;
    } else {
#pragma unroll
        for (int u = 0; u < GC; ++u) z[u] = ptr[u];
    }
}

// fp16 / bf16 bits -> f32; bf16 goes through fp16 first, the cast the reference applies
// before quantising (moe_experts.py:596-597). The dtype is a template parameter: a run-time
// flag compiles into one branch per element of the unrolled row code.
template <bool BF16>
__device__ __forceinline__ float dec_act_f32(uint32_t bits) {
    if constexpr (BF16) return __half2float(__float2half(__uint_as_float(bits << 16)));
    return __half2float(__ushort_as_half(static_cast<unsigned short>(bits)));
}

template <Epi EPI, int GPW, int KSPLIT, bool ABF16>
__global__ void __launch_bounds__(kDecThreads, 2) decode_gemv_kernel(DecodeParams p) {
    using C = DecCfg<EPI, GPW, KSPLIT>;
    __shared__ DecodeLists L;
    __shared__ float s_amax[4][16];
    __shared__ int s_oslot[4][16];
    __shared__ float s_oasc[4][16];
    extern __shared__ __attribute__((aligned(16))) uint8_t s_dyn[];
    v4f* s_part = reinterpret_cast<v4f*>(s_dyn);      // KSPLIT > 1: [wave][unit][FR][lane]

    build_lists(p, L);

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int q = lane >> 4;
    const int c16 = lane & 15;
    const int team = wave / KSPLIT;
    const int g0 = (wave % KSPLIT) * GPW;
    const int ncols = C::kSilu ? p.N / 2 : p.N;
    const int upe = ncols / (16 * C::CT);                 // units per expert
    const int U = L.n_touched * upe;
    const int nteams = (int)gridDim.x * C::TEAMS;
    const int tm = (int)blockIdx.x * C::TEAMS + team;
    const int ua = (int)((int64_t)U * tm / nteams);
    const int ub = (int)((int64_t)U * (tm + 1) / nteams);

    uint4 wv[2][C::GC * C::FR];
    uint32_t sw[2][C::FR][C::GC];
    int32_t zw[2][C::FR][C::GC];
    using B0 = std::integral_constant<int, 0>;
    using B1 = std::integral_constant<int, 1>;

    for (int u = ua; u < ub;) {                           // one expert segment per step
        const int r = u / upe;
        const int ue = min(ub, (r + 1) * upe);
        const int e = L.expert[r];
        const int s0 = L.first[r];
        const int cnt = L.first[r + 1] - s0;
        const int t0 = (u - r * upe) * C::CT;             // first column tile of the segment
        const int nunits = ue - u;
        const int nch = nunits * C::NB;
        const int32_t* we = p.w + (int64_t)e * p.N * (p.K / 8);
        const __half* se = p.scales + (int64_t)e * p.N * p.G;
        const int32_t* ze = p.zeros ? p.zeros + (int64_t)e * (p.N / 8) * p.G : nullptr;

        // weight row of fragment f, column cc of chunk c (its unit's tiles)
        auto row_of = [&](int c, int f, int cc) -> int {
            const int col = (t0 + (c / C::NB) * C::CT + f % C::CT) * 16 + cc;
            return (C::kSilu && f >= C::CT) ? col + ncols : col;
        };
        // chunk c: groups g0 + (c % NB) * GC .. + GC - 1 of the unit's FR fragments; chunks
        // past the end reload the expert's first 16 bytes (unconditional issues keep the
        // compiler's wait counts exact)
        auto issue = [&](int c, auto bufc) {
            constexpr int b = decltype(bufc)::value;
            const bool live = c < nch;
            const int g = g0 + (live ? (c % C::NB) * C::GC : 0);
#pragma unroll
            for (int f = 0; f < C::FR; ++f) {
                const int n = live ? row_of(c, f, c16) : 0;
                const int32_t* wr = we + (live ? ((int64_t)(n >> 4) * p.G + g) * 256 + lane * 4 : 0);
#pragma unroll
                for (int uu = 0; uu < C::GC; ++uu)
                    wv[b][uu * C::FR + f] = load_stream16(wr + (live ? uu * 256 : 0));
                dec_load_scales<C::GC>(se + (int64_t)n * p.G + g, sw[b][f]);
                dec_load_zeros<C::GC>(ze ? ze + (int64_t)(n >> 3) * p.G + g
                                         : reinterpret_cast<const int32_t*>(p.scales), zw[b][f]);
            }
        };

        for (int m0 = 0; m0 < cnt; m0 += 16) {            // 16 rows per pass
            const int mreal = min(16, cnt - m0);
            // activation rows of this pass (pad rows repeat the last real row), quantised in
            // registers: lane (q, c16) holds k in [128 g + 32 q, +32) of row c16. The rows go
            // out first and the first weight chunk right behind them (the memory counter
            // completes in order, so the wait for the rows leaves the chunk in flight); the
            // second chunk waits until the rows are quantised: with both chunks and the raw
            // rows in registers at once the kernel spills, and a spill reload waits for every
            // access in flight. (Staging the rows in LDS by direct loads instead frees the
            // registers but measured slower: the rows land later, and a read of directly
            // loaded LDS waits for every access in flight.)
            const int my_m = min(c16, mreal - 1);
            const int my_slot = L.slot[s0 + m0 + my_m];
            const int arow = p.a_per_token ? my_slot / p.top_k : my_slot;
            const uint16_t* xr = reinterpret_cast<const uint16_t*>(p.a) + (int64_t)arow * p.K + q * 32;
            uint4 raw[GPW][4];
#pragma unroll
            for (int g = 0; g < GPW; ++g)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    raw[g][i] = reinterpret_cast<const uint4*>(xr + (g0 + g) * kGroup)[i];
            issue(0, B0{});
            auto raw_at = [&](int g, int i) -> uint4 { return raw[g][i]; };
            // absmax on the magnitude bits (both conversions are monotone in them; NaNs,
            // which fmaxf skips, count as 0), then over the row's four quarter-lanes and the
            // team's K-split waves. Two values per instruction (packed 16-bit max); a maximum
            // above the infinity pattern means a NaN is present, and only then the exact
            // NaN-skipping pass runs.
            constexpr uint32_t nan_above = ABF16 ? 0x7F80u : 0x7C00u;
            u16x2 m2 = {0, 0};
#pragma unroll
            for (int g = 0; g < GPW; ++g)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const uint4 rv = raw_at(g, i);
                    const uint32_t wd[4] = {rv.x, rv.y, rv.z, rv.w};
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        m2 = __builtin_elementwise_max(m2, __builtin_bit_cast(u16x2, wd[j] & 0x7FFF7FFFu));
                }
            uint32_t mbits = max((uint32_t)m2.x, (uint32_t)m2.y);
            if (mbits > nan_above) {
                mbits = 0;
#pragma unroll
                for (int g = 0; g < GPW; ++g)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const uint4 rv = raw_at(g, i);
                        const uint32_t wd[4] = {rv.x, rv.y, rv.z, rv.w};
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            const uint32_t lo = wd[j] & 0x7FFFu, hi = (wd[j] >> 16) & 0x7FFFu;
                            mbits = max(mbits, lo > nan_above ? 0u : lo);
                            mbits = max(mbits, hi > nan_above ? 0u : hi);
                        }
                    }
            }
            float amax = dec_act_f32<ABF16>(mbits);
            {
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
            const float my_asc = act_scale_from_absmax(amax);
            const float inv = 1.0f / my_asc;
            v8i af[GPW];
#pragma unroll
            for (int g = 0; g < GPW; ++g)
#pragma unroll
                for (int i = 0; i < 4; ++i) {   // k8-interleaved bytes, as act_quant_kernel
                    const uint4 rv = raw_at(g, i);
                    const uint32_t wd[4] = {rv.x, rv.y, rv.z, rv.w};
                    float f[8];
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        f[2 * j] = dec_act_f32<ABF16>(wd[j] & 0xFFFFu) * inv;
                        f[2 * j + 1] = dec_act_f32<ABF16>(wd[j] >> 16) * inv;
                    }
                    af[g][2 * i] = (int)pack4_e4m3(f[0], f[2], f[4], f[6]);
                    af[g][2 * i + 1] = (int)pack4_e4m3(f[1], f[3], f[5], f[7]);
                }
            v4f sa[GPW];   // 2^-9 * group sums of rows 4q .. 4q + 3 (zero-point term)
#pragma unroll
            for (int g = 0; g < GPW; ++g) {
                const int one = (int)kDecOnes;
                sa[g] = mfma_16x16x128(af[g], v8i{one, one, one, one, one, one, one, one},
                                       v4f{0.f, 0.f, 0.f, 0.f});
#pragma unroll
                for (int i = 0; i < 4; ++i) sa[g][i] *= 1.0f / kNibbleScale;
            }
            issue(1, B1{});
            // this pass's output rows (slot, scale) for the stores, per wave
            if (q == 0) {
                s_oslot[wave][c16] = c16 < mreal ? L.slot[s0 + m0 + c16] : -1;
                s_oasc[wave][c16] = my_asc * kNibbleScale;
            }

            auto store = [&](int unit, int f0, const v4f& ra, const v4f& rb) {
                const int col = (t0 + unit * C::CT + f0) * 16 + c16;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int m = 4 * q + i;
                    if (m >= mreal) continue;
                    const int sl = s_oslot[wave][m];
                    const float a = s_oasc[wave][m];
                    if constexpr (C::kSilu) {
                        reinterpret_cast<__half*>(p.out)[(int64_t)sl * ncols + col] =
                            silu_mul_h(__float2half(as_f32(ra[i] * a)), __float2half(as_f32(rb[i] * a)));
                    } else {
                        reinterpret_cast<float*>(p.out)[(int64_t)sl * p.N + col] = ra[i] * a;
                    }
                }
            };

            v4f run[C::FR];
#pragma unroll
            for (int f = 0; f < C::FR; ++f) run[f] = v4f{0.f, 0.f, 0.f, 0.f};

            // split-K partials of up to kDecBatch units, summed in wave order and stored
            auto flush = [&](int unit_end, int nbu) {
                lds_barrier();
                for (int i = tid; i < nbu * 64; i += kDecThreads) {
                    const int bu = i >> 6;              // i & 63 == lane
                    v4f sum[C::FR];
#pragma unroll
                    for (int f = 0; f < C::FR; ++f) {
                        sum[f] = s_part[((0 * kDecBatch + bu) * C::FR + f) * 64 + lane];
#pragma unroll
                        for (int j = 1; j < KSPLIT; ++j) {
                            const v4f v = s_part[((j * kDecBatch + bu) * C::FR + f) * 64 + lane];
#pragma unroll
                            for (int k = 0; k < 4; ++k) sum[f][k] += v[k];
                        }
                    }
                    const int unit = unit_end - nbu + bu;
#pragma unroll
                    for (int ct = 0; ct < C::CT; ++ct)
                        store(unit, ct, sum[ct], C::kSilu ? sum[C::CT + ct] : sum[ct]);
                }
                lds_barrier();
            };

            auto consume = [&](int c, auto bufc) {
                constexpr int b = decltype(bufc)::value;
                constexpr int gb = C::NB == 2 ? b : 0;   // chunk parity == group batch when NB == 2
                const int unit = c / C::NB;
#pragma unroll
                for (int f = 0; f < C::FR; ++f) {
                    const int zsh = (row_of(c, f, c16) & 7) * 4;
#pragma unroll
                    for (int uu = 0; uu < C::GC; ++uu) {
                        const int ga = gb * C::GC + uu;
                        v4f acc = mfma_16x16x128(af[ga], spread_nibbles(wv[b][uu * C::FR + f]),
                                                 v4f{0.f, 0.f, 0.f, 0.f});
                        const float z = ze ? (float)((zw[b][f][uu] >> zsh) & 0xF) : 8.0f;
#pragma unroll
                        for (int i = 0; i < 4; ++i) acc[i] = fmaf(-z, sa[ga][i], acc[i]);
                        const float s = __half2float(__ushort_as_half((unsigned short)sw[b][f][uu]));
#pragma unroll
                        for (int i = 0; i < 4; ++i) run[f][i] = fmaf(acc[i], s, run[f][i]);
                    }
                }
                if (c % C::NB != C::NB - 1) return;
                // unit complete
                if constexpr (KSPLIT > 1) {
                    const int bu = unit % kDecBatch;
#pragma unroll
                    for (int f = 0; f < C::FR; ++f)
                        s_part[(((wave % KSPLIT) * kDecBatch + bu) * C::FR + f) * 64 + lane] = run[f];
                    if (bu == kDecBatch - 1 || unit == nunits - 1) flush(unit + 1, bu + 1);
                } else {
#pragma unroll
                    for (int ct = 0; ct < C::CT; ++ct)
                        store(unit, ct, run[ct], C::kSilu ? run[C::CT + ct] : run[ct]);
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
            if constexpr (KSPLIT == 1) __builtin_amdgcn_wave_barrier();
        }
        u = ue;
    }
}

struct DecSplit {
    int gpw, ksplit;
};
// K groups per wave and K-split for the decode GEMVs (a team is one wave or four)
DecSplit dec_split(int G) {
    switch (G) {
        case 1: return {1, 1};
        case 2: return {2, 1};
        case 3: return {3, 1};
        case 4: return {4, 1};
        case 8: return {2, 4};
        case 12: return {3, 4};
        case 16: return {4, 4};
        case 32: return {8, 4};
        default: return {0, 0};
    }
}

int persistent_grid() {
    int dev = 0, ncu = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        ncu <= 0)
        ncu = 256;
    return 2 * ncu;   // two four-wave work-groups per CU (two waves per SIMD)
}

template <Epi EPI, int GPW, int KSPLIT, bool ABF16>
int launch_dec_a(const DecodeParams& p, hipStream_t s) {
    using C = DecCfg<EPI, GPW, KSPLIT>;
    const size_t lds = C::LDS_BYTES;
    static bool attr_set = false;
    if (!attr_set) {
        if (hipFuncSetAttribute(reinterpret_cast<const void*>(&decode_gemv_kernel<EPI, GPW, KSPLIT, ABF16>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess) {
            set_error("decode_gemv_kernel: cannot reserve dynamic LDS");
            return W4A8_ERR_HIP;
        }
        attr_set = true;
    }
    static int grid = 0;
    if (grid == 0) grid = persistent_grid();
    launch_kernel(&decode_gemv_kernel<EPI, GPW, KSPLIT, ABF16>, dim3(grid), dim3(kDecThreads), lds,
                  s, p);
    return check_launch("decode_gemv_kernel");
}

// gemm1 reads x (fp16 or bf16); gemm2 reads the fp16 h rows
template <Epi EPI, int GPW, int KSPLIT>
int launch_dec_t(const DecodeParams& p, hipStream_t s) {
    if constexpr (EPI == Epi::kSiluHalf)
        if (p.a_bf16) return launch_dec_a<EPI, GPW, KSPLIT, true>(p, s);
    return launch_dec_a<EPI, GPW, KSPLIT, false>(p, s);
}

template <Epi EPI>
int launch_dec_e(const DecodeParams& p, hipStream_t s) {
    const DecSplit sp = dec_split(p.G);
    switch (sp.gpw * 8 + sp.ksplit) {
        case 1 * 8 + 1: return launch_dec_t<EPI, 1, 1>(p, s);
        case 2 * 8 + 1: return launch_dec_t<EPI, 2, 1>(p, s);
        case 3 * 8 + 1: return launch_dec_t<EPI, 3, 1>(p, s);
        case 4 * 8 + 1: return launch_dec_t<EPI, 4, 1>(p, s);
        case 2 * 8 + 4: return launch_dec_t<EPI, 2, 4>(p, s);
        case 3 * 8 + 4: return launch_dec_t<EPI, 3, 4>(p, s);
        case 4 * 8 + 4: return launch_dec_t<EPI, 4, 4>(p, s);
        case 8 * 8 + 4: return launch_dec_t<EPI, 8, 4>(p, s);
    }
    set_error("decode GEMV: unsupported number of K groups");
    return W4A8_ERR_INVALID;
}

}  // namespace

bool decode_layer_supported(int64_t numel, int64_t E, int64_t H, int64_t inter, int64_t gs) {
    return numel <= kDecMaxSlots && E <= kDecMaxExperts && gs == kGroup && H % kGroup == 0 &&
           inter % kGroup == 0 && dec_split((int)(H / kGroup)).gpw > 0 &&
           dec_split((int)(inter / kGroup)).gpw > 0;
}

int launch_decode_gemv(const DecodeLaunch& d, hipStream_t s) {
    if (d.numel == 0) return W4A8_OK;
    DecodeParams p;
    p.ids = d.topk_ids;
    p.emap = d.expert_map;
    p.emap_len = (int)d.emap_len;
    p.numel = (int)d.numel;
    p.top_k = (int)d.top_k;
    p.E = (int)d.E;
    p.a = d.a;
    p.a_bf16 = d.a_bf16 ? 1 : 0;
    p.a_per_token = d.silu ? 1 : 0;
    p.w = d.w;
    p.scales = reinterpret_cast<const __half*>(d.scales);
    p.zeros = d.zeros;
    p.out = d.out;
    p.K = (int)d.K;
    p.N = (int)d.N;
    p.G = (int)(d.K / kGroup);
    return d.silu ? launch_dec_e<Epi::kSiluHalf>(p, s) : launch_dec_e<Epi::kSlotF32>(p, s);
}

}  // namespace w4a8
