// Dense W4A8 GEMV for a few rows (gfx950 fp8 MFMA): the dense op's decode regime.
//
// Replaces the reference's dense decode path (dense_kernel.hip's GEMV behind
// mmq_fp8_gemm's "decode_gemv" name, vllm_adapter.py:296-324) for M <= 16 rows on op-layout
// weights (N, K/8) with group 128 and K = 1024 .. 4096. One work-group per 16-column tile:
// its eight waves split K (wave w takes groups [w GPW, (w + 1) GPW)), so every wave issues
// all of its weight, scale and row loads at once and the tile's bytes are in flight
// together. The rows are quantised inside the kernel (no act-quant launch): each wave
// takes the absmax of its K slice, the eight slices meet in LDS, and every wave then
// quantises its slice exactly as act_quant_kernel does (s = max(absmax / 448, 1e-8),
// e4m3 RNE of x / s, k8-interleaved). Per group, as in the decode GEMVs: one
// 16x16x128 MFMA on the raw nibbles, the zero-point term from the row sums (an MFMA against
// ones), the fp16 scale fold; the eight waves' partial sums are added in wave order.
#include "grouped_params.h"

namespace w4a8 {
namespace {

constexpr int kDgWaves = 8;
constexpr int kDgThreads = 64 * kDgWaves;
constexpr uint32_t kDgOnes = 0x38383838u;   // four e4m3 bytes of 1.0

struct DenseParams {
    const __half* x;       // (M, K)
    const int32_t* w;      // (N, K/8) op layout
    const __half* s;       // (N, G)
    const int32_t* z;      // (N/8, G) or null (uint4b8: zero point 8)
    __half* out;           // (M, N)
    int M, N, K, G;
};

template <int GPW, bool ZP>
__global__ void __launch_bounds__(kDgThreads) __attribute__((amdgpu_waves_per_eu(4))) dense_gemv_kernel(DenseParams p) {
    __shared__ float s_amax[kDgWaves][16];
    __shared__ v4f s_part[kDgWaves][64];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int q = lane >> 4;
    const int c16 = lane & 15;
    const int n = blockIdx.x * 16 + c16;                // this lane's weight column
    const int g0 = wave * GPW;

    // weights: column n, k in [128 g + 32 q, +32) of each group (16 bytes, raw nibbles)
    uint4 wv[GPW];
    const uint8_t* wrow = reinterpret_cast<const uint8_t*>(p.w) + (int64_t)n * (p.K / 2) + q * 16;
#pragma unroll
    for (int g = 0; g < GPW; ++g) wv[g] = load_stream16(wrow + (g0 + g) * 64);
    uint32_t sbits[GPW], zw[GPW];
#pragma unroll
    for (int g = 0; g < GPW; ++g) {
        sbits[g] = __half_as_ushort(p.s[(int64_t)n * p.G + g0 + g]);
        zw[g] = ZP ? (uint32_t)p.z[(int64_t)(n >> 3) * p.G + g0 + g] : 0u;
    }
    // activation row c16 (pad rows repeat the last real row): k in [128 g + 32 q, +32)
    const int row = min(c16, p.M - 1);
    const __half* xr = p.x + (int64_t)row * p.K + q * 32;
    uint4 raw[GPW][4];
#pragma unroll
    for (int g = 0; g < GPW; ++g)
#pragma unroll
        for (int i = 0; i < 4; ++i) raw[g][i] = *reinterpret_cast<const uint4*>(xr + (g0 + g) * kGroup + i * 8);

    // row absmax on the magnitude bits (monotone in the fp16 value); a NaN, which fmaxf
    // skips, lies above the infinity pattern and is dropped
    using u16x2 = unsigned short __attribute__((ext_vector_type(2)));
    u16x2 m2 = {0, 0};
#pragma unroll
    for (int g = 0; g < GPW; ++g)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t wd[4] = {raw[g][i].x, raw[g][i].y, raw[g][i].z, raw[g][i].w};
#pragma unroll
            for (int j = 0; j < 4; ++j)
                m2 = __builtin_elementwise_max(m2, __builtin_bit_cast(u16x2, wd[j] & 0x7FFF7FFFu));
        }
    uint32_t mbits = max((uint32_t)m2.x, (uint32_t)m2.y);
    if (mbits > 0x7C00u) {
        mbits = 0;
#pragma unroll
        for (int g = 0; g < GPW; ++g)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t wd[4] = {raw[g][i].x, raw[g][i].y, raw[g][i].z, raw[g][i].w};
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const uint32_t lo = wd[j] & 0x7FFFu, hi = (wd[j] >> 16) & 0x7FFFu;
                    mbits = max(mbits, lo > 0x7C00u ? 0u : lo);
                    mbits = max(mbits, hi > 0x7C00u ? 0u : hi);
                }
            }
    }
    float amax = __half2float(__ushort_as_half((unsigned short)mbits));
    {   // over the row's four quarter-lanes, then the eight waves' slices
        const auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(amax), __float_as_uint(amax), false, false);
        amax = fmaxf(__uint_as_float(r16[0]), __uint_as_float(r16[1]));
        const auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(amax), __float_as_uint(amax), false, false);
        amax = fmaxf(__uint_as_float(r32[0]), __uint_as_float(r32[1]));
    }
    if (q == 0) s_amax[wave][c16] = amax;
    __syncthreads();
#pragma unroll
    for (int j = 0; j < kDgWaves; ++j) amax = fmaxf(amax, s_amax[j][c16]);
    const float asc = act_scale_from_absmax(amax);
    const float inv = 1.0f / asc;
    v8i af[GPW];
#pragma unroll
    for (int g = 0; g < GPW; ++g)
#pragma unroll
        for (int i = 0; i < 4; ++i) {   // k8-interleaved bytes, as act_quant_kernel
            const uint32_t wd[4] = {raw[g][i].x, raw[g][i].y, raw[g][i].z, raw[g][i].w};
            float f[8];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                f[2 * j] = __half2float(__ushort_as_half((unsigned short)(wd[j] & 0xFFFFu))) * inv;
                f[2 * j + 1] = __half2float(__ushort_as_half((unsigned short)(wd[j] >> 16))) * inv;
            }
            af[g][2 * i] = (int)pack4_e4m3(f[0], f[2], f[4], f[6]);
            af[g][2 * i + 1] = (int)pack4_e4m3(f[1], f[3], f[5], f[7]);
        }

    // lane (q, c16) accumulates rows 4q .. 4q + 3 of column n
    v4f run = {0.f, 0.f, 0.f, 0.f};
    const int one = (int)kDgOnes;
#pragma unroll
    for (int g = 0; g < GPW; ++g) {
        // 2^-9 x the group sums of rows 4q .. 4q + 3 (zero-point term)
        v4f sa = mfma_16x16x128(af[g], v8i{one, one, one, one, one, one, one, one}, v4f{0.f, 0.f, 0.f, 0.f});
        v4f acc = mfma_16x16x128(af[g], spread_nibbles(wv[g]), v4f{0.f, 0.f, 0.f, 0.f});
        const float z = ZP ? (float)((zw[g] >> (4 * (n & 7))) & 0xFu) : 8.0f;
        const float s = __half2float(__ushort_as_half((unsigned short)sbits[g]));
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            acc[i] = fmaf(-z, sa[i] * (1.0f / kNibbleScale), acc[i]);
            run[i] = fmaf(acc[i], s, run[i]);
        }
    }
    s_part[wave][lane] = run;
    __syncthreads();
    if (wave == 0) {
        v4f sum = s_part[0][lane];
#pragma unroll
        for (int w = 1; w < kDgWaves; ++w) {
            const v4f v = s_part[w][lane];
#pragma unroll
            for (int i = 0; i < 4; ++i) sum[i] += v[i];
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int m = 4 * q + i;
            const float a = __shfl(asc * kNibbleScale, m, 64);
            if (m < p.M) p.out[(int64_t)m * p.N + n] = __float2half(as_f32(sum[i] * a));
        }
    }
}

template <int GPW, bool ZP>
int launch_dense_t(const DenseParams& p, hipStream_t s) {
    dense_gemv_kernel<GPW, ZP><<<dim3((unsigned)(p.N / 16)), dim3(kDgThreads), 0, s>>>(p);
    return check_launch("dense_gemv_kernel");
}

}  // namespace

bool dense_gemv_supported(int64_t M, int64_t N, int64_t K, int64_t group_size, bool e2m1) {
    return M >= 1 && M <= 16 && group_size == kGroup && !e2m1 && K % (kDgWaves * kGroup) == 0 &&
           K >= kDgWaves * kGroup && K <= 4 * kDgWaves * kGroup && N % 16 == 0 && N > 0 &&
           N * (K / 2) < ((int64_t)1 << 31);
}

int launch_dense_gemv(const void* x_f16, int64_t M, int64_t K, const int32_t* w, const void* scales_f16,
                      const int32_t* zeros, int64_t N, void* out_f16, hipStream_t s) {
    if (!dense_gemv_supported(M, N, K, kGroup, false)) {
        set_error("dense GEMV: needs 1 <= M <= 16, group 128, K a multiple of 1024 up to 4096, N % 16 == 0");
        return W4A8_ERR_INVALID;
    }
    DenseParams p;
    p.x = static_cast<const __half*>(x_f16);
    p.w = w;
    p.s = static_cast<const __half*>(scales_f16);
    p.z = zeros;
    p.out = static_cast<__half*>(out_f16);
    p.M = (int)M;
    p.N = (int)N;
    p.K = (int)K;
    p.G = (int)(K / kGroup);
    const int gpw = p.G / kDgWaves;
    const bool zp = zeros != nullptr;
    switch (gpw) {
        case 1: return zp ? launch_dense_t<1, true>(p, s) : launch_dense_t<1, false>(p, s);
        case 2: return zp ? launch_dense_t<2, true>(p, s) : launch_dense_t<2, false>(p, s);
        case 3: return zp ? launch_dense_t<3, true>(p, s) : launch_dense_t<3, false>(p, s);
        default: return zp ? launch_dense_t<4, true>(p, s) : launch_dense_t<4, false>(p, s);
    }
}

}  // namespace w4a8
