// Per-token e4m3 activation quantisation of one row by one wave (device side), shared by
// the act-quant kernel and the fused decode prologue.
#pragma once

#include "w4a8_common.h"

namespace w4a8 {

template <bool BF16>
__device__ __forceinline__ float load_act(const void* x, int64_t i) {
    if constexpr (BF16) {
        // Reference casts bf16 activations to fp16 first (moe_experts.py:596).
        const float f = __bfloat162float(reinterpret_cast<const __hip_bfloat16*>(x)[i]);
        return __half2float(__float2half(f));
    } else {
        return __half2float(reinterpret_cast<const __half*>(x)[i]);
    }
}

// Element j (0..7) of 8 consecutive fp16 / bf16 activations packed in a uint4, as
// load_act would read it.
template <bool BF16>
__device__ __forceinline__ float act_from_u4(const uint4& v, int j) {
    const uint32_t w = j < 2 ? v.x : j < 4 ? v.y : j < 6 ? v.z : v.w;
    const uint16_t b = (j & 1) ? (uint16_t)(w >> 16) : (uint16_t)(w & 0xFFFF);
    if constexpr (BF16) {
        const float f = __uint_as_float((uint32_t)b << 16);
        return __half2float(__float2half(f));
    } else {
        return __half2float(__ushort_as_half(b));
    }
}

template <bool BF16>
__device__ __forceinline__ void quantize_row_scalar(const void* __restrict__ x, int64_t row, int K,
                                                    uint8_t* __restrict__ q,
                                                    float* __restrict__ scales, bool k8,
                                                    float* __restrict__ gsum, int lane);

// A row of up to 4096 fp16 / bf16 values held by one wave: 16 bytes per lane and
// 512-wide pass.
struct RowRegs {
    static constexpr int kMaxPass = 8;
    uint4 v[kMaxPass];
};
__device__ __forceinline__ bool row_load(const void* __restrict__ x, int64_t row, int K, int lane,
                                         RowRegs& rr);
template <bool BF16>
__device__ __forceinline__ void quantize_row_regs(const RowRegs& rr, int64_t row, int K,
                                                  uint8_t* __restrict__ q,
                                                  float* __restrict__ scales, bool k8,
                                                  float* __restrict__ gsum, int lane);

// Group sum of one 512-wide pass (lanes 16j..16j+15 hold group k/128): fixed-order tree.
__device__ __forceinline__ void row_group_sum(uint32_t lo, uint32_t hi, int64_t row, int K, int k,
                                              float* __restrict__ gsum, int lane) {
    float t = e4m3_pair_sum(0.f, lo, hi);
    t = lane_allreduce<4>(t, SumOp{});
    if ((lane & 15) == 0 && k < K) gsum[row * (K / 128) + k / 128] = t;
}

// One wave quantises row `row` (moe_kernel.hip:87-127): s = max(absmax/448, 1e-8),
// q = e4m3_RNE(x * (1/s)). k8: bytes in the kernels' k8-interleaved order. gsum (optional,
// K % 128 == 0): per 128-wide group, the sum of the e4m3 values.
template <bool BF16>
__device__ __forceinline__ void quantize_row(const void* __restrict__ x, int64_t row, int K,
                                             uint8_t* __restrict__ q, float* __restrict__ scales,
                                             bool k8, float* __restrict__ gsum, int lane) {
    // Rows of up to 4096 values with 16-byte aligned starts: one 16-byte load per lane and
    // 512-wide pass, the row kept in registers between the absmax and the quantisation.
    // Same arithmetic as the element-wise form below, so the same bytes.
    RowRegs rr;
    if (!row_load(x, row, K, lane, rr)) {
        quantize_row_scalar<BF16>(x, row, K, q, scales, k8, gsum, lane);
        return;
    }
    quantize_row_regs<BF16>(rr, row, K, q, scales, k8, gsum, lane);
}

// The 16-byte loads of quantize_row: false (nothing loaded) when the row is longer than
// 4096 values or its start is not 16-byte aligned.
__device__ __forceinline__ bool row_load(const void* __restrict__ x, int64_t row, int K, int lane,
                                         RowRegs& rr) {
    const int npass = (K + 511) / 512;
    const char* rowp = reinterpret_cast<const char*>(x) + row * K * 2;
    if (npass > RowRegs::kMaxPass || (reinterpret_cast<uintptr_t>(rowp) & 15) != 0) return false;
#pragma unroll
    for (int ps = 0; ps < RowRegs::kMaxPass; ++ps) {
        const int k = ps * 512 + lane * 8;
        rr.v[ps] = make_uint4(0, 0, 0, 0);
        if (ps < npass && k < K) rr.v[ps] = *reinterpret_cast<const uint4*>(rowp + k * 2);
    }
    return true;
}

// quantize_row on a row already in registers (row_load).
template <bool BF16>
__device__ __forceinline__ void quantize_row_regs(const RowRegs& rr, int64_t row, int K,
                                                  uint8_t* __restrict__ q,
                                                  float* __restrict__ scales, bool k8,
                                                  float* __restrict__ gsum, int lane) {
    constexpr int kMaxPass = RowRegs::kMaxPass;
    const int npass = (K + 511) / 512;
    const uint4* v = rr.v;
    // absmax on the magnitude bits, two values per instruction (packed 16-bit max): the
    // conversions to the fp16-rounded fp32 value are monotone in them. NaNs, which the fmaxf
    // form below skips, lie above the infinity pattern; only a lane that holds one takes that
    // exact form.
    constexpr uint32_t nan_above = BF16 ? 0x7F80u : 0x7C00u;
    using u16x2 = unsigned short __attribute__((ext_vector_type(2)));
    u16x2 m2 = {0, 0};
#pragma unroll
    for (int ps = 0; ps < kMaxPass; ++ps) {
        if (ps >= npass) break;
        if (ps * 512 + lane * 8 >= K) continue;
        const uint32_t wd[4] = {v[ps].x, v[ps].y, v[ps].z, v[ps].w};
#pragma unroll
        for (int j = 0; j < 4; ++j)
            m2 = __builtin_elementwise_max(m2, __builtin_bit_cast(u16x2, wd[j] & 0x7FFF7FFFu));
    }
    const uint32_t mbits = max((uint32_t)m2.x, (uint32_t)m2.y);
    float amax;
    if (__builtin_expect(mbits <= nan_above, 1)) {
        amax = act_from_u4<BF16>(make_uint4(mbits, 0u, 0u, 0u), 0);
    } else {
        amax = 0.0f;
#pragma unroll
        for (int ps = 0; ps < kMaxPass; ++ps) {
            if (ps >= npass) break;
            if (ps * 512 + lane * 8 >= K) continue;
#pragma unroll
            for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fabsf(act_from_u4<BF16>(v[ps], j)));
        }
    }
    amax = wave_max(amax);
    const float s = act_scale_from_absmax(amax);
    if (lane == 0) scales[row] = s;
    const float inv = 1.0f / s;
    const int64_t base = row * K;
#pragma unroll
    for (int ps = 0; ps < kMaxPass; ++ps) {
        if (ps >= npass) break;
        const int k = ps * 512 + lane * 8;
        uint32_t lo = 0, hi = 0;
        if (k < K) {
            float f[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) f[j] = act_from_u4<BF16>(v[ps], j) * inv;
            if (k8) {
                lo = pack4_e4m3(f[0], f[2], f[4], f[6]);
                hi = pack4_e4m3(f[1], f[3], f[5], f[7]);
            } else {
                lo = pack4_e4m3(f[0], f[1], f[2], f[3]);
                hi = pack4_e4m3(f[4], f[5], f[6], f[7]);
            }
            *reinterpret_cast<uint2*>(q + base + k) = make_uint2(lo, hi);
        }
        if (gsum != nullptr) row_group_sum(lo, hi, row, K, k, gsum, lane);
    }
}

template <bool BF16>
__device__ __forceinline__ void quantize_row_scalar(const void* __restrict__ x, int64_t row, int K,
                                                    uint8_t* __restrict__ q,
                                                    float* __restrict__ scales, bool k8,
                                                    float* __restrict__ gsum, int lane) {
    const int64_t base = row * K;
    float amax = 0.0f;
    for (int k = lane * 8; k < K; k += 64 * 8) {
#pragma unroll
        for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fabsf(load_act<BF16>(x, base + k + j)));
    }
    amax = wave_max(amax);
    const float s = act_scale_from_absmax(amax);
    if (lane == 0) scales[row] = s;
    const float inv = 1.0f / s;
    // every lane runs every 512-wide pass (inactive lanes add zero) so the group-sum
    // shuffles always see a full wave
    for (int k0 = 0; k0 < K; k0 += 64 * 8) {
        const int k = k0 + lane * 8;
        uint32_t lo = 0, hi = 0;
        if (k < K) {
            float v[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) v[j] = load_act<BF16>(x, base + k + j) * inv;
            if (k8) {
                lo = pack4_e4m3(v[0], v[2], v[4], v[6]);
                hi = pack4_e4m3(v[1], v[3], v[5], v[7]);
            } else {
                lo = pack4_e4m3(v[0], v[1], v[2], v[3]);
                hi = pack4_e4m3(v[4], v[5], v[6], v[7]);
            }
            *reinterpret_cast<uint2*>(q + base + k) = make_uint2(lo, hi);
        }
        if (gsum != nullptr) row_group_sum(lo, hi, row, K, k, gsum, lane);
    }
}

}  // namespace w4a8
