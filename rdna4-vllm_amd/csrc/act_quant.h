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

// One wave quantises row `row` (moe_kernel.hip:87-127): s = max(absmax/448, 1e-8),
// q = e4m3_RNE(x * (1/s)). k8: bytes in the kernels' k8-interleaved order. gsum (optional,
// K % 128 == 0): per 128-wide group, the sum of the e4m3 values.
template <bool BF16>
__device__ __forceinline__ void quantize_row(const void* __restrict__ x, int64_t row, int K,
                                             uint8_t* __restrict__ q, float* __restrict__ scales,
                                             bool k8, float* __restrict__ gsum, int lane) {
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
        if (gsum != nullptr) {
            // lanes 16j..16j+15 hold group k/128 of this pass: fixed-order tree sum
            float t = 0.f;
#pragma unroll
            for (int b = 0; b < 4; ++b)
                t += e4m3_to_f32((lo >> (8 * b)) & 0xFF) + e4m3_to_f32((hi >> (8 * b)) & 0xFF);
            t = lane_allreduce<4>(t, SumOp{});
            if ((lane & 15) == 0 && k < K) gsum[row * (K / 128) + k / 128] = t;
        }
    }
}

}  // namespace w4a8
