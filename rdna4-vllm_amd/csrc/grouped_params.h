// Launch parameters and row resolution shared by the grouped GEMM schedules (device side).
#pragma once

#include "w4a8_common.h"
#include "w4a8_internal.h"

namespace w4a8 {

constexpr int kGroup = 128;          // K per group == K per fp8 MFMA
// Raw-nibble MFMA operands carry n * 2^-9; results are scaled back by 2^9.
constexpr float kNibbleScale = 512.0f;

// Fragment layout (repack.hip): per expert and 16-row tile, G 1 KB blocks (256 words each)
// and then G * 16 metadata words (row r, group g at word 256 G + r G + g: fp16 scale bits
// 0..15, zero-point bits 16..19).
__host__ __device__ constexpr int frag_tile_words(int G) { return 272 * G; }
__host__ __device__ constexpr int frag_meta_word(int G, int r, int g) { return 256 * G + r * G + g; }

struct Params {
    const uint8_t* xq;          // (x_rows, K) e4m3, k8-interleaved
    const float* asc;           // (x_rows,)
    const void* xh;             // (x_rows, K) fp16/bf16 rows (fused quantisation path)
    const int32_t* w;           // (E, N, K/8), or fragment layout when w_frag (E, N/16, 272 G)
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
    int xbf16;                  // xh holds bf16 (else fp16)
    int w_frag;                 // w in fragment layout (16-row tile, group, lane)
    const float* asum;          // (x_rows, K/128) sums of the e4m3 values per group, or null
    int xcd_slots;              // activation-resident tiles: work-groups one XCD runs at once
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

inline Params make_params(const GroupedArgs& a) {
    Params p;
    p.xq = a.x_fp8;
    p.asc = a.act_scales;
    p.xh = a.x;
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
    p.xbf16 = a.x_bf16 ? 1 : 0;
    p.asum = a.act_group_sums;
    p.w_frag = a.w_frag ? 1 : 0;
    p.xcd_slots = 0;
    return p;
}

__device__ __forceinline__ v4f mfma_16x16x128(const v8i& a, const v8i& b, const v4f& c) {
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}

// A word's eight nibbles as e4m3 bytes n * 2^-9 (the byte with value n, 0..15, is that
// number exactly: subnormals 0..7, exponent field 1 for 8..15), in k8-interleave order:
// low nibbles {k0,k2,k4,k6} then high nibbles {k1,k3,k5,k7}.
__device__ __forceinline__ v8i spread_nibbles(uint4 w) {
    constexpr uint32_t m = 0x0F0F0F0Fu;
    return v8i{(int)(w.x & m), (int)((w.x >> 4) & m), (int)(w.y & m), (int)((w.y >> 4) & m),
               (int)(w.z & m), (int)((w.z >> 4) & m), (int)(w.w & m), (int)((w.w >> 4) & m)};
}

}  // namespace w4a8
