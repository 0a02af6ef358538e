// Router selection of one token by one wave: softmax -> top-k -> renormalise (the vLLM
// fused_topk contract, moe_experts.py:587-589 call site), shared by the router kernel
// (routing.hip) and the decode layer's in-kernel routing (decode_gemv.hip).
#pragma once
#include "w4a8_common.h"

namespace w4a8 {

constexpr int kRouterMaxPerLane = 16;   // E <= 1024

// NV = logits per lane (E <= 64 * NV). Loads are unconditional (clamped index, the
// out-of-range entries masked to -inf afterwards) so they issue together.
// Selection key: the logit's bits mapped to an unsigned order (a larger key is a larger
// logit), at least 1; entries past E and entries already picked hold 0. Equal keys go to
// the lower expert id (the router's tie-break).
__device__ __forceinline__ uint32_t topk_key(float v) {
    uint32_t b = __float_as_uint(v);
    b = (b & 0x80000000u) ? ~b : (b | 0x80000000u);   // order-preserving float -> uint
    return b > 1u ? b : 1u;
}
__device__ __forceinline__ float topk_key_value(uint32_t key) {
    const uint32_t b = (key & 0x80000000u) ? (key & 0x7FFFFFFFu) : ~key;
    return __uint_as_float(b);
}
struct MaxU32Op {   // unsigned maximum of two words carried in float registers
    __device__ float operator()(float a, float b) const {
        return __uint_as_float(max(__float_as_uint(a), __float_as_uint(b)));
    }
};

// Softmax + top-k of one token's logits row l (E <= 64 * NV) by one wave: lane j < top_k
// writes pick j (weight, expert) to tw[j] / ids[j] and, if ids_lds is given, the expert to
// ids_lds[j] too. Picks are made on the logits (exact ids); the weights are
// exp(l - max) / sum exp(l - max), renormalised over the picks in pick order.
template <int NV>
__device__ __forceinline__ void topk_load(const float* __restrict__ l, int E, int lane, float (&v)[NV]) {
#pragma unroll
    for (int i = 0; i < NV; ++i) v[i] = l[min(lane + 64 * i, E - 1)];
}

// Selection of one token from its logits v (lane l holds entries l + 64 i).
template <int NV>
__device__ __forceinline__ void topk_select(float (&v)[NV], int E, int top_k, bool renorm,
                                            float* __restrict__ tw, int32_t* __restrict__ ids,
                                            int32_t* ids_lds, int lane) {
    float m = -INFINITY;
    uint32_t key[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const bool in = lane + 64 * i < E;
        if (!in) v[i] = -INFINITY;
        m = fmaxf(m, v[i]);
        key[i] = in ? topk_key(v[i]) : 0u;
    }
    m = wave_max(m);
    float ssum = 0.f;
#pragma unroll
    for (int i = 0; i < NV; ++i) ssum += lane + 64 * i < E ? expf(v[i] - m) : 0.f;
    ssum = wave_sum(ssum);
    uint32_t mine_key = 0;   // lane j < top_k: pick j
    int mine_e = 0;
    for (int j = 0; j < top_k; ++j) {
        uint32_t best = 0;
#pragma unroll
        for (int i = 0; i < NV; ++i) best = max(best, key[i]);
        best = __float_as_uint(lane_allreduce<6>(__uint_as_float(best), MaxU32Op{}));
        // the lowest expert holding it: lowest entry index i with a holder, lowest lane there
        int pick = 0;
#pragma unroll
        for (int i = NV - 1; i >= 0; --i) {
            const uint64_t h = __ballot(key[i] == best);
            if (h != 0) pick = (int)__builtin_ctzll(h) + 64 * i;
        }
#pragma unroll
        for (int i = 0; i < NV; ++i) key[i] = (lane + 64 * i == pick) ? 0u : key[i];   // taken
        mine_key = lane == j ? best : mine_key;
        mine_e = lane == j ? pick : mine_e;
    }
    const float p = expf(topk_key_value(mine_key) - m) / ssum;
    float sum_sel = 0.f;   // picks in order, as a sequential sum
    for (int j = 0; j < top_k; ++j)
        sum_sel += __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(p), j));
    if (lane < top_k) {
        if (tw != nullptr) {   // null: only the LDS copy of the ids is wanted
            tw[lane] = renorm ? p / sum_sel : p;
            ids[lane] = mine_e;
        }
        if (ids_lds != nullptr) ids_lds[lane] = mine_e;
    }
}

}  // namespace w4a8
