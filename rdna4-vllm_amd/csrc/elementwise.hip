// Activation quantisation, int4 dequant, SiLU*mul, reductions and casts (gfx950).
#include "w4a8_common.h"
#include "w4a8_internal.h"
#include "act_quant.h"

namespace w4a8 {
namespace {

constexpr int kWavesPerBlock = 4;

// One wave per row (moe_kernel.hip:87-127).
// Optional row filter (sorted_ids/ntp/num_valid): rows that are padding in the
// moe_align layout are skipped, so uninitialised padding rows are never read.
template <bool BF16>
__global__ void __launch_bounds__(256) act_quant_kernel(
    const void* __restrict__ x, int64_t rows, int K, uint8_t* __restrict__ q,
    float* __restrict__ scales, bool k8, const int32_t* __restrict__ sorted_ids,
    const int32_t* __restrict__ ntp, int64_t num_valid, float* __restrict__ gsum) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);
    if (row >= rows) return;
    if (sorted_ids != nullptr && (row >= ntp[0] || sorted_ids[row] >= num_valid)) return;
    quantize_row<BF16>(x, row, K, q, scales, k8, gsum, lane);
}

// One thread per (row, 8-wide k chunk): decode 8 nibbles through the same table path the
// GEMM kernels use, then restore natural k order for the caller.
__global__ void dequant_kernel(const int32_t* __restrict__ w, const int32_t* __restrict__ z,
                               int64_t E, int64_t N, int K, int gs, bool e2m1,
                               uint8_t* __restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int kw = K / kPackFactor;
    if (i >= E * N * kw) return;
    const int64_t row = i / kw;
    const int c = (int)(i % kw);
    const int64_t e = row / N;
    const int n = (int)(row % N);
    const int G = K / gs;
    const int g = (c * kPackFactor) / gs;
    const int* ze = z ? z + e * (N / 8) * G : nullptr;
    const uint4 t = load_table(table_index(ze, n, g, G, e2m1));
    uint32_t lo, hi;
    decode8(static_cast<uint32_t>(w[i]), t, lo, hi);
    // lo = {k0,k2,k4,k6}, hi = {k1,k3,k5,k7} -> natural order
    const uint32_t o0 = __builtin_amdgcn_perm(hi, lo, 0x05010400u);
    const uint32_t o1 = __builtin_amdgcn_perm(hi, lo, 0x07030602u);
    *reinterpret_cast<uint2*>(out + i * 8) = make_uint2(o0, o1);
}

__global__ void silu_and_mul_kernel(const __half* __restrict__ in, int64_t rows, int inter,
                                    __half* __restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= rows * inter) return;
    const int64_t r = i / inter;
    const int c = (int)(i % inter);
    out[i] = silu_mul_h(in[r * 2 * inter + c], in[r * 2 * inter + inter + c]);
}

// gpt-oss gated activation (vLLM's swigluoai_and_mul, the activation the reference's mxfp4
// hook passes to apply_moe_activation, moe_experts.py:1416-1424): gate and up interleaved
// along the row (gate = x[2c], up = x[2c + 1]); in fp32, g = min(gate, limit),
// u = clamp(up, -limit, limit), out = fp16((u + 1) * (g * (1 / (1 + exp(-g * alpha))))).
__global__ void swigluoai_and_mul_kernel(const __half* __restrict__ in, int64_t rows, int inter,
                                         float alpha, float limit, __half* __restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= rows * inter) return;
    const int64_t r = i / inter;
    const int c = (int)(i % inter);
    const __half2 gu = *reinterpret_cast<const __half2*>(in + r * 2 * inter + 2 * c);
    const float gate = __low2float(gu), up = __high2float(gu);
    const float g = gate > limit ? limit : gate;
    const float u = up > limit ? limit : (up < -limit ? -limit : up);
    const float sig = 1.0f / (1.0f + expf(as_f32(-g * alpha)));
    const float glu = as_f32(g * sig);
    out[i] = __float2half(as_f32((u + 1.0f) * glu));
}

__global__ void inverse_map_kernel(const int32_t* __restrict__ sorted_ids,
                                   const int32_t* __restrict__ ntp, int64_t P, int64_t m_tk,
                                   int32_t* __restrict__ slot_to_row) {
    const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= P || r >= ntp[0]) return;
    const int32_t s = sorted_ids[r];
    if (s >= 0 && s < m_tk) slot_to_row[s] = (int32_t)r;
}

__global__ void fill_i32_kernel(int32_t* __restrict__ p, int64_t n, int32_t v) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = v;
}

// out[t, n] = sum_{j asc} w[t*k+j] * out2[row(t,j), n] (moe_kernel.hip:1241-1258).
__global__ void gather_reduce_kernel(const __half* __restrict__ out2,
                                     const int32_t* __restrict__ slot_to_row,
                                     const float* __restrict__ tw, int64_t M, int N, int top_k,
                                     float* __restrict__ out) {
    const int64_t t = blockIdx.y;
    const int n = blockIdx.x * blockDim.x + threadIdx.x;
    if (n >= N || t >= M) return;
    float acc = 0.0f;
    for (int j = 0; j < top_k; ++j) {
        const int32_t r = slot_to_row[t * top_k + j];
        if (r >= 0) acc = fmaf(tw[t * top_k + j], __half2float(out2[(int64_t)r * N + n]), acc);
    }
    out[t * N + n] = acc;
}

template <bool BF16, int KMAX>
__global__ void slot_reduce_kernel(const float* __restrict__ y, const float* __restrict__ tw,
                                   const int32_t* __restrict__ ids,
                                   const int32_t* __restrict__ emap, int emap_len, int E,
                                   int64_t T, int N, int top_k, void* __restrict__ out,
                                   SlotReduceSync sync) {
    const int64_t t = blockIdx.y;
    const int n = (blockIdx.x * blockDim.x + threadIdx.x) * 4;
    // after the fused decode layer: its completion flags go back to 0 for the next call, and
    // a wait of this call that gave up (never expected) turns the whole output into NaN
    // instead of leaving rows that may have read unpublished h. Every work-group of that
    // launch has its own timeout word, which it clears itself when it starts, so a wait that
    // gave up in one call (or one graph replay) does not mark the next.
    bool failed = false;
    if (sync.timeout != nullptr) {   // uniform over the grid: every thread reaches the barrier
        bool mine = false;
        for (int i = threadIdx.x; i < sync.ntimeout; i += blockDim.x)
            mine = mine || sync.timeout[i] == sync.nonce;
        failed = __syncthreads_or(mine) != 0;
    }
    if (sync.flags != nullptr && blockIdx.x == 0 && blockIdx.y == 0)
        for (int i = threadIdx.x; i < sync.nflags; i += blockDim.x) sync.flags[i] = 0;
    if (n >= N || t >= T) return;
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    auto expert_of = [&](int j) {
        int e = ids[t * top_k + j];
        if (emap != nullptr) e = (e >= 0 && e < emap_len) ? emap[e] : -1;
        return e;
    };
    if constexpr (KMAX > 0) {
        // the token's ids, weights and all its slot rows requested together (every slot row
        // exists; a slot without a local expert is read and left out), then summed over j
        // ascending: one memory round trip instead of one per slot
        int e[KMAX];
        float w[KMAX];
        float4 v[KMAX];
#pragma unroll
        for (int j = 0; j < KMAX; ++j) {
            if (j < top_k) {
                e[j] = expert_of(j);
                w[j] = tw[t * top_k + j];
                v[j] = *reinterpret_cast<const float4*>(y + (t * top_k + j) * N + n);
            }
        }
#pragma unroll
        for (int j = 0; j < KMAX; ++j) {
            if (j < top_k && e[j] >= 0 && e[j] < E) {
                acc[0] = fmaf(w[j], v[j].x, acc[0]);
                acc[1] = fmaf(w[j], v[j].y, acc[1]);
                acc[2] = fmaf(w[j], v[j].z, acc[2]);
                acc[3] = fmaf(w[j], v[j].w, acc[3]);
            }
        }
    } else {
        for (int j = 0; j < top_k; ++j) {
            const int e = expert_of(j);
            if (e < 0 || e >= E) continue;
            const float w = tw[t * top_k + j];
            const float4 v = *reinterpret_cast<const float4*>(y + (t * top_k + j) * N + n);
            acc[0] = fmaf(w, v.x, acc[0]);
            acc[1] = fmaf(w, v.y, acc[1]);
            acc[2] = fmaf(w, v.z, acc[2]);
            acc[3] = fmaf(w, v.w, acc[3]);
        }
    }
    if (failed)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i] = __builtin_nanf("");
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        if constexpr (BF16)
            reinterpret_cast<__hip_bfloat16*>(out)[t * N + n + i] = __float2bfloat16(acc[i]);
        else
            reinterpret_cast<__half*>(out)[t * N + n + i] = __float2half(as_f32(acc[i]));
    }
}

// Prefill combine (moe_kernel.hip:1241-1258 with the inverse map built by the align):
// eight columns per thread, fp32 accumulation over j ascending. KMAX > 0: the token's rows
// and weights (top_k <= KMAX) are read first and all its row loads go out together;
// KMAX == 0: any top_k, one row at a time.
template <bool BF16, int KMAX>
__global__ void row_reduce_kernel(const __half* __restrict__ y, const int32_t* __restrict__ s2r,
                                  const float* __restrict__ tw, int64_t T, int N, int top_k,
                                  void* __restrict__ out) {
    const int64_t t = blockIdx.y;
    const int n = (blockIdx.x * blockDim.x + threadIdx.x) * 8;
    if (n >= N || t >= T) return;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    auto add_row = [&](float w, const uint4& v) {
        const uint32_t u[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            acc[2 * i] = fmaf(w, __half2float(__ushort_as_half((unsigned short)(u[i] & 0xFFFFu))), acc[2 * i]);
            acc[2 * i + 1] = fmaf(w, __half2float(__ushort_as_half((unsigned short)(u[i] >> 16))), acc[2 * i + 1]);
        }
    };
    if constexpr (KMAX > 0) {
        int32_t r[KMAX];
        float w[KMAX];
#pragma unroll
        for (int j = 0; j < KMAX; ++j) {
            r[j] = j < top_k ? s2r[t * top_k + j] : -1;
            w[j] = j < top_k ? tw[t * top_k + j] : 0.f;
        }
        uint4 v[KMAX];
#pragma unroll
        for (int j = 0; j < KMAX; ++j)
            v[j] = r[j] >= 0 ? *reinterpret_cast<const uint4*>(y + (int64_t)r[j] * N + n) : make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
        for (int j = 0; j < KMAX; ++j)
            if (r[j] >= 0) add_row(w[j], v[j]);
    } else {
        for (int j = 0; j < top_k; ++j) {
            const int32_t r = s2r[t * top_k + j];
            if (r < 0) continue;
            add_row(tw[t * top_k + j], *reinterpret_cast<const uint4*>(y + (int64_t)r * N + n));
        }
    }
    uint32_t o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        if constexpr (BF16) {
            const uint32_t lo = __bfloat16_as_ushort(__float2bfloat16(acc[2 * i]));
            const uint32_t hi = __bfloat16_as_ushort(__float2bfloat16(acc[2 * i + 1]));
            o[i] = lo | (hi << 16);
        } else {
            const uint32_t lo = __half_as_ushort(__float2half(as_f32(acc[2 * i])));
            const uint32_t hi = __half_as_ushort(__float2half(as_f32(acc[2 * i + 1])));
            o[i] = lo | (hi << 16);
        }
    }
    *reinterpret_cast<uint4*>(reinterpret_cast<uint16_t*>(out) + t * N + n) = make_uint4(o[0], o[1], o[2], o[3]);
}

template <bool BF16>
__global__ void cast_f32_kernel(const float* __restrict__ in, int64_t n, void* __restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    if constexpr (BF16)
        reinterpret_cast<__hip_bfloat16*>(out)[i] = __float2bfloat16(in[i]);
    else
        reinterpret_cast<__half*>(out)[i] = __float2half(in[i]);
}

__global__ void zero_f32_kernel(float* __restrict__ p, int64_t n) {
    const int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
    if (i + 3 < n) {
        *reinterpret_cast<float4*>(p + i) = make_float4(0.f, 0.f, 0.f, 0.f);
    } else {
        for (int64_t j = i; j < n; ++j) p[j] = 0.f;
    }
}

inline unsigned blocks_for(int64_t n, int per) { return (unsigned)((n + per - 1) / per); }

}  // namespace

int launch_act_quant(const void* x, bool x_bf16, int64_t rows, int64_t K, uint8_t* x_fp8,
                     float* scales, bool k8, hipStream_t stream, const int32_t* sorted_ids,
                     const int32_t* ntp, int64_t num_valid, float* group_sums) {
    if (rows == 0) return W4A8_OK;
    if (group_sums != nullptr && K % 128 != 0) {
        set_error("act_quant: group sums need K % 128 == 0");
        return W4A8_ERR_INVALID;
    }
    dim3 grid(blocks_for(rows, kWavesPerBlock)), block(64 * kWavesPerBlock);
    if (x_bf16)
        act_quant_kernel<true><<<grid, block, 0, stream>>>(x, rows, (int)K, x_fp8, scales, k8,
                                                          sorted_ids, ntp, num_valid, group_sums);
    else
        act_quant_kernel<false><<<grid, block, 0, stream>>>(x, rows, (int)K, x_fp8, scales, k8,
                                                           sorted_ids, ntp, num_valid, group_sums);
    return check_launch("act_quant_kernel");
}

int launch_dequant(const int32_t* w, const int32_t* z, int64_t E, int64_t N, int64_t K,
                   int64_t gs, bool e2m1, uint8_t* out, hipStream_t stream) {
    const int64_t n = E * N * (K / kPackFactor);
    if (n == 0) return W4A8_OK;
    dequant_kernel<<<blocks_for(n, 256), 256, 0, stream>>>(w, z, E, N, (int)K, (int)gs, e2m1,
                                                          out);
    return check_launch("dequant_kernel");
}

int launch_swigluoai_and_mul(const void* in, int64_t rows, int64_t inter, float alpha,
                             float limit, void* out, hipStream_t stream) {
    const int64_t n = rows * inter;
    if (n == 0) return W4A8_OK;
    swigluoai_and_mul_kernel<<<blocks_for(n, 256), 256, 0, stream>>>(
        static_cast<const __half*>(in), rows, (int)inter, alpha, limit, static_cast<__half*>(out));
    return check_launch("swigluoai_and_mul_kernel");
}

int launch_silu_and_mul(const void* in, int64_t rows, int64_t inter, void* out,
                        hipStream_t stream) {
    const int64_t n = rows * inter;
    if (n == 0) return W4A8_OK;
    silu_and_mul_kernel<<<blocks_for(n, 256), 256, 0, stream>>>(
        static_cast<const __half*>(in), rows, (int)inter, static_cast<__half*>(out));
    return check_launch("silu_and_mul_kernel");
}

int launch_gather_reduce(const void* out2, int64_t P, int64_t N, const int32_t* sorted_ids,
                         const float* tw, int64_t m_tk, const int32_t* ntp, int64_t top_k,
                         float* out, int32_t* slot_to_row, hipStream_t stream) {
    const int64_t M = m_tk / top_k;
    if (m_tk > 0) {
        fill_i32_kernel<<<blocks_for(m_tk, 256), 256, 0, stream>>>(slot_to_row, m_tk, -1);
        if (int rc = check_launch("fill_i32_kernel")) return rc;
    }
    if (P > 0) {
        inverse_map_kernel<<<blocks_for(P, 256), 256, 0, stream>>>(sorted_ids, ntp, P, m_tk,
                                                                  slot_to_row);
        if (int rc = check_launch("inverse_map_kernel")) return rc;
    }
    if (M == 0 || N == 0) return W4A8_OK;
    dim3 grid(blocks_for(N, 256), (unsigned)M);
    gather_reduce_kernel<<<grid, 256, 0, stream>>>(static_cast<const __half*>(out2),
                                                   slot_to_row, tw, M, (int)N, (int)top_k, out);
    return check_launch("gather_reduce_kernel");
}

int launch_slot_reduce(const float* y, const float* tw, const int32_t* ids,
                       const int32_t* emap, int64_t emap_len, int64_t E, int64_t T, int64_t N,
                       int64_t top_k, void* out, bool out_bf16, hipStream_t stream,
                       SlotReduceSync sync) {
    if (T == 0 || N == 0) return W4A8_OK;
    // 128 threads of four columns per work-group: a decode batch spreads over more CUs
    dim3 grid(blocks_for(N / 4, 128), (unsigned)T);
    auto go = [&](auto kernel) {
        kernel<<<grid, 128, 0, stream>>>(y, tw, ids, emap, (int)emap_len, (int)E, T, (int)N,
                                         (int)top_k, out, sync);
    };
    if (top_k <= 8) {
        if (out_bf16) go(slot_reduce_kernel<true, 8>);
        else go(slot_reduce_kernel<false, 8>);
    } else if (out_bf16) {
        go(slot_reduce_kernel<true, 0>);
    } else {
        go(slot_reduce_kernel<false, 0>);
    }
    return check_launch("slot_reduce_kernel");
}

int launch_row_reduce(const void* y, const int32_t* s2r, const float* tw, int64_t T,
                      int64_t N, int64_t top_k, void* out, bool out_bf16, hipStream_t stream) {
    if (T == 0 || N == 0) return W4A8_OK;
    if (N % 8 != 0) {
        set_error("row_reduce: N must be a multiple of 8");
        return W4A8_ERR_INVALID;
    }
    dim3 grid(blocks_for(N / 8, 256), (unsigned)T);
    const __half* yh = static_cast<const __half*>(y);
    if (top_k <= 8) {
        if (out_bf16)
            row_reduce_kernel<true, 8><<<grid, 256, 0, stream>>>(yh, s2r, tw, T, (int)N, (int)top_k, out);
        else
            row_reduce_kernel<false, 8><<<grid, 256, 0, stream>>>(yh, s2r, tw, T, (int)N, (int)top_k, out);
    } else if (out_bf16) {
        row_reduce_kernel<true, 0><<<grid, 256, 0, stream>>>(yh, s2r, tw, T, (int)N, (int)top_k, out);
    } else {
        row_reduce_kernel<false, 0><<<grid, 256, 0, stream>>>(yh, s2r, tw, T, (int)N, (int)top_k, out);
    }
    return check_launch("row_reduce_kernel");
}

int launch_cast_f32(const float* in, int64_t n, void* out, bool out_bf16, hipStream_t stream) {
    if (n == 0) return W4A8_OK;
    if (out_bf16)
        cast_f32_kernel<true><<<blocks_for(n, 256), 256, 0, stream>>>(in, n, out);
    else
        cast_f32_kernel<false><<<blocks_for(n, 256), 256, 0, stream>>>(in, n, out);
    return check_launch("cast_f32_kernel");
}

int launch_zero_f32(float* p, int64_t n, hipStream_t stream) {
    if (n == 0) return W4A8_OK;
    zero_f32_kernel<<<blocks_for((n + 3) / 4, 256), 256, 0, stream>>>(p, n);
    return check_launch("zero_f32_kernel");
}

}  // namespace w4a8
