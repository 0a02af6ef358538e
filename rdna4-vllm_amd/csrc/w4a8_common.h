// Shared device helpers for the gfx950 W4A8 MoE kernels.
//
// Numeric contract (patcarter883/rdna4-vllm, w4a8_fp8_wmma/):
//   * activations: per-row s = max(absmax/448, 1e-8), q = e4m3_RNE(x * (1/s))
//     (moe_kernel.hip:87-127);
//   * weights: the e4m3 byte of (nibble - zp), exact because |nibble - zp| <= 15
//     (tile_config.h:42-45); zp = 8 when no zero-points; E2M1 codebook when
//     weight_is_e2m1 (tile_config.h:59-71);
//   * per 128-wide K group: fp32 partial sum, then run += partial * scale[n, g]
//     (moe_gemm_tiled.h:144-151).
//
// fp8 byte order of activation scratch ("k8 interleave"): within every 8-byte block
// the byte at position p holds k = 8*block + kPerm8[p], kPerm8 = {0,2,4,6,1,3,5,7}.
// That is the order the nibble decoder below produces for weights (low nibbles of a
// dword, then high nibbles), so A and B fragments pair the same k in every MFMA
// without re-interleaving the decoded weights.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <hip/hip_bf16.h>
#include <cstdint>

namespace w4a8 {

constexpr int kPackFactor = 8;      // int4 nibbles per int32 word
constexpr float kE4m3Max = 448.0f;
constexpr float kActScaleFloor = 1e-8f;
constexpr int kMaxGroupSize = 128;
constexpr int kNumDecodeTables = 17;  // zp = 0..15, then the E2M1 codebook
constexpr int kE2m1Table = 16;

using v8i = int __attribute__((ext_vector_type(8)));
using v4i = int __attribute__((ext_vector_type(4)));
// 16-byte register staging of a load on its way to LDS. Arrays of the uint4 wrapper struct
// were kept in scratch (each piece stored there as soon as its load returned); arrays of
// this native vector stay in registers.
using u32x4 = uint32_t __attribute__((ext_vector_type(4)));

// An opaque copy of a per-lane 32-bit value. Loads at a wave-uniform base plus such an
// offset issue in the scalar-base form; without the copy, loop strength reduction and
// hoisting turn the addresses into 64-bit per-lane values held (and spilled) across loops.
__device__ __forceinline__ uint32_t opaque_u32(uint32_t v) {
    asm volatile("" : "+v"(v));
    return v;
}

// 16-byte streaming load (slc/nt): weights are read once per launch, so keep them from
// displacing reused data in the caches.
__device__ __forceinline__ uint4 load_stream16(const void* p) {
    const v4i v = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(p));
    return make_uint4((uint32_t)v.x, (uint32_t)v.y, (uint32_t)v.z, (uint32_t)v.w);
}
// cache-policy operand of the buffer intrinsics on gfx950: sc1 (agent coherence, the bit
// agent-scope atomics carry)
constexpr int kCpolSc1 = 16;
using v4f = float __attribute__((ext_vector_type(4)));
using v16f = float __attribute__((ext_vector_type(16)));

// Nibble -> e4m3 byte tables, 4 dwords each (entry i in byte i%4 of dword i/4).
// Table z < 16 holds e4m3(n - z) for n = 0..15; table 16 holds e4m3 of the OCP E2M1
// codebook {0,.5,1,1.5,2,3,4,6,-0,-.5,...,-6}. Every entry is exact in e4m3.
static __constant__ uint32_t g_decode_tables[kNumDecodeTables][4] = {
    {0x44403800u, 0x4E4C4A48u, 0x53525150u, 0x57565554u},  // zp=0
    {0x403800B8u, 0x4C4A4844u, 0x5251504Eu, 0x56555453u},  // zp=1
    {0x3800B8C0u, 0x4A484440u, 0x51504E4Cu, 0x55545352u},  // zp=2
    {0x00B8C0C4u, 0x48444038u, 0x504E4C4Au, 0x54535251u},  // zp=3
    {0xB8C0C4C8u, 0x44403800u, 0x4E4C4A48u, 0x53525150u},  // zp=4
    {0xC0C4C8CAu, 0x403800B8u, 0x4C4A4844u, 0x5251504Eu},  // zp=5
    {0xC4C8CACCu, 0x3800B8C0u, 0x4A484440u, 0x51504E4Cu},  // zp=6
    {0xC8CACCCEu, 0x00B8C0C4u, 0x48444038u, 0x504E4C4Au},  // zp=7
    {0xCACCCED0u, 0xB8C0C4C8u, 0x44403800u, 0x4E4C4A48u},  // zp=8
    {0xCCCED0D1u, 0xC0C4C8CAu, 0x403800B8u, 0x4C4A4844u},  // zp=9
    {0xCED0D1D2u, 0xC4C8CACCu, 0x3800B8C0u, 0x4A484440u},  // zp=10
    {0xD0D1D2D3u, 0xC8CACCCEu, 0x00B8C0C4u, 0x48444038u},  // zp=11
    {0xD1D2D3D4u, 0xCACCCED0u, 0xB8C0C4C8u, 0x44403800u},  // zp=12
    {0xD2D3D4D5u, 0xCCCED0D1u, 0xC0C4C8CAu, 0x403800B8u},  // zp=13
    {0xD3D4D5D6u, 0xCED0D1D2u, 0xC4C8CACCu, 0x3800B8C0u},  // zp=14
    {0xD4D5D6D7u, 0xD0D1D2D3u, 0xC8CACCCEu, 0x00B8C0C4u},  // zp=15
    {0x3C383000u, 0x4C484440u, 0xBCB8B080u, 0xCCC8C4C0u},  // E2M1
};

__device__ __forceinline__ uint32_t cvt_f32_e4m3(float v) {
    return static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(v, v, 0, false)) & 0xFFu;
}
// Four floats -> four e4m3 bytes (a in byte 0 ... d in byte 3).
__device__ __forceinline__ uint32_t pack4_e4m3(float a, float b, float c, float d) {
    const int lo = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
    return static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(c, d, lo, true));
}
__device__ __forceinline__ float e4m3_to_f32(uint32_t byte) {
    return __builtin_amdgcn_cvt_f32_fp8(static_cast<int>(byte), 0);
}
// Sum of a word's four e4m3 bytes, byte 0 first (bytes converted in pairs in place)
// plus the same of a second word: t + e(a0) + e(b0) + e(a1) + e(b1) + ... in that order.
__device__ __forceinline__ float e4m3_pair_sum(float t, uint32_t a, uint32_t b) {
    const auto a01 = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(a), false);
    const auto a23 = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(a), true);
    const auto b01 = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(b), false);
    const auto b23 = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(b), true);
    t += a01[0] + b01[0];
    t += a01[1] + b01[1];
    t += a23[0] + b23[0];
    t += a23[1] + b23[1];
    return t;
}

// 16-entry byte lookup of each byte of x (values 0..15) in table t.
// v_perm_b32 selects from 8 bytes; entries 8..15 come from a second select, and the
// third select turns (x + 5) >= 13 into an all-ones byte mask for x >= 8.
__device__ __forceinline__ uint32_t lut16(uint32_t x, uint4 t) {
    const uint32_t a = __builtin_amdgcn_perm(t.y, t.x, x);
    const uint32_t b = __builtin_amdgcn_perm(t.w, t.z, x ^ 0x08080808u);
    const uint32_t m = __builtin_amdgcn_perm(0u, 0u, x + 0x05050505u);
    return (a & ~m) | (b & m);
}

// One int32 of 8 nibbles (k = 0..7) -> 8 e4m3 bytes in k8-interleave order:
// lo = {k0,k2,k4,k6}, hi = {k1,k3,k5,k7}.
__device__ __forceinline__ void decode8(uint32_t w, uint4 t, uint32_t& lo, uint32_t& hi) {
    lo = lut16(w & 0x0F0F0F0Fu, t);
    hi = lut16((w >> 4) & 0x0F0F0F0Fu, t);
}

__device__ __forceinline__ uint4 load_table(int idx) {
    return make_uint4(g_decode_tables[idx][0], g_decode_tables[idx][1],
                      g_decode_tables[idx][2], g_decode_tables[idx][3]);
}

// Decode-table index for output row n, group g of one expert's packed zero-points
// (E, N/8, G) (moe_kernel.hip:172-176: (z[n/8][g] >> 4*(n%8)) & 0xF).
__device__ __forceinline__ int table_index(const int* __restrict__ zeros_e, int n, int g,
                                           int num_groups, bool e2m1) {
    if (e2m1) return kE2m1Table;
    if (zeros_e == nullptr) return 8;
    return (zeros_e[(n >> 3) * num_groups + g] >> ((n & 7) * 4)) & 0xF;
}

// Position of k inside the k8-interleaved activation row.
__device__ __host__ __forceinline__ int k8_pos(int k) {
    const int r = k & 7;
    return (k & ~7) | ((r >> 1) | ((r & 1) << 2));
}

// Work-group barrier for LDS hand-off only. __syncthreads() also orders global memory, so
// the compiler waits for every load in flight (vmcnt(0)) before it, which would drain the
// loads in flight; fencing LDS alone waits for the LDS writes only.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Index of the k-th (0-based) set bit of m; k < popcount(m).
__device__ __forceinline__ int nth_set_bit(uint64_t m, int k) {
    int pos = 0;
#pragma unroll
    for (int w = 32; w >= 1; w >>= 1) {
        const uint64_t low = m & ((1ull << w) - 1ull);
        const int c = __popcll(low);
        if (k >= c) {
            k -= c;
            m >>= w;
            pos += w;
        } else {
            m = low;
        }
    }
    return pos;
}

// Cross-lane moves on the VALU, without the LDS round trip of ds_bpermute (__shfl): DPP
// inside rows of 16 lanes, the gfx950 permlane swaps across rows and halves. lane_step<S>
// pairs lane l with a lane of the other half of its 2^(S+1)-lane group: lane l ^ 1, l ^ 2,
// then the mirrored lane of the 8- and 16-lane groups. Once the smaller groups hold one
// value each (true inside every reduction below) the mirrored lane holds what lane
// l ^ (1 << S) holds, so these reductions equal the xor butterfly bit for bit. Every lane
// of the wave must be active.
template <int S>
__device__ __forceinline__ uint32_t dpp_step(uint32_t v) {
    static_assert(S >= 0 && S < 4, "DPP steps stay inside a row of 16 lanes");
    constexpr int ctrl = S == 0 ? 0xB1 : S == 1 ? 0x4E : S == 2 ? 0x141 : 0x140;
    // every lane receives a value (full permutations inside rows), so the old value is never
    // kept; with it left undefined the compiler folds the move into the consuming VALU op
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, ctrl, 0xF, 0xF, true);
}

// v combined over aligned groups of 2^LOG2 lanes (op commutative and associative).
template <int LOG2, typename Op>
__device__ __forceinline__ float lane_allreduce(float v, Op op) {
    if constexpr (LOG2 > 0) v = op(v, __uint_as_float(dpp_step<0>(__float_as_uint(v))));
    if constexpr (LOG2 > 1) v = op(v, __uint_as_float(dpp_step<1>(__float_as_uint(v))));
    if constexpr (LOG2 > 2) v = op(v, __uint_as_float(dpp_step<2>(__float_as_uint(v))));
    if constexpr (LOG2 > 3) v = op(v, __uint_as_float(dpp_step<3>(__float_as_uint(v))));
    if constexpr (LOG2 > 4) {
        const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v),
                                                        false, false);
        v = op(__uint_as_float(r[0]), __uint_as_float(r[1]));
    }
    if constexpr (LOG2 > 5) {
        const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v),
                                                        false, false);
        v = op(__uint_as_float(r[0]), __uint_as_float(r[1]));
    }
    return v;
}

struct MaxOp {
    __device__ float operator()(float a, float b) const { return fmaxf(a, b); }
};
struct SumOp {
    __device__ float operator()(float a, float b) const { return a + b; }
};

// Wave64 reductions (every lane gets the result).
__device__ __forceinline__ float wave_max(float v) { return lane_allreduce<6>(v, MaxOp{}); }
__device__ __forceinline__ float wave_sum(float v) { return lane_allreduce<6>(v, SumOp{}); }

// Activation scale from an fp32 absmax (moe_kernel.hip:117-118).
__device__ __forceinline__ float act_scale_from_absmax(float amax) {
    float s = amax / kE4m3Max;
    if (s < kActScaleFloor) s = kActScaleFloor;
    return s;
}

// x as an fp32 value in a register. Conversions to fp16 go through it: without it the
// compiler may fold the product that forms x into the conversion (one f16-output FMA,
// v_fma_mixlo_f16) and round once, where the numerics contract rounds the fp32 product and
// then to fp16; the fused and unfused epilogues of one GEMM would then differ in rare
// elements. The empty asm only pins the value; it emits no instruction.
__device__ __forceinline__ float as_f32(float x) {
    asm("" : "+v"(x));
    return x;
}

// SiLU of an fp16 value, rounded to fp16: the bits of __float2half(g / (1.0f + expf(-g)))
// (vLLM silu_kernel<half>; moe_kernel.hip:549-561). Since g is one of 65536 fp16 values this
// is a fixed table, and a cheaper evaluation only has to land on the same fp16 values. Here
// 2^(-g log2 e) comes from the hardware exp2, with log2 e split so that g * kSiluL2eHi is
// exact (g has 11 significant bits, kSiluL2eHi 13), and the division from the hardware
// reciprocal. Over all fp16 inputs whose SiLU is a normal fp16 number this fp32 value lies
// within 5 fp32 ulps of the exact form's (measured over every input), so it rounds to the
// same fp16 unless it lies within a few ulps of an fp16 rounding midpoint: values within
// kSiluGuard ulps of one (0.13% of the inputs), results below the fp16 normal range (where
// the hardware operations flush denormals) and non-finite inputs take the exact form. The
// tests check every input against a table of the exact form.
constexpr float kSiluL2eHi = 1.442626953125f;                 // 5909 / 4096 (0x3FB8A800)
constexpr float kSiluL2eLo = 1.44269504088896340736f - 1.442626953125f;
constexpr uint32_t kSiluGuard = 8;                            // fp32 ulps around a midpoint
// The fast form's fp32 SiLU of g (an fp16 value); ok: it rounds to the exact form's fp16.
__device__ __forceinline__ float silu_fast_f32(float g, bool& ok) {
    const float d = fmaf(__builtin_amdgcn_exp2f(g * -kSiluL2eHi),
                         __builtin_amdgcn_exp2f(g * -kSiluL2eLo), 1.0f);
    const float r = g * __builtin_amdgcn_rcpf(d);
    const uint32_t a = __float_as_uint(r) & 0x7FFFFFFFu;
    // fp16 keeps 10 of the 23 fraction bits: the midpoint between two fp16 neighbours has
    // low 13 bits 0x1000
    const uint32_t mid = (a & 0x1FFFu) - (0x1000u - kSiluGuard);   // <= 2 * guard: near it
    ok = a >= 0x38800000u && a < 0x7F800000u && mid > 2u * kSiluGuard;
    return r;
}
__device__ __forceinline__ float silu_exact_f32(float g) { return g / (1.0f + expf(-g)); }

__device__ __forceinline__ __half silu_h(__half gate_h) {
    const float g = __half2float(gate_h);
    bool ok;
    const float r = silu_fast_f32(g, ok);
    return __float2half(__builtin_expect(ok, 1) ? r : silu_exact_f32(g));
}

// vLLM silu_and_mul on fp16 gate/up stores (moe_kernel.hip:555-561).
__device__ __forceinline__ __half silu_mul_h(__half gate_h, __half up_h) {
    return __hmul(silu_h(gate_h), up_h);
}

// silu_mul_h of four (gate, up) pairs given as fp32 values (each rounded to fp16 first): the
// fast form of all four first, so that their chains interleave, then the exact form of those
// it does not cover (each a branch that the wave skips unless one of its lanes needs it).
__device__ __forceinline__ void silu_mul_h4(const float (&gate)[4], const float (&up)[4],
                                            __half (&out)[4]) {
    float g[4], r[4];
    bool ok[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        g[k] = __half2float(__float2half(gate[k]));
        r[k] = silu_fast_f32(g[k], ok[k]);
    }
#pragma unroll
    for (int k = 0; k < 4; ++k)
        if (__builtin_expect(!ok[k], 0)) r[k] = silu_exact_f32(g[k]);
#pragma unroll
    for (int k = 0; k < 4; ++k) out[k] = __hmul(__float2half(r[k]), __float2half(up[k]));
}

}  // namespace w4a8
