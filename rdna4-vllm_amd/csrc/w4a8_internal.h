// Host-side internals shared by the C-ABI translation units (not part of the ABI).
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>
#include <cstdint>
#include <cstddef>
#include <string>

#include "../../include/w4a8_moe.h"

namespace w4a8 {

// Thread-local error slot behind w4a8_last_error().
void set_error(const std::string& msg);
void clear_error();

// Returns W4A8_ERR_HIP (with message) if the last launch failed, else W4A8_OK.
int check_launch(const char* what);

// Per-device launch facts, looked up once per (current device, kernel) under a lock, so
// several threads and several GPUs in one process each get their own values.
// Reserves `bytes` of dynamic LDS for `kernel` on the current device (hipFuncSetAttribute;
// more than 64 KB needs the opt-in); W4A8_OK or W4A8_ERR_HIP with a message naming `what`.
int reserve_dyn_lds(const void* kernel, int bytes, const char* what);
// Compute units of the current device (256 if the query fails).
int device_cu_count();
// Work-groups of `threads` threads and `lds` dynamic LDS bytes one CU holds at once
// (hipOccupancyMaxActiveBlocksPerMultiprocessor; 0 if the query fails).
int blocks_per_cu(const void* kernel, int threads, size_t lds);

inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// Kernel-exact timing (measurement aid): when set, the next launch made through
// launch_kernel() on this thread records `start` when that kernel begins and `stop` when it
// ends (hipExtLaunchKernel stamps the events from the dispatch itself, so the interval is
// the kernel's own duration, as a kernel trace reports it); the slot is then cleared.
struct KernelStamp {
    hipEvent_t start = nullptr;
    hipEvent_t stop = nullptr;
};
KernelStamp& next_kernel_stamp();

template <typename... Params, typename... Args>
inline void launch_kernel(void (*kernel)(Params...), dim3 grid, dim3 block, size_t lds,
                          hipStream_t s, Args... args) {
    KernelStamp& st = next_kernel_stamp();
    if (st.start != nullptr) {
        hipExtLaunchKernelGGL(kernel, grid, block, (uint32_t)lds, s, st.start, st.stop, 0u,
                              static_cast<Params>(args)...);
        st = KernelStamp{};
    } else {
        kernel<<<grid, block, lds, s>>>(static_cast<Params>(args)...);
    }
}

// Bump allocator over a caller workspace (256-byte aligned carve-outs).
struct Workspace {
    char* base;
    size_t size;
    size_t used = 0;
    Workspace(void* p, size_t n) : base(static_cast<char*>(p)), size(n) {}
    template <typename T>
    T* take(size_t count) {
        used = align_up(used, 256);
        T* p = reinterpret_cast<T*>(base + used);
        used += count * sizeof(T);
        return p;
    }
    bool ok() const { return used <= size; }
};

// Bytes a Workspace needs for a sequence of carve-outs.
struct WorkspaceSize {
    size_t used = 0;
    template <typename T>
    void take(size_t count) { used = align_up(used, 256) + count * sizeof(T); }
};

// ---- launchers implemented in the .hip files (all enqueue on `stream`) ----
int launch_act_quant(const void* x, bool x_bf16, int64_t rows, int64_t K, uint8_t* x_fp8,
                     float* scales, bool k8_interleave, hipStream_t stream,
                     const int32_t* sorted_ids = nullptr, const int32_t* ntp = nullptr,
                     int64_t num_valid = 0, float* group_sums = nullptr);
int launch_dequant(const int32_t* w, const int32_t* z, int64_t E, int64_t N, int64_t K,
                   int64_t gs, bool e2m1, uint8_t* out, hipStream_t stream);
int launch_silu_and_mul(const void* in, int64_t rows, int64_t inter, void* out,
                        hipStream_t stream);
int launch_swigluoai_and_mul(const void* in, int64_t rows, int64_t inter, float alpha,
                             float limit, void* out, hipStream_t stream);
// x non-null: the routing wave of token t also quantises row t of x (act_quant_kernel's
// arithmetic, k8-interleaved, group sums when gsum is non-null).
int launch_topk_softmax(const float* logits, int64_t T, int64_t E, int64_t top_k,
                        bool renorm, float* w, int32_t* ids, hipStream_t stream,
                        const void* x = nullptr, bool x_bf16 = false, int64_t K = 0,
                        uint8_t* xq = nullptr, float* xs = nullptr, float* gsum = nullptr);
size_t align_workspace_bytes(int64_t numel, int64_t num_experts);
// Decode prologue in one launch (numel <= 1024): the single-work-group align plus per-row
// act-quant of x (k8-interleaved) with optional group sums.
// emap (emap_len entries) maps routed ids to local experts in [0, E); slots without a
// local expert are dropped.
int launch_align_quant(const int32_t* ids, int64_t numel, int64_t E, int64_t block_m,
                       const int32_t* emap, int64_t emap_len, int32_t* sorted_ids,
                       int64_t sorted_len,
                       int32_t* expert_ids, int32_t* ntp, int32_t* slot_to_row,
                       const void* x, bool x_bf16, int64_t rows, int64_t K, uint8_t* xq,
                       float* xs, float* gsum, hipStream_t stream);
int launch_align(const int32_t* topk_ids, int64_t numel, int64_t E, int64_t block_m,
                 const int32_t* expert_map, int64_t emap_len, int32_t* sorted_ids,
                 int64_t sorted_len,
                 int32_t* expert_ids, int32_t* ntp, void* ws, size_t ws_bytes,
                 hipStream_t stream, int32_t* slot_to_row = nullptr);   // optional inverse map
int launch_gather_reduce(const void* out2, int64_t P, int64_t N, const int32_t* sorted_ids,
                         const float* tw, int64_t m_tk, const int32_t* ntp, int64_t top_k,
                         float* out, int32_t* slot_to_row, hipStream_t stream);
// out[t, n] = cast(sum_{j asc} w[t*k+j] * y[(t*k+j), n]) with y fp32 (rows = T*k);
// slots whose (mapped) expert is outside [0, E) are skipped (map as launch_align_quant).
// sync (after the fused decode layer): flags[0..nflags) are reset to 0, and the output is
// NaN when any of timeout[0..ntimeout) == nonce (an in-kernel wait of this call gave up).
struct SlotReduceSync {
    uint64_t* flags = nullptr;
    int nflags = 0;
    const uint64_t* timeout = nullptr;
    int ntimeout = 0;
    uint64_t nonce = 0;
};
int launch_slot_reduce(const float* y, const float* tw, const int32_t* topk_ids,
                       const int32_t* expert_map, int64_t emap_len, int64_t E, int64_t T,
                       int64_t N, int64_t top_k, void* out, bool out_bf16, hipStream_t stream,
                       SlotReduceSync sync = SlotReduceSync{});
int launch_cast_f32(const float* in, int64_t n, void* out, bool out_bf16, hipStream_t stream);
// out[t, n] = cast(sum_{j asc} w[t*k+j] * f32(y[slot_to_row[t*k+j], n])), y fp16 (rows, N);
// rows < 0 (slots dropped by expert_map) contribute nothing. N % 8 == 0.
int launch_row_reduce(const void* y, const int32_t* slot_to_row, const float* tw, int64_t T,
                      int64_t N, int64_t top_k, void* out, bool out_bf16, hipStream_t stream);
int launch_zero_f32(float* p, int64_t n, hipStream_t stream);

// Grouped GEMM epilogue modes.
enum class Epi : int {
    kHalf = 0,      // out[row_pad, n] = fp16(run * asc)            (P, N)
    kSiluHalf = 1,  // out[row_pad, n] = silu_mul(gate, up)          (P, N/2)
    kScatter = 2,   // atomicAdd(out[slot / top_k, n], w[slot] * run * asc)
    kSlotF32 = 3,   // out[slot, n] = run * asc (fp32, rows = M*top_k)
};

struct GroupedArgs {
    const void* x;          // activation rows: fp16 (or bf16 when x_bf16)
    bool x_bf16;
    int64_t x_rows;         // rows of x
    int64_t K;
    const int32_t* w;       // (E, N, K/8), or fragment layout when w_frag
    bool w_frag;            // w repacked by launch_repack_fragments (decode GEMV / prefill only)
    const uint16_t* scales; // (E, N, G) fp16 bits
    const int32_t* zeros;   // (E, N/8, G) or null
    int64_t E, N, group_size;
    const int32_t* sorted_ids;
    int64_t P;
    const int32_t* expert_ids;
    const int32_t* ntp;
    int64_t top_k;          // gather row = slot / top_k (ignored when identity)
    bool identity_gather;   // gather row = padded row index
    int64_t num_valid;      // slots >= num_valid are padding
    int64_t block_m;
    bool e2m1;
    Epi epi;
    void* out;              // see Epi
    const float* topk_weights;  // kScatter
    int64_t out_top_k;      // kScatter: token = slot / out_top_k
    // scratch for the prequantised path
    uint8_t* x_fp8;         // (x_rows, K) k8-interleaved, or null
    float* act_scales;      // (x_rows,)
    float* act_group_sums;  // (x_rows, K/128) per-group sums of the e4m3 values, or null
};

// Dense GEMV for 1 <= M <= 16 rows of fp16 x on op-layout weights (dense_gemv.hip): group
// 128, K a multiple of 1024 up to 4096, N % 16 == 0; quantises the rows itself.
bool dense_gemv_supported(int64_t M, int64_t N, int64_t K, int64_t group_size, bool e2m1);
int launch_dense_gemv(const void* x_f16, int64_t M, int64_t K, const int32_t* w, const void* scales_f16,
                      const int32_t* zeros, int64_t N, void* out_f16, hipStream_t s);
int launch_grouped_scalar(const GroupedArgs& a, hipStream_t stream);
int launch_grouped_mfma(const GroupedArgs& a, hipStream_t stream);   // prefill tiles
int launch_grouped_gemv(const GroupedArgs& a, hipStream_t stream);   // decode GEMV
// Prefill, activation-resident schedule (prefill_ares.hip): 64-row tiles, all N per tile.
bool prefill_ares_supported(int64_t K, int64_t N, int64_t group_size, bool e2m1, int64_t block_m,
                            Epi epi);
int launch_grouped_prefill_ares(const GroupedArgs& a, hipStream_t stream);
// The activation-resident tiles can take fp16 rows (x, no x_fp8) and quantise them in their
// prologue, bit-identical to act_quant_kernel with group sums (each tile owns its rows).
bool prefill_ares_quantises_rows(int64_t K, Epi epi);
// gemm1+SiLU and the self-quantising gemm2 of the same 64-row tiles in one launch (each
// work-group runs a tile's gemm1, then its gemm2 on the h rows it just wrote).
bool prefill_ares_pair_supported(const GroupedArgs& a1, const GroupedArgs& a2);
int launch_grouped_prefill_ares_pair(const GroupedArgs& a1, const GroupedArgs& a2,
                                     hipStream_t stream);
// (E, N, K/8) int32 op layout -> fragment layout: per expert, 16-row tile t and 128-wide
// group g, a 1 KB block whose 16-byte lane l holds row 16t + l % 16, k in
// [128g + 32 (l / 16), +32) (the MFMA B operand of lane l). N % 16 == 0, K % 128 == 0.
int launch_repack_fragments(const int32_t* w, const void* scales, const int32_t* zeros,
                            int64_t E, int64_t N, int64_t K, int32_t* out, hipStream_t stream);
// int32 words of the fragment layout of E experts of N rows and K columns (K % 128 == 0)
int64_t fragments_words(int64_t E, int64_t N, int64_t K);
// Prefill tiles with raw-nibble B in registers; needs x_fp8, act_scales and act_group_sums.
int launch_grouped_prefill(const GroupedArgs& a, hipStream_t stream);
bool prefill_supported(int64_t K, int64_t group_size, bool e2m1);   // g128, K <= 4096, no E2M1
// Same, with an explicit column-tile count per wave team (0 = default heuristic).
int launch_grouped_gemv_tpt(const GroupedArgs& a, int tiles_per_team, hipStream_t stream);
// the matrix-core tiles take the shape (int4: group 128; E2M1: groups of 32, 64 or 128)
bool mfma_supported(int64_t K, int64_t group_size, bool e2m1 = false);
// mfma_supported and K / group_size in {1,2,3,4,6,8,12,16,32} (split-K table of the GEMV)
bool gemv_supported(int64_t K, int64_t group_size);

// Whole-layer decode GEMV on fragment-layout weights (decode_gemv.hip): each work-group
// groups the slots by expert from topk_ids itself and quantises its activation rows in
// registers. silu: gemm1 (a = x (T, K) by token, out = h (numel, N/2) fp16 after SiLU*mul);
// else gemm2 (a = h (numel, K) fp16 by slot, out = y (numel, N) fp32).
// Hand-over of the decode lists from the gemm1 launch to the gemm2 launch (workspace):
// the touched experts, their slot lists and pass counts.
constexpr int kDecHandExperts = 1024;
constexpr int kDecHandSlots = 1024;
struct DecHandover {
    int n_touched;
    int16_t expert[kDecHandExperts + 1];
    int16_t first[kDecHandExperts + 1];
    int pp[kDecHandExperts + 1];
    int16_t slot[kDecHandSlots];
};

struct DecodeLaunch {
    const int32_t* topk_ids;
    // gemm1 only: route in the kernel from these logits (decode_routes_in_kernel), writing
    // topk_weights_out / topk_ids_out; null: topk_ids come from an earlier launch
    const float* logits = nullptr;
    int64_t n_router = 0;
    bool renormalize = true;
    float* topk_weights_out = nullptr;
    int32_t* topk_ids_out = nullptr;
    const int32_t* expert_map;
    int64_t emap_len, numel, top_k, E;
    const void* a;
    bool a_bf16;
    // gemm1 (silu) only: a's rows quantised already by the router launch (k8-interleaved
    // e4m3 (T, K) and their scales, act_quant_kernel's bytes), or null
    const uint8_t* aq = nullptr;
    const float* asc = nullptr;
    // list hand-over: gemm1 writes it (hand_out), gemm2 reads it (hand_in)
    DecHandover* hand_out = nullptr;
    const DecHandover* hand_in = nullptr;
    bool silu;
    const int32_t* w;
    const void* scales;
    const int32_t* zeros;
    void* out;
    int64_t K, N;
};
bool decode_layer_supported(int64_t numel, int64_t E, int64_t H, int64_t inter, int64_t gs);
// T tokens over n_router experts: the decode gemm1 launch can route them itself
bool decode_routes_in_kernel(int64_t T, int64_t n_router, int64_t top_k);
int launch_decode_gemv(const DecodeLaunch& d, hipStream_t stream);
// Both GEMVs in one launch (gemm2 waits in-kernel for the gemm1 rows it reads): d1 is gemm1,
// d2 gemm2. flags: kDecodeFlagSlots words, 0 or a value other than nonce on entry (the slot
// reduce resets them to 0); timeout: kDecodeFlagSlots words, word w set to nonce if a wait
// of work-group w gave up (each work-group clears its own word when it starts). The grid
// is decode_layer_grid() work-groups.
constexpr int64_t kDecodeFlagSlots = 1024;
bool decode_layer_fused_supported(int64_t H, int64_t inter);
int decode_layer_grid();
int launch_decode_layer(const DecodeLaunch& d1, const DecodeLaunch& d2, uint64_t* flags,
                        uint64_t nonce, uint64_t* timeout, hipStream_t stream);
// Test hook of the fused layer (g_dec_fault): on != 0 makes its waits give up.
int decode_fused_set_fault(int on);

}  // namespace w4a8
