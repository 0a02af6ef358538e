/*
 * w4a8_moe.h - C ABI of the MI355X (gfx950) W4A8 MoE expert path.
 *
 * This is the boundary the torch-op layer (w4a8_fp8_wmma/_ops.py) binds through
 * ctypes; any other host (C++, cgo, JNI) can bind the same symbols. Every entry point
 * takes raw device pointers, sizes and a hipStream_t (passed as void*), enqueues its
 * kernels on that stream without synchronising, and returns a status code. Nothing
 * here allocates device memory: scratch is a caller-owned workspace whose size the
 * matching *_workspace_size() function returns.
 *
 * The reference (patcarter883/rdna4-vllm) exposes this path as torch ops
 * (w4a8_fp8_wmma/bindings.cpp:388-424) over host launchers
 * (w4a8_fp8_wmma/moe_kernel.hip:1327-1464); each entry point below names the
 * reference interface it replaces.
 *
 * Tensor layouts (reference op layout, moe_kernel.hip:7-17):
 *   x          (rows, K)          fp16 (or bf16 where stated), row-major
 *   w_packed   (E, N, K/8)        int32, nibble j of word w is k = 8w + j (low first)
 *   scales     (E, N, K/group)    fp16
 *   w_zeros    (E, N/8, K/group)  int32, nibble n%8 of word n/8, or NULL (zp = 8)
 *   sorted_token_ids (P,), expert_ids (P/block_m,), num_tokens_post_padded (1,) int32
 *   topk_weights (M*top_k,) fp32, topk_ids (M, top_k) int32
 */
#ifndef W4A8_MOE_H_
#define W4A8_MOE_H_

#include <stddef.h>
#include <stdint.h>

#if defined(__GNUC__) || defined(__clang__)
#define W4A8_API __attribute__((visibility("default")))
#else
#define W4A8_API
#endif

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes. A non-zero return leaves a message for w4a8_last_error(). */
#define W4A8_OK 0
#define W4A8_ERR_INVALID 1      /* argument violates the contract (TORCH_CHECK in the reference) */
#define W4A8_ERR_HIP 2          /* a HIP runtime call or kernel launch failed */
#define W4A8_ERR_WORKSPACE 3    /* workspace pointer NULL or smaller than required */

/* Kernel ids carried over the ABI (w4a8_fp8_wmma/kernel_names.h:41-48). */
#define W4A8_MOE_KERNEL_SCALAR 0   /* scalar golden grouped GEMM */
#define W4A8_MOE_KERNEL_WMMA 6     /* tiled matrix-core grouped GEMM (fp8 MFMA on gfx950) */
#define W4A8_MOE_KERNEL_GEMV 7     /* decode grouped GEMV (fp8 MFMA, token rows compacted) */

/* x dtype selector for w4a8_moe_apply. */
#define W4A8_DTYPE_F16 0
#define W4A8_DTYPE_BF16 1

/* Version of this ABI (bumped on any signature change). */
W4A8_API int w4a8_abi_version(void);

/* Thread-local message of the last failing call on this thread ("" if none). */
W4A8_API const char* w4a8_last_error(void);

/* ---------------------------------------------------------------------------------
 * Per-token fp8 e4m3 activation quantisation.
 * Replaces moe_compute_act_fp8_kernel (moe_kernel.hip:87-127) and the dense twin
 * compute_act_fp8_and_scales_kernel (w4a8_fp8_wmma_kernel.hip:153-200).
 * x_fp8 bytes are in natural k order when k8_interleave == 0, else in the
 * kernels' k8-interleaved order (byte p of each 8-byte block holds k = {0,2,4,6,1,3,5,7}[p]).
 */
W4A8_API int w4a8_act_quant_fp8(const void* x_f16, int64_t rows, int64_t K, uint8_t* x_fp8,
                       float* act_scales, int k8_interleave, void* stream);

/* ---------------------------------------------------------------------------------
 * int4 -> e4m3 dequant of op-layout weights: out (rows, K) bytes = e4m3(nibble - zp),
 * natural k order. Exposes the exact decode the GEMM kernels run in registers
 * (tile_config.h:42-71, moe_kernel.hip:63-83). rows = E*N; w_zeros NULL => zp = 8.
 */
W4A8_API int w4a8_dequant_fp8(const int32_t* w_packed, const int32_t* w_zeros, int64_t E, int64_t N,
                     int64_t K, int64_t group_size, int weight_is_e2m1, uint8_t* out,
                     void* stream);

/* ---------------------------------------------------------------------------------
 * Router: softmax over E logits -> top_k -> optional renormalise.
 * Replaces vLLM fused_topk/topk_softmax, which the reference calls through vLLM
 * (not in the reference tree; contract from the layer the reference patches).
 * Selection is on logits, ties to the lower expert id; output order descending.
 */
W4A8_API int w4a8_topk_softmax(const float* logits, int64_t T, int64_t E, int64_t top_k,
                      int renormalize, float* topk_weights, int32_t* topk_ids, void* stream);

/* ---------------------------------------------------------------------------------
 * moe_align_block_size (vLLM op called at moe_experts.py:587-589, contract mirrored
 * by test_moe_experts.py:136-152). Groups slots t*top_k+j by expert ascending, slot
 * ascending, pads each expert to a multiple of block_m with the sentinel numel.
 * sorted_len must equal w4a8_moe_align_sorted_len(); entries past ntp hold the
 * sentinel and expert_ids -1. num_experts is the global count (the range of topk_ids);
 * expert_map (num_experts entries, -1 = not local) may be NULL; mapped ids must be below
 * num_experts and slots mapped to -1 are dropped. Deterministic (no atomics decide the
 * order).
 */
W4A8_API int64_t w4a8_moe_align_sorted_len(int64_t numel, int64_t num_experts, int64_t block_m);
W4A8_API size_t w4a8_moe_align_workspace_size(int64_t numel, int64_t num_experts);
W4A8_API int w4a8_moe_align_block_size(const int32_t* topk_ids, int64_t numel, int64_t num_experts,
                              int64_t block_m, const int32_t* expert_map,
                              int32_t* sorted_token_ids, int64_t sorted_len,
                              int32_t* expert_ids, int32_t* num_tokens_post_padded,
                              void* workspace, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------------
 * Grouped GEMM, padded sorted layout: out (P, N) fp16.
 * Replaces mmq_fp8_moe_gemm (bindings.cpp:178-228 -> moe_kernel.hip:1358-1392).
 * Row r with slot s = sorted_token_ids[r] < T*top_k (and r < ntp) gathers x[s/top_k];
 * other rows are not written. The workspace (w4a8_moe_gemm_workspace_size) holds the
 * quantised rows; with the GEMV kernel, int4 weights, group 128 and K / 128 one of
 * 1, 2, 3, 4, 6, 8, 12, 16, 32 it may be NULL, and each work-group then quantises its block's rows itself (same bytes,
 * no act-quant launch). Other calls without it return W4A8_ERR_WORKSPACE.
 */
W4A8_API size_t w4a8_moe_gemm_workspace_size(int64_t x_rows, int64_t K);
W4A8_API int w4a8_mmq_fp8_moe_gemm(const void* x_f16, int64_t T, int64_t K,
                          const int32_t* w_packed, const void* scales_f16,
                          const int32_t* w_zeros, int64_t E, int64_t N, int64_t group_size,
                          const int32_t* sorted_token_ids, int64_t P,
                          const int32_t* expert_ids, const int32_t* num_tokens_post_padded,
                          int64_t top_k, int64_t block_m, int64_t kernel, int weight_is_e2m1,
                          void* out_f16, void* workspace, size_t workspace_bytes, void* stream);

/* Fused gemm1 + silu_and_mul: w_packed is w13 (E, 2*inter, K/8); out (P, inter) fp16.
 * Replaces mmq_fp8_moe_gemm1_silu (bindings.cpp:235-287 -> moe_kernel.hip:1327-1356).
 * Same workspace as w4a8_mmq_fp8_moe_gemm. kernel must be WMMA. */
W4A8_API int w4a8_mmq_fp8_moe_gemm1_silu(const void* x_f16, int64_t T, int64_t K,
                                const int32_t* w_packed, const void* scales_f16,
                                const int32_t* w_zeros, int64_t E, int64_t N,
                                int64_t group_size, const int32_t* sorted_token_ids,
                                int64_t P, const int32_t* expert_ids,
                                const int32_t* num_tokens_post_padded, int64_t top_k,
                                int64_t block_m, int64_t kernel, int weight_is_e2m1,
                                void* out_f16, void* workspace, size_t workspace_bytes,
                                void* stream);

/* Fused gemm2 + top-k weight + atomic scatter into a pre-zeroed fp32 output (M, N).
 * x is the (P, K) post-activation buffer, gathered by identity.
 * Replaces mmq_fp8_moe_gemm_scatter (bindings.cpp:293-353 -> moe_kernel.hip:1398-1433).
 * Workspace: w4a8_moe_gemm_workspace_size(P, K). */
W4A8_API int w4a8_mmq_fp8_moe_gemm_scatter(const void* x_f16, int64_t P_rows, int64_t K,
                                  const int32_t* w_packed, const void* scales_f16,
                                  const int32_t* w_zeros, int64_t E, int64_t N,
                                  int64_t group_size, const int32_t* sorted_token_ids,
                                  int64_t P, const int32_t* expert_ids,
                                  const int32_t* num_tokens_post_padded,
                                  const float* topk_weights, float* output, int64_t M,
                                  int64_t top_k, int64_t block_m, int64_t kernel,
                                  int weight_is_e2m1, void* workspace,
                                  size_t workspace_bytes, void* stream);

/* Deterministic weighted gather-reduce: out (M, N) fp32 = sum_j w * out2[row(t, j)].
 * Replaces mmq_fp8_moe_gather_reduce (bindings.cpp:357-380 -> moe_kernel.hip:1437-1464).
 * Workspace: w4a8_gather_reduce_workspace_size(M*top_k). */
W4A8_API size_t w4a8_gather_reduce_workspace_size(int64_t m_times_topk);
W4A8_API int w4a8_mmq_fp8_moe_gather_reduce(const void* out2_f16, int64_t P, int64_t N,
                                   const int32_t* sorted_token_ids,
                                   const float* topk_weights, int64_t m_times_topk,
                                   const int32_t* num_tokens_post_padded, int64_t top_k,
                                   float* out, void* workspace, size_t workspace_bytes,
                                   void* stream);

/* vLLM silu_and_mul on (rows, 2*inter) fp16 -> (rows, inter) fp16, the unfused
 * activation the reference decode path calls (moe_experts.py:627-630). */
W4A8_API int w4a8_silu_and_mul(const void* in_f16, int64_t rows, int64_t inter, void* out_f16,
                      void* stream);

/* vLLM swigluoai_and_mul (gpt-oss) on (rows, 2*inter) fp16 with gate and up interleaved
 * (gate = row[2c], up = row[2c + 1]) -> (rows, inter) fp16: in fp32, g = min(gate, limit),
 * u = clamp(up, -limit, limit), out = fp16((u + 1) * g * sigmoid(alpha * g)); vLLM's defaults
 * are alpha = 1.702, limit = 7. The activation the reference's mxfp4 (gpt-oss) hook applies
 * between the unfused GEMMs (moe_experts.py:1416-1424 -> apply_moe_activation). */
W4A8_API int w4a8_swigluoai_and_mul(const void* in_f16, int64_t rows, int64_t inter, float alpha,
                                    float limit, void* out_f16, void* stream);

/* ---------------------------------------------------------------------------------
 * Dense W4A8 GEMM: x (M, K) fp16, w (N, K/8), scales (N, K/g), zeros (N/8, K/g) or NULL
 * -> out (M, N) fp16. Replaces mmq_fp8_gemm (bindings.cpp:98-146 ->
 * launch_mmq_fp8_gemm_gfx1201, w4a8_fp8_wmma_kernel.hip:2507). kernel = a DenseKernel
 * id (kernel_names.h:18-36); 0 runs the scalar golden, every other valid id the fp8
 * MFMA path. Workspace: w4a8_moe_gemm_workspace_size(M, K). */
W4A8_API int w4a8_mmq_fp8_gemm(const void* x_f16, int64_t M, int64_t K, const int32_t* w_packed,
                      const void* scales_f16, const int32_t* w_zeros, int64_t N,
                      int64_t group_size, int64_t kernel, int weight_is_e2m1, void* out_f16,
                      void* workspace, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------------
 * Whole gated MoE expert path: the _run_grouped_moe composition
 * (moe_experts.py:493-665) behind the patched MoeWNA16Method.apply
 * (moe_experts.py:1308-1332). x (T, H) in x_dtype -> out (T, H) in x_dtype.
 * w13 (E, 2*inter, H/8), w2 (E, H, inter/8); scales/zeros as above (zeros may be
 * NULL per weight). topk_ids (T, top_k) int32, topk_weights (T, top_k) fp32.
 * E is the LOCAL expert count (w13.shape[0]). topk_ids hold global expert ids in
 * [0, num_global_experts) (vLLM's global_num_experts, moe_experts.py:587-589); with an
 * expert_map (num_global_experts int32 entries, -1 = not local) each id is mapped to a local
 * expert in [0, E) and slots without one contribute nothing. Without a map,
 * num_global_experts must be E (or <= 0, meaning E). Chooses the decode (T <= 96) or
 * prefill schedule itself. The prefill GEMMs take the activation-resident tiles only while
 * their activation rows hold fewer than 2^31 elements (gemm1: T * H; gemm2: padded rows *
 * inter), since those tiles address rows in 32 bits; larger calls run the streamed-K tiles
 * (same results).
 */
W4A8_API size_t w4a8_moe_apply_workspace_size(int64_t T, int64_t H, int64_t inter, int64_t E,
                                     int64_t top_k);
W4A8_API int w4a8_moe_apply(const void* x, int x_dtype, int64_t T, int64_t H, int64_t inter,
                   int64_t E, int64_t top_k, int64_t group_size,
                   const int32_t* w13, const void* w13_scales_f16, const int32_t* w13_zeros,
                   const int32_t* w2, const void* w2_scales_f16, const int32_t* w2_zeros,
                   const float* topk_weights, const int32_t* topk_ids,
                   const int32_t* expert_map, int64_t num_global_experts, int weight_is_e2m1,
                   void* out, void* workspace, size_t workspace_bytes, void* stream);

/* Load-time repack of int4 weights, their scales and zero-points from the op layout
 * (moe_kernel.hip:7-17) into the fragment layout the gfx950 kernels stream, with each
 * 16-row tile's metadata next to its weights. Per expert and 16-row tile t, G = K/128 blocks
 * of 1 KB, then G * 16 metadata words (w4a8_fragments_words() words in all, out is
 * (E, N/16, 272 G) int32):
 *   - block g's 16-byte lane l holds row 16t + l % 16, k in [128g + 32 (l / 16), +32) (the
 *     fp8 MFMA B operand of lane l), so a wave's fragment-group is one contiguous KB;
 *   - metadata word r * G + g is row 16t + r, group g: fp16 scale bits in bits 0..15, the
 *     zero-point in bits 16..19 (8 when w_zeros is NULL).
 * The int4 words are a pure permutation of 16-byte words. Needs N % 16 == 0, K % 128 == 0,
 * group size 128; out must not alias w_packed. No reference counterpart: the reference
 * streams the op layout, and its load hook (moe_experts.py:1277-1306) is where a caller runs
 * this once. */
W4A8_API int w4a8_repack_int4_fragments(const int32_t* w_packed, const void* scales_f16,
                                        const int32_t* w_zeros, int64_t E, int64_t N, int64_t K,
                                        int32_t* out, void* stream);

/* int32 words of w4a8_repack_int4_fragments' output for E experts of N rows and K columns
 * (E * N/16 * 272 * K/128), or -1 for sizes it does not take. No reference counterpart. */
W4A8_API int64_t w4a8_fragments_words(int64_t E, int64_t N, int64_t K);

/* w4a8_moe_apply on weights repacked by w4a8_repack_int4_fragments (w13 and w2). The
 * op-layout scales and zero-points are still passed (the schedules that do not read the
 * copies inside the fragment layout use them) and must be the ones the repack read. Same
 * workspace (w4a8_moe_apply_workspace_size) and
 * bit-identical results. Needs group_size 128 and int4 weights (no E2M1); hidden and
 * intermediate sizes must be multiples of 128 that the schedule chosen for T takes: the
 * decode GEMV (T <= 96) needs K/128 in {1,2,3,4,6,8,12,16,32}, the prefill tiles K <= 4096.
 * No reference counterpart (the reference's composition, moe_experts.py:493-665, runs on
 * the op layout). */
W4A8_API int w4a8_moe_apply_fragments(const void* x, int x_dtype, int64_t T, int64_t H,
                                      int64_t inter, int64_t E, int64_t top_k, int64_t group_size,
                                      const int32_t* w13_frag, const void* w13_scales_f16,
                                      const int32_t* w13_zeros, const int32_t* w2_frag,
                                      const void* w2_scales_f16, const int32_t* w2_zeros,
                                      const float* topk_weights, const int32_t* topk_ids,
                                      const int32_t* expert_map, int64_t num_global_experts,
                                      void* out, void* workspace, size_t workspace_bytes,
                                      void* stream);

/* 1 when w4a8_moe_apply_fragments accepts weights of this shape for every T (both the
 * decode and the prefill schedule take it), else 0: what a load hook checks before it
 * repacks. No reference counterpart (layout query). */
W4A8_API int w4a8_moe_fragments_supported(int64_t H, int64_t inter, int64_t group_size);

/* Weight layouts for w4a8_moe_forward. */
#define W4A8_WEIGHTS_OP 0          /* (E, N, K/8) int32, the reference op layout */
#define W4A8_WEIGHTS_FRAGMENTS 1   /* w4a8_repack_int4_fragments output */

/* Router + expert path in one call: softmax / top-k / renormalise of router_logits
 * (T, num_global_experts) fp32 (the vLLM fused_topk the reference's caller runs before apply;
 * ties go to the lower expert id), then w4a8_moe_apply (op layout) or
 * w4a8_moe_apply_fragments on the result (expert_map / num_global_experts as there).
 * topk_weights (T, top_k) fp32 and topk_ids (T, top_k) int32 (global ids) are outputs. Same
 * workspace size as w4a8_moe_apply. No single reference counterpart (fused_topk is vLLM's,
 * moe_experts.py:493-665 the rest). */
W4A8_API int w4a8_moe_forward(const void* x, int x_dtype, int64_t T, int64_t H, int64_t inter,
                              int64_t E, int64_t top_k, int64_t group_size,
                              const float* router_logits, int renormalize, const int32_t* w13,
                              const void* w13_scales_f16, const int32_t* w13_zeros,
                              const int32_t* w2, const void* w2_scales_f16,
                              const int32_t* w2_zeros, int weights_layout,
                              const int32_t* expert_map, int64_t num_global_experts,
                              float* topk_weights, int32_t* topk_ids, void* out,
                              void* workspace, size_t workspace_bytes, void* stream);

/* Size in bytes of the library-owned scratch of w4a8_moe_forward_noalloc (one per GPU). */
#define W4A8_NOALLOC_SCRATCH_BYTES ((size_t)32 << 20)

/* w4a8_moe_forward with no workspace argument that allocates nothing: the intermediates live
 * in a static device array of W4A8_NOALLOC_SCRATCH_BYTES that the library holds on every GPU
 * it runs on until the process ends (its address is looked up once per device, on that
 * device's first call, with the device current). Shapes whose w4a8_moe_apply_workspace_size
 * exceeds the array are refused with W4A8_ERR_WORKSPACE (decode, T <= 96, fits at the
 * reference's shapes; large prefill does not). Results are bit-identical to
 * w4a8_moe_forward. Every call on a GPU uses that GPU's one array, which keeps the last
 * call's contents (the path writes every intermediate before reading it): calls that overlap
 * on one GPU (two streams or two threads) race and must be ordered by the caller. The stream
 * must belong to the current device. No counterpart in the reference: it is for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid allocation). */
W4A8_API int w4a8_moe_forward_noalloc(const void* x, int x_dtype, int64_t T, int64_t H,
                                      int64_t inter, int64_t E, int64_t top_k, int64_t group_size,
                                      const float* router_logits, int renormalize,
                                      const int32_t* w13, const void* w13_scales_f16,
                                      const int32_t* w13_zeros, const int32_t* w2,
                                      const void* w2_scales_f16, const int32_t* w2_zeros,
                                      int weights_layout, const int32_t* expert_map,
                                      int64_t num_global_experts, float* topk_weights,
                                      int32_t* topk_ids, void* out, void* stream);

/* Optional per-stage timing of the whole-layer calls on the calling thread: when count >= 8,
 * the next w4a8_moe_apply / _fragments / w4a8_moe_forward calls record events[0] before the
 * first expert-path launch and events[i] after stage i (1 align, 2 act-quant x, 3 reserved
 * (empty), 4 gemm1+SiLU, 5 act-quant h, 6 gemm2, 7 reduce/cast) on their stream. With
 * count == 12, events[8] / events[9] are also stamped at the start / end of the gemm1 kernel
 * itself and events[10] / events[11] of the gemm2 kernel (hipExtLaunchKernel: the kernel's
 * own duration, no marker latency). Events are hipEvent_t handles owned by the caller;
 * count == 0 switches recording off. No reference counterpart (measurement aid). */
W4A8_API int w4a8_moe_apply_set_stage_events(void* const* events, int count);

/* Fused decode layer switch: on != 0 makes the decode schedule on fragment-layout weights
 * run gemm1+SiLU and gemm2 as one persistent launch (both GEMVs on the same expert lists;
 * gemm2 teams wait inside the kernel, with bounded waits, for the gemm1 rows they read).
 * The default comes from W4A8_DECODE_FUSED=1 in the environment, read once. Returns the
 * previous setting. The launch needs every work-group (one per CU) resident at once: eager
 * calls use a cooperative launch, which the runtime refuses otherwise; under graph capture
 * the launch is an ordinary one, and a wait that gives up makes that call's output NaN.
 * Process-wide. No reference counterpart (the reference runs separate launches). */
W4A8_API int w4a8_set_decode_fused(int on);

/* Prefill pair switch: on != 0 (the default; W4A8_PREFILL_PAIR=0 in the environment, read
 * once, turns it off) lets the many-token schedule run gemm1+SiLU and gemm2 of the
 * activation-resident tiles as one launch where both apply (hidden size <= 2048,
 * intermediate size <= 1536): each work-group takes a 64-row tile through gemm1, then through
 * gemm2 on the h rows it has just written. Results are the same bits as the two launches.
 * Returns the previous setting. Process-wide. No reference counterpart (the reference runs
 * separate launches). */
W4A8_API int w4a8_set_prefill_pair(int on);

/* Test hook of the fused decode layer: while on != 0 (a device-side word of the current
 * device, so captured graphs see it between replays), its in-kernel waits wait for a flag
 * value no work-group publishes, with a short spin limit, so they give up and the call's
 * output is NaN; every kernel still ends normally. For failure-path tests only. No
 * reference counterpart. */
W4A8_API int w4a8_decode_fused_test_fault(int on);

#ifdef __cplusplus
}
#endif

#endif /* W4A8_MOE_H_ */
