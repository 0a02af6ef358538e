// C ABI entry points (include/w4a8_moe.h): argument validation mirroring the reference's
// TORCH_CHECKs (w4a8_fp8_wmma/bindings.cpp), workspace carving, kernel-id dispatch and the
// whole-layer composition (moe_experts.py:493-665).
#include <atomic>
#include <cstdlib>
#include <map>
#include <mutex>
#include <string>
#include <tuple>

#include "w4a8_common.h"
#include "w4a8_internal.h"

namespace w4a8 {

namespace {
thread_local std::string g_error;

hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

#define W4A8_REQUIRE(cond, msg)            \
    do {                                   \
        if (!(cond)) {                     \
            ::w4a8::set_error(msg);        \
            return W4A8_ERR_INVALID;       \
        }                                  \
    } while (0)

bool moe_kernel_valid(int64_t k) { return k == 0 || k == 6 || k == 7; }
bool dense_kernel_valid(int64_t v) { return v == 0 || v == 1 || v == 2 || (v >= 4 && v <= 14); }

// Shapes shared by every grouped GEMM entry (bindings.cpp:191-221).
int check_grouped(int64_t rows, int64_t K, int64_t E, int64_t N, int64_t gs, int64_t P,
                  int64_t block_m, int64_t top_k, int64_t kernel, const void* x,
                  const void* w, const void* scales, const int32_t* sti, const int32_t* eid,
                  const int32_t* ntp) {
    W4A8_REQUIRE(rows >= 0 && K > 0 && E > 0 && N > 0 && P >= 0, "invalid sizes");
    W4A8_REQUIRE(K % kPackFactor == 0, "K must be a multiple of 8 (w_packed last dim is K/8)");
    W4A8_REQUIRE(gs > 0 && K % gs == 0, "K not divisible by group_size");
    W4A8_REQUIRE(gs % 16 == 0 && gs <= kMaxGroupSize,
                 "group_size must be a multiple of 16 and <= 128");
    W4A8_REQUIRE(block_m > 0 && P % block_m == 0, "P not divisible by block_m");
    W4A8_REQUIRE(top_k > 0, "top_k must be positive");
    W4A8_REQUIRE(moe_kernel_valid(kernel),
                 "moe kernel id must be 0 (scalar) / 6 (wmma) / 7 (gemv)");
    if (kernel == W4A8_MOE_KERNEL_WMMA)
        W4A8_REQUIRE(block_m % 16 == 0 && block_m <= 128,
                     "wmma block_m must be a multiple of 16 and <= 128");
    if (kernel == W4A8_MOE_KERNEL_GEMV)
        W4A8_REQUIRE(block_m % 8 == 0 && block_m <= 64 && K % 32 == 0 && gs % 32 == 0,
                     "gemv needs block_m mult of 8 <= 64, K%32==0, group_size%32==0");
    W4A8_REQUIRE(x != nullptr && w != nullptr && scales != nullptr, "null tensor pointer");
    W4A8_REQUIRE(P == 0 || (sti != nullptr && eid != nullptr && ntp != nullptr),
                 "null routing pointer");
    return W4A8_OK;
}

int run_grouped(GroupedArgs& a, int64_t kernel, void* ws, size_t ws_bytes, hipStream_t s) {
    const bool mfma = mfma_supported(a.K, a.group_size, a.e2m1);
    // E2M1 codebook weights take the matrix-core tiles (the GEMV feeds raw nibbles)
    const bool gemv = gemv_supported(a.K, a.group_size) && !a.e2m1;
    Workspace w(ws, ws_bytes);
    a.x_fp8 = w.take<uint8_t>((size_t)(a.x_rows * a.K));
    a.act_scales = w.take<float>((size_t)a.x_rows);
    float* gsum = w.take<float>((size_t)(a.x_rows * ((a.K + 127) / 128)));
    const bool have_ws = !(a.x_rows > 0 && ws == nullptr) && w.ok();
    // identity-gathered inputs (gemm2 / scatter) have one row per padded row: skip padding.
    const bool filter = a.identity_gather && a.sorted_ids != nullptr;
    if (kernel == W4A8_MOE_KERNEL_GEMV && gemv) {
        if (!have_ws) {
            // no workspace: the GEMV quantises its block's rows itself (bit-identical to
            // act_quant, but repeated by every work-group that reads a row)
            a.x_fp8 = nullptr;
            a.act_scales = nullptr;
            return launch_grouped_gemv(a, s);
        }
        if (int rc = launch_act_quant(a.x, a.x_bf16, a.x_rows, a.K, a.x_fp8, a.act_scales, true,
                                      s, filter ? a.sorted_ids : nullptr,
                                      filter ? a.ntp : nullptr, a.num_valid, nullptr))
            return rc;
        return launch_grouped_gemv(a, s);
    }
    if (!have_ws) {
        set_error("workspace smaller than w4a8_moe_gemm_workspace_size()");
        return W4A8_ERR_WORKSPACE;
    }
    // gemv for K-group counts outside its split-K table runs the matrix-core tiles
    const bool tiles = (kernel == W4A8_MOE_KERNEL_WMMA || kernel == W4A8_MOE_KERNEL_GEMV) && mfma;
    // E2M1 tiles take fp4 operands against activations in natural k order; every other
    // kernel (the scalar one included) takes k8-interleaved activations
    const bool k8 = !(a.e2m1 && tiles);
    const bool prefill = tiles && prefill_supported(a.K, a.group_size, a.e2m1);
    a.act_group_sums = prefill ? gsum : nullptr;
    if (int rc = launch_act_quant(a.x, a.x_bf16, a.x_rows, a.K, a.x_fp8, a.act_scales, k8, s,
                                  filter ? a.sorted_ids : nullptr, filter ? a.ntp : nullptr,
                                  a.num_valid, a.act_group_sums))
        return rc;
    // activation-resident tiles where the shape allows (the whole-layer prefill kernel, so
    // the op API and moe_apply share it), the streamed-K tiles otherwise. An ares work-group
    // owns all N columns of its rows, so one expert (the dense GEMM) fills the chip only with
    // >= 512 row tiles; below that the streamed-K tiles also split N.
    const bool ares_fills = a.E > 1 || a.P >= 512 * 64;
    if (prefill && ares_fills &&
        prefill_ares_supported(a.K, a.N, a.group_size, a.e2m1, a.block_m, a.epi) &&
        a.x_rows * a.K < ((int64_t)1 << 31))
        return launch_grouped_prefill_ares(a, s);
    if (prefill) return launch_grouped_prefill(a, s);
    if (tiles) return launch_grouped_mfma(a, s);
    return launch_grouped_scalar(a, s);
}

}  // namespace

void set_error(const std::string& msg) { g_error = msg; }

KernelStamp& next_kernel_stamp() {
    thread_local KernelStamp stamp;
    return stamp;
}
void clear_error() { g_error.clear(); }

int check_launch(const char* what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_error(std::string(what) + ": " + hipGetErrorString(e));
        return W4A8_ERR_HIP;
    }
    return W4A8_OK;
}

namespace {
std::mutex g_dev_mu;
// (device, kind, kernel, threads, lds) -> cached value; kind 0: LDS reserved, 1: blocks
// per CU, 2: CU count
std::map<std::tuple<int, int, const void*, int, size_t>, int> g_dev_facts;
int current_device() {
    int dev = 0;
    return hipGetDevice(&dev) == hipSuccess ? dev : 0;
}
}  // namespace

int reserve_dyn_lds(const void* kernel, int bytes, const char* what) {
    const auto key = std::make_tuple(current_device(), 0, kernel, 0, (size_t)bytes);
    std::lock_guard<std::mutex> lock(g_dev_mu);
    if (g_dev_facts.count(key)) return W4A8_OK;
    const hipError_t e =
        hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    if (e != hipSuccess) {
        set_error(std::string(what) + ": cannot reserve dynamic LDS: " + hipGetErrorString(e));
        return W4A8_ERR_HIP;
    }
    g_dev_facts[key] = 1;
    return W4A8_OK;
}

int device_cu_count() {
    const int dev = current_device();
    const auto key = std::make_tuple(dev, 2, (const void*)nullptr, 0, (size_t)0);
    std::lock_guard<std::mutex> lock(g_dev_mu);
    auto it = g_dev_facts.find(key);
    if (it != g_dev_facts.end()) return it->second;
    int ncu = 0;
    if (hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        ncu <= 0)
        ncu = 256;
    g_dev_facts[key] = ncu;
    return ncu;
}

int blocks_per_cu(const void* kernel, int threads, size_t lds) {
    const auto key = std::make_tuple(current_device(), 1, kernel, threads, lds);
    std::lock_guard<std::mutex> lock(g_dev_mu);
    auto it = g_dev_facts.find(key);
    if (it != g_dev_facts.end()) return it->second;
    int occ = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, kernel, threads, lds) != hipSuccess ||
        occ < 0)
        occ = 0;
    g_dev_facts[key] = occ;
    return occ;
}

}  // namespace w4a8

// ---------------------------------------------------------------------------------------
// whole layer
// ---------------------------------------------------------------------------------------
namespace w4a8 {
namespace {
constexpr int64_t kAlignSmallMax = 1024;  // numel handled by the one-work-group align
constexpr int64_t kGemvMaxM = 96;   // moe_experts.py:563 GEMV_MAX_M
constexpr int64_t kDecodeBlockM = 16;
constexpr int64_t kPrefillBlockM = 64;    // 64-row tiles; empty 16-row fragments are skipped
// the activation-resident tiles address their rows in 32 bits: rows * K < 2^31, else the
// streamed-K tiles run
constexpr int64_t kAresMaxElems = (int64_t)1 << 31;

struct ApplyPlan {
    bool decode;
    int64_t block_m, P, nblk;
};

ApplyPlan plan_apply(int64_t T, int64_t E, int64_t top_k) {
    ApplyPlan pl;
    pl.decode = T <= kGemvMaxM;
    pl.block_m = pl.decode ? kDecodeBlockM : kPrefillBlockM;
    pl.P = w4a8_moe_align_sorted_len(T * top_k, E, pl.block_m);
    pl.nblk = pl.P / pl.block_m;
    return pl;
}

template <typename WS>
void carve_apply(WS& w, const ApplyPlan& pl, int64_t T, int64_t H, int64_t inter, int64_t E,
                 int64_t top_k, int32_t** sti, int32_t** eid, int32_t** ntp, void** align_ws,
                 size_t* align_bytes, uint8_t** xq, float** s1, __half** h, uint8_t** hq,
                 float** s2, float** acc, float** gs1, float** gs2, __half** y,
                 int32_t** s2r, uint64_t** dflags, DecHandover** dhand) {
    *sti = w.template take<int32_t>((size_t)pl.P);
    *eid = w.template take<int32_t>((size_t)pl.nblk);
    *ntp = w.template take<int32_t>(1);
    *align_bytes = align_workspace_bytes(T * top_k, E);
    *align_ws = w.template take<uint8_t>(*align_bytes);
    *xq = w.template take<uint8_t>((size_t)(T * H));
    *s1 = w.template take<float>((size_t)T);
    *h = w.template take<__half>((size_t)(pl.P * inter));
    *hq = w.template take<uint8_t>((size_t)(pl.P * inter));
    *s2 = w.template take<float>((size_t)pl.P);
    // decode: per-slot fp32 rows (T*k, H); prefill: fp16 rows (P, H) in padded order and the
    // slot -> padded-row map the combine reads
    *acc = pl.decode ? w.template take<float>((size_t)(T * top_k * H)) : nullptr;
    *y = pl.decode ? nullptr : w.template take<__half>((size_t)(pl.P * H));
    *s2r = pl.decode ? nullptr : w.template take<int32_t>((size_t)(T * top_k));
    // prefill: per-group sums of the quantised rows (zero-point term of the tiles)
    *gs1 = pl.decode ? nullptr : w.template take<float>((size_t)(T * ((H + 127) / 128)));
    *gs2 = pl.decode ? nullptr : w.template take<float>((size_t)(pl.P * ((inter + 127) / 128)));
    // decode: completion flags of the fused layer's work-groups and their timeout words
    *dflags = pl.decode ? w.template take<uint64_t>((size_t)(2 * kDecodeFlagSlots)) : nullptr;
    // decode: the lists the gemm1 launch hands to the gemm2 launch
    *dhand = pl.decode ? w.template take<DecHandover>(1) : nullptr;
}

// Per-call value of the fused decode layer's completion flags (never 0).
uint64_t next_decode_nonce() {
    static std::atomic<uint64_t> counter{0x9E3779B97F4A7C15ull};
    uint64_t v = counter.fetch_add(1, std::memory_order_relaxed);
    return v == 0 ? counter.fetch_add(1, std::memory_order_relaxed) : v;
}

// The decode layer's two GEMVs as one launch (decode_layer_kernel): W4A8_DECODE_FUSED=1 in
// the environment when the library first needs the setting, or w4a8_set_decode_fused().
// Off by default: on MI355X it measures slower than the two launches (the in-kernel wait for
// h through agent-coherent loads costs more than the launch boundary it removes).
std::atomic<int> g_decode_fused{-1};   // -1: not read yet
bool decode_fused_enabled() {
    int v = g_decode_fused.load(std::memory_order_relaxed);
    if (v < 0) {
        const char* e = std::getenv("W4A8_DECODE_FUSED");
        int want = (e != nullptr && e[0] == '1') ? 1 : 0;
        int expected = -1;
        g_decode_fused.compare_exchange_strong(expected, want, std::memory_order_relaxed);
        v = g_decode_fused.load(std::memory_order_relaxed);
    }
    return v == 1;
}

// gemm1+SiLU and gemm2 of the activation-resident prefill tiles as one launch
// (prefill_ares_pair_kernel) where both tiles apply; W4A8_PREFILL_PAIR=0 in the environment
// (read once per process) or w4a8_set_prefill_pair(0) keeps two launches.
std::atomic<int> g_prefill_pair{-1};   // -1: not read yet
bool prefill_pair_enabled() {
    int v = g_prefill_pair.load(std::memory_order_relaxed);
    if (v < 0) {
        const char* e = std::getenv("W4A8_PREFILL_PAIR");
        int want = (e != nullptr && e[0] == '0') ? 0 : 1;
        int expected = -1;
        g_prefill_pair.compare_exchange_strong(expected, want, std::memory_order_relaxed);
        v = g_prefill_pair.load(std::memory_order_relaxed);
    }
    return v == 1;
}

constexpr int kStageEvents = 8;
constexpr int kStampEvents = 4;   // optional: kernel-exact start / stop of gemm1 and gemm2
thread_local hipEvent_t g_stage_events[kStageEvents + kStampEvents];
thread_local bool g_stage_on = false;
thread_local bool g_stage_stamps = false;

inline void stage_mark(int i, hipStream_t s) {
    if (!g_stage_on) return;
    (void)hipEventRecord(g_stage_events[i], s);
}

// Arms (gemm = 0 / 1) or clears (gemm < 0) the kernel-exact stamps of the next GEMM launch.
inline void stamp_gemm(int gemm) {
    if (!g_stage_on || !g_stage_stamps) return;
    KernelStamp& st = next_kernel_stamp();
    if (gemm < 0) {
        st = KernelStamp{};
        return;
    }
    st.start = g_stage_events[kStageEvents + 2 * gemm];
    st.stop = g_stage_events[kStageEvents + 2 * gemm + 1];
}

// Fragment-layout weights are read by the decode GEMV and the prefill tiles only.
bool fragments_schedule_ok(bool decode, int64_t H, int64_t inter, int64_t gs) {
    if (gs != 128 || H % 128 != 0 || inter % 128 != 0) return false;
    if (decode) return gemv_supported(H, gs) && gemv_supported(inter, gs);
    return prefill_supported(H, gs, false) && prefill_supported(inter, gs, false);
}

struct SizeProbe {
    WorkspaceSize s;
    template <typename T>
    T* take(size_t n) { s.take<T>(n); return nullptr; }
};
}  // namespace
}  // namespace w4a8


using namespace w4a8;

namespace w4a8 {
// frag: w13 / w2 in the fragment layout (launch_repack_fragments); only the GEMV and the
// prefill tiles read it, so every other schedule is refused up front.
// logits: when given, the router runs first and topk_weights / topk_ids are its outputs
// (the decode schedule folds it into the prologue launch).
int moe_apply_impl(const void* x, int x_dtype, int64_t T, int64_t H, int64_t inter, int64_t E,
                   int64_t top_k, int64_t group_size, const int32_t* w13,
                   const void* w13_scales_f16, const int32_t* w13_zeros, const int32_t* w2,
                   const void* w2_scales_f16, const int32_t* w2_zeros,
                   const float* topk_weights, const int32_t* topk_ids,
                   const int32_t* expert_map, int64_t n_global, int weight_is_e2m1, void* out,
                   void* workspace, size_t workspace_bytes, void* stream, bool frag,
                   const float* logits = nullptr, bool renormalize = true) {
    W4A8_REQUIRE(x_dtype == W4A8_DTYPE_F16 || x_dtype == W4A8_DTYPE_BF16, "x dtype must be fp16 or bf16");
    W4A8_REQUIRE(T >= 0 && H > 0 && inter > 0 && E > 0 && top_k > 0, "moe_apply: invalid sizes");
    W4A8_REQUIRE(group_size > 0 && H % group_size == 0 && inter % group_size == 0 &&
                 group_size % 16 == 0 && group_size <= kMaxGroupSize,
                 "moe_apply: group_size must divide hidden and intermediate, mult of 16, <= 128");
    W4A8_REQUIRE(H % 8 == 0 && inter % 8 == 0, "moe_apply: sizes must be multiples of 8");
    W4A8_REQUIRE(!(weight_is_e2m1 && (w13_zeros || w2_zeros)),
                 "mxfp4 (E2M1) weights are symmetric; w_zeros must be empty");
    if (n_global <= 0) n_global = E;
    W4A8_REQUIRE(expert_map != nullptr || n_global == E,
                 "moe_apply: global expert count differs from the local one; pass expert_map");
    W4A8_REQUIRE(n_global <= (int64_t)1 << 20, "moe_apply: too many global experts");
    const ApplyPlan pl = plan_apply(T, E, top_k);
    W4A8_REQUIRE(!frag || (!weight_is_e2m1 && fragments_schedule_ok(pl.decode, H, inter, group_size)),
                 "fragment-layout weights need int4 g128 with hidden and intermediate sizes the "
                 "chosen schedule takes (decode GEMV: K/128 in {1,2,3,4,6,8,12,16,32}; prefill "
                 "tiles: K <= 4096)");
    if (T == 0) return W4A8_OK;
    W4A8_REQUIRE(x && w13 && w13_scales_f16 && w2 && w2_scales_f16 && topk_weights && topk_ids && out,
                 "moe_apply: null pointer");
    W4A8_REQUIRE(logits == nullptr || n_global <= 1024,
                 "moe_forward: the router takes at most 1024 experts");
    hipStream_t s = as_stream(stream);
    Workspace w(workspace, workspace_bytes);
    int32_t *sti, *eid, *ntp; void* aws; size_t abytes; uint8_t* xq; float* s1; __half* h;
    uint8_t* hq; float* s2; float* acc; float* gs1; float* gs2; __half* y; int32_t* s2r;
    uint64_t* dflags;
    DecHandover* dhand;
    carve_apply(w, pl, T, H, inter, E, top_k, &sti, &eid, &ntp, &aws, &abytes, &xq, &s1, &h, &hq,
                &s2, &acc, &gs1, &gs2, &y, &s2r, &dflags, &dhand);
    if (workspace == nullptr || !w.ok()) {
        set_error("moe_apply: workspace smaller than w4a8_moe_apply_workspace_size()");
        return W4A8_ERR_WORKSPACE;
    }
    const bool bf16 = x_dtype == W4A8_DTYPE_BF16;
    const bool e2m1 = weight_is_e2m1 != 0;
    const int64_t numel = T * top_k;
    const bool mfma = mfma_supported(H, group_size, e2m1) && mfma_supported(inter, group_size, e2m1);
    // E2M1 tiles take fp4 operands against activations in natural k order; the scalar
    // kernel takes k8-interleaved ones
    const bool k8 = !(e2m1 && mfma);
    // prefill tiles need the per-group sums of the quantised rows (zero-point term)
    const bool pf1 = !pl.decode && mfma && prefill_supported(H, group_size, e2m1);
    const bool pf2 = !pl.decode && mfma && prefill_supported(inter, group_size, e2m1);
    // router: one wave per token over the whole grid (folding it into the align launch
    // would serialise the tokens on the align work-group)
    // many-token schedule: the routing waves also quantise x (one launch less)
    const bool route_quant = logits != nullptr && !(pl.decode && numel <= kAlignSmallMax) && k8;
    const bool frag_decode =
        frag && pl.decode && !e2m1 && decode_layer_supported(numel, E, H, inter, group_size);
    // few tokens: the decode gemm1 launch routes them itself (no router launch)
    const bool route_in_gemm1 = logits != nullptr && frag_decode &&
                                decode_routes_in_kernel(T, n_global, top_k);
    // decode on fragment weights after a router launch: the routing waves quantise x as well,
    // and the separate gemm1 launch reads those rows instead of quantising in registers at
    // every pass start (the fused layer keeps its in-register quantisation)
    const bool decode_preq = logits != nullptr && frag_decode && !route_in_gemm1 && k8 &&
                             !(decode_fused_enabled() && decode_layer_fused_supported(H, inter));
    if (logits != nullptr && !route_in_gemm1)
        if (int rc = launch_topk_softmax(logits, T, n_global, top_k, renormalize,
                                         const_cast<float*>(topk_weights),
                                         const_cast<int32_t*>(topk_ids), s,
                                         route_quant || decode_preq ? x : nullptr, bf16, H, xq,
                                         s1, pf1 ? gs1 : nullptr))
            return rc;
    stage_mark(0, s);
    if (frag_decode) {
        // decode on fragment-layout weights: two GEMVs that group the slots by expert
        // themselves (no align launch) and quantise their rows in registers (no act-quant
        // launches), then the slot reduce
        stage_mark(1, s);
        stage_mark(2, s);
        stage_mark(3, s);
        DecodeLaunch d{};
        d.topk_ids = topk_ids; d.expert_map = expert_map; d.emap_len = n_global;
        d.numel = numel; d.top_k = top_k; d.E = E;
        d.a = x; d.a_bf16 = bf16; d.silu = true;
        d.w = w13; d.scales = w13_scales_f16; d.zeros = w13_zeros; d.out = h;
        d.K = H; d.N = 2 * inter;
        DecodeLaunch d2 = d;
        if (route_in_gemm1) {
            d.logits = logits; d.n_router = n_global; d.renormalize = renormalize;
            d.topk_weights_out = const_cast<float*>(topk_weights);
            d.topk_ids_out = const_cast<int32_t*>(topk_ids);
        }
        d2.a = h; d2.a_bf16 = false; d2.silu = false;
        if (decode_preq) {
            d.aq = xq;
            d.asc = s1;
        }
        d2.w = w2; d2.scales = w2_scales_f16; d2.zeros = w2_zeros; d2.out = acc;
        d2.K = inter; d2.N = H;
        SlotReduceSync sync;
        int rc;
        if (decode_fused_enabled() && decode_layer_fused_supported(H, inter)) {
            // one launch for both GEMVs; the slot reduce resets the completion flags
            sync.flags = dflags;
            sync.nflags = (int)kDecodeFlagSlots;
            sync.timeout = dflags + kDecodeFlagSlots;
            sync.ntimeout = decode_layer_grid();
            sync.nonce = next_decode_nonce();
            stamp_gemm(0);
            rc = launch_decode_layer(d, d2, dflags, sync.nonce, dflags + kDecodeFlagSlots, s);
            stamp_gemm(-1);
            if (rc) return rc;
            stage_mark(4, s);
            stage_mark(5, s);
        } else {
            // gemm1 hands its expert lists to the gemm2 launch
            d.hand_out = dhand;
            d2.hand_in = dhand;
            stamp_gemm(0);
            rc = launch_decode_gemv(d, s);
            stamp_gemm(-1);
            if (rc) return rc;
            stage_mark(4, s);
            stage_mark(5, s);
            stamp_gemm(1);
            rc = launch_decode_gemv(d2, s);
            stamp_gemm(-1);
            if (rc) return rc;
        }
        stage_mark(6, s);
        rc = launch_slot_reduce(acc, topk_weights, topk_ids, expert_map, n_global, E, T, H, top_k,
                                out, bf16, s, sync);
        stage_mark(7, s);
        return rc;
    }
    if (pl.decode && numel <= kAlignSmallMax && k8) {
        // one launch: align in work-group 0, act-quant of x in the others
        if (int rc = launch_align_quant(topk_ids, numel, E, pl.block_m, expert_map, n_global, sti,
                                        pl.P, eid, ntp, s2r, x, bf16, T, H, xq, s1, nullptr, s))
            return rc;
        stage_mark(1, s);
    } else {
        if (int rc = launch_align(topk_ids, numel, E, pl.block_m, expert_map, n_global, sti, pl.P,
                                  eid, ntp, aws, abytes, s, s2r))
            return rc;
        stage_mark(1, s);
        if (!route_quant)
            if (int rc = launch_act_quant(x, bf16, T, H, xq, s1, k8, s, nullptr, nullptr, 0,
                                          pf1 ? gs1 : nullptr))
                return rc;
    }
    stage_mark(2, s);
    stage_mark(3, s);

    // gemm1 + SiLU*mul -> h (P, inter)
    GroupedArgs g1{};
    g1.x_rows = T; g1.K = H; g1.w = w13; g1.scales = static_cast<const uint16_t*>(w13_scales_f16);
    g1.zeros = w13_zeros; g1.E = E; g1.N = 2 * inter; g1.group_size = group_size;
    g1.sorted_ids = sti; g1.P = pl.P; g1.expert_ids = eid; g1.ntp = ntp; g1.top_k = top_k;
    g1.identity_gather = false; g1.num_valid = numel; g1.block_m = pl.block_m; g1.e2m1 = e2m1;
    g1.epi = Epi::kSiluHalf; g1.out = h; g1.out_top_k = top_k; g1.x_fp8 = xq; g1.act_scales = s1;
    g1.act_group_sums = pf1 ? gs1 : nullptr;
    g1.w_frag = frag;
    const bool ares1 = pf1 && prefill_ares_supported(H, 2 * inter, group_size, e2m1, pl.block_m,
                                                     Epi::kSiluHalf) && T * H < kAresMaxElems;
    // act-quant of h over real rows only, once per row (quantising inside the decode GEMV
    // would repeat it for every work-group that reads the row); the activation-resident
    // prefill tiles quantise their own rows instead (a tile is the only reader of its rows)
    const bool gemv2 = pl.decode && !e2m1 && gemv_supported(inter, group_size);
    const bool ares2 = pf2 && prefill_ares_supported(inter, H, group_size, e2m1, pl.block_m, Epi::kHalf) &&
                       pl.P * inter < kAresMaxElems;
    const bool ares2_quant = ares2 && prefill_ares_quantises_rows(inter, Epi::kHalf);
    // gemm2 (identity gather) -> per-slot rows (decode) or scatter (prefill)
    GroupedArgs g2{};
    g2.x_rows = pl.P; g2.K = inter; g2.w = w2; g2.scales = static_cast<const uint16_t*>(w2_scales_f16);
    g2.zeros = w2_zeros; g2.E = E; g2.N = H; g2.group_size = group_size;
    g2.sorted_ids = sti; g2.P = pl.P; g2.expert_ids = eid; g2.ntp = ntp; g2.top_k = top_k;
    g2.identity_gather = true; g2.num_valid = numel; g2.block_m = pl.block_m; g2.e2m1 = e2m1;
    g2.epi = pl.decode ? Epi::kSlotF32 : Epi::kHalf; g2.out = pl.decode ? (void*)acc : (void*)y;
    g2.topk_weights = topk_weights; g2.out_top_k = top_k;
    g2.x = h; g2.x_bf16 = false;
    g2.x_fp8 = ares2_quant ? nullptr : hq;
    g2.act_scales = ares2_quant ? nullptr : s2;
    g2.act_group_sums = pf2 && !ares2_quant ? gs2 : nullptr;
    g2.w_frag = frag;
    int rc;
    if (ares1 && ares2_quant && prefill_pair_enabled() && prefill_ares_pair_supported(g1, g2)) {
        // both GEMMs in one launch, each work-group taking a tile through gemm1 and gemm2
        stamp_gemm(0);
        rc = launch_grouped_prefill_ares_pair(g1, g2, s);
        stamp_gemm(-1);
        if (rc) return rc;
        stage_mark(4, s);
        stage_mark(5, s);
        stage_mark(6, s);
        rc = launch_row_reduce(y, s2r, topk_weights, T, H, top_k, out, bf16, s);
        stage_mark(7, s);
        return rc;
    }
    stamp_gemm(0);
    if (!mfma) rc = launch_grouped_scalar(g1, s);
    else if (pl.decode && !e2m1 && gemv_supported(H, group_size)) rc = launch_grouped_gemv(g1, s);
    else if (ares1) rc = launch_grouped_prefill_ares(g1, s);
    else if (pf1) rc = launch_grouped_prefill(g1, s);
    else rc = launch_grouped_mfma(g1, s);
    stamp_gemm(-1);
    if (rc) return rc;
    stage_mark(4, s);
    if (!ares2_quant && (rc = launch_act_quant(h, false, pl.P, inter, hq, s2, k8, s, sti, ntp,
                                               numel, pf2 ? gs2 : nullptr)))
        return rc;
    stage_mark(5, s);
    stamp_gemm(1);
    if (!mfma) rc = launch_grouped_scalar(g2, s);
    else if (gemv2) rc = launch_grouped_gemv(g2, s);
    else if (ares2) rc = launch_grouped_prefill_ares(g2, s);
    else if (pf2) rc = launch_grouped_prefill(g2, s);
    else rc = launch_grouped_mfma(g2, s);
    stamp_gemm(-1);
    if (rc) return rc;
    stage_mark(6, s);
    // slots whose expert is not local / out of range contribute nothing
    if (pl.decode)
        rc = launch_slot_reduce(acc, topk_weights, topk_ids, expert_map, n_global, E, T, H, top_k,
                                out, bf16, s);
    else
        rc = launch_row_reduce(y, s2r, topk_weights, T, H, top_k, out, bf16, s);
    stage_mark(7, s);
    return rc;
}
}  // namespace w4a8

namespace w4a8 {
namespace {

// Scratch of w4a8_moe_forward_noalloc: device data of the code object, one copy per GPU,
// allocated when the library's code is loaded onto that GPU and held until the process
// ends. In host code the array's name is only a stand-in for the symbol; the device address
// of each GPU's copy comes from hipGetSymbolAddress with that GPU current.
constexpr size_t kNoAllocScratchBytes = W4A8_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// The current device's scratch address, looked up on the device's first call.
int noalloc_scratch(void** out) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        set_error("moe_forward_noalloc: no usable current HIP device");
        return W4A8_ERR_HIP;
    }
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr[dev] == nullptr) {
        void* p = nullptr;
        const hipError_t err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (err != hipSuccess || p == nullptr) {
            set_error(std::string("moe_forward_noalloc: hipGetSymbolAddress(scratch) failed: ") +
                      hipGetErrorString(err));
            return W4A8_ERR_HIP;
        }
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return W4A8_OK;
}

}  // namespace
}  // namespace w4a8

extern "C" {

int w4a8_abi_version(void) { return 3; }

const char* w4a8_last_error(void) { return g_error.c_str(); }

int w4a8_act_quant_fp8(const void* x_f16, int64_t rows, int64_t K, uint8_t* x_fp8,
                       float* act_scales, int k8_interleave, void* stream) {
    clear_error();
    W4A8_REQUIRE(rows >= 0 && K > 0 && K % 8 == 0, "act_quant: K must be a positive multiple of 8");
    W4A8_REQUIRE(rows == 0 || (x_f16 && x_fp8 && act_scales), "act_quant: null pointer");
    return launch_act_quant(x_f16, false, rows, K, x_fp8, act_scales, k8_interleave != 0,
                            as_stream(stream));
}

int w4a8_dequant_fp8(const int32_t* w_packed, const int32_t* w_zeros, int64_t E, int64_t N,
                     int64_t K, int64_t group_size, int weight_is_e2m1, uint8_t* out,
                     void* stream) {
    clear_error();
    W4A8_REQUIRE(E > 0 && N > 0 && K > 0 && K % 8 == 0, "dequant: invalid sizes");
    W4A8_REQUIRE(group_size > 0 && K % group_size == 0 && group_size % 8 == 0,
                 "dequant: group_size must divide K and be a multiple of 8");
    W4A8_REQUIRE(w_zeros == nullptr || N % 8 == 0, "dequant: zero-points need N % 8 == 0");
    W4A8_REQUIRE(!(weight_is_e2m1 && w_zeros), "mxfp4 (E2M1) weights are symmetric; w_zeros must be empty");
    W4A8_REQUIRE(w_packed && out, "dequant: null pointer");
    return launch_dequant(w_packed, w_zeros, E, N, K, group_size, weight_is_e2m1 != 0, out,
                          as_stream(stream));
}

int w4a8_topk_softmax(const float* logits, int64_t T, int64_t E, int64_t top_k,
                      int renormalize, float* topk_weights, int32_t* topk_ids, void* stream) {
    clear_error();
    W4A8_REQUIRE(T >= 0 && E > 0 && top_k > 0, "topk_softmax: invalid sizes");
    W4A8_REQUIRE(T == 0 || (logits && topk_weights && topk_ids), "topk_softmax: null pointer");
    return launch_topk_softmax(logits, T, E, top_k, renormalize != 0, topk_weights, topk_ids,
                               as_stream(stream));
}

int64_t w4a8_moe_align_sorted_len(int64_t numel, int64_t num_experts, int64_t block_m) {
    if (block_m <= 0) return -1;
    const int64_t m = numel + num_experts * (block_m - 1);
    return (m + block_m - 1) / block_m * block_m;
}

size_t w4a8_moe_align_workspace_size(int64_t numel, int64_t num_experts) {
    return align_workspace_bytes(numel, num_experts);
}

int w4a8_moe_align_block_size(const int32_t* topk_ids, int64_t numel, int64_t num_experts,
                              int64_t block_m, const int32_t* expert_map,
                              int32_t* sorted_token_ids, int64_t sorted_len,
                              int32_t* expert_ids, int32_t* num_tokens_post_padded,
                              void* workspace, size_t workspace_bytes, void* stream) {
    clear_error();
    W4A8_REQUIRE(numel >= 0 && num_experts > 0 && block_m > 0, "moe_align: invalid sizes");
    W4A8_REQUIRE(numel < (int64_t)1 << 30, "moe_align: too many slots");
    W4A8_REQUIRE(sorted_len == w4a8_moe_align_sorted_len(numel, num_experts, block_m),
                 "moe_align: sorted_len must equal round_up(numel + E*(block_m-1), block_m)");
    W4A8_REQUIRE(sorted_token_ids && expert_ids && num_tokens_post_padded,
                 "moe_align: null output pointer");
    W4A8_REQUIRE(numel == 0 || topk_ids, "moe_align: null topk_ids");
    return launch_align(topk_ids, numel, num_experts, block_m, expert_map, num_experts,
                        sorted_token_ids, sorted_len, expert_ids, num_tokens_post_padded,
                        workspace, workspace_bytes, as_stream(stream));
}

size_t w4a8_moe_gemm_workspace_size(int64_t x_rows, int64_t K) {
    WorkspaceSize s;
    s.take<uint8_t>((size_t)(x_rows * K));
    s.take<float>((size_t)x_rows);
    s.take<float>((size_t)(x_rows * ((K + 127) / 128)));   // per-group sums (prefill tiles)
    return s.used;
}

int w4a8_mmq_fp8_moe_gemm(const void* x_f16, int64_t T, int64_t K, const int32_t* w_packed,
                          const void* scales_f16, const int32_t* w_zeros, int64_t E, int64_t N,
                          int64_t group_size, const int32_t* sorted_token_ids, int64_t P,
                          const int32_t* expert_ids, const int32_t* ntp, int64_t top_k,
                          int64_t block_m, int64_t kernel, int weight_is_e2m1, void* out_f16,
                          void* workspace, size_t workspace_bytes, void* stream) {
    clear_error();
    if (int rc = check_grouped(T, K, E, N, group_size, P, block_m, top_k, kernel, x_f16,
                               w_packed, scales_f16, sorted_token_ids, expert_ids, ntp))
        return rc;
    W4A8_REQUIRE(w_zeros == nullptr || N % 8 == 0, "w_zeros must be (E, N/8, K/group) int32");
    W4A8_REQUIRE(!(weight_is_e2m1 && w_zeros), "mxfp4 (E2M1) weights are symmetric; w_zeros must be empty");
    W4A8_REQUIRE(P == 0 || out_f16, "null output");
    GroupedArgs a{};
    a.x = x_f16; a.x_rows = T; a.K = K; a.w = w_packed;
    a.scales = static_cast<const uint16_t*>(scales_f16); a.zeros = w_zeros;
    a.E = E; a.N = N; a.group_size = group_size;
    a.sorted_ids = sorted_token_ids; a.P = P; a.expert_ids = expert_ids; a.ntp = ntp;
    a.top_k = top_k; a.identity_gather = false; a.num_valid = T * top_k; a.block_m = block_m;
    a.e2m1 = weight_is_e2m1 != 0; a.epi = Epi::kHalf; a.out = out_f16; a.out_top_k = top_k;
    return run_grouped(a, kernel, workspace, workspace_bytes, as_stream(stream));
}

int w4a8_mmq_fp8_moe_gemm1_silu(const void* x_f16, int64_t T, int64_t K, const int32_t* w_packed,
                                const void* scales_f16, const int32_t* w_zeros, int64_t E,
                                int64_t N, int64_t group_size, const int32_t* sorted_token_ids,
                                int64_t P, const int32_t* expert_ids, const int32_t* ntp,
                                int64_t top_k, int64_t block_m, int64_t kernel,
                                int weight_is_e2m1, void* out_f16, void* workspace,
                                size_t workspace_bytes, void* stream) {
    clear_error();
    W4A8_REQUIRE(kernel == W4A8_MOE_KERNEL_WMMA,
                 "fused gemm1+silu needs the 'wmma' kernel");
    if (int rc = check_grouped(T, K, E, N, group_size, P, block_m, top_k, kernel, x_f16,
                               w_packed, scales_f16, sorted_token_ids, expert_ids, ntp))
        return rc;
    W4A8_REQUIRE(N % 2 == 0, "w13 N must be 2*inter (even)");
    W4A8_REQUIRE(w_zeros == nullptr || N % 8 == 0, "w_zeros must be (E, (2*inter)/8, K/group) int32");
    W4A8_REQUIRE(!(weight_is_e2m1 && w_zeros), "mxfp4 (E2M1) weights are symmetric; w_zeros must be empty");
    W4A8_REQUIRE(P == 0 || out_f16, "null output");
    GroupedArgs a{};
    a.x = x_f16; a.x_rows = T; a.K = K; a.w = w_packed;
    a.scales = static_cast<const uint16_t*>(scales_f16); a.zeros = w_zeros;
    a.E = E; a.N = N; a.group_size = group_size;
    a.sorted_ids = sorted_token_ids; a.P = P; a.expert_ids = expert_ids; a.ntp = ntp;
    a.top_k = top_k; a.identity_gather = false; a.num_valid = T * top_k; a.block_m = block_m;
    a.e2m1 = weight_is_e2m1 != 0; a.epi = Epi::kSiluHalf; a.out = out_f16; a.out_top_k = top_k;
    return run_grouped(a, kernel, workspace, workspace_bytes, as_stream(stream));
}

int w4a8_mmq_fp8_moe_gemm_scatter(const void* x_f16, int64_t P_rows, int64_t K,
                                  const int32_t* w_packed, const void* scales_f16,
                                  const int32_t* w_zeros, int64_t E, int64_t N,
                                  int64_t group_size, const int32_t* sorted_token_ids, int64_t P,
                                  const int32_t* expert_ids, const int32_t* ntp,
                                  const float* topk_weights, float* output, int64_t M,
                                  int64_t top_k, int64_t block_m, int64_t kernel,
                                  int weight_is_e2m1, void* workspace, size_t workspace_bytes,
                                  void* stream) {
    clear_error();
    if (int rc = check_grouped(P_rows, K, E, N, group_size, P, block_m, top_k, kernel, x_f16,
                               w_packed, scales_f16, sorted_token_ids, expert_ids, ntp))
        return rc;
    W4A8_REQUIRE(P_rows >= P, "x must have one row per padded row (P, K)");
    W4A8_REQUIRE(M >= 0 && (M == 0 || (output && topk_weights)), "null output/topk_weights");
    W4A8_REQUIRE(w_zeros == nullptr || N % 8 == 0, "w_zeros must be (E, N/8, K/group) int32");
    W4A8_REQUIRE(!(weight_is_e2m1 && w_zeros), "mxfp4 (E2M1) weights are symmetric; w_zeros must be empty");
    GroupedArgs a{};
    a.x = x_f16; a.x_rows = P_rows; a.K = K; a.w = w_packed;
    a.scales = static_cast<const uint16_t*>(scales_f16); a.zeros = w_zeros;
    a.E = E; a.N = N; a.group_size = group_size;
    a.sorted_ids = sorted_token_ids; a.P = P; a.expert_ids = expert_ids; a.ntp = ntp;
    a.top_k = top_k; a.identity_gather = true; a.num_valid = M * top_k; a.block_m = block_m;
    a.e2m1 = weight_is_e2m1 != 0; a.epi = Epi::kScatter; a.out = output;
    a.topk_weights = topk_weights; a.out_top_k = top_k;
    return run_grouped(a, kernel, workspace, workspace_bytes, as_stream(stream));
}

size_t w4a8_gather_reduce_workspace_size(int64_t m_times_topk) {
    WorkspaceSize s;
    s.take<int32_t>((size_t)m_times_topk);
    return s.used;
}

int w4a8_mmq_fp8_moe_gather_reduce(const void* out2_f16, int64_t P, int64_t N,
                                   const int32_t* sorted_token_ids, const float* topk_weights,
                                   int64_t m_times_topk, const int32_t* ntp, int64_t top_k,
                                   float* out, void* workspace, size_t workspace_bytes,
                                   void* stream) {
    clear_error();
    W4A8_REQUIRE(P >= 0 && N >= 0 && top_k > 0 && m_times_topk >= 0, "gather_reduce: invalid sizes");
    W4A8_REQUIRE(m_times_topk % top_k == 0, "topk_weights.numel() must be M*top_k");
    W4A8_REQUIRE(P == 0 || (out2_f16 && sorted_token_ids && ntp), "gather_reduce: null pointer");
    W4A8_REQUIRE(m_times_topk == 0 || (topk_weights && out), "gather_reduce: null pointer");
    Workspace w(workspace, workspace_bytes);
    int32_t* slot_to_row = w.take<int32_t>((size_t)m_times_topk);
    if ((m_times_topk > 0 && workspace == nullptr) || !w.ok()) {
        set_error("gather_reduce: workspace too small");
        return W4A8_ERR_WORKSPACE;
    }
    return launch_gather_reduce(out2_f16, P, N, sorted_token_ids, topk_weights, m_times_topk,
                                ntp, top_k, out, slot_to_row, as_stream(stream));
}

int w4a8_silu_and_mul(const void* in_f16, int64_t rows, int64_t inter, void* out_f16,
                      void* stream) {
    clear_error();
    W4A8_REQUIRE(rows >= 0 && inter >= 0, "silu_and_mul: invalid sizes");
    W4A8_REQUIRE(rows * inter == 0 || (in_f16 && out_f16), "silu_and_mul: null pointer");
    return launch_silu_and_mul(in_f16, rows, inter, out_f16, as_stream(stream));
}

int w4a8_swigluoai_and_mul(const void* in_f16, int64_t rows, int64_t inter, float alpha,
                           float limit, void* out_f16, void* stream) {
    clear_error();
    W4A8_REQUIRE(rows >= 0 && inter >= 0, "swigluoai_and_mul: invalid sizes");
    W4A8_REQUIRE(rows * inter == 0 || (in_f16 && out_f16), "swigluoai_and_mul: null pointer");
    return launch_swigluoai_and_mul(in_f16, rows, inter, alpha, limit, out_f16, as_stream(stream));
}

int w4a8_mmq_fp8_gemm(const void* x_f16, int64_t M, int64_t K, const int32_t* w_packed,
                      const void* scales_f16, const int32_t* w_zeros, int64_t N,
                      int64_t group_size, int64_t kernel, int weight_is_e2m1, void* out_f16,
                      void* workspace, size_t workspace_bytes, void* stream) {
    clear_error();
    W4A8_REQUIRE(M >= 0 && K > 0 && N > 0 && K % 8 == 0, "dense: invalid sizes");
    W4A8_REQUIRE(group_size > 0 && K % group_size == 0, "K not divisible by scales' K dim");
    W4A8_REQUIRE(group_size % 16 == 0 && group_size <= kMaxGroupSize,
                 "group_size must be a multiple of 16 and <= 128");
    W4A8_REQUIRE(dense_kernel_valid(kernel), "dense kernel id invalid (DenseKernel 0..14, no 3)");
    W4A8_REQUIRE(!(weight_is_e2m1 && w_zeros), "mxfp4 (E2M1) weights are symmetric; w_zeros must be empty");
    W4A8_REQUIRE(w_zeros == nullptr || N % 8 == 0, "w_zeros shape mismatch");
    W4A8_REQUIRE(M == 0 || (x_f16 && w_packed && scales_f16 && out_f16), "dense: null pointer");
    GroupedArgs a{};
    a.x = x_f16; a.x_rows = M; a.K = K; a.w = w_packed;
    a.scales = static_cast<const uint16_t*>(scales_f16); a.zeros = w_zeros;
    a.E = 1; a.N = N; a.group_size = group_size;
    a.sorted_ids = nullptr; a.P = M; a.expert_ids = nullptr; a.ntp = nullptr;
    a.top_k = 1; a.identity_gather = false; a.num_valid = M;
    a.e2m1 = weight_is_e2m1 != 0; a.epi = Epi::kHalf; a.out = out_f16; a.out_top_k = 1;
    // DenseKernel 0 = reference_scalar, 11 = decode_gemv, everything else = matrix cores.
    int64_t mk = W4A8_MOE_KERNEL_WMMA;
    a.block_m = 64;
    if (kernel == 0) { mk = W4A8_MOE_KERNEL_SCALAR; a.block_m = 1; }
    if (kernel == 11) { mk = W4A8_MOE_KERNEL_GEMV; a.block_m = 16; }
    // a few rows: the dense GEMV (rows quantised in the kernel, no act-quant launch)
    if (kernel == 11 && dense_gemv_supported(M, N, K, group_size, weight_is_e2m1 != 0))
        return launch_dense_gemv(x_f16, M, K, w_packed, scales_f16, w_zeros, N, out_f16,
                                 as_stream(stream));
    return run_grouped(a, mk, workspace, workspace_bytes, as_stream(stream));
}

int w4a8_moe_apply_set_stage_events(void* const* events, int count) {
    clear_error();
    if (count == 0) {
        g_stage_on = false;
        next_kernel_stamp() = KernelStamp{};
        return W4A8_OK;
    }
    W4A8_REQUIRE((count == kStageEvents || count == kStageEvents + kStampEvents) && events != nullptr,
                 "stage events: need 8 events (or 12 with the GEMM kernel stamps)");
    for (int i = 0; i < count; ++i) {
        W4A8_REQUIRE(events[i] != nullptr, "stage events: null event");
        g_stage_events[i] = reinterpret_cast<hipEvent_t>(events[i]);
    }
    g_stage_stamps = count == kStageEvents + kStampEvents;
    g_stage_on = true;
    return W4A8_OK;
}

size_t w4a8_moe_apply_workspace_size(int64_t T, int64_t H, int64_t inter, int64_t E,
                                     int64_t top_k) {
    const ApplyPlan pl = plan_apply(T, E, top_k);
    SizeProbe sp;
    int32_t *a, *b, *c; void* d; size_t db; uint8_t* e; float* f; __half* g; uint8_t* h;
    float *i, *j, *k, *l; __half* m; int32_t* n; uint64_t* o; DecHandover* q;
    carve_apply(sp, pl, T, H, inter, E, top_k, &a, &b, &c, &d, &db, &e, &f, &g, &h, &i, &j, &k,
                &l, &m, &n, &o, &q);
    return sp.s.used;
}

int w4a8_moe_apply(const void* x, int x_dtype, int64_t T, int64_t H, int64_t inter, int64_t E,
                   int64_t top_k, int64_t group_size, const int32_t* w13,
                   const void* w13_scales_f16, const int32_t* w13_zeros, const int32_t* w2,
                   const void* w2_scales_f16, const int32_t* w2_zeros,
                   const float* topk_weights, const int32_t* topk_ids,
                   const int32_t* expert_map, int64_t num_global_experts, int weight_is_e2m1,
                   void* out, void* workspace, size_t workspace_bytes, void* stream) {
    clear_error();
    return moe_apply_impl(x, x_dtype, T, H, inter, E, top_k, group_size, w13, w13_scales_f16,
                          w13_zeros, w2, w2_scales_f16, w2_zeros, topk_weights, topk_ids,
                          expert_map, num_global_experts, weight_is_e2m1, out, workspace,
                          workspace_bytes, stream, false);
}

int w4a8_moe_apply_fragments(const void* x, int x_dtype, int64_t T, int64_t H, int64_t inter,
                             int64_t E, int64_t top_k, int64_t group_size, const int32_t* w13_frag,
                             const void* w13_scales_f16, const int32_t* w13_zeros,
                             const int32_t* w2_frag, const void* w2_scales_f16,
                             const int32_t* w2_zeros, const float* topk_weights,
                             const int32_t* topk_ids, const int32_t* expert_map,
                             int64_t num_global_experts, void* out, void* workspace,
                             size_t workspace_bytes, void* stream) {
    clear_error();
    return moe_apply_impl(x, x_dtype, T, H, inter, E, top_k, group_size, w13_frag,
                          w13_scales_f16, w13_zeros, w2_frag, w2_scales_f16, w2_zeros,
                          topk_weights, topk_ids, expert_map, num_global_experts, 0, out,
                          workspace, workspace_bytes, stream, true);
}

int w4a8_moe_forward(const void* x, int x_dtype, int64_t T, int64_t H, int64_t inter, int64_t E,
                     int64_t top_k, int64_t group_size, const float* router_logits,
                     int renormalize, const int32_t* w13, const void* w13_scales_f16,
                     const int32_t* w13_zeros, const int32_t* w2, const void* w2_scales_f16,
                     const int32_t* w2_zeros, int weights_layout, const int32_t* expert_map,
                     int64_t num_global_experts, float* topk_weights, int32_t* topk_ids,
                     void* out, void* workspace, size_t workspace_bytes, void* stream) {
    clear_error();
    W4A8_REQUIRE(weights_layout == W4A8_WEIGHTS_OP || weights_layout == W4A8_WEIGHTS_FRAGMENTS,
                 "moe_forward: weights_layout must be W4A8_WEIGHTS_OP or W4A8_WEIGHTS_FRAGMENTS");
    W4A8_REQUIRE(T == 0 || (router_logits && topk_weights && topk_ids), "moe_forward: null pointer");
    return moe_apply_impl(x, x_dtype, T, H, inter, E, top_k, group_size, w13, w13_scales_f16,
                          w13_zeros, w2, w2_scales_f16, w2_zeros, topk_weights, topk_ids,
                          expert_map, num_global_experts, 0, out, workspace, workspace_bytes,
                          stream, weights_layout == W4A8_WEIGHTS_FRAGMENTS, router_logits,
                          renormalize != 0);
}

int w4a8_moe_forward_noalloc(const void* x, int x_dtype, int64_t T, int64_t H, int64_t inter,
                             int64_t E, int64_t top_k, int64_t group_size,
                             const float* router_logits, int renormalize, const int32_t* w13,
                             const void* w13_scales_f16, const int32_t* w13_zeros,
                             const int32_t* w2, const void* w2_scales_f16, const int32_t* w2_zeros,
                             int weights_layout, const int32_t* expert_map,
                             int64_t num_global_experts, float* topk_weights, int32_t* topk_ids,
                             void* out, void* stream) {
    clear_error();
    W4A8_REQUIRE(T >= 0 && H > 0 && inter > 0 && E > 0 && top_k > 0,
                 "moe_forward_noalloc: invalid sizes");
    const size_t need = w4a8_moe_apply_workspace_size(T, H, inter, E, top_k);
    if (need > w4a8::kNoAllocScratchBytes) {
        w4a8::set_error("moe_forward_noalloc: this shape needs " + std::to_string(need) +
                        " bytes of scratch; the library's static scratch holds " +
                        std::to_string(w4a8::kNoAllocScratchBytes) +
                        " (W4A8_NOALLOC_SCRATCH_BYTES): call w4a8_moe_forward with a workspace");
        return W4A8_ERR_WORKSPACE;
    }
    void* ws = nullptr;
    const int rc = w4a8::noalloc_scratch(&ws);
    if (rc != W4A8_OK) return rc;
    return w4a8_moe_forward(x, x_dtype, T, H, inter, E, top_k, group_size, router_logits,
                            renormalize, w13, w13_scales_f16, w13_zeros, w2, w2_scales_f16,
                            w2_zeros, weights_layout, expert_map, num_global_experts,
                            topk_weights, topk_ids, out, ws, w4a8::kNoAllocScratchBytes, stream);
}

int w4a8_set_decode_fused(int on) {
    clear_error();
    const int prev = decode_fused_enabled() ? 1 : 0;
    g_decode_fused.store(on != 0 ? 1 : 0, std::memory_order_relaxed);
    return prev;
}

int w4a8_set_prefill_pair(int on) {
    clear_error();
    const int prev = prefill_pair_enabled() ? 1 : 0;
    g_prefill_pair.store(on != 0 ? 1 : 0, std::memory_order_relaxed);
    return prev;
}

int w4a8_decode_fused_test_fault(int on) {
    clear_error();
    return decode_fused_set_fault(on);
}

int w4a8_moe_fragments_supported(int64_t H, int64_t inter, int64_t group_size) {
    return fragments_schedule_ok(true, H, inter, group_size) &&
           fragments_schedule_ok(false, H, inter, group_size);
}

int64_t w4a8_fragments_words(int64_t E, int64_t N, int64_t K) {
    if (E < 0 || N < 0 || K < 0 || N % 16 != 0 || K % 128 != 0) return -1;
    return fragments_words(E, N, K);
}

int w4a8_repack_int4_fragments(const int32_t* w_packed, const void* scales_f16,
                               const int32_t* w_zeros, int64_t E, int64_t N, int64_t K,
                               int32_t* out, void* stream) {
    clear_error();
    W4A8_REQUIRE(E >= 0 && N >= 0 && K >= 0, "repack: invalid sizes");
    W4A8_REQUIRE(N % 16 == 0 && K % 128 == 0, "repack: needs N % 16 == 0 and K % 128 == 0");
    W4A8_REQUIRE(E * N * K == 0 || (w_packed && scales_f16 && out), "repack: null pointer");
    W4A8_REQUIRE(w_packed != out, "repack: out must not alias w_packed");
    return launch_repack_fragments(w_packed, scales_f16, w_zeros, E, N, K, out, as_stream(stream));
}

}  // extern "C"
