// Decode expert GEMVs of the whole MoE layer (T <= 96) on fragment-layout weights, without
// an align launch and without act-quant launches (gfx950).
//
// Replaces, for the whole-layer decode schedule, the reference's chain of align
// (moe_experts.py:587-589), per-token act-quant (moe_kernel.hip:87-127) and decode GEMV
// (moe_kernel.hip:884-1062) for each of the two GEMMs. Arithmetic as in w4a8_common.h and
// bit-identical to the grouped GEMV of grouped_gemm.hip (same raw-nibble MFMA operands,
// zero-point term, scale fold order and split-K sum order). The schedule is this file's own:
//
//   * one four-wave work-group per CU (one wave per SIMD, so a wave holds four weight chunks
//     in registers); every work-group of gemm1 builds, in LDS, the list of touched experts
//     and each one's slots from topk_ids (the order of slots inside an expert does not
//     matter: every output row depends on its own activation row only), and work-group 0
//     writes the lists to the workspace, where gemm2's work-groups read them;
//   * the layer's work is a list of units (touched expert, column unit: 16 gate + 16 up
//     columns for gemm1+SiLU, 32 columns for gemm2), streamed once per 16-row pass over the
//     expert's slots; it is split over teams (a team is one wave, or the whole work-group
//     when the K groups are split over its 4 waves) in contiguous ranges of equal work, a
//     pass start (row load, and quantisation where the rows are not quantised already)
//     counting a GEMM's pass cost in units;
//   * a team walks its range expert by expert and pass by pass; at a pass start it loads the
//     activation rows (gemm1: x rows of the slots' tokens, fp16 or bf16; gemm2: the slots'
//     h rows) and quantises them in registers, bit-identical to act_quant_kernel; the weight
//     loads run three or four chunks ahead of the MFMAs across expert and pass boundaries,
//     each fragment's weight blocks and its row's scale / zero-point words (adjacent in the
//     16-row tile, repack.hip) loaded side by side;
//   * outputs are per slot: gemm1 writes h (numel, I) fp16 after SiLU*mul, gemm2 writes
//     y (numel, H) fp32, which the slot reduce sums in j order.
#include <algorithm>
#include <type_traits>

#include "grouped_params.h"
#include "router.h"

namespace w4a8 {
namespace {

constexpr int kDecThreads = 256;
constexpr int kDecMaxSlots = 1024;      // T * top_k
constexpr int kDecMaxExperts = 1024;
constexpr int kDecRing = 3;             // weight chunks in flight per wave (a ring slot each)
// partition cost of a pass start, in units: gemm1 loads quantised rows (or one row of x per
// token), gemm2 loads and quantises its h rows (measured best at c3: 1 and 3)
constexpr int kDecPassCost1 = 1;
constexpr int kDecPassCost2 = 3;
constexpr uint32_t kDecOnes = 0x38383838u;   // four e4m3 bytes of 1.0
using u16x2 = unsigned short __attribute__((ext_vector_type(2)));

struct DecodeParams {
    const int32_t* ids;      // (numel) routed expert ids (unused with logits)
    // router in the kernel (gemm1 only): every work-group routes the T tokens itself and
    // work-group 0 writes the weights and ids; null: ids come from an earlier launch
    const float* logits;     // (T, n_router) fp32
    int n_router, renorm;
    float* tw_out;           // (numel) fp32
    int32_t* ids_out;        // (numel)
    const int32_t* emap;     // global -> local expert map or null
    int emap_len, numel, top_k, E;
    const void* a;           // activation rows, fp16 / bf16
    int a_bf16;
    int a_per_token;         // 1: slot s reads row s / top_k (x); 0: row s (h)
    // gemm1 only: the rows already quantised (k8-interleaved e4m3 (rows, K) and their scales,
    // act_quant_kernel's bytes, written by the router launch); null: quantise a in registers
    const uint8_t* aq;
    const float* asc;
    // list hand-over between the two launches: gemm1 writes its lists (hand_out), gemm2 reads
    // them (hand_in) instead of loading the ids and building them again
    DecHandover* hand_out;
    const DecHandover* hand_in;
    const int32_t* w;        // fragment layout (E, N/16, 272 G): blocks, then scales/zeros
    void* out;               // kSiluHalf: (numel, N/2) fp16; kSlotF32: (numel, N) fp32
    int K, N, G;
};

static_assert(kDecMaxExperts == kDecHandExperts && kDecMaxSlots == kDecHandSlots,
              "the hand-over holds the lists whole");

struct DecodeLists {
    int n_touched;
    int16_t expert[kDecMaxExperts];        // touched expert r (ascending id)
    int16_t first[kDecMaxExperts + 1];     // its slots are slot[first[r] .. first[r + 1])
    int16_t slot[kDecMaxSlots];
    int cnt[kDecMaxExperts];
    int pp[kDecMaxExperts + 1];            // 16-row passes of the touched experts before r
    int wtot[3][kDecThreads / 64];
};

// Partition cost of the work before touched expert r for a GEMM with upe column units per
// expert: every 16-row pass streams the upe units once and starts with a row load charged
// as pc units.
__device__ __forceinline__ int dec_cost(const DecodeLists& L, int r, int upe, int pc) {
    return L.pp[r] * (upe + pc);
}

// Touched experts and their slot lists (the align's grouping, without padding) in LDS, and
// the number of 16-row passes before each touched expert (the partition cost, dec_cost).
__device__ void build_lists(const DecodeParams& p, const int32_t* ids, DecodeLists& L) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    constexpr int kPer = kDecMaxSlots / kDecThreads;
    for (int e = tid; e < p.E; e += kDecThreads) L.cnt[e] = 0;
    int es[kPer];
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
        const int s = tid + kDecThreads * i;
        int e = s < p.numel ? ids[s] : -1;
        if (p.emap != nullptr) e = (e >= 0 && e < p.emap_len) ? p.emap[e] : -1;
        es[i] = (e >= 0 && e < p.E) ? e : -1;
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kPer; ++i)
        if (es[i] >= 0) atomicAdd(&L.cnt[es[i]], 1);
    __syncthreads();
    // exclusive scans of (slots, touched, passes) over experts; thread t owns experts 4t .. 4t + 3
    int c[4], tot = 0, tch = 0, twk = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int e = 4 * tid + j;
        c[j] = e < p.E ? L.cnt[e] : 0;
        tot += c[j];
        tch += c[j] > 0 ? 1 : 0;
        twk += (c[j] + 15) >> 4;
    }
    int it = tot, ic = tch, iw = twk;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_up(it, o, 64), z = __shfl_up(ic, o, 64), v = __shfl_up(iw, o, 64);
        if (lane >= o) {
            it += y;
            ic += z;
            iw += v;
        }
    }
    if (lane == 63) {
        L.wtot[0][wave] = it;
        L.wtot[1][wave] = ic;
        L.wtot[2][wave] = iw;
    }
    __syncthreads();
    int off = it - tot, r = ic - tch, wk = iw - twk;
    for (int w = 0; w < wave; ++w) {
        off += L.wtot[0][w];
        r += L.wtot[1][w];
        wk += L.wtot[2][w];
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int e = 4 * tid + j;
        if (c[j] > 0) {
            L.expert[r] = (int16_t)e;
            L.first[r] = (int16_t)off;
            L.pp[r] = wk;
            wk += (c[j] + 15) >> 4;
            ++r;
        }
        if (e < p.E) L.cnt[e] = off;     // becomes the fill cursor of expert e
        off += c[j];
    }
    if (tid == kDecThreads - 1) {
        L.n_touched = r;
        L.first[r] = (int16_t)off;
        L.pp[r] = wk;
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kPer; ++i)
        if (es[i] >= 0) L.slot[atomicAdd(&L.cnt[es[i]], 1)] = (int16_t)(tid + kDecThreads * i);
    __syncthreads();
}

// In-kernel router (DecodeParams::logits): every work-group selects the top-k of all T
// tokens itself (wave w takes tokens w, w + 4, ..., eight logit rows in flight at a time),
// with the router kernel's selection (router.h), so the ids are the same bits; work-group 0
// also writes the weights and ids out. No other work-group's result is read, so there is
// no synchronisation between work-groups. One selection takes a wave ~2 us, so this pays
// only while each wave routes one token: T <= 4 (c2, T = 1: 32.4 -> 30.7 us per layer; at
// T = 32, eight tokens a wave, gemm1 grew by 17 us against the 4.7 us router launch it
// replaced). n_router <= 256.
constexpr int kDecRouteMaxT = 4;
constexpr int kDecRouteMaxE = 256;
__device__ void dec_route(const DecodeParams& p, int32_t* s_ids) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int T = p.numel / p.top_k;
    const bool writer = blockIdx.x == 0;
    constexpr int kRows = 8;
    for (int t0 = wave; t0 < T; t0 += 4 * kRows) {
        float v[kRows][4];
#pragma unroll
        for (int i = 0; i < kRows; ++i) {
            const int t = min(t0 + 4 * i, T - 1);
            topk_load<4>(p.logits + (int64_t)t * p.n_router, p.n_router, lane, v[i]);
        }
#pragma unroll
        for (int i = 0; i < kRows; ++i) {
            const int t = t0 + 4 * i;
            if (t < T)
                topk_select<4>(v[i], p.n_router, p.top_k, p.renorm != 0,
                               writer ? p.tw_out + (int64_t)t * p.top_k : nullptr,
                               writer ? p.ids_out + (int64_t)t * p.top_k : nullptr,
                               s_ids + t * p.top_k, lane);
        }
    }
    __syncthreads();
}

// First unit whose work start is at or past X: the work start of unit u of touched expert r
// is cost[r] + np (pc + u - r upe), np = its passes. Wave-wide 64-ary search.
__device__ int unit_at_cost(const DecodeLists& L, int n_t, int upe, int pc, int X) {
    const int lane = threadIdx.x & 63;
    const int step = (n_t + 64) / 64;       // candidates cost[0], cost[step], ... cover [0, n_t]
    int cand = lane * step;
    uint64_t m = __ballot(cand <= n_t && dec_cost(L, cand, upe, pc) <= X);   // bit 0: cost 0 <= X
    const int base = (63 - __clzll(m)) * step;
    cand = base + lane;
    m = __ballot(lane < step && cand <= n_t && dec_cost(L, cand, upe, pc) <= X);
    const int r = base + 63 - __clzll(m);    // largest r with cost[r] <= X
    if (r >= n_t) return n_t * upe;
    const int np = ((int)L.first[r + 1] - (int)L.first[r] + 15) >> 4;
    const int d = X - dec_cost(L, r, upe, pc) - np * pc;
    const int k = d <= 0 ? 0 : (d + np - 1) / np;
    return r * upe + min(k, upe);
}

// gemm1's side of the hand-over: work-group 0 writes the lists before its own work.
__device__ void dec_hand_lists(const DecodeParams& p, const DecodeLists& L) {
    if (blockIdx.x != 0) return;
    DecHandover* h = p.hand_out;
    const int n_t = L.n_touched;
    for (int i = threadIdx.x; i <= n_t; i += kDecThreads) {
        h->expert[i] = i < n_t ? L.expert[i] : (int16_t)0;
        h->first[i] = L.first[i];
        h->pp[i] = L.pp[i];
    }
    for (int i = threadIdx.x; i < p.numel; i += kDecThreads) h->slot[i] = L.slot[i];
    if (threadIdx.x == 0) h->n_touched = n_t;
}

// gemm2's side: the lists into LDS (one round of loads)
__device__ void dec_hand_read(const DecodeParams& p, DecodeLists& L) {
    const DecHandover* h = p.hand_in;
    const int nmax = min(p.E, p.numel);      // touched experts <= min(E, slots) <= 1024
    for (int i = threadIdx.x; i <= nmax; i += kDecThreads) {
        if (i < nmax) L.expert[i] = h->expert[i];
        L.first[i] = h->first[i];
        L.pp[i] = h->pp[i];
    }
    for (int i = threadIdx.x; i < p.numel; i += kDecThreads) L.slot[i] = h->slot[i];
    if (threadIdx.x == kDecThreads - 1) L.n_touched = h->n_touched;
    __syncthreads();
}

template <Epi EPI, int GPW, int KSPLIT>
struct DecCfg {
    static constexpr bool kSilu = EPI == Epi::kSiluHalf;
    static constexpr int NF = kSilu ? 2 : 1;      // fragments per column tile (gate, up)
    static constexpr int CT = kSilu ? 1 : 2;      // column tiles per unit
    static constexpr int FR = NF * CT;            // fragments per unit and group
    // groups per chunk: eight groups a wave (K = 4096) take 2-group chunks, so the ring of
    // four chunks holds one unit and its registers leave room for the 128 of fp16 rows a
    // pass start holds (4-group chunks spilled ring slots, each spill waiting for its load)
    static constexpr int GC = GPW < 4 ? GPW : (GPW == 8 ? 2 : 4);
    static constexpr int NB = GPW / GC;           // chunks per unit
    static constexpr int TEAMS = 4 / KSPLIT;      // teams per work-group
    static constexpr int PC = kSilu ? kDecPassCost1 : kDecPassCost2;   // pass-start cost
    static_assert(KSPLIT == 1 || KSPLIT == 4, "a team is one wave or the whole work-group");
    static_assert(GPW % GC == 0 && (NB == 1 || NB == 2 || NB == 4), "unsupported groups per wave");
    // ring slots: a multiple of NB, so a slot's group batch is fixed
    static constexpr int D = NB == 1 ? kDecRing : 4;
    static_assert(D % NB == 0 && D >= 3 && D <= 4, "ring of three or four slots");
    // split-K partials of a batch of up to D units (one per ring slot), double-buffered:
    // [batch parity][slot][wave][FR][lane]
    static constexpr int LDS_BYTES = KSPLIT > 1 ? 2 * D * KSPLIT * FR * 64 * 16 : 0;
};

// GC metadata words of one row (groups g .. g + GC - 1, adjacent in the tile): one 16-byte
// load for 4 groups and one 8-byte load for 2 (their offsets are multiples of that size:
// G % 4 == 0 and g % 4 == 0 where GC == 4, g even where GC == 2), single words otherwise
template <int GC>
__device__ __forceinline__ void dec_load_meta(const int32_t* ptr, uint32_t (&m)[GC]) {
    if constexpr (GC == 4) {
        const uint4 v = *reinterpret_cast<const uint4*>(ptr);
        m[0] = v.x; m[1] = v.y; m[2] = v.z; m[3] = v.w;
    } else if constexpr (GC == 2) {
        const uint2 v = *reinterpret_cast<const uint2*>(ptr);
        m[0] = v.x; m[1] = v.y;
    } else {
#pragma unroll
        for (int u = 0; u < GC; ++u) m[u] = (uint32_t)ptr[u];
    }
}

// fp16 / bf16 bits -> f32; bf16 goes through fp16 first, the cast the reference applies
// before quantising (moe_experts.py:596-597). The dtype is a template parameter: a run-time
// flag compiles into one branch per element of the unrolled row code.
template <bool BF16>
__device__ __forceinline__ float dec_act_f32(uint32_t bits) {
    if constexpr (BF16) return __half2float(__float2half(__uint_as_float(bits << 16)));
    return __half2float(__ushort_as_half(static_cast<unsigned short>(bits)));
}

// Position in a team's work: touched expert r, pass rows [m0, m0 + 16), unit u, chunk b.
struct DecCursor {
    int r, e, m0, u, b;
};

// In-kernel dependency of the fused layer's second GEMM on its first (decode_layer_kernel),
// on the agent-scope operations of the memory model only. Work-group w of the first GEMM
// stores `nonce` to flags[w] with release semantics at agent scope (its L2 written back)
// once every h row it writes is stored. A team of the second GEMM reads its rows only after
// every work-group that wrote a unit of the touched experts in its range has published, and
// reads flags and rows with agent-coherent loads (sc1, the loads of agent-scope atomics),
// which do not return lines another XCD's L2 may hold stale. The first GEMM's partition is
// a pure function of the lists, so its writers of an expert are computed, not recorded.
struct DecDep {
    const uint64_t* flags;    // one per work-group of the first GEMM
    uint64_t nonce;           // this call's value (never 0; the slot reduce resets flags to 0)
    int upe1;                 // column units per expert of the first GEMM
    int teams1;               // teams per work-group of the first GEMM
    // one word per work-group: cleared by the work-group at its start, set to nonce when one
    // of its waits gave up (bounded spin; not expected); the slot reduce reads them all
    uint64_t* timeout;
    uint64_t expect;          // the flag value a wait waits for (nonce; see g_dec_fault)
    int spin_limit;           // polls before a wait gives up
};
constexpr int kDecSpinLimit = 1 << 20;   // polls before a wait gives up (~1 s)
constexpr int kDecFaultSpinLimit = 64;

// Test hook (w4a8_decode_fused_test_fault): while non-zero, the fused layer's waits wait for a
// flag value no work-group publishes, with a short spin limit, so they give up and every
// kernel still ends normally. Read from device memory at each launch, so a captured graph
// sees changes between replays.
__device__ uint32_t g_dec_fault = 0;

// Last team of a GEMM partition (n teams over W cost units, team t starting at
// floor(W t / n)) whose start is at or before cost S: the team that runs the unit starting at S.
__device__ __forceinline__ int dec_owner(int S, int W, int n) {
    const int t = (int)((((int64_t)S + 1) * n - 1) / W);
    return min(t, n - 1);
}

// 8 bytes of a completion flag, agent-coherent
__device__ __forceinline__ uint64_t dec_flag(const uint64_t* flags, int w) {
    return __hip_atomic_load(flags + w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// 16 bytes of activation row: plain, or (DEP) agent-coherent (buffer load with sc1) for rows
// written earlier in the same kernel by other work-groups
template <bool DEP>
__device__ __forceinline__ uint4 dec_row16(const uint16_t* base, int64_t elem) {
    if constexpr (DEP) {
        using u32x4 = unsigned __attribute__((ext_vector_type(4)));
        const auto rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(base), (short)0,
                                                            0x7FFFFFFF, 0x00020000);
        const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rsrc, (int)(elem * 2), 0, kCpolSc1);
        return make_uint4(v.x, v.y, v.z, v.w);
    } else {
        return *reinterpret_cast<const uint4*>(base + elem);
    }
}

// L2 warm-up of the activation rows (one 128-byte line per lane; work-group b runs on XCD
// b % 8): they are cold (h was just written on other XCDs) and the row loads of a pass start
// are on the critical path. The value is only kept alive (dec_keep), never used.
__device__ __forceinline__ uint32_t dec_warm(const DecodeParams& p) {
    const int nrows = p.a_per_token ? p.numel / p.top_k : p.numel;
    const int lines = (int)(((int64_t)nrows * p.K * (p.aq ? 1 : 2) + 127) / 128);
    const int idx = ((int)(blockIdx.x / 8) * 4 + (int)(threadIdx.x >> 6)) * 64 + (int)(threadIdx.x & 63);
    const uint32_t* rows = p.aq ? reinterpret_cast<const uint32_t*>(p.aq) : reinterpret_cast<const uint32_t*>(p.a);
    return lines > 0 ? rows[(int64_t)min(idx, lines - 1) * 32] : 0u;
}
// keeps the warm-up load (its value never matches: a NaN pattern in a block that does not exist)
__device__ __forceinline__ void dec_keep(uint32_t warm, void* out) {
    if (warm == 0x7FC00001u && blockIdx.x == 0x7FFFFFFFu) reinterpret_cast<uint32_t*>(out)[0] = warm;
}

// One GEMM of the layer over the lists L by the whole grid (the body of decode_gemv_kernel).
// DEP: the activation rows are h written by the first GEMM of the same kernel (DecDep).
// PREQ: the rows come quantised (p.aq, p.asc); a pass start loads their e4m3 bytes straight
// into the MFMA operand registers.
template <Epi EPI, int GPW, int KSPLIT, bool ABF16, bool DEP, bool PREQ = false>
__device__ __forceinline__ void dec_run(const DecodeParams& p, const DecodeLists& L,
                                        float (&s_amax)[4][16], v4f* s_part, const DecDep& dep) {
    using C = DecCfg<EPI, GPW, KSPLIT>;
    const int ncols = C::kSilu ? p.N / 2 : p.N;
    const int upe = ncols / (16 * C::CT);                 // units per expert

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int q = lane >> 4;
    const int c16 = lane & 15;
    const int team = wave / KSPLIT;
    const int g0 = (wave % KSPLIT) * GPW;
    const int n_t = L.n_touched;
    const int nteams = (int)gridDim.x * C::TEAMS;
    const int tm = (int)blockIdx.x * C::TEAMS + team;
    // team tm starts at work floor(W tm / nteams), in 32-bit arithmetic (W < 2^25)
    const int work = dec_cost(L, n_t, upe, C::PC);
    const int wq = work / nteams, wr = work % nteams;
    auto work_at = [&](int t) { return wq * t + wr * t / nteams; };
    const int ua = __builtin_amdgcn_readfirstlane(unit_at_cost(L, n_t, upe, C::PC, work_at(tm)));
    const int ub = __builtin_amdgcn_readfirstlane(unit_at_cost(L, n_t, upe, C::PC, work_at(tm + 1)));
    if (ua >= ub) return;      // team-uniform; a K-split team is the whole work-group

    // the team's work in order: touched experts r, 16-row passes over each expert's slots,
    // the units of the team's range inside the expert, NB chunks per unit
    auto seg_lo = [&](int r) __attribute__((always_inline)) { return max(ua, r * upe); };
    auto seg_hi = [&](int r) __attribute__((always_inline)) { return min(ub, (r + 1) * upe); };
    // true: c entered a new pass
    auto advance = [&](DecCursor& c) __attribute__((always_inline)) -> bool {
        if (c.u >= ub) return false;
        if (++c.b < C::NB) return false;
        c.b = 0;
        if (++c.u < seg_hi(c.r)) return false;
        c.m0 += 16;
        if (c.m0 >= (int)L.first[c.r + 1] - (int)L.first[c.r]) {
            ++c.r;
            c.m0 = 0;
            c.e = c.r < n_t ? (int)L.expert[c.r] : 0;
        }
        c.u = seg_lo(c.r);
        return true;
    };

    uint4 wv[C::D][C::GC * C::FR];
    uint32_t mw[C::D][C::FR][C::GC];   // metadata words: fp16 scale | zero-point << 16
    uint4 raw[PREQ ? 1 : GPW][4];
    float rasc = 0.f;   // PREQ: the scale of this lane's row c16
    v8i af[GPW];
    v4f sa[GPW];   // 2^-9 * group sums of rows 4q .. 4q + 3 (zero-point term)
    v4f run[C::FR];
    // output rows of the pass for this lane: rows 4q .. 4q + 3 (one wave per row of the
    // four with a K split); pad rows store to the last real row's slot the value computed
    // for it (their activations repeat that row, so the value is the same)
    constexpr int NRO = KSPLIT > 1 ? 1 : 4;
    int osl[NRO];
    float oasc[NRO];

    // weight row of fragment f, column cc of unit column ucol
    auto row_of = [&](int ucol, int f, int cc) __attribute__((always_inline)) -> int {
        const int col = (ucol * C::CT + f % C::CT) * 16 + cc;
        return (C::kSilu && f >= C::CT) ? col + ncols : col;
    };
    // chunk at cursor c: groups g0 + b GC .. + GC - 1 of the unit's FR fragments; past the
    // team's end it reloads expert 0's first bytes (unconditional issues keep the compiler's
    // wait counts exact)
    auto issue = [&](const DecCursor& c, auto slot) __attribute__((always_inline)) {
        constexpr int b = decltype(slot)::value;
        const bool live = c.u < ub;
        const int g = g0 + (live ? c.b * C::GC : 0);
        const int ucol = live ? c.u - c.r * upe : 0;
        const int64_t e = live ? c.e : 0;
        const int tw = frag_tile_words(p.G);
        const int32_t* we = p.w + e * (int64_t)(p.N / 16) * tw;
#pragma unroll
        for (int f = 0; f < C::FR; ++f) {
            const int n = row_of(ucol, f, c16);
            // the 16-row tile of row n: its weight blocks, then its rows' scales and
            // zero-points (the lane's row, groups g .. g + GC - 1 adjacent)
            const int32_t* wt = we + (int64_t)(n >> 4) * tw;
            const int32_t* wr = wt + g * 256 + lane * 4;
#pragma unroll
            for (int uu = 0; uu < C::GC; ++uu) wv[b][uu * C::FR + f] = load_stream16(wr + uu * 256);
            dec_load_meta<C::GC>(wt + frag_meta_word(p.G, n & 15, g), mw[b][f]);
        }
    };

    // activation rows of pass c (pad rows repeat the last real row): lane (q, c16) holds k
    // in [128 g + 32 q, +32) of row c16
    auto load_rows = [&](const DecCursor& c) __attribute__((always_inline)) {
        const int s0 = (int)L.first[c.r] + c.m0;
        const int mreal = min(16, (int)L.first[c.r + 1] - s0);
        const int my_slot = L.slot[s0 + min(c16, mreal - 1)];
        const int arow = p.a_per_token ? my_slot / p.top_k : my_slot;
        const int64_t xr = (int64_t)arow * p.K + q * 32;
        if constexpr (PREQ) {
            // the 32 bytes of k in [128 g + 32 q, +32): the operand register order (k8
            // interleave inside each 8-byte block, as the in-register quantisation packs it)
#pragma unroll
            for (int g = 0; g < GPW; ++g) {
                const uint4* src = reinterpret_cast<const uint4*>(p.aq + xr + (g0 + g) * kGroup);
                const uint4 lo = src[0], hi = src[1];
                af[g] = v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w,
                            (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
            }
            rasc = p.asc[arow];
        } else {
#pragma unroll
            for (int g = 0; g < GPW; ++g)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    raw[g][i] = dec_row16<DEP>(reinterpret_cast<const uint16_t*>(p.a),
                                               xr + (g0 + g) * kGroup + i * 8);
        }
    };
    // DEP: wait until every work-group of the first GEMM that wrote a unit of the touched
    // experts in this team's range has published its rows. Lane i polls work-group
    // w_lo + i (+ 64 j); the partition is the first GEMM's (same lists, upe1 units).
    // work-groups [w_lo, w_hi] of the first GEMM that wrote units of the touched experts in
    // this team's range (its partition over the same lists, upe1 units an expert)
    auto producers = [&](int& w_lo, int& w_hi) __attribute__((always_inline)) {
        const int r_a = ua / upe, r_b = (ub - 1) / upe;
        const int n1 = (int)gridDim.x * dep.teams1;
        const int w1 = dec_cost(L, n_t, dep.upe1, kDecPassCost1);
        // start costs of the first unit of r_a and the last unit of r_b in the first GEMM
        const int np_a = ((int)L.first[r_a + 1] - (int)L.first[r_a] + 15) >> 4;
        const int np_b = ((int)L.first[r_b + 1] - (int)L.first[r_b] + 15) >> 4;
        const int s_lo = dec_cost(L, r_a, dep.upe1, kDecPassCost1) + np_a * kDecPassCost1;
        const int s_hi = dec_cost(L, r_b, dep.upe1, kDecPassCost1) + np_b * (kDecPassCost1 + dep.upe1 - 1);
        w_lo = dec_owner(s_lo, w1, n1) / dep.teams1;
        w_hi = dec_owner(s_hi, w1, n1) / dep.teams1;
    };
    // wait until work-groups w_lo .. w_hi (lane i: w_lo + i + 64 j) have published
    auto wait_rows = [&](int w_lo, int w_hi) __attribute__((always_inline)) {
        for (int w0 = w_lo; w0 <= w_hi; w0 += 64) {
            const int w = w0 + lane;
            bool ok = w > w_hi;
            for (int spin = 0; spin < dep.spin_limit; ++spin) {
                if (!ok) ok = dec_flag(dep.flags, w) == dep.expect;
                if (__ballot(!ok) == 0) break;
                __builtin_amdgcn_s_sleep(2);
            }
            if (__ballot(!ok) != 0 && lane == 0) dep.timeout[blockIdx.x] = dep.nonce;
        }
    };
    // quantise the pass's rows (PREQ: they are quantised already; only the group sums and
    // the output rows remain), bit-identical to act_quant_kernel: absmax on the magnitude
    // bits (both conversions are monotone in them; NaNs, which fmaxf skips, count as 0), then
    // over the row's four quarter-lanes and the team's K-split waves. Two values per
    // instruction (packed 16-bit max); a maximum above the infinity pattern means a NaN is
    // present, and only then the exact NaN-skipping pass runs.
    auto quantize = [&](const DecCursor& c) __attribute__((always_inline)) {
        float my_asc = rasc;
        if constexpr (!PREQ) {
            constexpr uint32_t nan_above = ABF16 ? 0x7F80u : 0x7C00u;
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
            if (mbits > nan_above) {
                mbits = 0;
#pragma unroll
                for (int g = 0; g < GPW; ++g)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const uint32_t wd[4] = {raw[g][i].x, raw[g][i].y, raw[g][i].z, raw[g][i].w};
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            const uint32_t lo = wd[j] & 0x7FFFu, hi = (wd[j] >> 16) & 0x7FFFu;
                            mbits = max(mbits, lo > nan_above ? 0u : lo);
                            mbits = max(mbits, hi > nan_above ? 0u : hi);
                        }
                    }
            }
            float amax = dec_act_f32<ABF16>(mbits);
            {
                const auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(amax), __float_as_uint(amax), false, false);
                amax = fmaxf(__uint_as_float(r16[0]), __uint_as_float(r16[1]));
                const auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(amax), __float_as_uint(amax), false, false);
                amax = fmaxf(__uint_as_float(r32[0]), __uint_as_float(r32[1]));
            }
            if constexpr (KSPLIT > 1) {
                if (q == 0) s_amax[wave][c16] = amax;
                lds_barrier();
#pragma unroll
                for (int j = 0; j < KSPLIT; ++j) amax = fmaxf(amax, s_amax[team * KSPLIT + j][c16]);
            }
            my_asc = act_scale_from_absmax(amax);
            const float inv = 1.0f / my_asc;
#pragma unroll
            for (int g = 0; g < GPW; ++g)
#pragma unroll
                for (int i = 0; i < 4; ++i) {   // k8-interleaved bytes, as act_quant_kernel
                    const uint32_t wd[4] = {raw[g][i].x, raw[g][i].y, raw[g][i].z, raw[g][i].w};
                    float f[8];
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        f[2 * j] = dec_act_f32<ABF16>(wd[j] & 0xFFFFu) * inv;
                        f[2 * j + 1] = dec_act_f32<ABF16>(wd[j] >> 16) * inv;
                    }
                    af[g][2 * i] = (int)pack4_e4m3(f[0], f[2], f[4], f[6]);
                    af[g][2 * i + 1] = (int)pack4_e4m3(f[1], f[3], f[5], f[7]);
                }
        }
#pragma unroll
        for (int g = 0; g < GPW; ++g) {
            const int one = (int)kDecOnes;
            sa[g] = mfma_16x16x128(af[g], v8i{one, one, one, one, one, one, one, one},
                                   v4f{0.f, 0.f, 0.f, 0.f});
#pragma unroll
            for (int i = 0; i < 4; ++i) sa[g][i] *= 1.0f / kNibbleScale;
        }
        // the pass's output rows (slot, scale) for the stores
        const int s0 = (int)L.first[c.r] + c.m0;
        const int mreal = min(16, (int)L.first[c.r + 1] - s0);
#pragma unroll
        for (int i = 0; i < NRO; ++i) {
            const int m = 4 * q + (KSPLIT > 1 ? wave % KSPLIT : i);
            osl[i] = L.slot[s0 + min(m, mreal - 1)];
            oasc[i] = __shfl(my_asc * kNibbleScale, m, 64);
        }
    };

    // column tile f0 of unit column ucol: value (ra, rb) of an output row (slot sl, scale a)
    auto store1 = [&](int ucol, int f0, int sl, float a, float ra, float rb) __attribute__((always_inline)) {
        const int col = (ucol * C::CT + f0) * 16 + c16;
        if constexpr (C::kSilu) {
            reinterpret_cast<__half*>(p.out)[(int64_t)sl * ncols + col] =
                silu_mul_h(__float2half(as_f32(ra * a)), __float2half(as_f32(rb * a)));
        } else {
            reinterpret_cast<float*>(p.out)[(int64_t)sl * p.N + col] = ra * a;
        }
    };

    // K split: the batch's completed units, per ring slot (column, and this wave's output row)
    int bp = 0;             // batch parity (LDS buffer)
    int bucol[C::D], bsl[C::D];
    float basc[C::D];
    auto part_of = [&](int parity, int slot) __attribute__((always_inline)) {
        return s_part + (parity * C::D + slot) * (KSPLIT * C::FR * 64);
    };
    // sum the K-split waves' partials of slot k's unit in wave order (wave w takes row 4q + w
    // of its lanes) and store it
    auto flush_slot = [&](int k) __attribute__((always_inline)) {
        const v4f* part = part_of(bp, k);
        const int i = wave % KSPLIT;
        float sum[C::FR];
#pragma unroll
        for (int f = 0; f < C::FR; ++f) {
            const float* pf = reinterpret_cast<const float*>(part + f * 64 + lane) + i;
            sum[f] = pf[0];
#pragma unroll
            for (int j = 1; j < KSPLIT; ++j) sum[f] += pf[j * C::FR * 64 * 4];
        }
#pragma unroll
        for (int ct = 0; ct < C::CT; ++ct)
            store1(bucol[k], ct, bsl[k], basc[k], sum[ct], C::kSilu ? sum[C::CT + ct] : sum[ct]);
    };
    auto consume = [&](const DecCursor& c, auto slot) __attribute__((always_inline)) {
        constexpr int b = decltype(slot)::value;
        constexpr int gb = b % C::NB;       // a pass has NB chunks per unit: slot parity == c.b
        const int ucol = c.u - c.r * upe;
#pragma unroll
        for (int f = 0; f < C::FR; ++f) {
#pragma unroll
            for (int uu = 0; uu < C::GC; ++uu) {
                const int ga = gb * C::GC + uu;
                v4f acc = mfma_16x16x128(af[ga], spread_nibbles(wv[b][uu * C::FR + f]),
                                         v4f{0.f, 0.f, 0.f, 0.f});
                const uint32_t m = mw[b][f][uu];
                const float z = (float)((m >> 16) & 0xF);
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[i] = fmaf(-z, sa[ga][i], acc[i]);
                const float s = __half2float(__ushort_as_half((unsigned short)(m & 0xFFFF)));
#pragma unroll
                for (int i = 0; i < 4; ++i) run[f][i] = fmaf(acc[i], s, run[f][i]);
            }
        }
        if constexpr (gb == C::NB - 1) {   // unit complete; every store is unconditional
            if constexpr (KSPLIT > 1) {
                // partials to LDS; the batch is summed and stored after the ring's last slot
                v4f* part = part_of(bp, b);
#pragma unroll
                for (int f = 0; f < C::FR; ++f) part[((wave % KSPLIT) * C::FR + f) * 64 + lane] = run[f];
                bucol[b] = ucol;
                bsl[b] = osl[0];
                basc[b] = oasc[0];
            } else {
#pragma unroll
                for (int ct = 0; ct < C::CT; ++ct)
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        store1(ucol, ct, osl[i], oasc[i], run[ct][i],
                               C::kSilu ? run[C::CT + ct][i] : run[ct][i]);
            }
#pragma unroll
            for (int f = 0; f < C::FR; ++f) run[f] = v4f{0.f, 0.f, 0.f, 0.f};
        }
        if constexpr (KSPLIT > 1 && b == C::D - 1) {   // batch complete (a full ring turn)
            lds_barrier();
#pragma unroll
            for (int k = C::NB - 1; k < C::D; k += C::NB) flush_slot(k);
            bp ^= 1;
        }
    };

    using S0 = std::integral_constant<int, 0>;
    using S1 = std::integral_constant<int, 1>;
    using S2 = std::integral_constant<int, 2>;
    using S3 = std::integral_constant<int, 3>;

    // chunks of the team's work
    int total = 0;
    for (int r = ua / upe; r * upe < ub; ++r)
        total += (((int)L.first[r + 1] - (int)L.first[r] + 15) >> 4) * (seg_hi(r) - seg_lo(r)) * C::NB;

    // The issue cursor runs D chunks (the ring slots) ahead of the consume cursor, across experts and
    // passes, so the next expert's weights are in flight while a pass boundary loads and
    // quantises rows. The rows go out before the chunk issued beside them: the memory counter
    // completes in order, so their wait leaves that chunk in flight. The compiler derives
    // its waits for the ring from the program order of loads, so the steady-state loop has a
    // fixed trip count (no exit inside), its steps are kept in order by scheduling barriers,
    // and its stores are unconditional; with these, each consume waits only for its own
    // chunk (D - 1 chunks stay in flight).
    const int r0 = ua / upe;
    DecCursor cc{r0, (int)L.expert[r0], 0, ua, 0};
    DecCursor ic = cc;
#pragma unroll
    for (int f = 0; f < C::FR; ++f) run[f] = v4f{0.f, 0.f, 0.f, 0.f};
    // DEP: the first poll of the producers' flags goes out, then the weight ring (weights do
    // not depend on the first GEMM), then the wait and the rows. The memory counter completes
    // in order, so reading the poll's result leaves the ring's loads in flight.
    int w_lo = 0, w_hi = -1;
    uint64_t fl0 = 0;
    if constexpr (DEP) {
        producers(w_lo, w_hi);
        // unconditional (a clamped address): a load under a branch gets its wait at the join
        fl0 = dec_flag(dep.flags, w_lo + min(lane, w_hi - w_lo));
    } else {
        load_rows(cc);
    }
    __builtin_amdgcn_sched_barrier(0);
    issue(ic, S0{}); advance(ic);
    __builtin_amdgcn_sched_barrier(0);
    issue(ic, S1{}); advance(ic);
    __builtin_amdgcn_sched_barrier(0);
    issue(ic, S2{}); advance(ic);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (C::D > 3) {
        issue(ic, S3{}); advance(ic);
        __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (DEP) {
        if (w_hi - w_lo >= 64 || __ballot(lane <= w_hi - w_lo && fl0 != dep.expect) != 0)
            wait_rows(w_lo, w_hi);
        // the row loads below must not be moved above the flag reads that allowed them (an
        // acquire at work-group scope orders them in the compiler; the loads themselves are
        // agent-coherent)
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
        load_rows(cc);
    }
    quantize(cc);

    auto step = [&](auto slot) __attribute__((always_inline)) {
        consume(cc, slot);
        const bool np = advance(cc) && cc.u < ub;
        if (np) load_rows(cc);
        issue(ic, slot);
        advance(ic);
        if (np) quantize(cc);
        __builtin_amdgcn_sched_barrier(0);
    };
    const int nq = total / C::D;
    for (int it = 0; it < nq; ++it) {
        step(S0{});
        step(S1{});
        step(S2{});
        if constexpr (C::D > 3) step(S3{});
    }
    const int rem = total % C::D;
    if (rem > 0) step(S0{});
    if (rem > 1) step(S1{});
    if constexpr (C::D > 3)
        if (rem > 2) step(S2{});
    if constexpr (KSPLIT > 1) {     // the last, partial batch (slots 0 .. rem - 1)
        lds_barrier();
#pragma unroll
        for (int k = 0; k < C::D - 1; ++k)
            if (k % C::NB == C::NB - 1 && k < rem) flush_slot(k);
    }
}

template <Epi EPI, int GPW, int KSPLIT, bool ABF16, bool PREQ>
__global__ void __launch_bounds__(kDecThreads, 1) decode_gemv_kernel(DecodeParams p) {
    __shared__ DecodeLists L;
    __shared__ float s_amax[4][16];
    extern __shared__ __attribute__((aligned(16))) uint8_t s_dyn[];
    __shared__ int32_t s_ids[kDecMaxSlots];
    const uint32_t warm = dec_warm(p);
    const int32_t* ids = p.ids;
    if (p.logits != nullptr) {
        dec_route(p, s_ids);
        ids = s_ids;
    }
    if (p.hand_in != nullptr) {
        dec_hand_read(p, L);
    } else {
        build_lists(p, ids, L);
        if (p.hand_out != nullptr) dec_hand_lists(p, L);
    }
    dec_run<EPI, GPW, KSPLIT, ABF16, false, PREQ>(p, L, s_amax, reinterpret_cast<v4f*>(s_dyn), DecDep{});
    dec_keep(warm, p.out);
}

// The decode layer's two GEMVs in one launch: gemm1 + SiLU*mul over x (h rows per slot),
// then gemm2 over h (fp32 rows per slot), on the same lists. Each work-group publishes its
// gemm1 rows (flags[blockIdx.x] = nonce) before its gemm2 part, whose weight ring fills
// while it waits for the rows it reads (DecDep). Every wait is bounded, so every wave
// reaches the end; one work-group per CU, all resident.
template <int GPW1, int KS1, int GPW2, int KS2, bool ABF16>
__global__ void __launch_bounds__(kDecThreads, 1) decode_layer_kernel(DecodeParams p1, DecodeParams p2,
                                                                      DecDep dep) {
    __shared__ DecodeLists L;
    __shared__ float s_amax[4][16];
    extern __shared__ __attribute__((aligned(16))) uint8_t s_dyn[];
    __shared__ int32_t s_ids[kDecMaxSlots];
    // this work-group's timeout word: the previous call's slot reduce has read it
    if (threadIdx.x == 0) dep.timeout[blockIdx.x] = 0;
    const uint32_t fault = g_dec_fault;
    const uint32_t warm = dec_warm(p1);
    const int32_t* ids = p1.ids;
    if (p1.logits != nullptr) {
        dec_route(p1, s_ids);
        ids = s_ids;
    }
    build_lists(p1, ids, L);
    if (fault != 0) {
        dep.expect = (dep.nonce ^ 0x8000000000000000ull) | 1ull;   // never published, never 0
        dep.spin_limit = kDecFaultSpinLimit;
    }
    dec_run<Epi::kSiluHalf, GPW1, KS1, ABF16, false>(p1, L, s_amax, reinterpret_cast<v4f*>(s_dyn), dep);
    // every wave's h stores complete (vmcnt(0)), then one release at agent scope publishes them
    __builtin_amdgcn_s_waitcnt(0x0F70);
    __syncthreads();
    if (threadIdx.x == 0)
        __hip_atomic_store(const_cast<uint64_t*>(dep.flags) + blockIdx.x, dep.nonce,
                           __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
    dec_run<Epi::kSlotF32, GPW2, KS2, false, true>(p2, L, s_amax, reinterpret_cast<v4f*>(s_dyn), dep);
    dec_keep(warm, p2.out);
}

struct DecSplit {
    int gpw, ksplit;
};
// K groups per wave and K-split for the decode GEMVs (a team is one wave or four)
DecSplit dec_split(int G) {
    switch (G) {
        case 1: return {1, 1};
        case 2: return {2, 1};
        case 3: return {3, 1};
        case 4: return {4, 1};
        case 8: return {2, 4};
        case 12: return {3, 4};
        case 16: return {4, 4};
        case 32: return {8, 4};
        default: return {0, 0};
    }
}

// one four-wave work-group per CU (one wave per SIMD, up to 512 registers)
int persistent_grid() { return device_cu_count(); }

template <Epi EPI, int GPW, int KSPLIT, bool ABF16, bool PREQ = false>
int launch_dec_a(const DecodeParams& p, hipStream_t s) {
    using C = DecCfg<EPI, GPW, KSPLIT>;
    const size_t lds = C::LDS_BYTES;
    auto* kern = &decode_gemv_kernel<EPI, GPW, KSPLIT, ABF16, PREQ>;
    if (int rc = reserve_dyn_lds(reinterpret_cast<const void*>(kern), (int)lds, "decode_gemv_kernel"))
        return rc;
    launch_kernel(kern, dim3(persistent_grid()), dim3(kDecThreads), lds, s, p);
    return check_launch("decode_gemv_kernel");
}

// gemm1 reads x (fp16 or bf16, or the router's quantised rows); gemm2 reads the fp16 h rows
template <Epi EPI, int GPW, int KSPLIT>
int launch_dec_t(const DecodeParams& p, hipStream_t s) {
    if constexpr (EPI == Epi::kSiluHalf) {
        if (p.aq != nullptr) return launch_dec_a<EPI, GPW, KSPLIT, false, true>(p, s);
        if (p.a_bf16) return launch_dec_a<EPI, GPW, KSPLIT, true>(p, s);
    }
    return launch_dec_a<EPI, GPW, KSPLIT, false>(p, s);
}

template <Epi EPI>
int launch_dec_e(const DecodeParams& p, hipStream_t s) {
    const DecSplit sp = dec_split(p.G);
    switch (sp.gpw * 8 + sp.ksplit) {
        case 1 * 8 + 1: return launch_dec_t<EPI, 1, 1>(p, s);
        case 2 * 8 + 1: return launch_dec_t<EPI, 2, 1>(p, s);
        case 3 * 8 + 1: return launch_dec_t<EPI, 3, 1>(p, s);
        case 4 * 8 + 1: return launch_dec_t<EPI, 4, 1>(p, s);
        case 2 * 8 + 4: return launch_dec_t<EPI, 2, 4>(p, s);
        case 3 * 8 + 4: return launch_dec_t<EPI, 3, 4>(p, s);
        case 4 * 8 + 4: return launch_dec_t<EPI, 4, 4>(p, s);
        case 8 * 8 + 4: return launch_dec_t<EPI, 8, 4>(p, s);
    }
    set_error("decode GEMV: unsupported number of K groups");
    return W4A8_ERR_INVALID;
}

// The fused layer for the K-group counts of the common shapes (gemm1 K = H, gemm2 K = I);
// other shapes run the two GEMVs as separate launches.
template <int GPW1, int KS1, int GPW2, int KS2, bool ABF16>
int launch_layer_a(const DecodeParams& p1, const DecodeParams& p2, const DecDep& dep, hipStream_t s) {
    constexpr size_t l1 = DecCfg<Epi::kSiluHalf, GPW1, KS1>::LDS_BYTES;
    constexpr size_t l2 = DecCfg<Epi::kSlotF32, GPW2, KS2>::LDS_BYTES;
    constexpr size_t lds = l1 > l2 ? l1 : l2;
    auto* kern = &decode_layer_kernel<GPW1, KS1, GPW2, KS2, ABF16>;
    const void* fn = reinterpret_cast<const void*>(kern);
    if (int rc = reserve_dyn_lds(fn, (int)lds, "decode_layer_kernel")) return rc;
    // gemm2 teams wait for other work-groups' flags: the whole grid (one work-group per CU)
    // must be resident at once
    if (blocks_per_cu(fn, kDecThreads, lds) < 1) {
        set_error("decode_layer_kernel: a work-group does not fit on one CU");
        return W4A8_ERR_INVALID;
    }
    const dim3 grid(persistent_grid());
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &cap) != hipSuccess) cap = hipStreamCaptureStatusActive;
    if (cap == hipStreamCaptureStatusNone && next_kernel_stamp().start == nullptr) {
        // eager: a cooperative launch, which the runtime refuses unless the grid can be
        // resident all at once (a graph capture takes the ordinary launch below; the bounded
        // waits and the NaN output of a wait that gave up cover that case)
        DecodeParams a1 = p1, a2 = p2;
        DecDep a3 = dep;
        void* args[] = {&a1, &a2, &a3};
        const hipError_t e = hipLaunchCooperativeKernel(fn, grid, dim3(kDecThreads), args,
                                                        (unsigned)lds, s);
        if (e != hipSuccess) {
            (void)hipGetLastError();
            set_error(std::string("decode_layer_kernel: cooperative launch refused: ") +
                      hipGetErrorString(e));
            return W4A8_ERR_HIP;
        }
        return W4A8_OK;
    }
    launch_kernel(kern, grid, dim3(kDecThreads), lds, s, p1, p2, dep);
    return check_launch("decode_layer_kernel");
}

template <int GPW1, int KS1, int GPW2, int KS2>
int launch_layer_t(const DecodeParams& p1, const DecodeParams& p2, const DecDep& dep, hipStream_t s) {
    if (p1.a_bf16) return launch_layer_a<GPW1, KS1, GPW2, KS2, true>(p1, p2, dep, s);
    return launch_layer_a<GPW1, KS1, GPW2, KS2, false>(p1, p2, dep, s);
}

// (K groups of gemm1, K groups of gemm2) with a fused instantiation
bool dec_fused_shape(int g1, int g2) {
    return (g1 == 16 && g2 == 4) || (g1 == 32 && g2 == 12) || (g1 == 4 && g2 == 2) ||
           (g1 == 2 && g2 == 1) || (g1 == 16 && g2 == 16) || (g1 == 8 && g2 == 4);
}

int launch_layer_e(const DecodeParams& p1, const DecodeParams& p2, const DecDep& dep, hipStream_t s) {
    switch (p1.G * 64 + p2.G) {
        case 16 * 64 + 4: return launch_layer_t<4, 4, 4, 1>(p1, p2, dep, s);
        case 32 * 64 + 12: return launch_layer_t<8, 4, 3, 4>(p1, p2, dep, s);
        case 4 * 64 + 2: return launch_layer_t<4, 1, 2, 1>(p1, p2, dep, s);
        case 2 * 64 + 1: return launch_layer_t<2, 1, 1, 1>(p1, p2, dep, s);
        case 16 * 64 + 16: return launch_layer_t<4, 4, 4, 4>(p1, p2, dep, s);
        case 8 * 64 + 4: return launch_layer_t<2, 4, 4, 1>(p1, p2, dep, s);
    }
    set_error("decode layer: no fused instantiation for these K-group counts");
    return W4A8_ERR_INVALID;
}

DecodeParams dec_params(const DecodeLaunch& d) {
    DecodeParams p;
    p.ids = d.topk_ids;
    p.logits = d.logits;
    p.n_router = (int)d.n_router;
    p.renorm = d.renormalize ? 1 : 0;
    p.tw_out = d.topk_weights_out;
    p.ids_out = d.topk_ids_out;
    p.emap = d.expert_map;
    p.emap_len = (int)d.emap_len;
    p.numel = (int)d.numel;
    p.top_k = (int)d.top_k;
    p.E = (int)d.E;
    p.a = d.a;
    p.a_bf16 = d.a_bf16 ? 1 : 0;
    p.aq = d.silu ? d.aq : nullptr;
    p.asc = d.silu ? d.asc : nullptr;
    p.hand_out = d.silu ? d.hand_out : nullptr;
    p.hand_in = d.silu ? nullptr : d.hand_in;
    p.a_per_token = d.silu ? 1 : 0;
    p.w = d.w;
    p.out = d.out;
    p.K = (int)d.K;
    p.N = (int)d.N;
    p.G = (int)(d.K / kGroup);
    return p;
}

}  // namespace

bool decode_layer_fused_supported(int64_t H, int64_t inter) {
    return dec_fused_shape((int)(H / kGroup), (int)(inter / kGroup));
}

int decode_layer_grid() { return persistent_grid(); }

int decode_fused_set_fault(int on) {
    const uint32_t v = on != 0 ? 1u : 0u;
    const hipError_t e = hipMemcpyToSymbol(HIP_SYMBOL(g_dec_fault), &v, sizeof(v), 0,
                                           hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        set_error(std::string("decode fused test hook: ") + hipGetErrorString(e));
        return W4A8_ERR_HIP;
    }
    return W4A8_OK;
}

int launch_decode_layer(const DecodeLaunch& d1, const DecodeLaunch& d2, uint64_t* flags,
                        uint64_t nonce, uint64_t* timeout, hipStream_t s) {
    if (d1.numel == 0) return W4A8_OK;
    if (persistent_grid() > kDecodeFlagSlots) {
        set_error("decode layer: more compute units than completion flags");
        return W4A8_ERR_INVALID;
    }
    const DecodeParams p1 = dec_params(d1), p2 = dec_params(d2);
    DecDep dep;
    dep.flags = flags;
    dep.nonce = nonce;
    dep.upe1 = (int)(d1.N / 2 / 16);                 // gemm1: 16 gate + 16 up columns a unit
    dep.teams1 = dec_split(p1.G).ksplit > 1 ? 1 : 4;
    dep.timeout = timeout;
    dep.expect = nonce;
    dep.spin_limit = kDecSpinLimit;
    return launch_layer_e(p1, p2, dep, s);
}

bool decode_routes_in_kernel(int64_t T, int64_t n_router, int64_t top_k) {
    return T <= kDecRouteMaxT && n_router <= kDecRouteMaxE && top_k <= n_router && top_k <= 64;
}

bool decode_layer_supported(int64_t numel, int64_t E, int64_t H, int64_t inter, int64_t gs) {
    return numel <= kDecMaxSlots && E <= kDecMaxExperts && gs == kGroup && H % kGroup == 0 &&
           inter % kGroup == 0 && dec_split((int)(H / kGroup)).gpw > 0 &&
           dec_split((int)(inter / kGroup)).gpw > 0;
}

int launch_decode_gemv(const DecodeLaunch& d, hipStream_t s) {
    if (d.numel == 0) return W4A8_OK;
    const DecodeParams p = dec_params(d);
    return d.silu ? launch_dec_e<Epi::kSiluHalf>(p, s) : launch_dec_e<Epi::kSlotF32>(p, s);
}

}  // namespace w4a8
