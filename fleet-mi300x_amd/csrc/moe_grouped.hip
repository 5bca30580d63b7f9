// Multi-token grouped-expert MoE step: T tokens, each routed to 6 of 64
// experts (ids and weights given), plus the shared expert on every token.
//
// The reference has no kernel for this (it is batch-1 only); the semantics are
// HF DeepseekV2MoE.moe_infer (reference/modeling_deepseek.py:591-664): count
// tokens per expert, permute the (token, slot) entries so each expert's rows
// are contiguous, run each expert's SwiGLU on its rows, un-permute and combine
// per token with the rounding of src/host/reference_decode.py:280-287.
//
// Launch shape. Work is cut into items that every workgroup takes from a
// contiguous range holding 1/256 of the step's cost (items priced by their
// measured time: VALU items by token count, MFMA items by live token tiles),
// after building the dispatch tables itself in LDS from the T x 6 ids
// (ballot-matched per-chunk counts, a scan, stable positions): units =
// [shared expert (T tokens), then every selected expert in id order (its
// tokens in token order)].
//   * VALU units (<= 8 tokens): items of two gate/up row pairs (16 KB) or 2-8
//     down rows; rows stream with 1 KB wave loads against the tokens' x / h
//     held in LDS (dot2, one multi-value wave reduction per item), one item
//     per wave from an LDS ticket.
//   * MFMA units (> 8 tokens): items of 32 rows x up to 64 tokens taken by
//     the whole workgroup, bf16 MFMA 16x16x32, all streamed (m_stream): each
//     wave keeps its 16 tokens' x or h fragments for one K parity in
//     registers, and the weight rows pass through a ring of 256-element K
//     slices in LDS (global_load_lds, 1 KB per instruction, XOR-swizzled so
//     the MFMA operand reads are conflict-free) kept 8 slices ahead across
//     items. The shared expert's down rows (K = 2816) run as two K halves
//     whose fp32 sums the combine adds.
// T <= 8 (every unit is a VALU unit): ONE launch, phases G (gate/up + SwiGLU)
//   -> D (down) -> C (combine) handing data over through self-validating words
//   (epoch << 32 | payload, device-scope stores and loads; no grid barrier).
// T > 8: two launches on the stream, G, then D + C; h crosses the kernel
//   boundary as plain bf16.
// Partials bf16(w * bf16(d)) (shared: bf16(d), or with two launches the two
// fp32 K-half sums) are published per (token, slot) as tagged words; phase C
// sums them in slot order: out[t] = bf16(bf16(sum_k part[t][k]) + shared[t]).
// The last workgroup to exit advances the epoch. Every wait is bounded and
// records FLEET_MOE_ABORT_GROUP_WAIT instead of hanging.
#include <stddef.h>

#include <mutex>
#include <vector>

#include "moe_common.h"

namespace fleet_moe {
namespace grouped {

constexpr int kMaxTokens = 256;
constexpr int kMaxEntries = kMaxTokens * kTopK;     // 1536
constexpr int kMaxChunks = kMaxEntries / kLanes;    // 24 chunks of 64 entries
constexpr int kWG = 256;
constexpr int kWaves = 8;
constexpr int kThreads = kWaves * kLanes;
constexpr int kVMax = 8;                // VALU path for units of at most 8 tokens
constexpr int kMGroup = 64;             // tokens per MFMA pass (4 tiles of 16)
constexpr int kUnitsMax = 1 + kRouted;
constexpr int kSegMax = 4;
constexpr int kSlots = kTopK + 1;       // partial slots per token: 6 routed + shared
constexpr int kPartWords = kHidden / 2; // 1024 words of two rows per (token, slot)
// h words per token over all units: 6 routed units of 704 + the shared 1408.
constexpr int kHWordsPerToken = kTopK * (kInter / 2) + kSharedInter / 2;   // 5632
// LDS staging, shared by phase G (x rows of <= 2 VALU units: 2 x 8 x 4 KB) and
// phase D (h rows of <= 3 VALU units: shared 8 x 5,632 B + routed 8 x 2,816 B,
// or 3 routed).
constexpr int kStageBytes = 3 * kVMax * kInter * 2;   // 67,584
static_assert(2 * kVMax * kHidden * 2 <= kStageBytes, "x staging fits");
static_assert(kVMax * (kSharedInter + kInter) * 2 <= kStageBytes, "h staging fits");

// MFMA items: 32 weight rows x up to 64 tokens; the rows pass through LDS in
// K slices of 256 (512 B of every row; a K of 1408 ends with a half slice).
constexpr int kMRows = 32;
constexpr int kKs = 256;
constexpr int kRowSlice = kKs * 2;                 // 512 B
constexpr int kSliceA = kMRows * kRowSlice;        // 16 KB
constexpr int kRing = 8;                           // slices in flight
constexpr int kXchBytes = 4 * 8 * kLanes * 4;      // odd-K-half partials, 8 KB

// Sticky status bit beside FLEET_MOE_ABORT_*: LDS staging overflow (the
// partition bounds make it unreachable; checked anyway).
constexpr uint32_t kAbortStage = 0x200u;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

struct Header {
    uint32_t epoch, exits, abort;
    uint32_t pad[61];
};
static_assert(offsetof(Header, abort) == 8, "status word offset");

// The dispatch tables launch 1 of a two-launch step leaves for launch 2
// (struct Tab below): three counts, the units, the sorted entries.
constexpr int kTabBytes = 16 + kUnitsMax * 6 * 4 + kMaxEntries * 2;

struct Layout {
    size_t tab, h, hp, part, sp, total;
};

__host__ __device__ constexpr size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

__host__ __device__ constexpr Layout layout(int max_tokens) {
    Layout L{};
    L.tab = align256(sizeof(Header));
    L.h = L.tab + align256(kTabBytes);
    L.hp = L.h + align256((size_t)(max_tokens < kVMax ? max_tokens : kVMax) * kHWordsPerToken * 8);
    L.part = L.hp + align256((size_t)max_tokens * kHWordsPerToken * 4);
    L.sp = L.part + align256((size_t)max_tokens * kSlots * kPartWords * 8);
    L.total = L.sp + align256((size_t)max_tokens * 2 * kHidden * 8);
    return L;
}

struct Params {
    const uint16_t* experts;
    const uint16_t* shared;
    int64_t expert_stride;
    const int32_t* ids;        // [T][6]
    const float* weights;      // [T][6]
    const uint16_t* x;         // bf16 [T][H]
    uint16_t* out;             // bf16 [T][H]
    Header* hdr;
    uint64_t* h;               // tagged h words (single launch)
    uint32_t* hp;              // plain h words, two bf16 each (two launches)
    uint64_t* part;            // tagged partial words [T][7][1024]
    uint64_t* sp;              // tagged fp32 shared down sums [T][2 K halves][2048] (two launches)
    struct Tab* tab;           // dispatch tables handed from launch 1 to launch 2
    size_t ws_tail16;          // 16-byte words of the workspace after the header
    int T;
};

struct Unit {
    int expert;     // -1: shared
    int m;          // tokens
    int tok0;       // first sorted position of its entries (routed)
    int h_off;      // first h word
    int gstart;     // first G cost unit
    int dstart;     // first D cost unit
};

struct Tab {
    int n_units, g_total, d_total, pad;
    Unit unit[kUnitsMax];
    int16_t ent[kMaxEntries];
};
static_assert(sizeof(Tab) <= kTabBytes && sizeof(Unit) == 6 * 4, "table blob");

struct Seg {
    int unit, lo, hi, base;   // items [lo, hi) of the unit; base = first ticket
    int stage;                // LDS staging offset (bytes) or -1
};

struct Lds {
    int16_t ent[kMaxEntries];          // sorted position -> flat entry (t * 6 + k)
    int cnt[kRouted];
    int off[kRouted];
    Unit unit[kUnitsMax];
    Seg gseg[kSegMax];
    Seg dseg[kSegMax];
    int n_units, g_total, d_total;
    int n_gseg, n_dseg, g_items, d_items;
    int gnext, dnext;
    int exit_last;                     // this workgroup exits last (the wrap call)
    float red[kWaves][kLanes];
    union {
        alignas(16) uint8_t stage[kStageBytes];          // VALU units: x or h rows
        alignas(16) uint8_t ring[kRing * kSliceA + kXchBytes];   // MFMA items
        struct {                                         // prologue only
            int8_t id[kMaxEntries];      // ids, clamped to [0, 64)
            int16_t rank[kMaxEntries];   // rank of an entry among equal ids of its chunk
            int ccnt[kMaxChunks][kRouted];   // per-chunk counts, then per-chunk offsets
        } pro;
    };
};

__device__ __forceinline__ bool is_v(int m) { return m <= kVMax; }
__device__ __forceinline__ int passes_of(int m) { return (m + kMGroup - 1) / kMGroup; }
__device__ __forceinline__ int gpairs_of(const Unit& u) { return u.expert < 0 ? kSharedInter : kInter; }

// Rows per VALU down item: R rows x M tokens values stay <= 32 accumulators.
__device__ __forceinline__ int d_rows_v(const Unit& u) {
    return u.expert < 0 ? (u.m > 4 ? 2 : 4) : (u.m > 4 ? 4 : 8);
}

// Items and their cost of a unit, in eighths of the time a one-token VALU
// item takes per 16 KB (G) or 11 KB (D) of weight rows, as measured on the
// DeepSeek-V2-Lite shapes with every CU streaming. A VALU item's time grows
// with its tokens (dot products and the reduction per weight byte; fewer rows
// in flight above 4 tokens in D); an MFMA item holds 8 units of weights, its
// live token tiles load LDS and the matrix cores, and its operand load delays
// its first copy. MFMA items run pass-minor: item i is row block i / passes,
// token pass i % passes; the shared expert's MFMA down items are two K halves
// of that sequence.
__device__ __forceinline__ int m_tiles(int m) { return min(kMGroup / 16, (m + 15) >> 4); }
__device__ __forceinline__ void g_items_of(const Unit& u, int& n, int& cost) {
    const int pairs = gpairs_of(u);
    if (is_v(u.m)) { n = pairs / 2; cost = u.m <= 3 ? 8 : 9; }
    else {
        n = 2 * pairs / kMRows * passes_of(u.m);
        constexpr int kCost[4] = {84, 84, 99, 103};
        cost = kCost[m_tiles(u.m) - 1];
    }
}
__device__ __forceinline__ void d_items_of(const Unit& u, int& n, int& cost) {
    const bool sh = u.expert < 0;
    if (is_v(u.m)) {
        const int R = d_rows_v(u);
        n = kHidden / R;
        const int units = sh ? R / 2 : R / 4;            // 11 KB units of weights
        cost = units * (u.m == 1 ? 8 : u.m == 2 ? 9 : u.m <= 4 ? 10 : 12);
    } else {
        n = (sh ? 2 : 1) * (kHidden / kMRows) * passes_of(u.m);
        constexpr int kCost[4] = {124, 132, 140, 150};
        cost = kCost[m_tiles(u.m) - 1];
    }
}

__device__ __forceinline__ void flag_abort(Header* hdr, uint32_t bit) {
    __hip_atomic_fetch_or(&hdr->abort, bit, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// A wait gives up early once another wait of the step has expired (or the
// staging bound was hit, which leaves work undone); the id warning bit does
// not stop anything.
__device__ __forceinline__ bool step_failed(Header* hdr) {
    return (ld_agent(&hdr->abort) & (FLEET_MOE_ABORT_GROUP_WAIT | kAbortStage)) != 0;
}

__device__ __forceinline__ void st_word(uint64_t* p, uint32_t epoch, uint32_t payload) {
    __hip_atomic_store(p, ((uint64_t)epoch << 32) | payload, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
    return bf16_bits(lo) | (bf16_bits(hi) << 16);
}

__device__ __forceinline__ f32x4 mfma16(const u32x4& a, const u32x4& b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

// Inclusive prefix sum over the 64 lanes (all lanes active), DPP only:
// row_shr 1, 2, 4, 8 within each row of 16 (lanes without a source add 0),
// then row_bcast 15 into rows 1 and 3 and row_bcast 31 into rows 2 and 3.
__device__ __forceinline__ int wave_incl_scan(int v) {
    v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, false);
    v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, false);
    v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, false);
    v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xF, 0xF, false);
    v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xA, 0xF, false);
    v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xC, 0xF, false);
    return v;
}

// Workgroup-local ticket, the same value in every lane.
__device__ __forceinline__ int claim(int* ctr, int limit) {
    int t = 0;
    if ((threadIdx.x & (kLanes - 1)) == 0)
        t = __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    t = wave_bcast(t);
    return t < limit ? t : -1;
}

// Workgroup barrier that orders LDS only (no wait for outstanding global
// loads, unlike __syncthreads).
__device__ __forceinline__ void lds_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

__device__ __forceinline__ void lds_wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// ---------------------------------------------------------------- prologue

// Wave 0: this workgroup's item ranges of the phases the launch runs (kG:
// gate/up, kD: down), items whose first cost unit lies in [ceil(w C / 256),
// ceil((w + 1) C / 256)), over up to 65 units, and the LDS staging of their
// VALU units (the units must be in LDS).
template <bool kG, bool kD>
__device__ void item_ranges(const Params& P, Lds& L) {
    const int lane = threadIdx.x & (kLanes - 1);
    const int wg = blockIdx.x;
#pragma unroll
    for (int ph = 0; ph < 2; ++ph) {
        if (ph == 0 ? !kG : !kD) continue;
        const int C = ph == 0 ? L.g_total : L.d_total;
        const int lo = (wg * C + kWG - 1) / kWG, hi = ((wg + 1) * C + kWG - 1) / kWG;
        Seg* S = ph == 0 ? L.gseg : L.dseg;
        int ns = 0, nitems = 0;
        for (int r0 = 0; r0 < L.n_units; r0 += kLanes) {
            const int ui = r0 + lane;
            const bool have = ui < L.n_units;
            int n = 0, cost = 1, start = 0;
            if (have) {
                const Unit& u = L.unit[ui];
                if (ph == 0) { g_items_of(u, n, cost); start = u.gstart; }
                else { d_items_of(u, n, cost); start = u.dstart; }
            }
            const int a = lo - start, b = hi - start;
            const int i0 = a <= 0 ? 0 : min(n, (a + cost - 1) / cost);
            const int i1 = b <= 0 ? 0 : min(n, (b + cost - 1) / cost);
            const bool seg = have && i0 < i1;
            const unsigned long long sm = __ballot(seg);
            const int si = ns + __builtin_popcountll(sm & ((1ull << lane) - 1ull));
            const int items = seg ? i1 - i0 : 0;
            const int incl = wave_incl_scan(items);
            if (seg && si < kSegMax) {
                // staging bytes of a VALU unit's x (G) or h (D) rows
                const Unit& u = L.unit[ui];
                const int need = !is_v(u.m) ? 0 : ph == 0 ? u.m * kHidden * 2
                                                            : u.m * gpairs_of(u) * 2;
                S[si] = Seg{ui, i0, i1, nitems + incl - items, need};
            }
            ns += __builtin_popcountll(sm);
            nitems += __builtin_amdgcn_readlane(incl, kLanes - 1);
        }
        const int nseg = min(ns, kSegMax);
        if (lane == 0) {
            if (ns > kSegMax) flag_abort(P.hdr, kAbortStage);
            if (ph == 0) { L.n_gseg = nseg; L.g_items = nitems; }
            else { L.n_dseg = nseg; L.d_items = nitems; }
        }
        lds_wave_sync();
        // lane s < nseg: its segment's staging offset (a running sum in
        // segment order), or -1 for an MFMA unit
        const int need = lane < nseg ? S[lane].stage : 0;
        const int end = wave_incl_scan(need);
        if (lane < nseg) {
            if (need > 0 && end > kStageBytes) flag_abort(P.hdr, kAbortStage);
            S[lane].stage = need > 0 && end <= kStageBytes ? end - need : -1;
        }
    }
}

// Dispatch tables and this workgroup's item ranges of the phases the launch
// runs (kG: gate/up, kD: down), all in LDS.
template <bool kG, bool kD>
__device__ void build_tables(const Params& P, Lds& L) {
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & (kLanes - 1);
    const int T = P.T, N = T * kTopK;
    const int nchunks = (N + kLanes - 1) / kLanes;
    for (int i = tid; i < nchunks * kRouted; i += kThreads) (&L.pro.ccnt[0][0])[i] = 0;
    if (tid == 0) {
        L.gnext = L.dnext = 0;
        L.n_gseg = L.n_dseg = L.g_items = L.d_items = 0;   // a phase the launch skips stays empty
    }
    __syncthreads();
    // per chunk of 64 entries: lanes with equal ids by 6 ballots; the rank of
    // an entry among them, and the count, kept by the lowest such lane
    for (int c = wave; c < nchunks; c += kWaves) {
        const int i = c * kLanes + lane;
        const bool valid = i < N;
        const int raw = valid ? P.ids[i] : 0;
        const int id = min(max(raw, 0), kRouted - 1);   // clamped: addresses stay in bounds
        if (valid) L.pro.id[i] = (int8_t)id;
        if (__ballot(raw != id) && lane == 0 && blockIdx.x == 0)
            flag_abort(P.hdr, FLEET_MOE_ABORT_BAD_ID);
        unsigned long long same = __ballot(valid);
#pragma unroll
        for (int b = 0; b < 6; ++b) {
            const unsigned long long ones = __ballot(valid && ((id >> b) & 1));
            same &= ((id >> b) & 1) ? ones : ~ones;
        }
        const int r = __builtin_popcountll(same & ((1ull << lane) - 1ull));
        if (valid) {
            L.pro.rank[i] = (int16_t)r;
            if (r == 0) L.pro.ccnt[c][id] = __builtin_popcountll(same);
        }
    }
    __syncthreads();
    if (tid < kRouted) {
        int run = 0;
        for (int c = 0; c < nchunks; ++c) {
            const int v = L.pro.ccnt[c][tid];
            L.pro.ccnt[c][tid] = run;
            run += v;
        }
        L.cnt[tid] = run;
    }
    __syncthreads();
    if (wave == 0) {
        const int c = L.cnt[lane];
        // exclusive scans over the 64 experts: entry offsets, h words, costs
        int s_off = c, s_h = c * (kInter / 2), s_g = 0, s_d = 0;
        if (c > 0) {
            int n, cost;
            g_items_of(Unit{lane, c, 0, 0, 0, 0}, n, cost);
            s_g = n * cost;
            d_items_of(Unit{lane, c, 0, 0, 0, 0}, n, cost);
            s_d = n * cost;
        }
        const int e_off = s_off, e_h = s_h, e_g = s_g, e_d = s_d;
        s_off = wave_incl_scan(s_off);
        s_h = wave_incl_scan(s_h);
        s_g = wave_incl_scan(s_g);
        s_d = wave_incl_scan(s_d);
        L.off[lane] = s_off - e_off;
        const unsigned long long sel = __ballot(c > 0);
        int g_sh, d_sh, n, cost;
        g_items_of(Unit{-1, T, 0, 0, 0, 0}, n, cost);
        g_sh = n * cost;
        d_items_of(Unit{-1, T, 0, 0, 0, 0}, n, cost);
        d_sh = n * cost;
        if (c > 0) {
            const int u = 1 + __builtin_popcountll(sel & ((1ull << lane) - 1ull));
            L.unit[u] = Unit{lane, c, s_off - e_off, T * (kSharedInter / 2) + s_h - e_h,
                             g_sh + s_g - e_g, d_sh + s_d - e_d};
        }
        if (lane == kLanes - 1) {
            L.unit[0] = Unit{-1, T, 0, 0, 0, 0};
            L.n_units = 1 + __builtin_popcountll(sel);
            L.g_total = g_sh + s_g;
            L.d_total = d_sh + s_d;
        }
    }
    __syncthreads();
    if (wave != 0) {
        // waves 1..7: sorted position -> entry
        for (int i = tid - kLanes; i < N; i += kThreads - kLanes) {
            const int id = L.pro.id[i];
            L.ent[L.off[id] + L.pro.ccnt[i >> 6][id] + L.pro.rank[i]] = (int16_t)i;
        }
    } else {
        // wave 0, meanwhile: this workgroup's item ranges
        item_ranges<kG, kD>(P, L);
    }
    __syncthreads();
}

// Launch 1 of a two-launch step (workgroup 0): the tables every workgroup
// built alike, for launch 2 (the kernel boundary orders the stores before
// launch 2's loads).
__device__ void store_tables(const Params& P, const Lds& L) {
    Tab* tb = P.tab;
    const int tid = threadIdx.x;
    if (tid == 0) {
        tb->n_units = L.n_units;
        tb->g_total = L.g_total;
        tb->d_total = L.d_total;
    }
    for (int i = tid; i < kUnitsMax * 6; i += kThreads)
        reinterpret_cast<int*>(tb->unit)[i] = reinterpret_cast<const int*>(L.unit)[i];
    for (int i = tid; i < P.T * kTopK; i += kThreads) tb->ent[i] = L.ent[i];
}

// Launch 2: launch 1's tables, then this launch's item ranges.
template <bool kG, bool kD>
__device__ void load_tables(const Params& P, Lds& L) {
    const Tab* tb = P.tab;
    const int tid = threadIdx.x;
    if (tid == 0) {
        L.gnext = L.dnext = 0;
        L.n_gseg = L.n_dseg = L.g_items = L.d_items = 0;
        L.n_units = tb->n_units;
        L.g_total = tb->g_total;
        L.d_total = tb->d_total;
    }
    for (int i = tid; i < kUnitsMax * 6; i += kThreads)
        reinterpret_cast<int*>(L.unit)[i] = reinterpret_cast<const int*>(tb->unit)[i];
    for (int i = tid; i < P.T * kTopK; i += kThreads) L.ent[i] = tb->ent[i];
    __syncthreads();
    if (tid < kLanes) item_ranges<kG, kD>(P, L);
    __syncthreads();
}

// Activation row (token) of unit position j.
__device__ __forceinline__ int token_of(const Lds& L, const Unit& u, int j) {
    return u.expert < 0 ? j : L.ent[u.tok0 + j] / kTopK;
}

// ---------------------------------------------------------------- phase G

// VALU item: row pairs 2i, 2i+1 of a unit with m <= 8 tokens whose x rows sit
// in LDS at `xs`. Writes h word i of every token (plain with two launches,
// tagged with one).
template <int M>
__device__ __forceinline__ void g_item_v(const Params& P, Lds& L, const Unit& u, int i,
                                         const uint8_t* xs, uint32_t epoch) {
    const int lane = threadIdx.x & (kLanes - 1);
    const uint16_t* blk = u.expert < 0 ? P.shared : P.experts + (int64_t)u.expert * P.expert_stride;
    const u32x4* base = reinterpret_cast<const u32x4*>(blk) + (int64_t)(2 * i) * 2 * kRowChunks;
    u32x4 W[16];   // rows g(2i), u(2i), g(2i+1), u(2i+1): 4 chunks each
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int c = 0; c < 4; ++c) W[4 * r + c] = ld_stream(base + r * kRowChunks + lane + kLanes * c);
    constexpr int NV = 4 * M;
    float acc[NV];
#pragma unroll
    for (int v = 0; v < NV; ++v) acc[v] = 0.f;
    const u32x4* xr = reinterpret_cast<const u32x4*>(xs);
#pragma unroll
    for (int j = 0; j < M; ++j) {
        if (j < u.m) {
            u32x4 xq[4];
#pragma unroll
            for (int c = 0; c < 4; ++c) xq[c] = xr[j * kRowChunks + lane + kLanes * c];
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int c = 0; c < 4; ++c) acc[r * M + j] = dot8_d2(W[4 * r + c], xq[c], acc[r * M + j]);
        }
    }
    const float tot = wave_msum<NV>(acc);
    const int wave = threadIdx.x >> 6;
    float* red = L.red[wave];
    red[msum_index<NV>(lane)] = tot;
    lds_wave_sync();
    if (lane < u.m) {
        const int j = lane;
        const float g0 = red[0 * M + j], u0 = red[1 * M + j];
        const float g1 = red[2 * M + j], u1 = red[3 * M + j];
        const float h0 = bf16r(bf16r(silu_rn(bf16r(g0))) * bf16r(u0));
        const float h1 = bf16r(bf16r(silu_rn(bf16r(g1))) * bf16r(u1));
        const int64_t w = u.h_off + (int64_t)j * (gpairs_of(u) / 2) + i;
        if (P.hp) P.hp[w] = pack_bf16(h0, h1);
        else st_word(P.h + w, epoch, pack_bf16(h0, h1));
    }
    lds_wave_sync();
}

// ---------------------------------------------------------------- phase D

// Partial words of `pos` (unit position) for rows 2w, 2w + 1: routed values
// are bf16(w * bf16(d)), shared bf16(d).
__device__ __forceinline__ void put_part(const Params& P, const Lds& L, const Unit& u, int pos,
                                         int word, float d0, float d1, uint32_t epoch) {
    int t, slot;
    float a, b;
    if (u.expert < 0) {
        t = pos;
        slot = kTopK;
        a = bf16r(d0);
        b = bf16r(d1);
    } else {
        const int e = L.ent[u.tok0 + pos];
        t = e / kTopK;
        slot = e - t * kTopK;
        const float w = P.weights[e];
        a = w * bf16r(d0);
        b = w * bf16r(d1);
    }
    st_word(P.part + ((int64_t)t * kSlots + slot) * kPartWords + word, epoch, pack_bf16(a, b));
}

// VALU item: R rows of the unit's down matrix (R x M <= 32), m <= M tokens
// whose h rows sit in LDS at `hs` (bf16 [m][I]).
template <int M, bool SH, int R>
__device__ __forceinline__ void d_item_v(const Params& P, Lds& L, const Unit& u, int i,
                                         const uint8_t* hs, uint32_t epoch) {
    constexpr int K = SH ? kSharedInter : kInter;
    constexpr int C = K / kChunk;          // 16-byte chunks per row: 176 / 352
    constexpr int G = (C + kLanes - 1) / kLanes;   // 3 / 6
    static_assert(R * M <= 32 && R % 2 == 0, "item shape");
    const int lane = threadIdx.x & (kLanes - 1);
    const int row0 = R * i;
    const uint16_t* dn = SH ? P.shared + (int64_t)2 * kSharedInter * kHidden
                            : P.experts + (int64_t)u.expert * P.expert_stride +
                                  (int64_t)2 * kInter * kHidden;
    const u32x4* base = reinterpret_cast<const u32x4*>(dn) + (int64_t)row0 * C;
    u32x4 W[R * G];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const int c = lane + kLanes * g;
            W[r * G + g] = c < C ? ld_stream(base + r * C + c) : u32x4{0u, 0u, 0u, 0u};
        }
    constexpr int NV = R * M;
    float acc[NV];
#pragma unroll
    for (int v = 0; v < NV; ++v) acc[v] = 0.f;
    const u32x4* hr = reinterpret_cast<const u32x4*>(hs);
#pragma unroll
    for (int j = 0; j < M; ++j) {
        if (j < u.m) {
            u32x4 H[G];
#pragma unroll
            for (int g = 0; g < G; ++g) {
                const int c = lane + kLanes * g;
                H[g] = c < C ? hr[j * C + c] : u32x4{0u, 0u, 0u, 0u};
            }
#pragma unroll
            for (int r = 0; r < R; ++r)
#pragma unroll
                for (int g = 0; g < G; ++g) acc[r * M + j] = dot8_d2(W[r * G + g], H[g], acc[r * M + j]);
        }
    }
    const float tot = wave_msum<NV>(acc);
    const int wave = threadIdx.x >> 6;
    float* red = L.red[wave];
    red[msum_index<NV>(lane)] = tot;
    lds_wave_sync();
    if (lane < u.m * (R / 2)) {
        const int j = lane / (R / 2), wp = lane - j * (R / 2);
        put_part(P, L, u, j, row0 / 2 + wp, red[(2 * wp) * M + j], red[(2 * wp + 1) * M + j],
                 epoch);
    }
    lds_wave_sync();
}

// ---------------------------------------------------------------- MFMA stream
// The MFMA items of a phase, taken by the whole workgroup in order, with the
// token operand held in registers. Wave w takes token tile tt = w % 4 (16
// tokens of the pass) and the 256-K slices of parity kh = w / 4; it loads that
// operand once per (unit, pass, K half): 16-byte fragments of its tokens' x
// (or h) rows, one per 32-K MFMA step. The weight rows (32 per item) stream
// through a ring of kRing 16 KB LDS slices, filled by every wave with 1 KB
// global_load_lds copies and kept kRing slices ahead across item boundaries,
// so an item boundary costs no pipeline restart. In a slice, row r sits at
// [r * 512 B) with its 16-byte chunk c in slot c ^ (r & 15), so the 16 rows an
// MFMA operand read touches hit 16 different slots (all 64 banks once). Each
// barrier covers two slices, one per parity, computed side by side; an item's
// two K halves are added (even half + odd half) by the even-parity waves after
// the next barrier, the odd half crossing in LDS. Every weight byte is read
// once and each token row once per (workgroup, unit, pass, K half).
// Phase D: the shared expert's down rows (K = 2816) run as two K halves of
// 1408, each item shaped like a routed one; their fp32 sums go out as tagged
// words, and the combine adds the two halves before the bf16 rounding.
constexpr int kBMax = 32;                      // fragments per wave: G 32, D 24
static_assert(kSliceA == kWaves * 2 * 1024, "two 1 KB copies per wave per slice");

struct MRef {
    int unit, rb, pass, half;
};

// n-th MFMA item of the phase in this workgroup's segments: row block rb,
// token pass, K half (shared down items only; item i of that unit is half
// i / (64 passes), then row block and pass as for the others).
template <bool kG>
__device__ __forceinline__ bool m_item_n(const Lds& L, int n, MRef& r) {
    const Seg* S = kG ? L.gseg : L.dseg;
    const int ns = kG ? L.n_gseg : L.n_dseg;
    for (int s = 0; s < ns; ++s) {
        const Unit& u = L.unit[S[s].unit];
        if (is_v(u.m)) continue;
        const int cnt = S[s].hi - S[s].lo;
        if (n < cnt) {
            const int pr = passes_of(u.m);
            int i = S[s].lo + n;
            r.unit = S[s].unit;
            r.half = 0;
            if (!kG && u.expert < 0) {
                r.half = i / ((kHidden / kMRows) * pr);
                i -= r.half * (kHidden / kMRows) * pr;
            }
            r.rb = i / pr;
            r.pass = i - r.rb * pr;
            return true;
        }
        n -= cnt;
    }
    return false;
}

// First weight row of item r and the row stride (elements).
template <bool kG>
__device__ __forceinline__ const uint16_t* m_rows(const Params& P, const Unit& u, const MRef& r,
                                                  int& ld) {
    if (kG) {
        ld = kHidden;
        const uint16_t* w = u.expert < 0 ? P.shared : P.experts + (int64_t)u.expert * P.expert_stride;
        return w + (int64_t)kMRows * r.rb * kHidden;
    }
    if (u.expert < 0) {
        ld = kSharedInter;
        return P.shared + (int64_t)2 * kSharedInter * kHidden +
               (int64_t)kMRows * r.rb * kSharedInter + r.half * kInter;
    }
    ld = kInter;
    return P.experts + (int64_t)u.expert * P.expert_stride + (int64_t)2 * kInter * kHidden +
           (int64_t)kMRows * r.rb * kInter;
}

// s_waitcnt vmcnt(n), n wave-uniform in [0, 2 kRing].
__device__ __forceinline__ void wait_vm(int n) {
    switch (n) {
        case 0: __builtin_amdgcn_s_waitcnt(0x0F70); break;
        case 1: __builtin_amdgcn_s_waitcnt(0x0F71); break;
        case 2: __builtin_amdgcn_s_waitcnt(0x0F72); break;
        case 3: __builtin_amdgcn_s_waitcnt(0x0F73); break;
        case 4: __builtin_amdgcn_s_waitcnt(0x0F74); break;
        case 5: __builtin_amdgcn_s_waitcnt(0x0F75); break;
        case 6: __builtin_amdgcn_s_waitcnt(0x0F76); break;
        case 7: __builtin_amdgcn_s_waitcnt(0x0F77); break;
        case 8: __builtin_amdgcn_s_waitcnt(0x0F78); break;
        case 9: __builtin_amdgcn_s_waitcnt(0x0F79); break;
        case 10: __builtin_amdgcn_s_waitcnt(0x0F7A); break;
        case 11: __builtin_amdgcn_s_waitcnt(0x0F7B); break;
        case 12: __builtin_amdgcn_s_waitcnt(0x0F7C); break;
        case 13: __builtin_amdgcn_s_waitcnt(0x0F7D); break;
        case 14: __builtin_amdgcn_s_waitcnt(0x0F7E); break;
        default: __builtin_amdgcn_s_waitcnt(0x0F7F); break;   // 15
    }
}

template <bool kG>
__device__ void m_stream(const Params& P, Lds& L, uint32_t epoch) {
    constexpr int K = kG ? kHidden : kInter;            // 2048 / 1408 per item
    constexpr int S = kG ? 8 : 6;                       // slices per item (D: 5 and a half)
    constexpr int KS = kG ? 32 : 24;                    // fragments per wave
    static_assert(KS <= kBMax && S % 2 == 0 && 2 * kRing <= 16, "stream shape");
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // uniform
    const int lane = threadIdx.x & (kLanes - 1);
    const int tt = wave & 3, kh = wave >> 2;
    int n_items = 0;
    {
        MRef r;
        while (m_item_n<kG>(L, n_items, r)) ++n_items;
    }
    if (n_items == 0) return;
    const int total = n_items * S;
    uint8_t* ring = L.ring;
    float* xch = reinterpret_cast<float*>(ring + kRing * kSliceA);   // [4 waves][8][64]

    // this wave's two 1 KB copies of a slice: rows 4 wave + 2 c + lane / 32;
    // the item's row base is looked up once per item (the copies of one item
    // are issued in order)
    int is_item = -1, is_ld = K;
    const uint8_t* is_rows = nullptr;
    auto issue = [&](int g) {
        const int item = g / S, s = g - item * S;
        if (item != is_item) {
            MRef r;
            m_item_n<kG>(L, item, r);
            is_rows = reinterpret_cast<const uint8_t*>(m_rows<kG>(P, L.unit[r.unit], r, is_ld));
            is_item = item;
        }
        const bool half = !kG && s == S - 1;
        uint8_t* dst = ring + (g % kRing) * kSliceA;
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            const int row = 4 * wave + 2 * c + (lane >> 5);
            const int key = row & 15, p = lane & 31;
            const uint8_t* src = is_rows + (int64_t)row * is_ld * 2 + kRowSlice * s;
            const int chunk = half ? ((p & 15) ^ key) : (p ^ key);
            __builtin_amdgcn_global_load_lds(src + chunk * 16, dst + (4 * wave + 2 * c) * kRowSlice,
                                             16, 0, 0);
        }
    };

    u32x4 bf[KS];
    MRef cur{-1, -1, -1, -1}, done{-1, -1, -1, -1};
    f32x4 acc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
    bool live = false;
    // phase D: where this lane's token of the current (unit, pass, half)
    // publishes (first word of its routed (token, slot) partial, or of its
    // shared half's fp32 sums) and its routing weight, set with the operand
    // so that the epilogue reads no memory but the exchange area (a global
    // or LDS-table load there would wait for the ring copies in flight); the
    // dn_ copies belong to the finished item whose epilogue is pending, as
    // the operand may already be the next unit's
    bool ep_ok = false, ep_sh = false, dn_ok = false, dn_sh = false;
    int64_t ep_base = 0, dn_base = 0;
    float ep_w = 1.f, dn_w = 1.f;

    // even-parity waves: the finished item's total and its outputs
    auto epilogue = [&](const MRef& r) {
        const int q = lane >> 4, j = lane & 15, jj = 16 * tt + j;
        int j0 = 0, m = 0;
        if (kG) {
            j0 = kMGroup * r.pass;
            m = min(kMGroup, L.unit[r.unit].m - j0);
            if (jj >= m) return;
        } else if (!dn_ok) {
            return;
        }
#pragma unroll
        for (int rt = 0; rt < 2; ++rt) {
            const float* o = xch + ((tt * 2 + rt) * 4) * kLanes + lane;
            const float t0 = acc[rt][0] + o[0], t1 = acc[rt][1] + o[kLanes];
            const float t2 = acc[rt][2] + o[2 * kLanes], t3 = acc[rt][3] + o[3 * kLanes];
            if (kG) {
                const Unit& u = L.unit[r.unit];
                P.hp[u.h_off + (int64_t)(j0 + jj) * (gpairs_of(u) / 2) + 8 * r.rb + 4 * rt + q] =
                    pack_bf16(bf16r(bf16r(silu_rn(bf16r(t0))) * bf16r(t1)),
                              bf16r(bf16r(silu_rn(bf16r(t2))) * bf16r(t3)));
            } else if (dn_sh) {
                // fp32 sums of rows 32 rb + 16 rt + 4 q + v
                uint64_t* o2 = P.sp + dn_base + 32 * r.rb + 16 * rt + 4 * q;
                st_word(o2, epoch, __float_as_uint(t0));
                st_word(o2 + 1, epoch, __float_as_uint(t1));
                st_word(o2 + 2, epoch, __float_as_uint(t2));
                st_word(o2 + 3, epoch, __float_as_uint(t3));
            } else {
                // words of rows (2 w0, 2 w0 + 1) and (2 w0 + 2, 2 w0 + 3):
                // bf16(w * bf16(d)), as put_part
                const int w0 = 16 * r.rb + 8 * rt + 2 * q;
                st_word(P.part + dn_base + w0, epoch, pack_bf16(dn_w * bf16r(t0), dn_w * bf16r(t1)));
                st_word(P.part + dn_base + w0 + 1, epoch,
                        pack_bf16(dn_w * bf16r(t2), dn_w * bf16r(t3)));
            }
        }
    };

    int issued = 0;
    for (int item = 0; item < n_items; ++item) {
        MRef r;
        m_item_n<kG>(L, item, r);
        if (r.unit != cur.unit || r.pass != cur.pass || r.half != cur.half) {
            // new token operand: everything in flight lands first, so the
            // slice waits below stay exact
            wait_vm(0);
            const Unit& u = L.unit[r.unit];
            const int j0 = kMGroup * r.pass;
            const int m = min(kMGroup, u.m - j0);
            live = 16 * tt < m;
            const int t = 16 * tt + (lane & 15);
            const int tc = j0 + (t < m ? t : 0);
            const uint16_t* row;
            if (kG) {
                row = P.x + (int64_t)token_of(L, u, tc) * kHidden;
            } else {
                row = reinterpret_cast<const uint16_t*>(P.hp + u.h_off) +
                      (int64_t)tc * gpairs_of(u) + r.half * kInter;
                ep_ok = t < m;
                ep_sh = u.expert < 0;
                if (ep_sh) {
                    ep_base = ((int64_t)tc * 2 + r.half) * kHidden;
                    ep_w = 1.f;
                } else {
                    const int e = L.ent[u.tok0 + tc];
                    const int tok = e / kTopK;
                    ep_base = ((int64_t)tok * kSlots + (e - tok * kTopK)) * kPartWords;
                    ep_w = P.weights[e];
                }
            }
            // (a wave whose token tile holds no token of the pass loads none)
#pragma unroll
            for (int f = 0; f < KS; ++f) {
                const int sl = kh + 2 * (f >> 3), ks = f & 7;
                const int e = kKs * sl + 32 * ks + 8 * (lane >> 4);
                bf[f] = live && e < K ? *reinterpret_cast<const u32x4*>(row + e)
                                      : u32x4{0u, 0u, 0u, 0u};
            }
            // the operand is complete from here on (an explicit wait the
            // compiler accounts for, so it adds none before the MFMAs, where
            // slice copies of unknown count are in flight)
            wait_vm(0);
            cur = r;
        }
        if (item == 0)   // the ring fills behind the first operand, not before it
            for (; issued < total && issued < kRing; ++issued) issue(issued);
        // step j: slices 2j (even-parity waves) and 2j + 1 (odd) of the item
#pragma unroll
        for (int j = 0; j < S / 2; ++j) {
            const int g0 = item * S + 2 * j;
            // this wave's copies of both slices have landed when at most the
            // later slices' copies are outstanding (copies complete in order)
            wait_vm(2 * (issued - g0 - 2));
            lds_barrier();
            if (j == 0 && item > 0 && kh == 0) epilogue(done);
            // the slots of the previous step are free: keep the ring full
            while (issued < total && issued < g0 + kRing) issue(issued++);
            if (j == 0) acc[0] = acc[1] = f32x4{0.f, 0.f, 0.f, 0.f};
            if (live) {
                const uint8_t* base = ring + ((g0 + kh) % kRing) * kSliceA;
                const int rr = lane & 15, kq = lane >> 4;
                const int nks = (!kG && j == S / 2 - 1 && kh == 1) ? 4 : 8;   // the half slice
#pragma unroll
                for (int rt = 0; rt < 2; ++rt) {
                    u32x4 a[8];
#pragma unroll
                    for (int ks = 0; ks < 8; ++ks)
                        a[ks] = *reinterpret_cast<const u32x4*>(
                            base + (16 * rt + rr) * kRowSlice + (((4 * ks + kq) ^ rr) * 16));
#pragma unroll
                    for (int ks = 0; ks < 8; ++ks)
                        if (ks < nks) acc[rt] = mfma16(a[ks], bf[8 * j + ks], acc[rt]);
                }
            }
            if (j == S / 2 - 1) {
                if (kh == 1) {
                    float* o = xch + ((tt * 2) * 4) * kLanes + lane;
#pragma unroll
                    for (int rt = 0; rt < 2; ++rt)
#pragma unroll
                        for (int i = 0; i < 4; ++i) o[(rt * 4 + i) * kLanes] = acc[rt][i];
                }
                done = r;
                dn_ok = ep_ok;
                dn_sh = ep_sh;
                dn_base = ep_base;
                dn_w = ep_w;
            }
        }
    }
    lds_barrier();
    if (kh == 0) epilogue(done);
    __syncthreads();    // the ring and the staging area are reused afterwards
}

// h rows of a VALU unit (plain words, written by the previous launch) into
// LDS as bf16 [m][I].
__device__ void stage_h_plain(const Params& P, const Unit& u, uint8_t* stage) {
    const int n = u.m * gpairs_of(u) / 8;      // 16-byte chunks
    const u32x4* src = reinterpret_cast<const u32x4*>(P.hp + u.h_off);
    for (int k = threadIdx.x; k < n; k += kThreads) reinterpret_cast<u32x4*>(stage)[k] = src[k];
}

// Poll the unit's h words [j0, j0 + m) x [0, K / 2) until all carry `epoch`
// (all threads of the workgroup share the words); when `stage` is not null the
// bf16 payloads are written there as [m][K]. Returns false on timeout.
__device__ bool poll_h(const Params& P, const Unit& u, int j0, int m, uint8_t* stage,
                       uint32_t epoch) {
    const int wpt = gpairs_of(u) / 2;
    const int n = m * wpt / 2;             // 16-byte units (two words)
    const __amdgpu_buffer_rsrc_t rs = rsrc(P.h + u.h_off + (int64_t)j0 * wpt);
    bool ok = true;
    for (int k = threadIdx.x; k < n; k += kThreads) {
        u32x4 v;
        uint32_t it = 0;
        for (;; ++it) {
            v = ld_dev16(rs, 16 * k);
            if (v.y == epoch && v.w == epoch) break;
            if (it >= kSpinLimit || ((it & 1023) == 1023 && step_failed(P.hdr))) {
                ok = false;
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
        if (!ok) break;
        if (stage) reinterpret_cast<uint2*>(stage)[k] = make_uint2(v.x, v.z);
    }
    if (!ok) flag_abort(P.hdr, FLEET_MOE_ABORT_GROUP_WAIT);
    return ok;
}

// ---------------------------------------------------------------- kernel

__device__ __forceinline__ bool item_at(const Seg* S, int ns, int t, int& s, int& i) {
    for (s = 0; s < ns; ++s)
        if (t < S[s].base + (S[s].hi - S[s].lo)) {
            i = S[s].lo + (t - S[s].base);
            return true;
        }
    return false;
}

__device__ __forceinline__ void g_item_v_any(const Params& P, Lds& L, const Unit& u, int i,
                                             const uint8_t* xs, uint32_t epoch) {
    if (u.m == 1) g_item_v<1>(P, L, u, i, xs, epoch);
    else if (u.m == 2) g_item_v<2>(P, L, u, i, xs, epoch);
    else if (u.m <= 4) g_item_v<4>(P, L, u, i, xs, epoch);
    else g_item_v<8>(P, L, u, i, xs, epoch);
}

__device__ __forceinline__ void d_item_v_any(const Params& P, Lds& L, const Unit& u, int i,
                                             const uint8_t* hs, uint32_t epoch) {
    if (u.expert < 0) {
        if (u.m == 1) d_item_v<1, true, 4>(P, L, u, i, hs, epoch);
        else if (u.m == 2) d_item_v<2, true, 4>(P, L, u, i, hs, epoch);
        else if (u.m <= 4) d_item_v<4, true, 4>(P, L, u, i, hs, epoch);
        else d_item_v<8, true, 2>(P, L, u, i, hs, epoch);
    } else {
        if (u.m == 1) d_item_v<1, false, 8>(P, L, u, i, hs, epoch);
        else if (u.m == 2) d_item_v<2, false, 8>(P, L, u, i, hs, epoch);
        else if (u.m <= 4) d_item_v<4, false, 8>(P, L, u, i, hs, epoch);
        else d_item_v<8, false, 4>(P, L, u, i, hs, epoch);
    }
}

// VALU items of a phase, one per wave from the LDS ticket (MFMA segments are
// skipped: the whole workgroup has run them already).
template <bool kG>
__device__ void v_items(const Params& P, Lds& L, uint32_t epoch) {
    const Seg* S = kG ? L.gseg : L.dseg;
    const int ns = kG ? L.n_gseg : L.n_dseg;
    int* next = kG ? &L.gnext : &L.dnext;
    const int limit = kG ? L.g_items : L.d_items;
    for (;;) {
        const int t = claim(next, limit);
        if (t < 0) break;
        int s, i;
        if (!item_at(S, ns, t, s, i)) break;
        const Seg& sg = S[s];
        const Unit& u = L.unit[sg.unit];
        if (!is_v(u.m) || sg.stage < 0) continue;
        if (kG) g_item_v_any(P, L, u, i, L.stage + sg.stage, epoch);
        else d_item_v_any(P, L, u, i, L.stage + sg.stage, epoch);
    }
}

// x rows of this workgroup's VALU units of phase G into their LDS slots.
__device__ void stage_x(const Params& P, Lds& L) {
    for (int s = 0; s < L.n_gseg; ++s) {
        const Seg& sg = L.gseg[s];
        if (sg.stage < 0) continue;
        const Unit& u = L.unit[sg.unit];
        u32x4* dst = reinterpret_cast<u32x4*>(L.stage + sg.stage);
        for (int k = threadIdx.x; k < u.m * kRowChunks; k += kThreads) {
            const int j = k / kRowChunks, c = k - j * kRowChunks;
            dst[k] = reinterpret_cast<const u32x4*>(P.x + (int64_t)token_of(L, u, j) * kHidden)[c];
        }
    }
}

// Phase C: the 4T output words of this workgroup. kSplit (two launches): the
// shared expert's value of a row is bf16(lo + hi) of its two fp32 K-half
// sums; otherwise it is the bf16 partial of slot 6.
template <bool kSplit>
__device__ void combine(const Params& P, uint32_t epoch) {
    Header* hdr = P.hdr;
    const int nw = P.T * (kPartWords / kWG);
    constexpr int NS = kSplit ? kTopK : kSlots;
    const __amdgpu_buffer_rsrc_t rp = rsrc(P.part);
    const __amdgpu_buffer_rsrc_t rs = rsrc(kSplit ? P.sp : P.part);
    for (int k = threadIdx.x; k < nw; k += kThreads) {
        const int g = blockIdx.x * nw + k;
        const int t = g / kPartWords, w = g - t * kPartWords;
        uint32_t pay[kSlots];
        bool ready = false;
        for (uint32_t it = 0; !ready; ++it) {
            ready = true;
#pragma unroll
            for (int s = 0; s < NS; ++s) {
                const int o = (((t * kSlots + s) * kPartWords) + w) * 8;
                const uint2 v =
                    __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rp, o, 0, 16));
                pay[s] = v.x;
                ready &= v.y == epoch;
            }
            if (kSplit) {
                // rows 2w, 2w + 1 of each K half: one 16-byte load of two words
                const u32x4 lo = ld_dev16(rs, ((t * 2) * kHidden + 2 * w) * 8);
                const u32x4 hi = ld_dev16(rs, ((t * 2 + 1) * kHidden + 2 * w) * 8);
                ready &= lo.y == epoch && lo.w == epoch && hi.y == epoch && hi.w == epoch;
                pay[kTopK] = pack_bf16(__uint_as_float(lo.x) + __uint_as_float(hi.x),
                                       __uint_as_float(lo.z) + __uint_as_float(hi.z));
            }
            if (!ready) {
                if (it >= kSpinLimit || ((it & 1023) == 1023 && step_failed(hdr))) {
                    flag_abort(hdr, FLEET_MOE_ABORT_GROUP_WAIT);
                    break;
                }
                __builtin_amdgcn_s_sleep(1);
            }
        }
        float y0 = 0.f, y1 = 0.f;
#pragma unroll
        for (int s = 0; s < kTopK; ++s) {
            y0 += bf_lo(pay[s]);
            y1 += bf_hi(pay[s]);
        }
        const float o0 = bf16r(bf16r(y0) + bf_lo(pay[kTopK]));
        const float o1 = bf16r(bf16r(y1) + bf_hi(pay[kTopK]));
        reinterpret_cast<uint32_t*>(P.out)[(int64_t)t * kPartWords + w] = pack_bf16(o0, o1);
    }
}

// The last workgroup to exit publishes the epoch the next call starts from.
// After the call numbered 2^32 - 1 the tags would wrap (and tag 0 is what a
// zero-filled word carries), so that workgroup first clears every tagged word
// and restarts the count from 0, which leaves the workspace as it was when
// new; the next launch on the stream starts after this one has finished.
// (The flag for that call lives in the workgroup's Lds: a __shared__ variable
// of its own beside it moved the Lds and made the two-launch step's MFMA
// streaming ~9 us slower at 64 tokens.)
__device__ void exit_epoch(const Params& P, Lds& L, uint32_t epoch) {
    Header* hdr = P.hdr;
    __syncthreads();
    if (epoch != 0xffffffffu) {
        if (threadIdx.x == 0) {
            const uint32_t old = __hip_atomic_fetch_add(&hdr->exits, 1u, __ATOMIC_RELAXED,
                                                        __HIP_MEMORY_SCOPE_AGENT);
            if (old + 1u == epoch * (uint32_t)kWG) st_agent(&hdr->epoch, epoch);
        }
        return;
    }
    if (threadIdx.x == 0) {
        const uint32_t old = __hip_atomic_fetch_add(&hdr->exits, 1u, __ATOMIC_RELAXED,
                                                    __HIP_MEMORY_SCOPE_AGENT);
        L.exit_last = old + 1u == epoch * (uint32_t)kWG;
    }
    __syncthreads();
    if (!L.exit_last) return;
    u32x4* w = reinterpret_cast<u32x4*>(reinterpret_cast<char*>(hdr) + sizeof(Header));
    const u32x4 z = {0u, 0u, 0u, 0u};
    for (size_t i = threadIdx.x; i < P.ws_tail16; i += kThreads) w[i] = z;
    __syncthreads();
    if (threadIdx.x == 0) {
        st_agent(&hdr->exits, 0u);
        st_agent(&hdr->epoch, 0u);
    }
}

// T <= 8: G -> D -> C in one launch, h as tagged words.
__global__ __launch_bounds__(kThreads, 1) void grouped_fused_kernel(Params P) {
    __shared__ Lds L;
    Header* hdr = P.hdr;
    const uint32_t epoch = ld_agent(&hdr->epoch) + 1u;
    build_tables<true, true>(P, L);
    stage_x(P, L);
    __syncthreads();
    v_items<true>(P, L, epoch);
    __syncthreads();
    for (int s = 0; s < L.n_dseg; ++s) {
        const Seg& sg = L.dseg[s];
        if (sg.stage >= 0) poll_h(P, L.unit[sg.unit], 0, L.unit[sg.unit].m, L.stage + sg.stage, epoch);
    }
    __syncthreads();
    v_items<false>(P, L, epoch);
    combine<false>(P, epoch);
    exit_epoch(P, L, epoch);
}

// T > 8, launch 1: phase G, h as plain words.
__global__ __launch_bounds__(kThreads, 1) void grouped_g_kernel(Params P) {
    __shared__ Lds L;
    build_tables<true, false>(P, L);
    if (blockIdx.x == 0) store_tables(P, L);
    m_stream<true>(P, L, 0);
    stage_x(P, L);
    __syncthreads();
    v_items<true>(P, L, 0);
}

// T > 8, launch 2: phases D and C.
__global__ __launch_bounds__(kThreads, 1) void grouped_dc_kernel(Params P) {
    __shared__ Lds L;
    Header* hdr = P.hdr;
    const uint32_t epoch = ld_agent(&hdr->epoch) + 1u;
    load_tables<false, true>(P, L);
    m_stream<false>(P, L, epoch);
    for (int s = 0; s < L.n_dseg; ++s) {
        const Seg& sg = L.dseg[s];
        if (sg.stage >= 0) stage_h_plain(P, L.unit[sg.unit], L.stage + sg.stage);
    }
    __syncthreads();
    v_items<false>(P, L, epoch);
    combine<true>(P, epoch);
    exit_epoch(P, L, epoch);
}

}  // namespace grouped
}  // namespace fleet_moe

using namespace fleet_moe;

int fleet_moe_check_dims(const fleet_moe_dims* d);
int fleet_moe_check_device(int min_cus);
int fleet_moe_check_resident(const void* fn, int threads, int grid);

static bool aligned(const void* p, size_t a) { return ((uintptr_t)p % a) == 0; }

extern "C" size_t fleet_moe_grouped_workspace_bytes(const fleet_moe_dims* dims, int32_t max_tokens) {
    if (fleet_moe_check_dims(dims) != 0) return 0;
    if (max_tokens < 1 || max_tokens > grouped::kMaxTokens) return 0;
    return grouped::layout(max_tokens).total;
}

// Argument checks shared by both entry points (everything but the workspace).
static int check_grouped_args(const fleet_moe_layer* layer, int32_t n_tokens, const int32_t* ids,
                              const float* weights, const uint16_t* x_norm, uint16_t* out,
                              const fleet_moe_dims* dims) {
    if (!layer || !dims) return FLEET_MOE_ERR_ARG;
    if (int e = fleet_moe_check_dims(dims)) return e;
    if (!layer->experts || !layer->shared || !ids || !weights || !x_norm || !out)
        return FLEET_MOE_ERR_ARG;
    if (n_tokens < 1 || n_tokens > grouped::kMaxTokens) return FLEET_MOE_ERR_ARG;
    if (!aligned(layer->experts, 16) || !aligned(layer->shared, 16) || !aligned(x_norm, 16) ||
        !aligned(out, 4) || !aligned(ids, 4) || !aligned(weights, 4))
        return FLEET_MOE_ERR_ARG;
    if (layer->expert_stride < kExpertStride || layer->expert_stride % kChunk != 0)
        return FLEET_MOE_ERR_DIMS;
    return 0;
}

// Every grouped kernel waits on other workgroups (tagged words) except launch
// 1 of a two-launch step; all three are checked so either plan can run.
static int check_grouped_resident() {
    using namespace grouped;
    if (int e = fleet_moe_check_resident(reinterpret_cast<const void*>(&grouped_fused_kernel),
                                         kThreads, kWG))
        return e;
    if (int e = fleet_moe_check_resident(reinterpret_cast<const void*>(&grouped_g_kernel),
                                         kThreads, kWG))
        return e;
    return fleet_moe_check_resident(reinterpret_cast<const void*>(&grouped_dc_kernel), kThreads,
                                    kWG);
}

// Enqueue the step on a workspace laid out for `max_tokens` (arguments checked).
static int launch_grouped(const fleet_moe_layer* layer, int32_t n_tokens, const int32_t* ids,
                          const float* weights, const uint16_t* x_norm, uint16_t* out,
                          char* ws, int max_tokens, hipStream_t stream) {
    const grouped::Layout L = grouped::layout(max_tokens);
    grouped::Params P;
    P.experts = layer->experts;
    P.shared = layer->shared;
    P.expert_stride = layer->expert_stride;
    P.ids = ids;
    P.weights = weights;
    P.x = x_norm;
    P.out = out;
    P.hdr = reinterpret_cast<grouped::Header*>(ws);
    P.h = reinterpret_cast<uint64_t*>(ws + L.h);
    P.part = reinterpret_cast<uint64_t*>(ws + L.part);
    P.sp = reinterpret_cast<uint64_t*>(ws + L.sp);
    P.tab = reinterpret_cast<grouped::Tab*>(ws + L.tab);
    P.ws_tail16 = (L.total - sizeof(grouped::Header)) / 16;
    P.T = n_tokens;
    if (n_tokens <= grouped::kVMax) {
        P.hp = nullptr;
        hipLaunchKernelGGL(grouped::grouped_fused_kernel, dim3(grouped::kWG),
                           dim3(grouped::kThreads), 0, stream, P);
    } else {
        P.hp = reinterpret_cast<uint32_t*>(ws + L.hp);
        hipLaunchKernelGGL(grouped::grouped_g_kernel, dim3(grouped::kWG), dim3(grouped::kThreads),
                           0, stream, P);
        hipLaunchKernelGGL(grouped::grouped_dc_kernel, dim3(grouped::kWG),
                           dim3(grouped::kThreads), 0, stream, P);
    }
    return (int)hipGetLastError();
}

extern "C" int fleet_moe_grouped(const fleet_moe_layer* layer, int32_t n_tokens,
                                 const int32_t* ids, const float* weights,
                                 const uint16_t* x_norm, uint16_t* out, void* workspace,
                                 size_t workspace_bytes, const fleet_moe_dims* dims,
                                 hipStream_t stream) {
    if (int e = check_grouped_args(layer, n_tokens, ids, weights, x_norm, out, dims)) return e;
    if (!workspace || !aligned(workspace, 256)) return FLEET_MOE_ERR_ARG;
    // The workspace is laid out for the max_tokens it was sized for; recover it.
    int max_tokens = 0;
    for (int t = grouped::kMaxTokens; t >= 1; --t)
        if (grouped::layout(t).total <= workspace_bytes) { max_tokens = t; break; }
    if (max_tokens < n_tokens) return FLEET_MOE_ERR_WORKSPACE;
    if (int e = check_grouped_resident()) return e;
    return launch_grouped(layer, n_tokens, ids, weights, x_norm, out,
                          static_cast<char*>(workspace), max_tokens, stream);
}

// ------------------------------------------------- the variant that allocates nothing
//
// fleet_moe_grouped_noalloc runs the same kernels on `scratch`, a file-scope
// device array laid out exactly like a caller workspace sized for
// kScratchTokens tokens. Each device holds its own copy at its own address;
// host code never passes the array's name to a kernel (on the host it is only
// a stand-in for the symbol), only the per-device address that
// hipGetSymbolAddress returns at the first call on that device.
namespace fleet_moe {
namespace grouped {

constexpr int kScratchTokens = 64;
constexpr size_t kScratchBytes = layout(kScratchTokens).total;   // 7,574,528 B

__global__ __launch_bounds__(256) void scratch_clear_kernel(u32x4* p, size_t n16) {
    const u32x4 z = {0u, 0u, 0u, 0u};
    for (size_t i = blockIdx.x * (size_t)256 + threadIdx.x; i < n16; i += gridDim.x * (size_t)256)
        p[i] = z;
}

// Reads and clears the step's status word (ordered after the step's kernels
// on the stream, so it sees every bit they raised).
__global__ void status_take_kernel(Header* hdr, uint32_t* status) {
    if (threadIdx.x == 0)
        status[0] = __hip_atomic_exchange(&hdr->abort, 0u, __ATOMIC_RELAXED,
                                          __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace grouped
}  // namespace fleet_moe

static __device__ __align__(256) uint8_t scratch[grouped::kScratchBytes];

namespace {
std::mutex g_scratch_mu;
std::vector<char*> g_scratch;   // per device: the address of `scratch`, once set up
}  // namespace

// The calling thread's current device's copy of `scratch`. At the first call on
// a device: look up its address and zero it (a fill kernel on `stream`, then a
// synchronize, so later calls on any stream see it cleared). That first call
// must not be under graph capture.
static int scratch_of_current_device(hipStream_t stream, char** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return (int)e;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if ((int)g_scratch.size() <= dev) g_scratch.resize(dev + 1, nullptr);
    if (!g_scratch[dev]) {
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        e = hipStreamIsCapturing(stream, &cs);
        if (e != hipSuccess) return (int)e;
        if (cs != hipStreamCaptureStatusNone) return FLEET_MOE_ERR_CAPTURE;
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return (int)e;
        if (!p || !aligned(p, 256)) return FLEET_MOE_ERR_DEVICE;
        hipLaunchKernelGGL(grouped::scratch_clear_kernel, dim3(1024), dim3(256), 0, stream,
                           static_cast<u32x4*>(p), grouped::kScratchBytes / 16);
        e = hipGetLastError();
        if (e == hipSuccess) e = hipStreamSynchronize(stream);
        if (e != hipSuccess) return (int)e;
        g_scratch[dev] = static_cast<char*>(p);
    }
    *out = g_scratch[dev];
    return 0;
}

extern "C" int fleet_moe_grouped_noalloc(const fleet_moe_layer* layer, int32_t n_tokens,
                                         const int32_t* ids, const float* weights,
                                         const uint16_t* x_norm, uint16_t* out,
                                         uint32_t* status, const fleet_moe_dims* dims,
                                         hipStream_t stream) {
    if (int e = check_grouped_args(layer, n_tokens, ids, weights, x_norm, out, dims)) return e;
    if (!status || !aligned(status, 4)) return FLEET_MOE_ERR_ARG;
    if (n_tokens > grouped::kScratchTokens) return FLEET_MOE_ERR_CAPACITY;
    if (int e = check_grouped_resident()) return e;
    char* ws = nullptr;
    if (int e = scratch_of_current_device(stream, &ws)) return e;
    if (int e = launch_grouped(layer, n_tokens, ids, weights, x_norm, out, ws,
                               grouped::kScratchTokens, stream))
        return e;
    hipLaunchKernelGGL(grouped::status_take_kernel, dim3(1), dim3(64), 0, stream,
                       reinterpret_cast<grouped::Header*>(ws), status);
    return (int)hipGetLastError();
}
