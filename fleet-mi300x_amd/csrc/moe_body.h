// Device code of the batch-1 MoE layer, shared by its own launch
// (moe_decode.hip) and the whole-step kernel (step_decode.hip).
//
// Batch-1 MoE layer for DeepSeek-V2-Lite on MI355X (gfx950): RMSNorm, router,
// greedy top-6, six routed SwiGLU experts, the merged shared expert, the
// weighted combine and the bf16 residual add, in ONE launch of 256
// workgroups (one per CU, 8 waves each).
//
// What it replaces in the reference: the NORM_ROUTER / EXPERT_GATE_UP /
// EXPERT_DOWN task bodies of the persistent decode kernel
// (src/kernels/fleet_kernel.hip:398-456, 469-500, 826-889, built on
// src/kernels/expert.h and gemv.h) and the fold of the eight expert partials
// in the next layer's prologue (fleet_kernel.hip:146-201). The reference
// gives each of its 8 XCDs one 17.3 MB "unit" and synchronises with XCD-local
// and global events; this kernel spreads every gate/up row pair of all seven
// experts over all 256 CUs and keeps cross-CU communication off the critical
// path:
//
//   routing: every workgroup computes all 64 router logits itself from L2
//     (bf16 dot2, fp32 accumulate) together with a rigorous error bound, and
//     selects the top 6. If the gap between the 6th and 7th logit exceeds
//     twice the bound, that set is provably the exact one and routed
//     streaming starts at once; otherwise (a near tie, ~1% of tokens) the
//     workgroup waits for the exact logits below. Independently, the control
//     wave of workgroups 0..63 computes one router row exactly (fp64 sum of
//     the exact bf16 x bf16 products, rounded once) and publishes it; the
//     routing weights and the slot order come from those exact logits, and
//     they are only needed at the final combine.
//   phase G (gate/up): the 11,264 row pairs of [shared | routed slot 0..5]
//     are dealt round-robin to the 256 workgroups (44 pairs each, the first
//     11 of them shared and routing-independent). Seven streaming waves pull
//     pairs from an LDS ticket; a pair is 8 x 16-byte non-temporal loads per
//     lane against x_norm (bf16 pairs in registers);
//     h = bf16(bf16(silu(bf16(g))) * bf16(u)), every dot exactly rounded
//     (an fp32 evaluation certified by an error bound, fp64 when the bound
//     cannot decide).
//   phase D (down + combine): workgroup w owns output rows [8w, 8w+8). Waves
//     0..5 take routed slot 0..5 for the 8 rows (8 x 2,816 B), waves 6..7 the
//     shared expert's rows (4 x 5,632 B each): 22.5 KB per wave, issued
//     before the wave waits for its unit's h. The seven row dots of a row are
//     combined in the owning workgroup's LDS in one fixed order: no partial
//     buffers, no float atomics.
//
// Cross-workgroup data is self-validating: every h value is published as one
// 32-bit word (epoch tag << 16 | bf16 h) and every exact router logit as one
// 64-bit word (epoch << 32 | fp32 bits), written and read with device-scope
// (sc1) accesses. A consumer polls the words it needs until every tag equals
// the current call's epoch: no flags, no release fences, no L2 write-backs.
// Workgroup 0 advances the call count once it has seen every workgroup's
// tagged h. Every wait is bounded and
// records an abort reason instead of hanging.
#pragma once
#include <stddef.h>

#include "moe_common.h"

#ifndef FLEET_MOE_TRACE
#define FLEET_MOE_TRACE 0
#endif

namespace fleet_moe {
namespace decode {

constexpr int kWG = 256;                       // one workgroup per CU
constexpr int kWaves = 8;
constexpr int kThreads = kWaves * kLanes;      // 512
constexpr int kUnits = 1 + kTopK;              // unit 0 = shared, 1..6 = routed slots
constexpr int kSharedPairs = kSharedInter;     // 2816 gate/up row pairs
constexpr int kPairs = kSharedPairs + kTopK * kInter;   // 11264
constexpr int kItems = kPairs / kWG;           // 44 pairs per workgroup
constexpr int kSharedItems = kSharedPairs / kWG;   // 11
constexpr int kRowsPerWG = kHidden / kWG;      // 8 output rows per workgroup
constexpr int kCtlWave = kWaves - 1;           // control wave: exact router row, routing
constexpr int kRouterRowsPerWave = kRouted / kWaves;   // 8 local router rows per wave
constexpr int kSharedRowBytes = kSharedInter * 2;              // 5,632 B per shared down row
constexpr int kSharedBlockBytes = kRowsPerWG * kSharedRowBytes;  // 45,056 B = 44 x 1 KB
static_assert(kSharedBlockBytes % 1024 == 0, "shared down block is whole 1 KB wave loads");
static_assert(kPairs % kWG == 0 && kSharedPairs % kWG == 0, "pair split");
static_assert(kRowsPerWG == 8 && kWaves == 8, "down split assumes 8 rows x 8 waves");
static_assert(kSharedItems >= kWaves - 1, "streaming waves start on routing-independent pairs");
static_assert(kRouted <= kWG, "one exact router row per workgroup");

// Sticky status bit (beside the header's FLEET_MOE_ABORT_* bits): the locally
// selected expert set disagreed with the exact logits. The margin test makes
// this impossible; it is checked anyway.
constexpr uint32_t kAbortRouteMismatch = 0x100u;

// Device workspace (zero-filled once by the caller). The header keeps the
// offsets fleet_moe_workspace_status relies on.
struct Workspace {
    uint32_t epoch;        // calls completed on this workspace
    uint32_t pad_exits;
    uint32_t abort;        // sticky FLEET_MOE_ABORT_* bits
    uint32_t pad0[61];
    uint64_t logit[kRouted];   // (epoch << 32) | fp32 exact logit bits
    uint32_t h[kPairs];        // (epoch & 0xffff) << 16 | bf16 h; shared [0, 2816),
                               // routed slot k at 2816 + k * 1408
};
static_assert(offsetof(Workspace, abort) == 8, "status word offset");
static_assert(offsetof(Workspace, h) % 16 == 0, "h is read with 16-byte loads");

__device__ __forceinline__ int h_offset(int unit) {
    return unit == 0 ? 0 : kSharedInter + (unit - 1) * kInter;
}

struct Params {
    const uint16_t* norm;      // bf16[H] or null
    const u32x4* router;       // bf16[64][H]
    const uint16_t* experts;   // packed routed experts
    const uint16_t* shared;    // packed shared expert
    const float* x;            // fp32[H]
    float* x_out;              // fp32[H]
    uint16_t* moe_out;         // bf16[H] or null
    int32_t* ids_out;          // int32[6] or null
    float* w_out;              // fp32[6] or null
    Workspace* ws;
    int64_t expert_stride;     // elements
    float eps;
    float scaling;
    // the whole-step kernel only
    uint32_t epoch;            // this layer's call count
    const uint32_t* xin;       // tagged x [kXCopies][kHidden], or null: xin_f32
    const float* xin_f32;      // x itself (the first stage of a launch)
    uint32_t xin_tag;
    uint32_t* xout;            // tagged x_out [kXCopies][kHidden]
    uint32_t xout_tag;
    bool router_first;         // all eight router rows per wave before x (see the prologue)
#if FLEET_MOE_TRACE
    unsigned long long* trace; // [kWG][kWaves][16] s_memrealtime stamps, or null
#endif
};

#if FLEET_MOE_TRACE
#define FLEET_TRACE(k)                                                                   \
    do {                                                                                 \
        if (P.trace && (fm_tid() & 63) == 0)                                          \
            P.trace[((size_t)blockIdx.x * kWaves + (fm_tid() >> 6)) * 16 + (k)] =     \
                __builtin_amdgcn_s_memrealtime();                                        \
    } while (0)
#else
#define FLEET_TRACE(k) do {} while (0)
#endif

struct Lds {
    alignas(16) uint32_t xb[kHidden / 2];  // x_norm as bf16 pairs
    alignas(16) float xraw[kHidden];       // x itself (the whole-step kernel)
    double red[kWaves];
    double xsq[kWaves];
    float llog[kRouted];       // local (fp32) logits
    float lnrm[kRouted];       // local sum of squares of each router row
    int ids[8];                // slot -> expert id (slot order = local selection order)
    float w[8];                // slot -> routing weight (exact)
    int order[8];              // exact selection order: order[j] = slot
    float part[kUnits][kRowsPerWG];
    int next;
    int route;                 // 0 pending, 2 ready, 3 failed
    int sdown_ready;           // the shared down rows have landed in sdown
    alignas(16) uint8_t sdown[kSharedBlockBytes];   // this workgroup's 8 shared down rows
};

// Pair `j` of workgroup `wg`: shared pairs wg + 256 j for j < 11, then the
// routed pairs 2816 + wg + 256 (j - 11), which walk slots 0..5 in order.
__device__ __forceinline__ void item_of(int wg, int j, int& unit, int& pair) {
    if (j < kSharedItems) {
        unit = 0;
        pair = wg + kWG * j;
    } else {
        const int r = wg + kWG * (j - kSharedItems);
        unit = 1 + r / kInter;
        pair = r - (unit - 1) * kInter;
    }
}

// Polls the 64 exact router words (one per lane) until every tag is this
// call's epoch; four polls in flight. Returns false if the bound ran out.
__device__ bool poll_exact_logits(const Params& P, uint32_t epoch, float& logit) {
    const int lane = fm_tid() & (kLanes - 1);
    Workspace* ws = P.ws;
    const uint64_t* src = &ws->logit[lane];
    auto poll = [&]() {
        return __hip_atomic_load(src, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    };
    auto ready = [&](uint64_t w) { return __all((uint32_t)(w >> 32) == epoch); };
    uint64_t a = poll();
    __builtin_amdgcn_s_sleep(4);
    uint64_t b = poll();
    __builtin_amdgcn_s_sleep(4);
    uint64_t c = poll();
    __builtin_amdgcn_s_sleep(4);
    uint64_t d = poll();
    for (uint32_t it = 0; it < kSpinLimit; it += 4) {
        if (ready(a)) { logit = __uint_as_float((uint32_t)a); return true; }
        __builtin_amdgcn_s_sleep(4);
        a = poll();
        if (ready(b)) { logit = __uint_as_float((uint32_t)b); return true; }
        __builtin_amdgcn_s_sleep(4);
        b = poll();
        if (ready(c)) { logit = __uint_as_float((uint32_t)c); return true; }
        __builtin_amdgcn_s_sleep(4);
        c = poll();
        if (ready(d)) { logit = __uint_as_float((uint32_t)d); return true; }
        __builtin_amdgcn_s_sleep(4);
        d = poll();
        if ((it & 1023) == 1020 && ld_agent(&ws->abort) != 0) break;
    }
    if (lane == 0)
        __hip_atomic_fetch_or(&ws->abort, FLEET_MOE_ABORT_ROUTER_WAIT, __ATOMIC_RELAXED,
                              __HIP_MEMORY_SCOPE_AGENT);
    return false;
}

// a2 (exact): router row `row`, fp64 accumulation of the exact bf16 x bf16
// products rounded once to fp32, published as a tagged 64-bit word.
__device__ void publish_exact_row(const Params& P, const u32x4 (&er)[4], const u32x4 (&xq)[4],
                                  int row, uint32_t epoch) {
    const int lane = fm_tid() & (kLanes - 1);
    double acc = 0.0;
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        const uint32_t wv[4] = {er[m].x, er[m].y, er[m].z, er[m].w};
        const uint32_t xw[4] = {xq[m].x, xq[m].y, xq[m].z, xq[m].w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            acc += (double)(bf_lo(wv[q]) * bf_lo(xw[q]));
            acc += (double)(bf_hi(wv[q]) * bf_hi(xw[q]));
        }
    }
    acc = wave_sum64(acc);
    if (lane == 0)
        __hip_atomic_store(&P.ws->logit[row], ((uint64_t)epoch << 32) | __float_as_uint((float)acc),
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    FLEET_TRACE(8);
}

// Control wave, once the local logits are in LDS: top-7 by local logit (ties
// to the lower index). The fp32 dot2 sum of a row differs from the exact dot
// product by at most eps_row = 4 * 56 * 2^-24 * ||w_row||_2 * ||x_norm||_2
// (at most 48 roundings along a lane's chain plus 8 in the reduction,
// Cauchy-Schwarz for sum |w_i x_i|, a factor 4 of headroom). If the 6th-7th
// gap exceeds twice the largest eps, the selected set equals the exact top 6
// (and no softmax tie can reorder it: the gap is far above fp32 resolution);
// otherwise the exact logits are fetched and selected from directly.
__device__ bool select_routing(const Params& P, Lds& L, uint32_t epoch, float xnorm2,
                               bool publish_row, const u32x4 (&er)[4], const u32x4 (&xq)[4],
                               bool& exact) {
    const int lane = fm_tid() & (kLanes - 1);
    const float l = L.llog[lane];
    const float eps =
        4.0f * 56.0f * 5.9604645e-8f * __fsqrt_rn(L.lnrm[lane]) * __fsqrt_rn(xnorm2);
    const float eps_max = wave_max(eps);
    float q = l;
    float sel_val[7];
    int sel_id[7];
#pragma unroll
    for (int j = 0; j < 7; ++j) {
        const float best = wave_max(q);
        const unsigned long long hit = __ballot(q == best);
        sel_id[j] = (int)__builtin_ctzll(hit);
        sel_val[j] = best;
        if (lane == sel_id[j]) q = -INFINITY;
    }
    exact = false;
    if (sel_val[5] - sel_val[6] > 2.0f * eps_max) {
        if (lane < kTopK) {
            int id = sel_id[0];
#pragma unroll
            for (int j = 1; j < kTopK; ++j) id = lane == j ? sel_id[j] : id;
            L.ids[lane] = id;
        }
        return true;
    }
    // Near tie: every workgroup reaches the same decision, so the row owners
    // publish their exact rows before anyone waits for them.
    exact = true;
    if (publish_row) publish_exact_row(P, er, xq, blockIdx.x, epoch);
    float el;
    if (!poll_exact_logits(P, epoch, el)) return false;
    wave_softmax_topk(el, kRouted, kTopK, P.scaling, L.ids, L.w, nullptr);
    if (lane < kTopK) L.order[lane] = lane;
    return true;
}

// Exact weights and order for a locally selected set, from the exact logit
// of this lane's expert: softmax (fp64, as the standalone router computes
// it), then each slot's weight and the slots sorted by (p descending, id
// ascending), one ballot per slot. Also checks that the set is the exact
// top 6.
__device__ void exact_weights_from(const Params& P, Lds& L, float el) {
    const int lane = fm_tid() & (kLanes - 1);
    const float m = wave_max(el);
    const double e = exp((double)el - (double)m);
    const double sum = wave_sum64(e);
    const float p = (float)(e / sum);
    float pk = 0.f;
    int rk = 0;
#pragma unroll
    for (int k = 0; k < kTopK; ++k) {
        const int id = wave_bcast(L.ids[k]);
        const float q = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(p), id));
        const int rank = __popcll(__ballot(p > q || (p == q && lane < id)));
        pk = lane == k ? q : pk;
        rk = lane == k ? rank : rk;
    }
    if (lane < kTopK) {
        L.w[lane] = pk * P.scaling;
        if (rk < kTopK) L.order[rk] = lane;
        else __hip_atomic_fetch_or(&P.ws->abort, kAbortRouteMismatch, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
    }
}
// One poll of this lane's exact router word (tag = epoch in the high half).
__device__ __forceinline__ uint64_t ld_exact_logit(const Params& P) {
    return __hip_atomic_load(&P.ws->logit[fm_tid() & (kLanes - 1)], __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
}
__device__ void exact_weights(const Params& P, Lds& L, uint32_t epoch) {
    float el;
    if (poll_exact_logits(P, epoch, el)) exact_weights_from(P, L, el);
}

// Base of gate/up row pair `pair` of `unit`, as 16-byte chunks. ids are in
// [0, 64) by construction (ballot lanes / softmax lanes).
__device__ __forceinline__ const u32x4* pair_base(const Params& P, const Lds& L, int unit,
                                                  int pair) {
    const uint16_t* blk = unit == 0
        ? P.shared
        : P.experts + (int64_t)L.ids[unit - 1] * P.expert_stride;
    return reinterpret_cast<const u32x4*>(blk) + (int64_t)pair * 2 * kRowChunks;
}

__device__ __forceinline__ void issue_pair(const u32x4* base, int lane, u32x4 (&b)[8]) {
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        b[m] = ld_stream(base + lane + kLanes * m);
        b[4 + m] = ld_stream(base + kRowChunks + lane + kLanes * m);
    }
}

// Exact dot of a K = 2048 row (4 chunks per lane) with x: the fp64 sum of the
// exact products, rounded once to fp32.
__device__ __forceinline__ float exact_row2048(const u32x4* w, const u32x4 (&xq)[4]) {
    double a = 0.0;
#pragma unroll
    for (int m = 0; m < 4; ++m) a = dot8_x(w[m], xq[m], a);
    return (float)wave_sum64(a);
}
// Reduce one gate/up pair and publish its tagged h word. bf16(g) and bf16(u)
// are the exactly rounded values: the fp32 evaluation (four v_dot2 chains of
// depth 8, a two-level tree, the wave sum: 16 roundings) is certified against
// ||w|| ||x_norm||, and a row near a bf16 boundary is evaluated exactly. The
// four sums (g, u, |g row|^2, |u row|^2) are reduced together into lanes
// 0..3; lanes 0 and 1 certify g and u.
__device__ __forceinline__ void finish_pair(const Params& P, int unit, int pair,
                                            const u32x4 (&b)[8], const u32x4 (&xq)[4],
                                            uint32_t tag, float xnorm) {
    const int lane = fm_tid() & (kLanes - 1);
    float g[4], u[4], gw[4], uw[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        g[m] = dot8_d2(b[m], xq[m], 0.f);
        u[m] = dot8_d2(b[4 + m], xq[m], 0.f);
        gw[m] = dot8_d2(b[m], b[m], 0.f);
        uw[m] = dot8_d2(b[4 + m], b[4 + m], 0.f);
    }
    float v[4] = {(g[0] + g[1]) + (g[2] + g[3]), (u[0] + u[1]) + (u[2] + u[3]),
                  (gw[0] + gw[1]) + (gw[2] + gw[3]), (uw[0] + uw[1]) + (uw[2] + uw[3])};
    const float s = wave_nsum(v);                  // lane % 4: g, u, gw, uw
    const float w2 = __int_as_float(FLEET_DPP(__float_as_int(s), 0x4E));   // lane ^ 2
    float r;
    const bool ok = certify_bf16(s, w2, xnorm, cert_gamma(16), r);
    const uint64_t bad = __ballot(!ok) & 3ull;
    if (bad & 1ull) {
        const float e = bf16r(exact_row2048(b, xq));
        r = lane == 0 ? e : r;
    }
    if (bad & 2ull) {
        const float e = bf16r(exact_row2048(b + 4, xq));
        r = lane == 1 ? e : r;
    }
    const float ub = __int_as_float(FLEET_DPP(__float_as_int(r), 0xB1));   // lane ^ 1
    if (lane == 0) {
        const float h = bf16r(bf16r(silu_rn(r)) * ub);
        st_agent(&P.ws->h[h_offset(unit) + pair], tag | bf16_bits(h));
    }
}

// Poll the tagged h words of chunks c = lane + 64 m (m < NM, c < n_chunks)
// until all carry `tag`, returning the bf16 values as 16-byte chunks.
template <int NM>
__device__ bool wait_h(const Params& P, int unit, int n_chunks, uint32_t tag,
                       u32x4 (&H)[NM]) {
    const int lane = fm_tid() & (kLanes - 1);
    const __amdgpu_buffer_rsrc_t r = rsrc(P.ws->h + h_offset(unit));
    for (uint32_t it = 0;; ++it) {
        bool ok = true;
#pragma unroll
        for (int m = 0; m < NM; ++m) {
            const int c = lane + kLanes * m;
            if (c < n_chunks) {
                const u32x4 a = ld_dev16(r, 32 * c);
                const u32x4 b = ld_dev16(r, 32 * c + 16);
                ok &= (a.x & 0xffff0000u) == tag && (a.y & 0xffff0000u) == tag &&
                      (a.z & 0xffff0000u) == tag && (a.w & 0xffff0000u) == tag &&
                      (b.x & 0xffff0000u) == tag && (b.y & 0xffff0000u) == tag &&
                      (b.z & 0xffff0000u) == tag && (b.w & 0xffff0000u) == tag;
                H[m] = u32x4{(a.x & 0xffffu) | (a.y << 16), (a.z & 0xffffu) | (a.w << 16),
                             (b.x & 0xffffu) | (b.y << 16), (b.z & 0xffffu) | (b.w << 16)};
            } else {
                H[m] = u32x4{0u, 0u, 0u, 0u};
            }
        }
        if (__all(ok)) return true;
        if (it >= kSpinLimit || ((it & 1023) == 1023 && ld_agent(&P.ws->abort) != 0)) {
            if (lane == 0)
                __hip_atomic_fetch_or(&P.ws->abort, FLEET_MOE_ABORT_UNIT_WAIT, __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_AGENT);
            return false;
        }
        __builtin_amdgcn_s_sleep(1);
    }
}

// An LDS word read through inline asm: the compiler, which cannot tell the
// word from the shared down rows the control wave copies into LDS by DMA,
// would otherwise wait for every vector memory operation of the wave
// (vmcnt(0)) before reading it. For words the DMA never writes.
__device__ __forceinline__ int lds_word(const int* p) {
    const uint32_t a = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) int*)p;
    int v;
    asm volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(a) : "memory");
    return v;
}

// Any wave that needs the routing waits for the control wave's LDS
// publication (bounded, because the control wave's own waits are bounded).
__device__ __forceinline__ bool wait_routing(Lds& L) {
    int st;
    while ((st = __hip_atomic_load(&L.route, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_WORKGROUP)) < 2)
        __builtin_amdgcn_s_sleep(1);
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    return st == 2;
}

// A streaming wave's first pair (shared pair wg + 256 wave; the control wave
// has none), issued into `b`. The whole-step kernel issues it from the stage
// before this one, once that stage's last wait is done, so it is in flight
// while that stage finishes and the residual is handed over.
__device__ __forceinline__ void issue_first_pair(const uint16_t* shared, u32x4 (&b)[8]) {
    const int wave = __builtin_amdgcn_readfirstlane(fm_tid() >> 6);
    if (wave == kCtlWave) {
        // written all the same: a buffer that is not rewritten on every path
        // would stay live through the stages in between
#pragma unroll
        for (int m = 0; m < 8; ++m) b[m] = u32x4{0u, 0u, 0u, 0u};
        return;
    }
    issue_pair(reinterpret_cast<const u32x4*>(shared) +
                   (int64_t)(blockIdx.x + kWG * wave) * 2 * kRowChunks,
               fm_tid() & (kLanes - 1), b);
}

// The layer. kMega: inside the whole-step kernel (fleet_decode_step): the
// call count comes from the step (P.epoch), x from the tagged exchange buffer
// P.xin and x_out goes to the exchange buffer P.xout (and to P.x_out when
// that is not null). `pre` is the first pair's buffer; with pre_in the pair
// was issued by the stage before (otherwise here). `next` runs once this
// layer's last wait is done: the whole-step kernel issues the next stage's
// first loads there.
template <bool kMega, class Next>
__device__ __forceinline__ void moe_layer(const Params& P, Lds& L, u32x4 (&pre)[8], bool pre_in,
                                          Next&& next) {
    const int wg = blockIdx.x;
    const int tid = fm_tid();
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // uniform: branches on it are scalar
    const int lane = tid & (kLanes - 1);
    Workspace* ws = P.ws;
    const bool ctl = wave == kCtlWave;

    // Issue order matters: vmcnt retires loads in order, so the first values
    // needed (the epoch, x, the norm weight) go first. Then this wave's first four local router rows (L2-resident
    // after the first workgroup of an XCD touches them), the exact router row
    // (control wave of workgroups 0..63), then each streaming wave's first
    // shared pair.
    // the call count, written by the previous launch: a plain load (current
    // after the launch boundary; a device-scope load of one word by every
    // wave would queue at its memory channel)
    const uint32_t epoch = kMega ? P.epoch : ws->epoch + 1u;
    const uint32_t tag = (epoch & 0xffffu) << 16;
    float4 xv = make_float4(0.f, 0.f, 0.f, 0.f);
    if constexpr (!kMega) xv = reinterpret_cast<const float4*>(P.x)[tid];
    const uint2 gb = P.norm ? ld_global_u2(P.norm, tid)
                            : make_uint2(0x3f803f80u, 0x3f803f80u);   // bf16 1.0
    const int rrow0 = wave * kRouterRowsPerWave;
    u32x4 ra[4][4];
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int m = 0; m < 4; ++m)
            ra[r][m] = ld_global(P.router + (int64_t)(rrow0 + r) * kRowChunks + lane + kLanes * m);
    // The second half of the wave's router rows goes out here too in the FFN
    // column (after an FFN stage x comes late, and the rows are in by the
    // time it is normed: column 728 -> 721 us/token); otherwise after the
    // first step of the RMSNorm (after an attention stage, or in a launch of
    // its own, issuing them here is slower).
    u32x4 rb[4][4];
    const bool rb_first = kMega && P.router_first;
    if (rb_first) {
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int m = 0; m < 4; ++m)
                rb[r][m] = ld_global(P.router + (int64_t)(rrow0 + 4 + r) * kRowChunks + lane + kLanes * m);
    }
    const bool exact_row = ctl && wg < kRouted;
    u32x4 er[4];
    if (exact_row) {
#pragma unroll
        for (int m = 0; m < 4; ++m) er[m] = ld_global(P.router + (int64_t)wg * kRowChunks + lane + kLanes * m);
    }
    u32x4 (&bufA)[8] = pre;
    int cur;
    if (!(kMega && pre_in)) issue_first_pair(P.shared, bufA);
    FLEET_TRACE(0);
    {
        // (an opaque zero: with constants the whole-step kernel kept these
        // values in registers from its start, through every stage)
        int z = 0;
        asm volatile("" : "+v"(z));
        if (tid == 0) { L.next = kWaves - 1 + z; L.route = z; L.sdown_ready = z; }
        if (tid < 8) { L.ids[tid] = z; L.w[tid] = (float)z; L.order[tid] = tid; }
    }
    if constexpr (kMega) {
        // x: every workgroup's published rows (polled behind this wave's first
        // router rows and pair, which are in flight already), or the launch's
        // input vector
        if (P.xin_f32)
            xv = reinterpret_cast<const float4*>(P.xin_f32)[tid];
        else
            xv = poll_x4(P.xin + (wg % kXCopies) * kHidden, P.xin_tag, &ws->abort,
                         FLEET_MOE_ABORT_STEP_WAIT);
        reinterpret_cast<float4*>(L.xraw)[tid] = xv;
    }

    // a1: RMSNorm of x (every workgroup, identical arithmetic): fp64 sum of
    // squares in a fixed order, var = fp32(ssq / H), inv = 1 / sqrt(var + eps)
    // in correctly rounded fp32, y = bf16(bf16(x * inv) * gamma).
    double ss = (double)xv.x * xv.x + (double)xv.y * xv.y + (double)xv.z * xv.z +
                (double)xv.w * xv.w;
    ss = wave_sum64(ss);
    if (lane == 0) L.red[wave] = ss;
    __syncthreads();
    double ssq = 0.0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) ssq += L.red[w];
    const float var = (float)(ssq / (double)kHidden);
    const float inv = __fdiv_rn(1.0f, sqrt_rn(var + P.eps));
    float y[4] = {bf16r(xv.x * inv), bf16r(xv.y * inv), bf16r(xv.z * inv), bf16r(xv.w * inv)};
    y[0] = bf16r(y[0] * bf_lo(gb.x));
    y[1] = bf16r(y[1] * bf_hi(gb.x));
    y[2] = bf16r(y[2] * bf_lo(gb.y));
    y[3] = bf16r(y[3] * bf_hi(gb.y));
    L.xb[2 * tid] = bf16_bits(y[0]) | (bf16_bits(y[1]) << 16);
    L.xb[2 * tid + 1] = bf16_bits(y[2]) | (bf16_bits(y[3]) << 16);
    {
        const double q = (double)y[0] * y[0] + (double)y[1] * y[1] + (double)y[2] * y[2] +
                         (double)y[3] * y[3];
        const double qs = wave_sum64(q);
        if (lane == 0) L.xsq[wave] = qs;
    }
    // the second half of this wave's local router rows
    if (!rb_first) {
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int m = 0; m < 4; ++m)
                rb[r][m] = ld_global(P.router + (int64_t)(rrow0 + 4 + r) * kRowChunks + lane + kLanes * m);
    }
    __syncthreads();
    u32x4 xq[4];
#pragma unroll
    for (int m = 0; m < 4; ++m)
        xq[m] = reinterpret_cast<const u32x4*>(L.xb)[lane + kLanes * m];
    float xnorm;                              // ||x_norm||_2, for the certified GEMVs
    {
        double xs = 0.0;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) xs += L.xsq[w];
        xnorm = (float)__builtin_sqrt(xs);
    }
    FLEET_TRACE(1);

    // a2 (local): eight router rows per wave, dot2 with fp32 accumulation,
    // plus each row's sum of squares for the error bound; the 16 sums are
    // reduced together, lane r < 8 ending with row r's logit and lane 8 + r
    // with its sum of squares.
    {
        float v[16];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            float a = 0.f, n = 0.f;
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                a = dot8_d2(ra[r][m], xq[m], a);
                n = dot8_d2(ra[r][m], ra[r][m], n);
            }
            v[r] = a;
            v[8 + r] = n;
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            float a = 0.f, n = 0.f;
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                a = dot8_d2(rb[r][m], xq[m], a);
                n = dot8_d2(rb[r][m], rb[r][m], n);
            }
            v[4 + r] = a;
            v[12 + r] = n;
        }
        const float s = wave_nsum(v);
        if (lane < kRouterRowsPerWave) L.llog[rrow0 + lane] = s;
        else if (lane < 2 * kRouterRowsPerWave) L.lnrm[rrow0 + lane - kRouterRowsPerWave] = s;
    }

    __syncthreads();

    // Pairs of this workgroup are handed out by an LDS ticket.
    auto claim = [&]() -> int {
        int t = 0;
        if (lane == 0)
            t = __hip_atomic_fetch_add(&L.next, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        t = wave_bcast(t);
        return t < kItems ? t : -1;
    };
    auto issue = [&](int item, u32x4 (&b)[8]) {
        int u, p;
        item_of(wg, item, u, p);
        if (u != 0) wait_routing(L);
        issue_pair(pair_base(P, L, u, p), lane, b);
    };
    auto finish = [&](int item, const u32x4 (&b)[8]) {
        int u, p;
        item_of(wg, item, u, p);
        finish_pair(P, u, p, b, xq, tag, xnorm);
    };
    bool exact_sel = false, weights_pending = false;
    uint64_t ew = 0;
    cur = ctl ? -1 : wave;
    if (ctl) {
        __builtin_amdgcn_s_setprio(2);
        double xs = 0.0;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) xs += L.xsq[w];
        const bool ok = select_routing(P, L, epoch, (float)xs * 1.0001f, exact_row, er, xq,
                                       exact_sel);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
        if (lane == 0)
            __hip_atomic_store(&L.route, ok ? 2 : 3, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_WORKGROUP);
        __builtin_amdgcn_s_setprio(0);
        FLEET_TRACE(10);
        if (exact_row && !exact_sel) publish_exact_row(P, er, xq, wg, epoch);
        // This workgroup's eight shared-expert down rows (44 KB, needed in
        // phase D) go straight into LDS now. Issued any earlier they would
        // push the wave past the 63 loads a wave can have outstanding and
        // stall the RMSNorm / routing path on the first load's return.
        {
            const uint8_t* src = reinterpret_cast<const uint8_t*>(
                                     P.shared + (int64_t)2 * kSharedInter * kHidden) +
                                 (int64_t)wg * kSharedBlockBytes + lane * 16;
#pragma unroll 4
            for (int k = 0; k < kSharedBlockBytes / 1024; ++k)
                __builtin_amdgcn_global_load_lds(src + k * 1024, L.sdown + k * 1024, 16, 0, 0);
        }
        weights_pending = ok && !exact_sel;
        // In the whole-step kernel the control wave takes no pairs: its
        // copies hold its first pair back until ~13 us into the stage, and it
        // was then the workgroup's last wave to finish phase G in a third of
        // the workgroups (column 760 -> 750 us/token without it; the
        // single-layer launch is 0.2 us faster with it).
        cur = kMega ? -1 : claim();
        if (weights_pending && cur >= 0) ew = ld_exact_logit(P);
        if (cur >= 0) issue(cur, bufA);
    }
    FLEET_TRACE(2);

    // Phase G: gate/up pairs, one in flight per streaming wave. The control
    // wave also polls the exact router logits (for the weights of a locally
    // selected set) as soon as they may be published: each poll is issued
    // just before a pair's loads, so the pair's wait covers it and the wave
    // never stalls on it alone.
    // The control wave's loop (it also polls the exact logits) is kept apart
    // from the streaming waves' loop, and it consumes its last poll before
    // the paths join: a poll's destination register, possibly still loading
    // on some path, made the compiler wait for every load in flight before
    // the routed waves' down rows (vmcnt(0) on reuse of that register).
    if (ctl) {
        while (cur >= 0) {
            const int nxt = claim();
            finish(cur, bufA);
            if (weights_pending) {
                if (__all((uint32_t)(ew >> 32) == epoch)) {
                    exact_weights_from(P, L, __uint_as_float((uint32_t)ew));
                    weights_pending = false;
                } else if (nxt >= 0) {
                    ew = ld_exact_logit(P);
                }
            }
            if (nxt >= 0) issue(nxt, bufA);
            cur = nxt;
        }
        asm volatile("" ::"v"(ew));
    } else {
        while (cur >= 0) {
            const int nxt = claim();
            finish(cur, bufA);
            if (nxt >= 0) issue(nxt, bufA);
            cur = nxt;
        }
    }
    FLEET_TRACE(3);

    // Phase D: this workgroup's 8 output rows. Waves 0..5 stream routed slot
    // 0..5's rows (8 x 2,816 B), all loads in flight before the wave waits for
    // its unit's h; waves 6..7 take the shared expert's rows from LDS.
    const int row0 = wg * kRowsPerWG;
    const bool routed = wave < kTopK;
    const int unit = routed ? 1 + wave : 0;
    if (routed) {
        // the routing (published long before phase G ends) and this slot's
        // expert, read without waiting for this wave's h stores
        while (lds_word(&L.route) < 2) __builtin_amdgcn_s_sleep(1);
        const int expert = __builtin_amdgcn_readfirstlane(lds_word(&L.ids[wave]));
        u32x4 W[24];
        const u32x4* base = reinterpret_cast<const u32x4*>(
                                P.experts + (int64_t)expert * P.expert_stride +
                                (int64_t)2 * kInter * kHidden) +
                            (int64_t)row0 * kInterChunks;
        // Every lane loads all 24 chunks: lanes 48..63 read chunk 175 of the
        // row again for m = 2 (their chunk 176 + would be past the row), and
        // that copy is left out where it is used (the row norms below; in the
        // dots h is zero there), so no per-lane condition splits the issue.
        // The rows go out in three groups, rows 0-1, 2-3, then 4-7, each after
        // the one before has landed: a workgroup done with phase G early then
        // leaves more of the memory system to the workgroups still streaming
        // their pairs, whose h every workgroup waits for (all 24 loads at
        // once: single layer +0.4 us, column +12 us/token; in three groups:
        // single layer -0.2 us, column -8 us, decode step -20 us/token).
        const bool tail = lane + 2 * kLanes < kInterChunks;
#pragma unroll
        for (int r = 0; r < 8; ++r) {
            if (r == 2 || r == 4) asm volatile("" ::"v"(W[3 * r - 1].x));   // the group before has landed
#pragma unroll
            for (int m = 0; m < 3; ++m) {
                const int c = m < 2 ? lane + kLanes * m : min(lane + kLanes * m, kInterChunks - 1);
                W[3 * r + m] = ld_stream(base + r * kInterChunks + c);
            }
        }
        FLEET_TRACE(4);
        // the 8 rows' sums of squares (lane r < 8: row r), while the h this
        // wave waits for below is still being produced
        float nv[8];
#pragma unroll
        for (int r = 0; r < 8; ++r) {
            const u32x4* w = &W[3 * r];
            const float t = dot8_d2(w[2], w[2], 0.f);
            nv[r] = (dot8_d2(w[0], w[0], 0.f) + dot8_d2(w[1], w[1], 0.f)) + (tail ? t : 0.f);
        }
        const float w2 = wave_nsum(nv);
        u32x4 H[3];
        wait_h<3>(P, unit, kInterChunks, tag, H);
        FLEET_TRACE(5);
        float hv[1] = {(dot8_d2(H[0], H[0], 0.f) + dot8_d2(H[1], H[1], 0.f)) +
                       dot8_d2(H[2], H[2], 0.f)};
        const float hn = __builtin_sqrtf(wave_nsum(hv)) * 1.0001f;
        // the 8 rows' dots reduced together: lane r < 8 holds row r's
        float v[8];
#pragma unroll
        for (int r = 0; r < 8; ++r) {
            const u32x4* w = &W[3 * r];
            v[r] = (dot8_d2(w[0], H[0], 0.f) + dot8_d2(w[1], H[1], 0.f)) +
                   dot8_d2(w[2], H[2], 0.f);
        }
        const float s = wave_nsum(v);
        float d;
        const bool ok = certify_bf16(s, w2, hn, cert_gamma(16), d);  // v_dot2 chain 8, tree 2, sum 6
        const uint64_t bad = __ballot(!ok) & 0xffull;
        if (bad) {
#pragma unroll
            for (int r = 0; r < 8; ++r) {
                if (bad & (1ull << r)) {
                    double acc = 0.0;
#pragma unroll
                    for (int m = 0; m < 3; ++m) acc = dot8_x(W[3 * r + m], H[m], acc);
                    const float e = bf16r((float)wave_sum64(acc));
                    d = lane == r ? e : d;
                }
            }
        }
        if (lane < kRowsPerWG) L.part[unit][lane] = d;
    } else {
        if (ctl) {
            // the shared down rows this wave put in flight at the start
            __builtin_amdgcn_s_waitcnt(0x0F70);
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
            if (lane == 0)
                __hip_atomic_store(&L.sdown_ready, 1, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_WORKGROUP);
            // exact weights and order, if phase G ended before the exact
            // logits were seen (they are needed only by the final combine)
            if (weights_pending) exact_weights(P, L, epoch);
            FLEET_TRACE(9);
        } else {
            while (__hip_atomic_load(&L.sdown_ready, __ATOMIC_RELAXED,
                                     __HIP_MEMORY_SCOPE_WORKGROUP) == 0)
                __builtin_amdgcn_s_sleep(1);
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
        }
        FLEET_TRACE(4);
        u32x4 H[6];
        const int rs = 4 * (wave - kTopK);
        auto srow = [&](int r, u32x4 (&w)[6]) {
            const u32x4* wr = reinterpret_cast<const u32x4*>(L.sdown + (rs + r) * kSharedRowBytes);
#pragma unroll
            for (int m = 0; m < 6; ++m) {
                const int c = lane + kLanes * m;
                w[m] = c < kSharedChunks ? wr[c] : u32x4{0u, 0u, 0u, 0u};
            }
        };
        // the 4 rows' sums of squares (lane r < 4: row rs + r), while the h
        // this wave waits for below is still being produced
        float nq[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            u32x4 w[6];
            srow(r, w);
            float nv[6];
#pragma unroll
            for (int m = 0; m < 6; ++m) nv[m] = dot8_d2(w[m], w[m], 0.f);
            nq[r] = ((nv[0] + nv[1]) + (nv[2] + nv[3])) + (nv[4] + nv[5]);
        }
        const float w2 = wave_nsum(nq);
        wait_h<6>(P, unit, kSharedChunks, tag, H);
        FLEET_TRACE(5);
        float hq[6];
#pragma unroll
        for (int m = 0; m < 6; ++m) hq[m] = dot8_d2(H[m], H[m], 0.f);
        float hv[1] = {((hq[0] + hq[1]) + (hq[2] + hq[3])) + (hq[4] + hq[5])};
        const float hn = __builtin_sqrtf(wave_nsum(hv)) * 1.0001f;
        // the 4 rows' dots reduced together: lane r < 4 holds row rs + r's
        float v[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            u32x4 w[6];
            srow(r, w);
            float av[6];
#pragma unroll
            for (int m = 0; m < 6; ++m) av[m] = dot8_d2(w[m], H[m], 0.f);
            v[r] = ((av[0] + av[1]) + (av[2] + av[3])) + (av[4] + av[5]);
        }
        const float s = wave_nsum(v);
        float d;
        const bool ok = certify_bf16(s, w2, hn, cert_gamma(17), d);  // v_dot2 chain 8, tree 3, sum 6
        const uint64_t bad = __ballot(!ok) & 0xfull;
        if (bad) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                if (bad & (1ull << r)) {
                    const u32x4* wr =
                        reinterpret_cast<const u32x4*>(L.sdown + (rs + r) * kSharedRowBytes);
                    double acc = 0.0;
#pragma unroll
                    for (int m = 0; m < 6; ++m) {
                        const int c = lane + kLanes * m;
                        const u32x4 w = c < kSharedChunks ? wr[c] : u32x4{0u, 0u, 0u, 0u};
                        acc = dot8_x(w, H[m], acc);
                    }
                    const float e = bf16r((float)wave_sum64(acc));
                    d = lane == r ? e : d;
                }
            }
        }
        if (lane < 4) L.part[0][rs + lane] = d;
    }
    FLEET_TRACE(6);
    next();
    __syncthreads();

    // a7: bf16(w_k * d_k) summed in exact selection order, then the shared
    // expert and the bf16 residual add.
    if (tid < kRowsPerWG) {
        const int n = row0 + tid;
        float y = 0.f;
#pragma unroll
        for (int j = 0; j < kTopK; ++j) {
            const int k = L.order[j];
            y += bf16r(L.w[k] * L.part[1 + k][tid]);
        }
        const float out = bf16r(bf16r(y) + L.part[0][tid]);
        const float xo = bf16r((kMega ? L.xraw[n] : P.x[n]) + out);
        if (!kMega || P.x_out) P.x_out[n] = xo;
        if constexpr (kMega) publish_x(P.xout, n, xo, P.xout_tag);
        if (P.moe_out) P.moe_out[n] = (uint16_t)bf16_bits(out);
    }
    if (wg == 0 && tid < kTopK) {
        const int k = L.order[tid];
        if (P.ids_out) P.ids_out[tid] = L.ids[k];
        if (P.w_out) P.w_out[tid] = L.w[k];
    }
    // Every workgroup published h words with this call's tag (each unit's
    // pairs are spread over all of them), and this workgroup has seen all of
    // them, so every workgroup has read the call count: workgroup 0 advances
    // it for the next call (which starts after this launch has ended).
    if (!kMega && wg == 0 && tid == 0) st_agent(&ws->epoch, epoch);
    FLEET_TRACE(7);
}

}  // namespace decode
}  // namespace fleet_moe
