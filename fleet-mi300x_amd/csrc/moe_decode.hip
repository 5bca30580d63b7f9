// Batch-1 MoE layer for DeepSeek-V2-Lite on MI355X (gfx950): RMSNorm, router,
// greedy top-6, six routed SwiGLU experts, the merged shared expert, the
// weighted combine and the bf16 residual add, in ONE launch of 256
// workgroups (one per CU).
//
// What it replaces in the reference: the NORM_ROUTER / EXPERT_GATE_UP /
// EXPERT_DOWN task bodies of the persistent decode kernel
// (src/kernels/fleet_kernel.hip:398-456, 469-500, 826-889, built on
// src/kernels/expert.h and gemv.h) and the fold of the eight expert partials
// in the next layer's prologue (fleet_kernel.hip:146-201). The reference
// gives each of its 8 XCDs one 17.3 MB "unit" and synchronises with XCD-local
// and global events; this kernel spreads every gate/up row pair of all seven
// experts over all 256 CUs and orders the work so that a CU always has
// weight loads in flight while it waits on a dependency:
//
//   phase G (gate/up): the 11,264 row pairs of [shared | routed slot 0..5]
//     are dealt round-robin to the 256 workgroups (44 pairs each, the first
//     11 of them shared). Shared pairs come first: they do not depend on the
//     routing, so they stream while 64 workgroups compute one router row
//     each. Inside a workgroup, 8 waves pull pairs from an LDS ticket and
//     double-buffer them (the next pair's 8 KB is in flight while the
//     current one is reduced). A pair is 8 x 16-byte non-temporal loads per
//     lane against x_norm held in registers;
//     h = bf16(bf16(silu(bf16(g))) * bf16(u)).
//   phase D (down + combine): workgroup w owns output rows [8w, 8w+8). Waves
//     0..5 take routed slot 0..5 for the 8 rows (8 x 2,816 B), waves 6..7 the
//     shared expert's rows (4 x 5,632 B each): 22.5 KB per wave, issued
//     before the wave waits for its unit's h, so the gate/up -> down
//     dependency is hidden behind in-flight loads. The seven row dots of a
//     row are combined in the owning workgroup's LDS in one fixed order: no
//     partial buffers, no float atomics.
//
// Cross-workgroup data is self-validating: every h value is published as one
// 32-bit word (epoch tag << 16 | bf16 h) and every router logit as one 64-bit
// word (epoch << 32 | fp32 bits), written and read with device-scope
// (sc1) accesses. A consumer polls the words it needs until every tag equals
// the current call's epoch, so there are no flags, no release fences and no
// L2 write-backs; the words of the previous call carry the previous epoch.
// The last workgroup to exit advances the epoch. Every wait is bounded and
// records an abort reason instead of hanging.
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
constexpr int kRouterWave = kWaves - 1;        // wave that computes a router row
static_assert(kPairs % kWG == 0 && kSharedPairs % kWG == 0, "pair split");
static_assert(kRowsPerWG == 8 && kWaves == 8, "down split assumes 8 rows x 8 waves");
static_assert(kSharedItems >= kWaves, "every wave starts on a routing-independent pair");
static_assert(kRouted <= kWG, "one router row per workgroup");

// Device workspace (zero-filled once by the caller). The header keeps the
// offsets fleet_moe_workspace_status relies on.
struct Workspace {
    uint32_t epoch;        // calls completed on this workspace
    uint32_t exits;        // workgroup exits over all calls
    uint32_t abort;        // sticky FLEET_MOE_ABORT_* bits
    uint32_t pad0[61];
    uint64_t logit[kRouted];   // (epoch << 32) | fp32 logit bits
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
#if FLEET_MOE_TRACE
    unsigned long long* trace; // [kWG][kWaves][8] s_memrealtime stamps, or null
#endif
};

#if FLEET_MOE_TRACE
#define FLEET_TRACE(k)                                                                   \
    do {                                                                                 \
        if (P.trace && (threadIdx.x & 63) == 0)                                          \
            P.trace[((size_t)blockIdx.x * kWaves + (threadIdx.x >> 6)) * 8 + (k)] =      \
                __builtin_amdgcn_s_memrealtime();                                        \
    } while (0)
#else
#define FLEET_TRACE(k) do {} while (0)
#endif

struct Lds {
    float xn[kHidden];
    double red[kWaves];
    int ids[8];
    float w[8];
    float part[kUnits][kRowsPerWG];
    int next;
    int route;                 // 0 idle, 1 being fetched, 2 ready, 3 failed
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

__device__ __forceinline__ int wave_bcast(int v) { return __shfl(v, 0, kLanes); }

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, 0x7fffffff, 0x00020000);
}
// 16-byte device-scope (sc1) load: sees the latest values written by any CU.
__device__ __forceinline__ u32x4 ld_dev16(__amdgpu_buffer_rsrc_t r, int byte_off) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 16);
}

// First wave of the workgroup to need the routing fetches it: polls the 64
// tagged router words (one per lane) until every tag is this call's epoch,
// runs softmax + top-6 on this one wave, and publishes ids/weights to LDS.
// Other waves wait on LDS.
__device__ bool ensure_routing(const Params& P, Lds& L, uint32_t epoch) {
    const int lane = threadIdx.x & (kLanes - 1);
    int st = __hip_atomic_load(&L.route, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    if (st >= 2) return st == 2;
    int old = 0;
    if (lane == 0) {
        int expected = 0;
        __hip_atomic_compare_exchange_strong(&L.route, &expected, 1, __ATOMIC_RELAXED,
                                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        old = expected;
    }
    old = wave_bcast(old);
    if (old == 0) {
        Workspace* ws = P.ws;
        uint64_t v = 0;
        bool ok = false;
        for (uint32_t it = 0;; ++it) {
            v = __hip_atomic_load(&ws->logit[lane], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (__all((uint32_t)(v >> 32) == epoch)) { ok = true; break; }
            if (it >= kSpinLimit || ld_agent(&ws->abort) != 0) {
                if (lane == 0)
                    __hip_atomic_fetch_or(&ws->abort, FLEET_MOE_ABORT_ROUTER_WAIT,
                                          __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
        if (ok) {
            wave_softmax_topk(__uint_as_float((uint32_t)v), kRouted, kTopK, P.scaling, L.ids,
                              L.w, nullptr);
            if (lane < kTopK) {
                L.ids[lane] = min(max(L.ids[lane], 0), kRouted - 1);
                if (blockIdx.x == 0 && P.ids_out) P.ids_out[lane] = L.ids[lane];
                if (blockIdx.x == 0 && P.w_out) P.w_out[lane] = L.w[lane];
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
        if (lane == 0)
            __hip_atomic_store(&L.route, ok ? 2 : 3, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_WORKGROUP);
        return ok;
    }
    // Bounded because the fetching wave's own wait is bounded.
    while ((st = __hip_atomic_load(&L.route, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_WORKGROUP)) < 2)
        __builtin_amdgcn_s_sleep(1);
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    return st == 2;
}

// Base of gate/up row pair `pair` of `unit`, as 16-byte chunks. ids were
// clamped to [0, 64) when they were published.
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

// Reduce one gate/up pair and publish its tagged h word.
__device__ __forceinline__ void finish_pair(const Params& P, int unit, int pair,
                                            const u32x4 (&b)[8], const float (&xr)[4][8],
                                            uint32_t tag) {
    const int lane = threadIdx.x & (kLanes - 1);
    float g = 0.f, u = 0.f;
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        g = dot8(b[m], xr[m], g);
        u = dot8(b[4 + m], xr[m], u);
    }
    g = wave_sum(g);
    u = wave_sum(u);
    if (lane == 0) {
        const float h = bf16r(bf16r(silu_rn(bf16r(g))) * bf16r(u));
        st_agent(&P.ws->h[h_offset(unit) + pair], tag | bf16_bits(h));
    }
}

// Poll the tagged h words of chunks c = lane + 64 m (m < NM, c < n_chunks)
// until all carry `tag`, returning the bf16 values as 16-byte chunks.
template <int NM>
__device__ bool wait_h(const Params& P, int unit, int n_chunks, uint32_t tag,
                       u32x4 (&H)[NM]) {
    const int lane = threadIdx.x & (kLanes - 1);
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
        if (it >= kSpinLimit || ld_agent(&P.ws->abort) != 0) {
            if (lane == 0)
                __hip_atomic_fetch_or(&P.ws->abort, FLEET_MOE_ABORT_UNIT_WAIT, __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_AGENT);
            return false;
        }
        __builtin_amdgcn_s_sleep(1);
    }
}

__global__ __launch_bounds__(kThreads, 1) void moe_decode_kernel(Params P) {
    __shared__ Lds L;
    const int wg = blockIdx.x;
    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & (kLanes - 1);
    Workspace* ws = P.ws;

    // Issue order: x (needed first), the router row, then this wave's first
    // (shared, routing-independent) pair.
    const float4 xv = reinterpret_cast<const float4*>(P.x)[tid];
    const bool router_wave = wave == kRouterWave && wg < kRouted;
    u32x4 rrow[4];
    if (router_wave) {
        const u32x4* r = P.router + (int64_t)wg * kRowChunks;
#pragma unroll
        for (int m = 0; m < 4; ++m) rrow[m] = r[lane + kLanes * m];
    }
    u32x4 bufA[8], bufB[8];
    int cur = wave;
    issue_pair(reinterpret_cast<const u32x4*>(P.shared) + (int64_t)(wg + kWG * cur) * 2 * kRowChunks,
               lane, bufA);
    const uint32_t epoch = ld_agent(&ws->epoch) + 1u;
    const uint32_t tag = (epoch & 0xffffu) << 16;
    FLEET_TRACE(0);
    if (tid == 0) { L.next = kWaves; L.route = 0; }
    if (tid < 8) { L.ids[tid] = 0; L.w[tid] = 0.f; }

    // a1: RMSNorm of x (every workgroup, identical arithmetic): fp64 sum of
    // squares in a fixed tree, var = fp32(ssq / H), inv = 1 / sqrt(var + eps)
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
    {
        float y[4] = {bf16r(xv.x * inv), bf16r(xv.y * inv), bf16r(xv.z * inv), bf16r(xv.w * inv)};
        if (P.norm) {
            const uint2 gb = reinterpret_cast<const uint2*>(P.norm)[tid];
            y[0] = bf16r(y[0] * bf_lo(gb.x));
            y[1] = bf16r(y[1] * bf_hi(gb.x));
            y[2] = bf16r(y[2] * bf_lo(gb.y));
            y[3] = bf16r(y[3] * bf_hi(gb.y));
        }
        reinterpret_cast<float4*>(L.xn)[tid] = make_float4(y[0], y[1], y[2], y[3]);
    }
    __syncthreads();
    float xr[4][8];
#pragma unroll
    for (int m = 0; m < 4; ++m)
#pragma unroll
        for (int i = 0; i < 8; ++i) xr[m][i] = L.xn[kChunk * (lane + kLanes * m) + i];
    FLEET_TRACE(1);

    // a2: one router row per workgroup (fp64 accumulation of the exact
    // bf16 x bf16 products), published as a tagged 64-bit word.
    if (router_wave) {
        double acc = 0.0;
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            const uint32_t wv[4] = {rrow[m].x, rrow[m].y, rrow[m].z, rrow[m].w};
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                acc += (double)(bf_lo(wv[q]) * xr[m][2 * q]);
                acc += (double)(bf_hi(wv[q]) * xr[m][2 * q + 1]);
            }
        }
        acc = wave_sum64(acc);
        if (lane == 0)
            __hip_atomic_store(&ws->logit[wg],
                               ((uint64_t)epoch << 32) | __float_as_uint((float)acc),
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }

    // Phase G: gate/up pairs, double-buffered.
    auto grab = [&]() {
        int t = 0;
        if (lane == 0)
            t = __hip_atomic_fetch_add(&L.next, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        return wave_bcast(t);
    };
    bool traced_route = false;
    auto issue = [&](int j, u32x4 (&b)[8]) {
        int u, p;
        item_of(wg, j, u, p);
        if (u != 0 && ensure_routing(P, L, epoch) && !traced_route) {
            FLEET_TRACE(2);
            traced_route = true;
        }
        issue_pair(pair_base(P, L, u, p), lane, b);
    };
    auto finish = [&](int j, const u32x4 (&b)[8]) {
        int u, p;
        item_of(wg, j, u, p);
        finish_pair(P, u, p, b, xr, tag);
    };
    while (true) {
        int nxt = grab();
        if (nxt < kItems) issue(nxt, bufB);
        finish(cur, bufA);
        if (nxt >= kItems) break;
        cur = nxt;
        nxt = grab();
        if (nxt < kItems) issue(nxt, bufA);
        finish(cur, bufB);
        if (nxt >= kItems) break;
        cur = nxt;
    }
    FLEET_TRACE(3);

    // Phase D: this wave's down rows, all loads in flight before the wait.
    const int row0 = wg * kRowsPerWG;
    u32x4 W[24];
    const bool routed = wave < kTopK;
    const int unit = routed ? 1 + wave : 0;
    float wk = 0.f;
    if (routed) {
        ensure_routing(P, L, epoch);
        wk = L.w[wave];
        const u32x4* base = reinterpret_cast<const u32x4*>(
                                P.experts + (int64_t)L.ids[wave] * P.expert_stride +
                                (int64_t)2 * kInter * kHidden) +
                            (int64_t)row0 * kInterChunks;
#pragma unroll
        for (int r = 0; r < 8; ++r)
#pragma unroll
            for (int m = 0; m < 3; ++m) {
                const int c = lane + kLanes * m;
                W[3 * r + m] = c < kInterChunks ? ld_stream(base + r * kInterChunks + c)
                                                : u32x4{0u, 0u, 0u, 0u};
            }
    } else {
        const int r0 = row0 + 4 * (wave - kTopK);
        const u32x4* base = reinterpret_cast<const u32x4*>(
                                P.shared + (int64_t)2 * kSharedInter * kHidden) +
                            (int64_t)r0 * kSharedChunks;
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int m = 0; m < 6; ++m) {
                const int c = lane + kLanes * m;
                W[6 * r + m] = c < kSharedChunks ? ld_stream(base + r * kSharedChunks + c)
                                                 : u32x4{0u, 0u, 0u, 0u};
            }
    }
    FLEET_TRACE(4);
    if (routed) {
        u32x4 H[3];
        wait_h<3>(P, unit, kInterChunks, tag, H);
        FLEET_TRACE(5);
#pragma unroll
        for (int r = 0; r < 8; ++r) {
            float acc = 0.f;
#pragma unroll
            for (int m = 0; m < 3; ++m) acc = dot8_bb(W[3 * r + m], H[m], acc);
            acc = wave_sum(acc);
            if (lane == 0) L.part[unit][r] = bf16r(wk * bf16r(acc));
        }
    } else {
        u32x4 H[6];
        wait_h<6>(P, unit, kSharedChunks, tag, H);
        FLEET_TRACE(5);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            float acc = 0.f;
#pragma unroll
            for (int m = 0; m < 6; ++m) acc = dot8_bb(W[6 * r + m], H[m], acc);
            acc = wave_sum(acc);
            if (lane == 0) L.part[0][4 * (wave - kTopK) + r] = bf16r(acc);
        }
    }
    FLEET_TRACE(6);
    __syncthreads();

    // a7: combine in slot order, then the bf16 residual add.
    if (tid < kRowsPerWG) {
        const int n = row0 + tid;
        float y = 0.f;
#pragma unroll
        for (int k = 0; k < kTopK; ++k) y += L.part[1 + k][tid];
        const float out = bf16r(bf16r(y) + L.part[0][tid]);
        const float xo = bf16r(P.x[n] + out);
        P.x_out[n] = xo;
        if (P.moe_out) P.moe_out[n] = (uint16_t)bf16_bits(out);
    }
    if (tid == 0) {
        const uint32_t old = __hip_atomic_fetch_add(&ws->exits, 1u, __ATOMIC_RELAXED,
                                                    __HIP_MEMORY_SCOPE_AGENT);
        if (old + 1u == epoch * (uint32_t)kWG) st_agent(&ws->epoch, epoch);
    }
    FLEET_TRACE(7);
}

}  // namespace decode
}  // namespace fleet_moe

using namespace fleet_moe;

static bool aligned(const void* p, size_t a) { return ((uintptr_t)p % a) == 0; }

int fleet_moe_check_dims(const fleet_moe_dims* d);   // moe_abi.hip
int fleet_moe_check_device(int min_cus);              // moe_abi.hip

#if FLEET_MOE_TRACE
static unsigned long long* g_trace = nullptr;
extern "C" void fleet_moe_debug_set_trace(void* p) { g_trace = (unsigned long long*)p; }
#endif

extern "C" size_t fleet_moe_layer_workspace_bytes(const fleet_moe_dims* dims) {
    (void)dims;
    return (sizeof(decode::Workspace) + 255) & ~(size_t)255;
}

extern "C" int fleet_moe_layer_decode(const fleet_moe_layer* layer, const float* x,
                                      float* x_out, uint16_t* moe_out, int32_t* ids,
                                      float* weights, void* workspace, size_t workspace_bytes,
                                      const fleet_moe_dims* dims, hipStream_t stream) {
    if (!layer || !dims) return FLEET_MOE_ERR_ARG;
    if (int e = fleet_moe_check_dims(dims)) return e;
    if (!layer->router || !layer->experts || !layer->shared || !x || !x_out || !workspace)
        return FLEET_MOE_ERR_ARG;
    if (!aligned(layer->router, 16) || !aligned(layer->experts, 16) ||
        !aligned(layer->shared, 16) || !aligned(x, 16) || !aligned(x_out, 4) ||
        !aligned(workspace, 256) || (layer->norm && !aligned(layer->norm, 8)) ||
        (moe_out && !aligned(moe_out, 2)) || (ids && !aligned(ids, 4)) ||
        (weights && !aligned(weights, 4)))
        return FLEET_MOE_ERR_ARG;
    if (layer->expert_stride < kExpertStride || layer->expert_stride % kChunk != 0)
        return FLEET_MOE_ERR_DIMS;
    if (workspace_bytes < fleet_moe_layer_workspace_bytes(dims)) return FLEET_MOE_ERR_WORKSPACE;
    if (int e = fleet_moe_check_device(decode::kWG)) return e;

    decode::Params P;
    P.norm = layer->norm;
    P.router = reinterpret_cast<const u32x4*>(layer->router);
    P.experts = layer->experts;
    P.shared = layer->shared;
    P.x = x;
    P.x_out = x_out;
    P.moe_out = moe_out;
    P.ids_out = ids;
    P.w_out = weights;
    P.ws = reinterpret_cast<decode::Workspace*>(workspace);
    P.expert_stride = layer->expert_stride;
    P.eps = dims->rms_eps;
    P.scaling = dims->routed_scaling;
#if FLEET_MOE_TRACE
    P.trace = g_trace;
#endif
    hipLaunchKernelGGL(decode::moe_decode_kernel, dim3(decode::kWG), dim3(decode::kThreads), 0,
                       stream, P);
    return (int)hipGetLastError();
}
