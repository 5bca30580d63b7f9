// Device code of the batch-1 dense layer, shared by its own launch
// (moe_dense.hip) and the whole-step kernel (step_decode.hip).
//
// Batch-1 dense SwiGLU layer of DeepSeek-V2-Lite (layer 0, intermediate 10944):
// x_out = bf16(x + down(bf16(bf16(silu(bf16(g))) * bf16(u)))), g/u = gate/up
// rows . rms_norm(x), in ONE launch of 256 workgroups (one per CU, 8 waves).
//
// What it replaces in the reference: the DENSE_GATE_UP / DENSE_DOWN task
// bodies of the persistent decode kernel (src/kernels/fleet_kernel.hip:891-903,
// emitted by src/host/taskgraph.py:444-474) and the layer's NORM_ROUTER
// prologue; semantics of src/host/reference_decode.py:290-302 (dense_mlp =
// mlp_unit at the dense width, bf16 residual add).
//
//   prologue  RMSNorm exactly as the MoE decode kernel computes it (fp64 sum of
//             squares, correctly rounded sqrt and division), x_norm as packed
//             bf16 in registers.
//   phase G   the 10944 gate/up row pairs (interleaved, 8 KB each) are dealt
//             round-robin to the 256 workgroups (42 or 43 each); the 8 waves
//             pull them from an LDS ticket, one in flight per wave, and publish
//             h as tagged words (epoch << 16 | bf16) with device-scope stores.
//   phase D   workgroup w owns output rows [8w, 8w + 8): wave r streams row
//             8w + r (21,888 B) into registers, then the workgroup polls the
//             10944 h words once into LDS (bf16) and every wave takes its dot.
// Every wait is bounded and records FLEET_MOE_ABORT_UNIT_WAIT instead of
// hanging; workgroup 0 advances the call count once it has seen every
// workgroup's h.
#pragma once
#include <stddef.h>

#include "moe_common.h"

namespace fleet_moe {
namespace dense {

constexpr int kDenseInter = 10944;
constexpr int kWG = 256;
constexpr int kWaves = 8;
constexpr int kThreads = kWaves * kLanes;
constexpr int kRowsPerWG = kHidden / kWG;                  // 8 down rows per workgroup
constexpr int kDnChunks = kDenseInter / kChunk;             // 1368 chunks per down row
constexpr int kDnIters = (kDnChunks + kLanes - 1) / kLanes; // 22
constexpr int kPollUnits = kDenseInter / 4;                 // 16-byte units of h words
static_assert(kRowsPerWG == kWaves, "one down row per wave");
static_assert(kDenseInter % 4 == 0, "h polled in 16-byte units");

struct Workspace {
    uint32_t epoch;
    uint32_t pad_exits;
    uint32_t abort;
    uint32_t pad0[61];
    uint32_t h[kDenseInter];   // (epoch & 0xffff) << 16 | bf16 h
};
static_assert(offsetof(Workspace, abort) == 8, "status word offset");
static_assert(offsetof(Workspace, h) % 16 == 0, "h is read with 16-byte loads");

struct Params {
    const uint16_t* norm;      // bf16[H] or null
    const uint16_t* w;         // [2I][H] interleaved gate/up, then [H][I] down
    const float* x;
    float* x_out;
    uint16_t* mlp_out;         // bf16[H] or null
    Workspace* ws;
    float eps;
    // the whole-step kernel only
    uint32_t epoch;            // this layer's call count
    const uint32_t* xin;       // tagged x [kXCopies][kHidden], or null: xin_f32
    const float* xin_f32;      // x itself (the first stage of a launch)
    uint32_t xin_tag;
    uint32_t* xout;            // tagged x_out [kXCopies][kHidden]
    uint32_t xout_tag;
};

struct Lds {
    alignas(16) uint32_t xb[kHidden / 2];
    alignas(16) float xraw[kHidden];           // x itself (the whole-step kernel)
    double red[kWaves];
    double xsq[kWaves];
    alignas(16) uint32_t hb[kDenseInter / 2];   // h as bf16 pairs
    int next;
};

__device__ __forceinline__ int pairs_of(int wg) {
    return kDenseInter / kWG + (wg < kDenseInter % kWG ? 1 : 0);   // 43 or 42
}

__device__ __forceinline__ void issue_pair(const u32x4* base, int lane, u32x4 (&b)[8]) {
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        b[m] = ld_stream(base + lane + kLanes * m);
        b[4 + m] = ld_stream(base + kRowChunks + lane + kLanes * m);
    }
}

// A wave's first gate/up pair (pair wg + 256 wave), issued into `b`. The
// whole-step kernel issues it from the stage before this one, once that
// stage's last wait is done. Every wave has one (a workgroup has at least 42
// pairs), and the issue is unconditional: behind a branch, the compiler
// waited for every load in flight (the pair too) before the RMSNorm read x.
static_assert(kDenseInter / kWG >= kWaves, "every wave has a first pair");
__device__ __forceinline__ void issue_first_pair(const uint16_t* w, u32x4 (&b)[8]) {
    const int wg = blockIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(fm_tid() >> 6);
    issue_pair(reinterpret_cast<const u32x4*>(w) + (int64_t)(wg + kWG * wave) * 2 * kRowChunks,
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
__device__ __forceinline__ void dense_layer(const Params& P, Lds& L, u32x4 (&pre)[8], bool pre_in,
                                            Next&& next) {
    const int wg = blockIdx.x, tid = fm_tid();
    const int wave = tid >> 6, lane = tid & (kLanes - 1);
    Workspace* ws = P.ws;
    // the call count, written by the previous launch: a plain load (current
    // after the launch boundary; a device-scope load of one word by every
    // wave would queue at its memory channel)
    const uint32_t epoch = kMega ? P.epoch : ws->epoch + 1u;
    const uint32_t tag = (epoch & 0xffffu) << 16;
    float4 xv = make_float4(0.f, 0.f, 0.f, 0.f);
    if constexpr (!kMega) xv = reinterpret_cast<const float4*>(P.x)[tid];
    const uint2 gb = P.norm ? ld_global_u2(P.norm, tid)
                            : make_uint2(0x3f803f80u, 0x3f803f80u);   // bf16 1.0
    const u32x4* gu = reinterpret_cast<const u32x4*>(P.w);
    const int n_items = pairs_of(wg);
    u32x4 (&buf)[8] = pre;
    int cur = wave;                           // every wave's first pair (see above)
    if (!(kMega && pre_in)) issue_first_pair(P.w, buf);
    if (tid == 0) L.next = kWaves;
    if constexpr (kMega) {
        // x: every workgroup's published rows (polled behind this wave's first
        // pair), or the launch's input vector
        if (P.xin_f32)
            xv = reinterpret_cast<const float4*>(P.xin_f32)[tid];
        else
            xv = poll_x4(P.xin + (wg % kXCopies) * kHidden, P.xin_tag, &ws->abort,
                         FLEET_MOE_ABORT_STEP_WAIT);
        reinterpret_cast<float4*>(L.xraw)[tid] = xv;
    }

    // RMSNorm (identical arithmetic to the MoE decode kernel)
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
    __syncthreads();
    u32x4 xq[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) xq[m] = reinterpret_cast<const u32x4*>(L.xb)[lane + kLanes * m];
    float xnorm;                              // ||x_norm||_2, for the certified GEMVs
    {
        double xs = 0.0;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) xs += L.xsq[w];
        xnorm = (float)__builtin_sqrt(xs);
    }

    // Phase G
    auto claim = [&]() -> int {
        int t = 0;
        if (lane == 0)
            t = __hip_atomic_fetch_add(&L.next, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        t = wave_bcast(t);
        return t < n_items ? t : -1;
    };
    while (cur >= 0) {
        const int nxt = claim();
        // bf16(g), bf16(u) exactly rounded: certified fp32 evaluation (depth
        // 8 + 2 + 6), the exact fp64 sum for a row the bound cannot decide.
        // The four sums (g, u, |g row|^2, |u row|^2) are reduced together
        // into lanes 0..3; lanes 0 and 1 certify g and u.
        float g[4], u[4], gw[4], uw[4];
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            g[m] = dot8_d2(buf[m], xq[m], 0.f);
            u[m] = dot8_d2(buf[4 + m], xq[m], 0.f);
            gw[m] = dot8_d2(buf[m], buf[m], 0.f);
            uw[m] = dot8_d2(buf[4 + m], buf[4 + m], 0.f);
        }
        float v4[4] = {tree_sum(g), tree_sum(u), tree_sum(gw), tree_sum(uw)};
        const float s = wave_nsum(v4);                                         // lane % 4: g, u, gw, uw
        const float w2 = __int_as_float(FLEET_DPP(__float_as_int(s), 0x4E));   // lane ^ 2
        float r;
        const bool okc = certify_bf16(s, w2, xnorm, cert_gamma(16), r);
        const uint64_t bad = __ballot(!okc) & 3ull;
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            if (bad & (1ull << q)) {
                double a = 0.0;
#pragma unroll
                for (int m = 0; m < 4; ++m) a = dot8_x(buf[4 * q + m], xq[m], a);
                const float e = bf16r((float)wave_sum64(a));
                r = lane == q ? e : r;
            }
        }
        const float ub = __int_as_float(FLEET_DPP(__float_as_int(r), 0xB1));   // lane ^ 1
        if (lane == 0) {
            const float h = bf16r(bf16r(silu_rn(r)) * ub);
            st_agent(&ws->h[wg + kWG * cur], tag | bf16_bits(h));
        }
        if (nxt >= 0) issue_pair(gu + (int64_t)(wg + kWG * nxt) * 2 * kRowChunks, lane, buf);
        cur = nxt;
    }

    // Phase D: this wave's down row in flight before the h wait
    const int n = kRowsPerWG * wg + wave;
    const u32x4* drow = gu + (int64_t)2 * kDenseInter * kRowChunks + (int64_t)n * kDnChunks;
    u32x4 W[kDnIters];
#pragma unroll
    for (int i = 0; i < kDnIters; ++i) {
        const int c = lane + kLanes * i;
        W[i] = c < kDnChunks ? ld_stream(drow + c) : u32x4{0u, 0u, 0u, 0u};
    }
    // h, polled once per workgroup (16 bytes = four words per step)
    const __amdgpu_buffer_rsrc_t rh = rsrc(ws->h);
    bool ok = true;
    for (int k = tid; k < kPollUnits; k += kThreads) {
        u32x4 v;
        for (uint32_t it = 0;; ++it) {
            v = ld_dev16(rh, 16 * k);
            if ((v.x & 0xffff0000u) == tag && (v.y & 0xffff0000u) == tag &&
                (v.z & 0xffff0000u) == tag && (v.w & 0xffff0000u) == tag)
                break;
            if (it >= kSpinLimit || ((it & 1023) == 1023 && ld_agent(&ws->abort) != 0)) {
                ok = false;
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
        if (!ok) break;
        L.hb[2 * k] = (v.x & 0xffffu) | (v.y << 16);
        L.hb[2 * k + 1] = (v.z & 0xffffu) | (v.w << 16);
    }
    if (!ok)
        __hip_atomic_fetch_or(&ws->abort, FLEET_MOE_ABORT_UNIT_WAIT, __ATOMIC_RELAXED,
                              __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    // every workgroup's h words carried this call's tag, so every workgroup
    // has read the call count: workgroup 0 advances it for the next call
    if (!kMega && wg == 0 && tid == 0) st_agent(&ws->epoch, epoch);
    // bf16(down . h) exactly rounded: certified fp32 evaluation (v_dot2
    // chain 8, a 22-value tree 5, wave sum 6), exact fp64 sum as fallback
    // (h is read from LDS where it is used rather than held: 88 registers
    // fewer, which the whole-step kernel needs)
    auto h_chunk = [&](int i) {
        const int c = lane + kLanes * i;
        return c < kDnChunks ? reinterpret_cast<const u32x4*>(L.hb)[c] : u32x4{0u, 0u, 0u, 0u};
    };
    float av[kDnIters], wv[kDnIters], hq[kDnIters];
#pragma unroll
    for (int i = 0; i < kDnIters; ++i) {
        const u32x4 hv = h_chunk(i);
        av[i] = dot8_d2(W[i], hv, 0.f);
        wv[i] = dot8_d2(W[i], W[i], 0.f);
        hq[i] = dot8_d2(hv, hv, 0.f);
    }
    // the three sums reduced together: lane % 4 = 0, 1, 2 holds the dot,
    // the row's and h's sums of squares; every lane of a quad takes all three.
    // Quads can hold different roundings of the same sum (wave_nsum), so the
    // decision is lane 0's (lane 0 writes the row) and the wave follows it:
    // decided per lane, a wave split near the bound ran the fp64 fallback
    // with lanes masked off, and its wave sum missed their terms.
    float v4[4] = {tree_sum(av), tree_sum(wv), tree_sum(hq), 0.f};
    const float s = wave_nsum(v4);
    const float w2 = __int_as_float(FLEET_DPP(__float_as_int(s), 0x55));   // quad lane 1
    const float h2 = __int_as_float(FLEET_DPP(__float_as_int(s), 0xAA));   // quad lane 2
    const float a0 = __int_as_float(FLEET_DPP(__float_as_int(s), 0x00));   // quad lane 0
    const float hn = __builtin_sqrtf(h2) * 1.0001f;
    float out;
    const bool okc = certify_bf16(a0, w2, hn, cert_gamma(8 + tree_depth(kDnIters) + 6), out);
    if (__ballot(!okc) & 1ull) {
        double acc = 0.0;
#pragma unroll
        for (int i = 0; i < kDnIters; ++i) acc = dot8_x(W[i], h_chunk(i), acc);
        out = bf16r((float)wave_sum64(acc));
    }
    next();
    if (lane == 0) {
        const float xo = bf16r((kMega ? L.xraw[n] : P.x[n]) + out);
        if (!kMega || P.x_out) P.x_out[n] = xo;
        if constexpr (kMega) publish_x(P.xout, n, xo, P.xout_tag);
        if (P.mlp_out) P.mlp_out[n] = (uint16_t)bf16_bits(out);
    }
}

}  // namespace dense
}  // namespace fleet_moe
