// Device helpers shared by the MoE kernels (gfx950, wave64).
//
// Numerics contract (the CPU oracle follows the same one):
//   * bf16 rounding is round-to-nearest-even on the fp32 bit pattern;
//   * reductions whose result must be reproducible bit for bit (RMSNorm mean of
//     squares, router logits, softmax) run in fp64 and are rounded once to fp32;
//   * expert GEMVs accumulate in fp32 and reduce with a fixed butterfly.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fleet_moe.h"

namespace fleet_moe {

// DeepSeek-V2-Lite MoE shape (reference/dsv2lite_config.json).
constexpr int kHidden = 2048;
constexpr int kInter = 1408;          // routed expert intermediate
constexpr int kRouted = 64;
constexpr int kShared = 2;
constexpr int kSharedInter = kShared * kInter;   // 2816
constexpr int kTopK = 6;
constexpr int64_t kExpertStride = 3ll * kHidden * kInter;   // 8,650,752 elements

constexpr int kLanes = 64;
constexpr int kChunk = 8;             // bf16 per 16-byte load
constexpr int kRowChunks = kHidden / kChunk;        // 256 16-byte chunks per K=2048 row
constexpr int kInterChunks = kInter / kChunk;       // 176 per K=1408 row
constexpr int kSharedChunks = kSharedInter / kChunk;  // 352 per K=2816 row

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// Streaming weight load: 16 bytes per lane, non-temporal (weights are read
// exactly once per call, so they should not displace the small shared
// vectors from L2).
__device__ __forceinline__ u32x4 ld_stream(const u32x4* p) {
    return __builtin_nontemporal_load(p);
}

__device__ __forceinline__ float bf_lo(uint32_t v) { return __uint_as_float(v << 16); }
__device__ __forceinline__ float bf_hi(uint32_t v) { return __uint_as_float(v & 0xffff0000u); }

__device__ __forceinline__ uint32_t bf16_bits(float f) {
    const uint32_t u = __float_as_uint(f);
    return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}
__device__ __forceinline__ float bf16r(float f) { return __uint_as_float(bf16_bits(f) << 16); }

// 8-element dot of one 16-byte bf16 chunk with 8 fp32 values, fp32 FMA chain.
__device__ __forceinline__ float dot8(const u32x4& w, const float* x, float acc) {
    acc = fmaf(bf_lo(w.x), x[0], acc);
    acc = fmaf(bf_hi(w.x), x[1], acc);
    acc = fmaf(bf_lo(w.y), x[2], acc);
    acc = fmaf(bf_hi(w.y), x[3], acc);
    acc = fmaf(bf_lo(w.z), x[4], acc);
    acc = fmaf(bf_hi(w.z), x[5], acc);
    acc = fmaf(bf_lo(w.w), x[6], acc);
    acc = fmaf(bf_hi(w.w), x[7], acc);
    return acc;
}

// Same, both operands bf16 chunks.
__device__ __forceinline__ float dot8_bb(const u32x4& w, const u32x4& h, float acc) {
    acc = fmaf(bf_lo(w.x), bf_lo(h.x), acc);
    acc = fmaf(bf_hi(w.x), bf_hi(h.x), acc);
    acc = fmaf(bf_lo(w.y), bf_lo(h.y), acc);
    acc = fmaf(bf_hi(w.y), bf_hi(h.y), acc);
    acc = fmaf(bf_lo(w.z), bf_lo(h.z), acc);
    acc = fmaf(bf_hi(w.z), bf_hi(h.z), acc);
    acc = fmaf(bf_lo(w.w), bf_lo(h.w), acc);
    acc = fmaf(bf_hi(w.w), bf_hi(h.w), acc);
    return acc;
}

// Fixed butterfly over the 64 lanes: every lane ends with the same sum, and
// the order of additions never changes, so results are bitwise reproducible.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = kLanes / 2; off; off >>= 1) v += __shfl_xor(v, off, kLanes);
    return v;
}
__device__ __forceinline__ double wave_sum64(double v) {
#pragma unroll
    for (int off = kLanes / 2; off; off >>= 1) v += __shfl_xor(v, off, kLanes);
    return v;
}
__device__ __forceinline__ double wave_max64(double v) {
#pragma unroll
    for (int off = kLanes / 2; off; off >>= 1) v = fmax(v, __shfl_xor(v, off, kLanes));
    return v;
}

// Correctly rounded fp32 square root. The hardware square root is within one
// ulp; the candidate is corrected by comparing `a` with the squares of the
// midpoints to its neighbours, which are exact in fp64 (a midpoint has at
// most 25 significant bits). Positive normal inputs only (a >= eps here).
__device__ __forceinline__ float sqrt_rn(float a) {
    float s = __builtin_sqrtf(a);
    const double ad = (double)a;
    const float up = __uint_as_float(__float_as_uint(s) + 1u);
    const float dn = __uint_as_float(__float_as_uint(s) - 1u);
    const double mu = 0.5 * ((double)s + (double)up);
    const double md = 0.5 * ((double)s + (double)dn);
    if (ad > mu * mu) s = up;
    else if (ad < md * md) s = dn;
    return s;
}

// fp32 SiLU of a bf16-valued input, evaluated in fp64 and rounded once.
__device__ __forceinline__ float silu_rn(float g) {
    const double d = (double)g;
    return (float)(d / (1.0 + exp(-d)));
}

// Sleep-poll bound: ~2^22 polls of s_sleep(2) (about 0.2 s at 2.4 GHz). A
// wait that runs out records an abort reason and the kernel drains normally.
constexpr uint32_t kSpinLimit = 1u << 22;

__device__ __forceinline__ uint32_t ld_agent(const uint32_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent(uint32_t* p, uint32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Whole-wave wait until flags[0..n) all equal `target` (n <= 256), then an
// agent-scope acquire. Returns false (after recording `reason` in *abort)
// when the bound runs out or another wave already aborted.
__device__ inline bool wave_wait_flags(const uint32_t* flags, int n, uint32_t target,
                                       uint32_t* abort_word, uint32_t reason) {
    const int lane = threadIdx.x & (kLanes - 1);
    for (uint32_t it = 0;; ++it) {
        bool ok = true;
        for (int i = lane; i < n; i += kLanes) ok &= ld_agent(flags + i) == target;
        if (__all(ok)) break;
        if (it >= kSpinLimit || ld_agent(abort_word) != 0) {
            if (lane == 0) __hip_atomic_fetch_or(abort_word, reason, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT);
            return false;
        }
        __builtin_amdgcn_s_sleep(2);
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    return true;
}

// Softmax in fp64 over one logit per lane (lanes >= n hold -inf) and greedy
// top-k with ties to the lowest index: k passes of a butterfly argmax over
// (p, lane). Writes ids[0..k) and p[ids] * scaling to LDS arrays on lane 0's
// side (every lane computes the same values; lanes < k store slot `lane`).
// Rule of select_experts_from, src/kernels/fleet_kernel.hip:469-494.
__device__ inline void wave_softmax_topk(float logit, int n, int k, float scaling,
                                         int* ids_out, float* w_out, const float* bias) {
    const int lane = threadIdx.x & (kLanes - 1);
    const bool valid = lane < n;
    // A bias is added in fp32 (z = fp32(logit + bias)); the softmax is fp64.
    const float z32 = valid ? (bias ? logit + bias[lane] : logit) : 0.f;
    const double zz = valid ? (double)z32 : -INFINITY;
    const double mx = wave_max64(zz);
    const double e = valid ? exp(zz - mx) : 0.0;
    const double s = wave_sum64(e);
    float p = valid ? (float)(e / s) : -INFINITY;
    int my_slot = -1;
    float my_val = 0.f;
    for (int j = 0; j < k; ++j) {
        float bv = p;
        int bi = valid ? lane : 0x7fffffff;
#pragma unroll
        for (int off = kLanes / 2; off; off >>= 1) {
            const float ov = __shfl_xor(bv, off, kLanes);
            const int oi = __shfl_xor(bi, off, kLanes);
            if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
        }
        if (lane == j) { my_slot = bi; my_val = bv; }
        if (lane == bi) p = -INFINITY;
    }
    if (lane < k) {
        ids_out[lane] = my_slot;
        w_out[lane] = my_val * scaling;
    }
}

}  // namespace fleet_moe
