// The attention half of a DeepSeek-V2-Lite decoder layer (absorbed MLA) and
// the lm_head + argmax at batch 1, as device code shared by their own
// launches (attn_decode.hip) and the whole-step kernel (step_decode.hip).
//
// Semantics of src/host/reference_decode.py:210-256 (attention_absorbed) and
// of the kernel's EMBED / LM_HEAD / ARGMAX tasks (src/kernels/fleet_kernel.hip:
// 68-78, 509-585, 905-920): bf16 rounding after q / kv_a, after
// kv_a_layernorm, after RoPE (both the cached k_pe and q_pe), after the
// concatenated head outputs and after o_proj; bf16 logits; argmax with the
// lowest index on ties. Every dot product is the exact value rounded once to
// fp32 (fp64 accumulation of exact products); q_c is that fp32 value; the
// scores, the softmax and its weighted sum of c stay in fp64 (chunk partials
// merged in fp64) and o_c is rounded once to fp32, so no result depends on
// how positions are split into chunks.
//
// One layer is ONE launch of 256 workgroups (one per CU, 8 waves each) that
// runs five stages; the data a stage needs from other workgroups crosses as
// self-validating words (each carries the call's epoch, written and polled
// with device-scope accesses), so a stage starts as soon as its own inputs
// are published, and every weight slice and cache row a workgroup will need
// is put in flight at the start, before the first wait:
//   S1 qkv    RMSNorm(x) in every workgroup, then the 3648 rows of
//             [q_proj ; kv_a]: head h's 192 q rows in its 16 workgroups
//             (row 192 h + k + 16 i in workgroup (h, k)), kv_a row 3072 + j
//             in workgroup j % 256.
//   S2 q_c    workgroup (h, k): columns 32k .. 32k+31 of head h's absorbed
//             query q_c = W_UK^T q_nope (128 rows x 32 columns of W_UK).
//   S3 mla    workgroup (h3, k3): positions chunk k3 of head h3 (16 chunks of
//             ceil((pos+1)/16)): scores, then the chunk's fp64 softmax partial
//             (max, sum of exp, sum exp * c); the workgroups holding the
//             current position derive its cache row (kv_a_layernorm of c,
//             RoPE of k_pe) from kv_a themselves, and (0, k3) writes it.
//   S4 merge  workgroup (h, k): columns 32k .. 32k+31 of o_c merged from the
//             chunk partials and rounded once; then rows 8k .. 8k+7 of
//             W_UV o_c, bf16.
//   S5 oproj  workgroup w: rows 8w .. 8w+7 of o_proj, bf16, residual add.
// Workgroup w has (h, k) = (w % 8 + 8 ((w / 8) % 2), w / 16) in S1, S2, S4
// and S5: workgroups are dealt to the 8 XCDs round-robin (w % 8), so all 16
// workgroups of a head share one XCD and its q rows, q_c and o_c pass through
// that XCD. In S3 it has (h3, k3) = ((w / 8) % 16, 2 (w % 8) + w / 128): XCD
// x takes position chunks 2x and 2x + 1 of every head, so each cached row is
// fetched from HBM into one XCD's L2 (which serves it to all 16 heads)
// instead of into all eight. Every word is published with a device-scope
// store, so the protocol does not depend on the placement, only its speed
// does.
// The position can come from the host (an argument) or from device memory
// (pos_dev), so a whole decode step can be captured once in a HIP graph and
// replayed: the argmax kernel then advances *pos_dev itself. A device
// position outside [0, max_pos) raises FLEET_MOE_ABORT_POSITION and the layer
// does nothing past the check; a token outside the vocabulary raises
// FLEET_MOE_ABORT_TOKEN in the embedding, which then writes zeros. Every
// cross-workgroup wait is bounded (FLEET_MOE_ABORT_ATTN_WAIT).
//
// Cache layout [max_pos][512 + 64] bf16 per layer: c after kv_a_layernorm,
// then k_pe after RoPE in DeepseekV2's reordered basis. RoPE tables (cos, sin
// [max_pos][64] fp32) are the caller's.
#pragma once
#include <stddef.h>

#include <cmath>

#include "moe_common.h"

#ifndef FLEET_ATTN_TRACE
#define FLEET_ATTN_TRACE 0
#endif

namespace fleet_moe {
namespace attn {

constexpr int kHeads = 16;
constexpr int kLora = 512;
constexpr int kNope = 128;
constexpr int kRope = 64;
constexpr int kV = 128;
constexpr int kQDim = kHeads * (kNope + kRope);          // 3072
constexpr int kQkvRows = kQDim + kLora + kRope;          // 3648
constexpr int kKvbRowsPerHead = kNope + kV;              // 256
constexpr int kRowElems = kLora + kRope;                 // 576: one cache row
constexpr int kMaxPos = 4096;
constexpr int kVocab = 102400;
constexpr int kWG = 256;
constexpr int kThreads = 512;
constexpr int kWaves = kThreads / kLanes;
constexpr int kChunks = kWG / kHeads;                    // 16 position chunks per head
constexpr int kQcCols = kLora / kChunks;                 // 32 columns of q_c / o_c per workgroup
constexpr int kUkRows = kNope / kWaves;                  // 16 W_UK rows per wave
constexpr int kUvRows = kV / kChunks;                    // 8 W_UV rows per workgroup
constexpr int kOpRows = kHidden / kWG;                   // 8 o_proj rows per workgroup
// The head outputs are read by every workgroup (S5): they are published in
// kOutCopies copies and workgroup w polls copy w % kOutCopies, so each line
// sees 32 pollers instead of 256 (same-address device-scope requests queue at
// the line's memory channel).
constexpr int kOutCopies = 8;
constexpr int kBatch = 9;                                // cache rows a wave holds at once (72-row chunks: one batch)
static_assert(kHeads * kChunks == kWG && kQcCols * kChunks == kLora, "work split");
static_assert(kUvRows == kWaves && kOpRows == kWaves, "one row per wave in the epilogues");
static_assert(kBatch <= kLanes, "one lane per row for the exponentials");

struct Workspace {
    uint32_t epoch;                            // calls completed on this workspace
    uint32_t pad0;
    uint32_t abort;                            // offset 8: sticky status
    uint32_t pad1[61];
    float qkv[kQkvRows];                       // plain copies of the published values
    float qc[kHeads][kLora];
    float qpe[kHeads][kRope];
    // Published values. Every 32-bit word is (epoch & 0xffff) << 16 | 16
    // payload bits: a bf16 in one word, an fp32 in two (high half first), an
    // fp64 in four, so a word read with any tearing of wider accesses still
    // proves its own freshness. Every call rewrites every one of these words
    // (chunks without positions publish neutral partials), so a 16-bit tag
    // only has to differ from the previous call's.
    uint32_t qkv_t[kQkvRows];                  // bf16 q / kv_a
    uint32_t qc_t[kHeads][kLora][2];           // fp32 q_c
    uint32_t ml_t[kHeads][kChunks][8];         // fp64 chunk max, then fp64 chunk sum of exp
    uint32_t o_t[kHeads][kChunks][kLora][4];   // fp64 chunk sum of exp * c
    uint32_t oc_t[kHeads][kLora][2];           // fp32 o_c
    uint32_t out_t[kOutCopies][kHeads * kV];   // bf16 head outputs, kOutCopies copies
    float cand_v[kWG];                         // lm_head: best logit per workgroup
    int32_t cand_i[kWG];
    uint64_t cand_t[kWG][2];                   // the same, tagged (epoch << 32 | bits), for the
                                               // whole-step kernel
};
static_assert(offsetof(Workspace, abort) == 8, "status word offset");
static_assert(offsetof(Workspace, qkv) == 256, "plain copies follow the header");
static_assert(offsetof(Workspace, qkv_t) % 16 == 0 && offsetof(Workspace, qc_t) % 16 == 0 &&
                  offsetof(Workspace, ml_t) % 16 == 0 && offsetof(Workspace, o_t) % 16 == 0 &&
                  offsetof(Workspace, oc_t) % 16 == 0 && offsetof(Workspace, out_t) % 16 == 0,
              "polled arrays are read with 16-byte loads");
static_assert(sizeof(Workspace) < (1u << 31), "32-bit buffer offsets");

__device__ __forceinline__ void raise(Workspace* ws, uint32_t bit) {
    __hip_atomic_fetch_or(&ws->abort, bit, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// RMSNorm of a 2048-vector held 4 per thread (512 threads), the arithmetic of
// the MoE decode kernel (fp64 sum of squares, correctly rounded sqrt and
// division, two bf16 roundings); writes the bf16 result as packed pairs and
// returns its 2-norm (for the certified GEMVs). red: 16 doubles of LDS.
__device__ float norm2048(const float4 xv, const uint2 gb, float eps, uint32_t* xb, double* red) {
    const int tid = fm_tid(), wave = tid >> 6, lane = tid & (kLanes - 1);
    double ss = (double)xv.x * xv.x + (double)xv.y * xv.y + (double)xv.z * xv.z +
                (double)xv.w * xv.w;
    ss = wave_sum64(ss);
    if (lane == 0) red[wave] = ss;
    __syncthreads();
    double ssq = 0.0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) ssq += red[w];
    const float var = (float)(ssq / (double)kHidden);
    const float inv = __fdiv_rn(1.0f, sqrt_rn(var + eps));
    float y[4] = {bf16r(xv.x * inv), bf16r(xv.y * inv), bf16r(xv.z * inv), bf16r(xv.w * inv)};
    y[0] = bf16r(y[0] * bf_lo(gb.x));
    y[1] = bf16r(y[1] * bf_hi(gb.x));
    y[2] = bf16r(y[2] * bf_lo(gb.y));
    y[3] = bf16r(y[3] * bf_hi(gb.y));
    xb[2 * tid] = bf16_bits(y[0]) | (bf16_bits(y[1]) << 16);
    xb[2 * tid + 1] = bf16_bits(y[2]) | (bf16_bits(y[3]) << 16);
    const double q = wave_sum64((double)y[0] * y[0] + (double)y[1] * y[1] +
                                (double)y[2] * y[2] + (double)y[3] * y[3]);
    if (lane == 0) red[kWaves + wave] = q;
    __syncthreads();
    double qs = 0.0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) qs += red[kWaves + w];
    return (float)__builtin_sqrt(qs);
}

__device__ __forceinline__ void load_row(const uint16_t* W, int64_t row, u32x4 (&w)[4]) {
    const int lane = fm_tid() & (kLanes - 1);
    const u32x4* r = reinterpret_cast<const u32x4*>(W + row * kHidden);
#pragma unroll
    for (int m = 0; m < 4; ++m) w[m] = ld_stream(r + lane + kLanes * m);
}

// Exactly rounded dot of a K = 2048 bf16 row with a bf16 vector (wave total).
__device__ __forceinline__ float dot_row(const u32x4 (&w)[4], const u32x4 (&xq)[4]) {
    double a = 0.0;
#pragma unroll
    for (int m = 0; m < 4; ++m) a = dot8_x(w[m], xq[m], a);
    return (float)wave_sum64(a);
}

// Two rows at once (the second only if `two`): their dots and sums of
// squares reduced together (lane % 4: a0, a1, n0, n1), lanes 0 and 1
// certify, a row the bound cannot decide is evaluated exactly. r0 / r1
// receive the exactly rounded bf16 results in every lane.
__device__ __forceinline__ void dot_rows2_bf16(const u32x4 (&w0)[4], const u32x4 (&w1)[4],
                                               bool two, const u32x4 (&xq)[4], float xnorm,
                                               float& r0, float& r1) {
    const int lane = fm_tid() & (kLanes - 1);
    float a0[4], a1[4], n0[4], n1[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        a0[m] = dot8_d2(w0[m], xq[m], 0.f);
        a1[m] = dot8_d2(w1[m], xq[m], 0.f);
        n0[m] = dot8_d2(w0[m], w0[m], 0.f);
        n1[m] = dot8_d2(w1[m], w1[m], 0.f);
    }
    float v[4] = {tree_sum(a0), tree_sum(a1), tree_sum(n0), tree_sum(n1)};
    const float sv = wave_nsum(v);
    const float w2 = __int_as_float(FLEET_DPP(__float_as_int(sv), 0x4E));   // lane ^ 2
    float r;
    const bool ok = certify_bf16(sv, w2, xnorm, cert_gamma(16), r);
    const uint64_t bad = __ballot(!ok) & (two ? 3ull : 1ull);
    if (bad & 1ull) {
        const float e = bf16r(dot_row(w0, xq));
        r = lane == 0 ? e : r;
    }
    if (bad & 2ull) {
        const float e = bf16r(dot_row(w1, xq));
        r = lane == 1 ? e : r;
    }
    r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(r), 0));
    r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(r), 1));
}

// Sum over the 8 lanes of each aligned group of 8 (quad exchanges, then the
// half-row mirror); every lane of the group returns the group total.
__device__ __forceinline__ double sum8_lanes(double v) {
    v += dpp64<0xB1>(v);
    v += dpp64<0x4E>(v);
    v += dpp64<0x141>(v);
    return v;
}

__device__ __forceinline__ double wave_max64(double v) {
    v = fmax(v, dpp64<0xB1>(v));
    v = fmax(v, dpp64<0x4E>(v));
    v = fmax(v, dpp64<0x141>(v));
    v = fmax(v, dpp64<0x140>(v));
    return fmax(fmax(readlane64(v, 0), readlane64(v, 16)), fmax(readlane64(v, 32), readlane64(v, 48)));
}

// The fp64 counterpart of wave_msum (moe_common.h): N values per lane summed
// over the wave in six exchange steps (lane L with L ^ {1, 2, 7, 15, 16, 32});
// v[0] of lane L returns the total of value msum_index<N>(L).
template <int K>
__device__ __forceinline__ double msum_xchg64(double x) {
    const long long b = __double_as_longlong(x);
    int lo = (int)(b & 0xffffffffll), hi = (int)(b >> 32);
    if constexpr (K == 0) {
        lo = FLEET_DPP(lo, 0xB1); hi = FLEET_DPP(hi, 0xB1);
    } else if constexpr (K == 1) {
        lo = FLEET_DPP(lo, 0x4E); hi = FLEET_DPP(hi, 0x4E);
    } else if constexpr (K == 2) {
        lo = FLEET_DPP(lo, 0x141); hi = FLEET_DPP(hi, 0x141);
    } else if constexpr (K == 3) {
        lo = FLEET_DPP(lo, 0x140); hi = FLEET_DPP(hi, 0x140);
    } else if constexpr (K == 4) {
        lo = __builtin_amdgcn_ds_swizzle(lo, 0x401F); hi = __builtin_amdgcn_ds_swizzle(hi, 0x401F);
    } else {
        const int a = (int)(((fm_tid() & (kLanes - 1)) ^ 32u) << 2);
        lo = __builtin_amdgcn_ds_bpermute(a, lo); hi = __builtin_amdgcn_ds_bpermute(a, hi);
    }
    return __longlong_as_double(((long long)hi << 32) | (unsigned int)lo);
}

// x plus its step-K partner's x. The cross-row steps (K = 4: lane ^ 16,
// K = 5: lane ^ 32) go through permlane swaps of both halves: the swap's two
// results hold the lane's own value and its partner's, in an order that
// depends on the row, and their sum is the same either way.
template <int K>
__device__ __forceinline__ double msum_pair64(double x) {
    if constexpr (K >= 4) {
        const long long b = __double_as_longlong(x);
        const uint32_t lo = (uint32_t)(b & 0xffffffffll), hi = (uint32_t)(b >> 32);
        const auto sl = K == 4 ? __builtin_amdgcn_permlane16_swap(lo, lo, false, false)
                               : __builtin_amdgcn_permlane32_swap(lo, lo, false, false);
        const auto sh = K == 4 ? __builtin_amdgcn_permlane16_swap(hi, hi, false, false)
                               : __builtin_amdgcn_permlane32_swap(hi, hi, false, false);
        const double a = __longlong_as_double((long long)(((uint64_t)sh[0] << 32) | sl[0]));
        const double c = __longlong_as_double((long long)(((uint64_t)sh[1] << 32) | sl[1]));
        return a + c;
    } else {
        return x + msum_xchg64<K>(x);
    }
}

template <int K, int LEN, int N>
__device__ __forceinline__ void msum_step64(double (&v)[N]) {
    if constexpr (K < 6) {
        if constexpr (LEN > 1) {
            const bool up = __builtin_popcount((fm_tid() & (kLanes - 1)) & kMsumDual[K]) & 1;
#pragma unroll
            for (int j = 0; j < LEN / 2; ++j) {
                const double lo = msum_pair64<K>(v[j]);
                const double hi = msum_pair64<K>(v[j + LEN / 2]);
                v[j] = up ? hi : lo;
            }
            msum_step64<K + 1, LEN / 2, N>(v);
        } else {
            v[0] = msum_pair64<K>(v[0]);
            msum_step64<K + 1, 1, N>(v);
        }
    }
}

template <int N>
__device__ __forceinline__ double wave_msum64(double (&v)[N]) {
    static_assert(N >= 1 && N <= 64 && (N & (N - 1)) == 0, "N is a power of two <= 64");
    msum_step64<0, N, N>(v);
    return v[0];
}

// The lowest lane that receives value i of wave_msum<N> / wave_msum64<N>.
constexpr int msum_index_c(int n, int lane) {
    int idx = 0;
    for (int k = 0; (1 << k) < n; ++k) {
        int m = lane & kMsumDual[k], p = 0;
        while (m) { p ^= m & 1; m >>= 1; }
        idx = (idx << 1) | p;
    }
    return idx;
}
constexpr int msum_lane_of(int n, int i) {
    for (int lane = 0; lane < kLanes; ++lane)
        if (msum_index_c(n, lane) == i) return lane;
    return -1;
}
struct LaneTable16 {
    int lane[16];
};
constexpr LaneTable16 make_lane_table16() {
    LaneTable16 t{};
    for (int i = 0; i < 16; ++i) t.lane[i] = msum_lane_of(16, i);
    return t;
}
constexpr LaneTable16 kMsumLane16 = make_lane_table16();
static_assert(kMsumLane16.lane[0] == 0 && kMsumLane16.lane[15] >= 0, "lane table");

// bf16 chunk against 8 fp64 values (fp32 values widened once): each product
// is exact in fp64 and rounded once into the fp64 sum.
__device__ __forceinline__ double dot8_xd(const u32x4& w, const double* x, double acc) {
    acc = fma((double)bf_lo(w.x), x[0], acc);
    acc = fma((double)bf_hi(w.x), x[1], acc);
    acc = fma((double)bf_lo(w.y), x[2], acc);
    acc = fma((double)bf_hi(w.y), x[3], acc);
    acc = fma((double)bf_lo(w.z), x[4], acc);
    acc = fma((double)bf_hi(w.z), x[5], acc);
    acc = fma((double)bf_lo(w.w), x[6], acc);
    acc = fma((double)bf_hi(w.w), x[7], acc);
    return acc;
}

// DeepseekV2 RoPE of 64 bf16-valued inputs v: reordered basis y = [v0, v2, ..,
// v62, v1, v3, .., v63]; out[i] = y[i] cos[i] - y[i+32] sin[i] (i < 32),
// y[i] cos[i] + y[i-32] sin[i] (i >= 32), two products and a sum, unfused, as
// the fp32 reference computes them; rounded to bf16. Returns out[i].
// Contraction is off for these three operations (HIP compiles with
// -ffp-contract=fast, and its __fmul_rn / __fadd_rn carry that flag into the
// inlined code): a fused multiply-add rounds twice instead of three times and
// moves about one result in 2^16 to the neighbouring bf16 value.
__device__ __forceinline__ float rope_one(const float* v, float cs_i, float sn_i, int i) {
#pragma clang fp contract(off)
    const int half = kRope / 2;
    const float y = i < half ? v[2 * i] : v[2 * (i - half) + 1];
    const float r = i < half ? -v[2 * i + 1] : v[2 * (i - half)];
    const float a = y * cs_i;
    const float b = r * sn_i;
    return bf16r(a + b);
}

// ---------------------------------------------------------------- polling
// A 16-byte group of published words is complete when each of its four
// 32-bit words carries this call's 16-bit tag.
__device__ __forceinline__ bool tagged(const u32x4& v, uint32_t tag) {
    return ((v.x & 0xffff0000u) == tag) & ((v.y & 0xffff0000u) == tag) &
           ((v.z & 0xffff0000u) == tag) & ((v.w & 0xffff0000u) == tag);
}

// Polls (device-scope 16-byte loads, a short sleep between rounds) until the
// group at byte offset `off` of `base` carries `tag` in every active lane.
// Called by whole waves; lanes with `active` false load nothing. A wait that
// runs out (or finds the sticky status set by another wait) raises
// FLEET_MOE_ABORT_ATTN_WAIT and returns false; the caller carries on with
// whatever was read, so the grid always drains.
// kOne: one poll in flight per wave (the layer's own launch: 21.0 -> 20.0 us
// against two); otherwise two, half a round trip apart (the whole-step
// kernel, where one in flight measured 0.2-0.5 us slower per layer).
template <bool kOne>
__device__ bool poll16(const void* base, int off, bool active, uint32_t tag, u32x4& v,
                       Workspace* ws) {
    const __amdgpu_buffer_rsrc_t r = rsrc(base);
    const u32x4 z = u32x4{0u, 0u, 0u, 0u};
    if constexpr (kOne) {
        // one poll in flight, a short sleep between rounds
        u32x4 a = active ? ld_dev16(r, off) : z;
        for (uint32_t it = 0;; ++it) {
            if (__all(!active || tagged(a, tag))) { v = a; return true; }
            __builtin_amdgcn_s_sleep(1);
            a = active ? ld_dev16(r, off) : z;
            if (it >= kSpinLimit || ((it & 1023) == 1023 && ld_agent(&ws->abort) != 0)) {
                if ((fm_tid() & (kLanes - 1)) == 0) raise(ws, FLEET_MOE_ABORT_ATTN_WAIT);
                v = a;
                return false;
            }
        }
    }
    // two polls in flight, half a round trip apart
    u32x4 a = active ? ld_dev16(r, off) : z;
    __builtin_amdgcn_s_sleep(8);
    u32x4 b = active ? ld_dev16(r, off) : z;
    for (uint32_t it = 0;; it += 2) {
        if (__all(!active || tagged(a, tag))) { v = a; return true; }
        a = active ? ld_dev16(r, off) : z;
        if (__all(!active || tagged(b, tag))) { v = b; return true; }
        b = active ? ld_dev16(r, off) : z;
        if (it >= kSpinLimit || ((it & 1022) == 1022 && ld_agent(&ws->abort) != 0)) {
            if ((fm_tid() & (kLanes - 1)) == 0) raise(ws, FLEET_MOE_ABORT_ATTN_WAIT);
            v = a;
            return false;
        }
        __builtin_amdgcn_s_sleep(1);
    }
}

// Payload of tagged words: an fp64 from four words, an fp32 from two.
__device__ __forceinline__ double tagged_f64(const u32x4& v) {
    const uint64_t b = ((uint64_t)(v.x & 0xffffu) << 48) | ((uint64_t)(v.y & 0xffffu) << 32) |
                       ((v.z & 0xffffu) << 16) | (v.w & 0xffffu);
    return __longlong_as_double((long long)b);
}
__device__ __forceinline__ float tagged_f32(uint32_t hi, uint32_t lo) {
    return __uint_as_float((hi << 16) | (lo & 0xffffu));
}
// Two tagged words (high payload half at the lower address) as one 64-bit
// device-scope store.
__device__ __forceinline__ void publish_pair(uint32_t* p, uint32_t bits, uint32_t tag) {
    const uint64_t w = ((uint64_t)(tag | (bits & 0xffffu)) << 32) | (tag | (bits >> 16));
    __hip_atomic_store(reinterpret_cast<uint64_t*>(p), w, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void publish_f32(uint32_t* p, float f, uint32_t tag) {
    publish_pair(p, __float_as_uint(f), tag);
}
__device__ __forceinline__ void publish_f64(uint32_t* p, double d, uint32_t tag) {
    const uint64_t b = (uint64_t)__double_as_longlong(d);
    publish_pair(p, (uint32_t)(b >> 32), tag);
    publish_pair(p + 2, (uint32_t)b, tag);
}

// ---------------------------------------------------------------- the layer kernel
struct Params {
    const float* x;
    float* x_out;
    const uint16_t* norm_in;
    const uint16_t* qkv;
    const uint16_t* kv_a_norm;
    const uint16_t* kv_b;
    const uint16_t* o_proj;
    uint16_t* cache;
    const float* cos;
    const float* sin;
    const int32_t* pos_dev;
    int32_t pos_host;
    int32_t max_pos;
    // the whole-step kernel only
    uint32_t epoch;             // this layer's call count
    const uint32_t* xin;        // tagged x [kXCopies][kHidden], or null: xin_row
    const uint16_t* xin_row;    // bf16 x (the embedding row)
    uint32_t xin_tag;
    uint32_t* xout;             // tagged x_out [kXCopies][kHidden]
    uint32_t xout_tag;
    double scale;
    float eps;
    Workspace* ws;
#if FLEET_ATTN_TRACE
    unsigned long long* trace;   // [kWG][kWaves][16] s_memrealtime stamps, or null
#endif
};

#if FLEET_ATTN_TRACE
#define ATTN_TRACE(k)                                                                    \
    do {                                                                                 \
        if (P.trace && lane == 0)                                                        \
            P.trace[((size_t)wg * kWaves + wave) * 16 + (k)] =                           \
                __builtin_amdgcn_s_memrealtime();                                        \
    } while (0)
#else
#define ATTN_TRACE(k) do {} while (0)
#endif

struct Lds {
    alignas(16) uint32_t xb[kHidden / 2];      // x_norm as bf16 pairs
    alignas(16) float xraw[kHidden];           // x itself (the whole-step kernel)
    double red[2 * kWaves];
    union {
        struct {                                // S2
            double uk[kWaves][kUkRows][kQcCols];
            double uk2[kUkRows][kQcCols];
        } s2;
        struct {                                // S3
            alignas(16) float qc[kLora];
            float qpe_raw[kRope];
            float qpe[kRope];
            float kva[kLora + kRope];
            alignas(16) uint16_t row[kRowElems];    // the cache row of the current position
            double wm[kWaves], wl[kWaves], wf[kWaves];
            double wo[kWaves][kLora];
        } s3;
        struct {                                // S4
            double mo[kChunks][kQcCols];
            double mm[kChunks], ml[kChunks], f[kChunks];
            alignas(16) float oc[kLora];
            double uvr[kWaves][kUvRows];
        } s4;
        struct {                                // S5
            alignas(16) uint16_t outv[kHeads * kV];
            double opr[kWaves][kOpRows];
        } s5;
    } u;
};

// The first stage's rows of this wave: q rows of head h, 12 per workgroup
// (i = wave, and wave + 8 for waves 0..3); kv_a rows 3072 + wg + 256 i for
// waves 4..6 (i = wave - 4, the last only for wg < 64). w[0..3] holds row r0,
// w[4..7] row r1 (zeros where the wave has no second row).
__device__ __forceinline__ void first_rows(const uint16_t* qkv, int& r0, int& r1,
                                           u32x4 (&w)[8], bool issue) {
    const int wg = blockIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(fm_tid() >> 6);
    const int lane = fm_tid() & (kLanes - 1);
    const int h = (wg & 7) + 8 * ((wg >> 3) & 1);
    const int k = wg >> 4;
    r0 = h * (kNope + kRope) + k + kChunks * wave;
    r1 = wave < 4 ? h * (kNope + kRope) + k + kChunks * (wave + kWaves)
       : wave < 7 ? kQDim + wg + kWG * (wave - 4) : kQkvRows;
    if (!issue) return;
    const u32x4* a = reinterpret_cast<const u32x4*>(qkv + (int64_t)r0 * kHidden);
#pragma unroll
    for (int m = 0; m < 4; ++m) w[m] = ld_stream(a + lane + kLanes * m);
    if (r1 < kQkvRows) {
        const u32x4* b = reinterpret_cast<const u32x4*>(qkv + (int64_t)r1 * kHidden);
#pragma unroll
        for (int m = 0; m < 4; ++m) w[4 + m] = ld_stream(b + lane + kLanes * m);
    } else {
#pragma unroll
        for (int m = 0; m < 4; ++m) w[4 + m] = u32x4{0u, 0u, 0u, 0u};
    }
}
// The whole-step kernel's hand-over: the stage before this one issues these
// rows once its own last wait is done (into `pre`), so they are in flight
// while that stage finishes and the residual is handed over.
__device__ __forceinline__ void issue_first_rows(const uint16_t* qkv, u32x4 (&pre)[8]) {
    int r0, r1;
    first_rows(qkv, r0, r1, pre, true);
}

// The layer. kMega: inside the whole-step kernel (fleet_decode_step): the
// call count and the position come from the step (P.epoch, P.pos_host), x
// from the tagged exchange buffer P.xin (or, for layer 0, the bf16 embedding
// row P.xin_row), and x_out goes to the exchange buffer P.xout (and to
// P.x_out when that is not null). `pre` holds the first stage's rows; with
// pre_in they were issued by the stage before (otherwise here). `next` runs
// once this layer's last wait is done: the whole-step kernel issues the next
// stage's first loads there.
template <bool kMega, class Next>
__device__ __forceinline__ void attn_layer(const Params& P, Lds& L, u32x4 (&pre)[8], bool pre_in,
                                           Next&& next) {
    const int wg = blockIdx.x, tid = fm_tid(), lane = tid & (kLanes - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // uniform: branches on it are scalar
    Workspace* ws = P.ws;
    // the position: the step's, the host's, or *pos_dev through the scalar
    // cache (invalidated at every launch, so current after the launch
    // boundary), its latency hidden behind the position-independent loads
    // below; a bad position is rejected only after they are issued
    int pos = P.pos_host;
    if constexpr (!kMega) {
        if (P.pos_dev) pos = *(const __attribute__((address_space(4))) int32_t*)P.pos_dev;
    }
    ATTN_TRACE(0);
    const int h = (wg & 7) + 8 * ((wg >> 3) & 1);
    const int k = wg >> 4;

    // ---- the inputs of the first stage
    // the call count, written by the previous launch: a plain load (after the
    // launch boundary it is current; device-scope loads of one word by every
    // wave would queue at its memory channel)
    const uint32_t epoch = kMega ? P.epoch : ws->epoch + 1u;
    const uint32_t tag = (epoch & 0xffffu) << 16;
    float4 xv = make_float4(0.f, 0.f, 0.f, 0.f);
    if constexpr (!kMega) xv = reinterpret_cast<const float4*>(P.x)[tid];
    const uint2 gb = P.norm_in ? ld_global_u2(P.norm_in, tid)
                               : make_uint2(0x3f803f80u, 0x3f803f80u);   // bf16 1.0
    float x_own = (!kMega && tid < kOpRows) ? P.x[kOpRows * wg + tid] : 0.f;
    // the kv_a_layernorm weight (thread i: element i), needed in S3; raw bf16
    // bits, widened where used (widened here, the wave would wait for this
    // load before issuing the weight rows below)
    const uint32_t kvn_b = P.kv_a_norm ? (uint32_t)ld_global(P.kv_a_norm + tid) : 0x3f80u;
    int r0, r1;
    first_rows(P.qkv, r0, r1, pre, !(kMega && pre_in));
    const u32x4 wq0[4] = {pre[0], pre[1], pre[2], pre[3]};
    const u32x4 wq1[4] = {pre[4], pre[5], pre[6], pre[7]};
    if (!kMega && (pos < 0 || pos >= P.max_pos)) {
        if (wg == 0 && tid == 0) raise(ws, FLEET_MOE_ABORT_POSITION);
        return;
    }
    const int n_pos = pos + 1;
    const int C = (n_pos + kChunks - 1) / kChunks;      // positions per chunk
    const int n_used = (n_pos + C - 1) / C;             // chunks holding positions
    // S3's (head, chunk): XCD x (wg % 8) takes chunks 2x and 2x + 1 of all 16 heads, so
    // each cached row is fetched into one XCD's L2 only
    const int h3 = (wg >> 3) & 15;
    const int k3 = 2 * (wg & 7) + (wg >> 7);
    const int t0 = k3 * C;
    const int t1 = min(t0 + C, n_pos);
    const bool has_rows = k3 < n_used;
    const bool last = k3 == n_used - 1;                 // the chunk holding `pos`
    // this position's RoPE angle (thread i < 64: element i), needed in S3
    const float cs_t = tid < kRope ? P.cos[(int64_t)pos * kRope + tid] : 0.f;
    const float sn_t = tid < kRope ? P.sin[(int64_t)pos * kRope + tid] : 0.f;
    if constexpr (kMega) {
        // x: the embedding row, or every workgroup's published rows
        if (P.xin_row) {
            const uint2 b = reinterpret_cast<const uint2*>(P.xin_row)[tid];
            xv = make_float4(bf_lo(b.x), bf_hi(b.x), bf_lo(b.y), bf_hi(b.y));
        } else {
            xv = poll_x4(P.xin + (wg % kXCopies) * kHidden, P.xin_tag, &ws->abort,
                         FLEET_MOE_ABORT_STEP_WAIT);
        }
        reinterpret_cast<float4*>(L.xraw)[tid] = xv;
    }
    ATTN_TRACE(1);
    // ---- S1: RMSNorm, then this wave's rows of [q_proj ; kv_a]
    const float xnorm = norm2048(xv, gb, P.eps, L.xb, L.red);
    if constexpr (kMega) x_own = tid < kOpRows ? L.xraw[kOpRows * wg + tid] : 0.f;
    ATTN_TRACE(2);
    {
        u32x4 xq[4];
#pragma unroll
        for (int m = 0; m < 4; ++m) xq[m] = reinterpret_cast<const u32x4*>(L.xb)[lane + kLanes * m];
        const bool two = r1 < kQkvRows;
        float a0, a1;
        dot_rows2_bf16(wq0, wq1, two, xq, xnorm, a0, a1);
        if (lane == 0) {
            ws->qkv[r0] = a0;
            st_agent(&ws->qkv_t[r0], tag | bf16_bits(a0));
            if (two) {
                ws->qkv[r1] = a1;
                st_agent(&ws->qkv_t[r1], tag | bf16_bits(a1));
            }
        }
    }

    // S2's weight slice and S3's cache rows go in flight now, behind the first
    // stage's inputs: issued before the RMSNorm, these ~10 loads per wave
    // would hold up x and the q / kv_a rows.
    // W_UK of head h: row 16 wave + lane / 4, columns 32 k + 8 (lane % 4) .. + 7
    const u32x4 wuk = ld_stream(reinterpret_cast<const u32x4*>(
        P.kv_b + ((int64_t)h * kKvbRowsPerHead + kUkRows * wave + (lane >> 2)) * kLora +
        kQcCols * k + 8 * (lane & 3)));
    // this wave's first cache rows of the chunk (rows before `pos`; row `pos`
    // is derived from kv_a below). In a launch of its own the wave issues
    // them three at a time, waiting for each three before the next: issued
    // all at once, these rows (20 MB of L2 reads over the chip) compete with
    // the first stage's weight rows of the workgroups still streaming them
    // (all at once 23.3 us, one at a time 21.5, two 21.1, three 20.9, four
    // 21.0, five 21.5). In the whole-step kernel the first stage's rows were
    // issued by the stage before, and all at once is ~1.7 us faster per layer.
    u32x4 c8[kBatch];
    uint32_t kp[kBatch];
    const int t_end = min(t1, pos);
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
        const int t = t0 + wave + kWaves * i;
        if (t < t_end) {
            const uint16_t* row = P.cache + (int64_t)t * kRowElems;
            c8[i] = ld_global(reinterpret_cast<const u32x4*>(row) + lane);
            kp[i] = ld_global(row + kLora + lane);
            if constexpr (!kMega)
                if (i % 3 == 2) asm volatile("" : "+v"(kp[i]));   // the wait
        } else {
            c8[i] = u32x4{0u, 0u, 0u, 0u};
            kp[i] = 0u;
        }
    }

    ATTN_TRACE(3);
    // ---- S2: q_c[h][32k .. 32k+31] = sum over the 128 rows of W_UK q_nope
    {
        u32x4 qn;
        poll16<!kMega>(ws->qkv_t, 4 * (h * (kNope + kRope) + kUkRows * wave) + 16 * lane, lane < 4,
               tag, qn, ws);
        ATTN_TRACE(4);
        // lane needs q_nope[16 wave + lane / 4]: word (lane / 4) % 4 of lane lane / 16
        const int src = (lane >> 4) << 2;
        const uint32_t c0 = __builtin_amdgcn_ds_bpermute(src, qn.x);
        const uint32_t c1 = __builtin_amdgcn_ds_bpermute(src, qn.y);
        const uint32_t c2 = __builtin_amdgcn_ds_bpermute(src, qn.z);
        const uint32_t c3 = __builtin_amdgcn_ds_bpermute(src, qn.w);
        const int comp = (lane >> 2) & 3;
        const uint32_t wd = comp == 0 ? c0 : comp == 1 ? c1 : comp == 2 ? c2 : c3;
        const float q = __uint_as_float(wd << 16);
        // bf16 x bf16 products are exact in fp32, so every sum below is exact
        const uint32_t ww[4] = {wuk.x, wuk.y, wuk.z, wuk.w};
        double* dst = &L.u.s2.uk[wave][lane >> 2][8 * (lane & 3)];
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
            dst[2 * jj] = (double)(q * bf_lo(ww[jj]));
            dst[2 * jj + 1] = (double)(q * bf_hi(ww[jj]));
        }
        __syncthreads();
        {
            const int col = tid & (kQcCols - 1), part = tid >> 5;
            double s = 0.0;
#pragma unroll
            for (int w = 0; w < kWaves; ++w) s += L.u.s2.uk[w][part][col];
            L.u.s2.uk2[part][col] = s;
        }
        __syncthreads();
        if (tid < kQcCols) {
            double s = 0.0;
#pragma unroll
            for (int p = 0; p < kUkRows; ++p) s += L.u.s2.uk2[p][tid];
            const float qc = (float)s;
            ws->qc[h][kQcCols * k + tid] = qc;
            publish_f32(ws->qc_t[h][kQcCols * k + tid], qc, tag);
        }
        __syncthreads();
    }
    ATTN_TRACE(5);

    // ---- S3: the chunk's scores and fp64 softmax partial
    // S4's and S5's weight slices go in flight once this stage's polls are
    // done: issued earlier, they would sit ahead of the polls (a wave's loads
    // complete in order) and ahead of the cache rows in the memory queues.
    u32x4 wuv, wo[4];
    auto load_tail = [&]() {
        // W_UV of head h: row 8 k + lane / 8, columns 64 wave + 8 (lane % 8) .. + 7
        wuv = ld_stream(reinterpret_cast<const u32x4*>(
            P.kv_b + ((int64_t)h * kKvbRowsPerHead + kNope + kUvRows * k + (lane >> 3)) * kLora +
            64 * wave + 8 * (lane & 7)));
        // o_proj: row 8 wg + lane / 8, columns 256 wave + 32 (lane % 8) .. + 31
        const u32x4* p = reinterpret_cast<const u32x4*>(
            P.o_proj + (int64_t)(kOpRows * wg + (lane >> 3)) * kHidden + 256 * wave +
            32 * (lane & 7));
#pragma unroll
        for (int m = 0; m < 4; ++m) wo[m] = ld_stream(p + m);
    };
    if (has_rows) {
        u32x4 v;
        if (wave < 4) {
            // q_c of head h: 512 tagged words, 2 per lane
            poll16<!kMega>(ws->qc_t, 8 * (h3 * kLora + 128 * wave + 2 * lane), true, tag, v, ws);
            L.u.s3.qc[128 * wave + 2 * lane] = tagged_f32(v.x, v.y);
            L.u.s3.qc[128 * wave + 2 * lane + 1] = tagged_f32(v.z, v.w);
        } else if (wave == 4) {
            // q_pe of head h before RoPE: 64 words, 4 per lane
            poll16<!kMega>(ws->qkv_t, 4 * (h3 * (kNope + kRope) + kNope) + 16 * lane, lane < 16,
                   tag, v, ws);
            if (lane < 16) {
                L.u.s3.qpe_raw[4 * lane] = __uint_as_float(v.x << 16);
                L.u.s3.qpe_raw[4 * lane + 1] = __uint_as_float(v.y << 16);
                L.u.s3.qpe_raw[4 * lane + 2] = __uint_as_float(v.z << 16);
                L.u.s3.qpe_raw[4 * lane + 3] = __uint_as_float(v.w << 16);
            }
        } else if (last) {
            // kv_a (576 words): waves 5, 6, 7 take words 0..255, 256..511, 512..575
            const int w0 = 256 * (wave - 5);
            const bool act = w0 + 4 * lane < kLora + kRope;
            poll16<!kMega>(ws->qkv_t, 4 * (kQDim + w0) + 16 * lane, act, tag, v, ws);
            if (act) {
                L.u.s3.kva[w0 + 4 * lane] = __uint_as_float(v.x << 16);
                L.u.s3.kva[w0 + 4 * lane + 1] = __uint_as_float(v.y << 16);
                L.u.s3.kva[w0 + 4 * lane + 2] = __uint_as_float(v.z << 16);
                L.u.s3.kva[w0 + 4 * lane + 3] = __uint_as_float(v.w << 16);
            }
        }
        ATTN_TRACE(6);
        load_tail();
        __syncthreads();
        if (tid < kRope) {
            const float qp = rope_one(L.u.s3.qpe_raw, cs_t, sn_t, tid);
            L.u.s3.qpe[tid] = qp;
            if (k3 == 0) ws->qpe[h3][tid] = qp;
        }
        if (last) {
            // c = kv_a_layernorm(kv_a[:512]) (two bf16 roundings), k_pe = RoPE(kv_a[512:])
            const float c = L.u.s3.kva[tid];
            const double ss = wave_sum64((double)c * c);
            if (lane == 0) L.red[wave] = ss;
            __syncthreads();
            double ssq = 0.0;
#pragma unroll
            for (int w = 0; w < kWaves; ++w) ssq += L.red[w];
            const float var = (float)(ssq / (double)kLora);
            const float inv = __fdiv_rn(1.0f, sqrt_rn(var + P.eps));
            uint32_t gbits = kvn_b;
            asm volatile("" : "+v"(gbits));                // keeps the widening here
            const float g = __uint_as_float(gbits << 16);
            const uint16_t cb = (uint16_t)bf16_bits(bf16r(bf16r(c * inv) * g));
            L.u.s3.row[tid] = cb;
            uint16_t kb = 0;
            if (tid < kRope) {
                kb = (uint16_t)bf16_bits(rope_one(L.u.s3.kva + kLora, cs_t, sn_t, tid));
                L.u.s3.row[kLora + tid] = kb;
            }
            if (h3 == 0) {
                uint16_t* crow = P.cache + (int64_t)pos * kRowElems;
                st_global(crow + tid, cb);
                if (tid < kRope) st_global(crow + kLora + tid, kb);
            }
        }
        __syncthreads();
        ATTN_TRACE(7);

        double qd[8];
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) qd[jj] = (double)L.u.s3.qc[8 * lane + jj];
        const float qp = L.u.s3.qpe[lane];
        constexpr int kSum = 16;                           // kBatch rows reduced together
        static_assert(kBatch < kSum, "one reduction per batch, and a free value index");
        int ri = 0;                                        // the row whose score this lane gets
#pragma unroll
        for (int k2 = 0; k2 < 4; ++k2)
            ri = (ri << 1) | (__builtin_popcount(lane & kMsumDual[k2]) & 1);
        double m_w = -INFINITY, l_w = 0.0;
        double o[8] = {0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0};
        // rows before `pos`, kBatch at a time (rows past the chunk are zeros);
        // online softmax: rescale by exp(m_old - m_new), add exp(s - m_new) c
        for (int base = t0 + wave, b = 0; base < t_end; base += kWaves * kBatch, ++b) {
            if (b > 0) {
#pragma unroll
                for (int i = 0; i < kBatch; ++i) {
                    const int t = min(base + kWaves * i, t_end - 1);   // clamped: a real row
                    const uint16_t* row = P.cache + (int64_t)t * kRowElems;
                    c8[i] = ld_global(reinterpret_cast<const u32x4*>(row) + lane);
                    kp[i] = ld_global(row + kLora + lane);
                }
            }
            double a[kSum];
#pragma unroll
            for (int i = 0; i < kSum; ++i)
                a[i] = i < kBatch ? dot8_xd(c8[i], qd, (double)(__uint_as_float(kp[i] << 16) * qp)) : 0.0;
            const double tot = wave_msum64(a);
            const bool valid = ri < kBatch && base + kWaves * ri < t_end;
            const double sv = valid ? tot * P.scale : -INFINITY;
            const double m_new = fmax(m_w, wave_max64(sv));
            // one exponential per lane: the rows' exp(s - m_new) in the lanes
            // that hold a row, the rescale exp(m_old - m_new) in the last lane
            // (whose value index, 15, holds no row)
            const double ev = exp(ri == kSum - 1 ? m_w - m_new : sv - m_new);
            const double fo = readlane64(ev, kMsumLane16.lane[kSum - 1]);   // 0 while nothing is accumulated
            l_w *= fo;
#pragma unroll
            for (int jj = 0; jj < 8; ++jj) o[jj] *= fo;
#pragma unroll
            for (int i = 0; i < kBatch; ++i) {
                const double e = readlane64(ev, kMsumLane16.lane[i]);
                uint32_t cw[4] = {c8[i].x, c8[i].y, c8[i].z, c8[i].w};
                // widen again rather than keep the score loop's 96 widened values
                // alive across the reduction (the compiler would share them)
                asm("" : "+v"(cw[0]), "+v"(cw[1]), "+v"(cw[2]), "+v"(cw[3]));
                l_w += e;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    o[2 * q] = fma(e, (double)bf_lo(cw[q]), o[2 * q]);
                    o[2 * q + 1] = fma(e, (double)bf_hi(cw[q]), o[2 * q + 1]);
                }
            }
            m_w = m_new;
        }
        // the row of `pos`, derived from kv_a above
        if (last && (pos - t0) % kWaves == wave) {
            const u32x4 rc = reinterpret_cast<const u32x4*>(L.u.s3.row)[lane];
            const float rk = __uint_as_float((uint32_t)L.u.s3.row[kLora + lane] << 16);
            const double sv = wave_sum64(dot8_xd(rc, qd, (double)(rk * qp))) * P.scale;
            const double m_new = fmax(m_w, sv);
            const double ex = exp(lane == 0 ? m_w - m_new : sv - m_new);   // one per lane
            const double fo = readlane64(ex, 0);
            const double e = readlane64(ex, 1);
            const uint32_t cw[4] = {rc.x, rc.y, rc.z, rc.w};
            l_w = fma(l_w, fo, e);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                o[2 * q] = fma(e, (double)bf_lo(cw[q]), o[2 * q] * fo);
                o[2 * q + 1] = fma(e, (double)bf_hi(cw[q]), o[2 * q + 1] * fo);
            }
            m_w = m_new;
        }
        ATTN_TRACE(8);
        if (lane == 0) {
            L.u.s3.wm[wave] = m_w;
            L.u.s3.wl[wave] = l_w;
        }
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) L.u.s3.wo[wave][8 * lane + jj] = o[jj];
        __syncthreads();
        double M = -INFINITY;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) M = fmax(M, L.u.s3.wm[w]);
        if (tid < kWaves) L.u.s3.wf[tid] = exp(L.u.s3.wm[tid] - M);
        __syncthreads();
        double O = 0.0, Ls = 0.0;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            O = fma(L.u.s3.wf[w], L.u.s3.wo[w][tid], O);
            Ls = fma(L.u.s3.wf[w], L.u.s3.wl[w], Ls);
        }
        publish_f64(ws->o_t[h3][k3][tid], O, tag);
        if (tid == 0) {
            publish_f64(&ws->ml_t[h3][k3][0], M, tag);
            publish_f64(&ws->ml_t[h3][k3][4], Ls, tag);
        }
    } else {
        load_tail();
        // A chunk without positions (pos < 15) still publishes, a neutral
        // partial (max -inf, sums 0) that no merge reads: every polled word
        // is then rewritten on every call, so a word is never older than one
        // call and its 16-bit tag can never equal the current one by wrapping.
        publish_f64(ws->o_t[h3][k3][tid], 0.0, tag);
        if (tid == 0) {
            publish_f64(&ws->ml_t[h3][k3][0], -INFINITY, tag);
            publish_f64(&ws->ml_t[h3][k3][4], 0.0, tag);
        }
    }
    ATTN_TRACE(9);
    __syncthreads();

    // ---- S4: o_c[h][32k .. 32k+31] from the chunk partials, then W_UV rows 8k .. 8k+7
    {
        // wave w: chunks 2w and 2w + 1 (column 32k + lane % 32), and their max / sum
        const int c = 2 * wave + (lane >> 5);
        u32x4 v;
        poll16<!kMega>(ws->o_t, (int)(((h * kChunks + c) * kLora + kQcCols * k + (lane & 31)) * 16),
               c < n_used, tag, v, ws);
        if (c < n_used) L.u.s4.mo[c][lane & 31] = tagged_f64(v);
        const int cm = 2 * wave + (lane >> 1);
        poll16<!kMega>(ws->ml_t, (int)(((h * kChunks + cm) * 8 + 4 * (lane & 1)) * 4),
               lane < 4 && cm < n_used, tag, v, ws);
        if (lane < 4 && cm < n_used) {
            if (lane & 1) L.u.s4.ml[cm] = tagged_f64(v);
            else L.u.s4.mm[cm] = tagged_f64(v);
        }
        ATTN_TRACE(10);
        __syncthreads();
        if (tid < kChunks) {
            double M = -INFINITY;
            for (int q = 0; q < n_used; ++q) M = fmax(M, L.u.s4.mm[q]);
            L.u.s4.f[tid] = tid < n_used ? exp(L.u.s4.mm[tid] - M) : 0.0;
        }
        __syncthreads();
        if (tid < kQcCols) {
            double O = 0.0, Ls = 0.0;
            for (int q = 0; q < n_used; ++q) {
                O = fma(L.u.s4.f[q], L.u.s4.mo[q][tid], O);
                Ls = fma(L.u.s4.f[q], L.u.s4.ml[q], Ls);
            }
            publish_f32(ws->oc_t[h][kQcCols * k + tid], (float)(O / Ls), tag);
        }
        ATTN_TRACE(11);
        // o_c of head h, columns 64 wave .. 64 wave + 63 (two per lane)
        poll16<!kMega>(ws->oc_t, 8 * (h * kLora + 64 * wave + 2 * lane), lane < 32, tag, v, ws);
        ATTN_TRACE(12);
        if (lane < 32) {
            L.u.s4.oc[64 * wave + 2 * lane] = tagged_f32(v.x, v.y);
            L.u.s4.oc[64 * wave + 2 * lane + 1] = tagged_f32(v.z, v.w);
        }
        __syncthreads();
        float ov[8];
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) ov[jj] = L.u.s4.oc[64 * wave + 8 * (lane & 7) + jj];
        const double a = sum8_lanes(dot8_xf(wuv, ov, 0.0));
        if ((lane & 7) == 0) L.u.s4.uvr[wave][lane >> 3] = a;
        __syncthreads();
        if (tid < kUvRows) {
            double s = 0.0;
#pragma unroll
            for (int w = 0; w < kWaves; ++w) s += L.u.s4.uvr[w][tid];
            const float ob = bf16r((float)s);
            const uint32_t word = tag | bf16_bits(ob);
#pragma unroll
            for (int c = 0; c < kOutCopies; ++c)
                st_agent(&ws->out_t[c][h * kV + kUvRows * k + tid], word);
        }
        __syncthreads();
    }
    ATTN_TRACE(13);

    // ---- S5: o_proj rows 8 wg .. 8 wg + 7 and the residual add
    {
        u32x4 v;
        poll16<!kMega>(ws->out_t[wg % kOutCopies], 4 * (256 * wave + 4 * lane), true, tag, v, ws);
        ATTN_TRACE(14);
        next();
        reinterpret_cast<uint2*>(L.u.s5.outv)[64 * wave + lane] =
            make_uint2((v.x & 0xffffu) | (v.y << 16), (v.z & 0xffffu) | (v.w << 16));
        __syncthreads();
        // Every workgroup published its head outputs with this call's tag, so
        // every one has read the call count: workgroup 0 can advance it now,
        // for the next call (which starts after this launch has ended).
        if (!kMega && wg == 0 && tid == 0) st_agent(&ws->epoch, epoch);
        const u32x4* hv = reinterpret_cast<const u32x4*>(L.u.s5.outv + 256 * wave + 32 * (lane & 7));
        double a = 0.0;
#pragma unroll
        for (int m = 0; m < 4; ++m) a = dot8_x(wo[m], hv[m], a);
        a = sum8_lanes(a);
        if ((lane & 7) == 0) L.u.s5.opr[wave][lane >> 3] = a;
        __syncthreads();
        if (tid < kOpRows) {
            double s = 0.0;
#pragma unroll
            for (int w = 0; w < kWaves; ++w) s += L.u.s5.opr[w][tid];
            const float xo = bf16r(x_own + bf16r((float)s));
            if (!kMega || P.x_out) P.x_out[kOpRows * wg + tid] = xo;
            if constexpr (kMega) publish_x(P.xout, kOpRows * wg + tid, xo, P.xout_tag);
        }
    }
    ATTN_TRACE(15);
}

// ---------------------------------------------------------------- embed / lm_head / argmax
// Workgroup w: rows w + 256 j (400 of them); logits bf16; its best (max,
// lowest index on ties) goes to the candidate arrays.
struct HeadLds {
    alignas(16) uint32_t xb[kHidden / 2];
    double red[2 * kWaves];
    float bv_s[kWaves];
    int bi_s[kWaves];
    float av[kWG];              // the whole-step kernel's argmax: the candidates
    int ai[kWG];
};

struct HeadParams {
    const float* x;
    const uint16_t* norm;
    const uint16_t* W;
    float eps;
    float* logits;
    Workspace* ws;
    // the whole-step kernel only: x from the exchange buffer, the candidates
    // tagged with the step's call count, and the argmax in workgroup 0
    const uint32_t* xin;
    uint32_t xin_tag;
    uint32_t epoch;
    int32_t* token_out;
    int32_t* token_next;
    int32_t* pos_advance;
};

// Lowest index among equal maxima over the 256 candidates in LDS (threads
// t < 128 step down a tree; every thread of the workgroup calls it).
__device__ __forceinline__ void argmax256(float* v, int* ix) {
    const int t = fm_tid();
    for (int s = kWG / 2; s > 0; s >>= 1) {
        if (t < s) {
            const bool take = v[t + s] > v[t] || (v[t + s] == v[t] && ix[t + s] < ix[t]);
            if (take) {
                v[t] = v[t + s];
                ix[t] = ix[t + s];
            }
        }
        __syncthreads();
    }
}

template <bool kMega>
__device__ __forceinline__ void lmhead_body(const HeadParams& H, HeadLds& S) {
    const uint16_t* W = H.W;
    float* logits = H.logits;
    Workspace* ws = H.ws;
    const int wave = fm_tid() >> 6, lane = fm_tid() & (kLanes - 1);
    const uint2 gb = H.norm ? ld_global_u2(H.norm, fm_tid())
                            : make_uint2(0x3f803f80u, 0x3f803f80u);
    float4 xv;
    if constexpr (kMega)
        xv = poll_x4(H.xin + (blockIdx.x % kXCopies) * kHidden, H.xin_tag, &ws->abort,
                     FLEET_MOE_ABORT_STEP_WAIT);
    else
        xv = reinterpret_cast<const float4*>(H.x)[fm_tid()];
    const float xnorm = norm2048(xv, gb, H.eps, S.xb, S.red);
    u32x4 xq[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) xq[m] = reinterpret_cast<const u32x4*>(S.xb)[lane + kLanes * m];
    // This wave's rows first + stride i (i < 50), two at a time from two
    // buffers in turn (each wait is for the older pair while the newer one
    // streams); lane i keeps row i's logit until the one store at the end,
    // since a store among the loads would make every wait a full drain.
    constexpr int kRowsPerWave = kVocab / (kWG * kWaves);   // 50
    constexpr int kPairsPerWave = kRowsPerWave / 2;          // 25
    static_assert(kVocab % (kWG * kWaves) == 0 && kRowsPerWave % 2 == 0 &&
                      kPairsPerWave % 2 == 1 && kRowsPerWave <= kLanes,
                  "lm_head rows: 25 pairs per wave, the last in buffer A");
    const int first = blockIdx.x + kWG * wave, stride = kWG * kWaves;
    float bv = -INFINITY, lg = 0.f;
    int bi = 0x7fffffff;
    auto take = [&](int i, float v0, float v1) {
        lg = lane == i ? v0 : lg;
        lg = lane == i + 1 ? v1 : lg;
        const int row = first + stride * i;
        if (v0 > bv) { bv = v0; bi = row; }        // rows ascend: ties keep the lower
        if (v1 > bv) { bv = v1; bi = row + stride; }
    };
    u32x4 a0[4], a1[4], b0[4], b1[4];
    load_row(W, first, a0);
    load_row(W, first + stride, a1);
    for (int p = 0; p + 1 < kPairsPerWave; p += 2) {
        load_row(W, first + stride * (2 * p + 2), b0);
        load_row(W, first + stride * (2 * p + 3), b1);
        float v0, v1;
        dot_rows2_bf16(a0, a1, true, xq, xnorm, v0, v1);
        take(2 * p, v0, v1);
        load_row(W, first + stride * (2 * p + 4), a0);
        load_row(W, first + stride * (2 * p + 5), a1);
        dot_rows2_bf16(b0, b1, true, xq, xnorm, v0, v1);
        take(2 * p + 2, v0, v1);
    }
    {
        float v0, v1;
        dot_rows2_bf16(a0, a1, true, xq, xnorm, v0, v1);
        take(kRowsPerWave - 2, v0, v1);
    }
    if (logits && lane < kRowsPerWave) logits[first + stride * lane] = lg;
    if (lane == 0) {
        S.bv_s[wave] = bv;
        S.bi_s[wave] = bi;
    }
    __syncthreads();
    if (fm_tid() == 0) {
        for (int w8 = 1; w8 < kWaves; ++w8)
            if (S.bv_s[w8] > bv || (S.bv_s[w8] == bv && S.bi_s[w8] < bi)) {
                bv = S.bv_s[w8];
                bi = S.bi_s[w8];
            }
        if constexpr (kMega) {
            const uint64_t t = (uint64_t)H.epoch << 32;
            __hip_atomic_store(&ws->cand_t[blockIdx.x][0], t | __float_as_uint(bv),
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(&ws->cand_t[blockIdx.x][1], t | (uint32_t)bi, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        } else {
            ws->cand_v[blockIdx.x] = bv;
            ws->cand_i[blockIdx.x] = bi;
        }
    }
    if constexpr (kMega) {
        // workgroup 0 takes the argmax of every workgroup's candidate
        if (blockIdx.x == 0) {
            const int t = fm_tid();
            if (t < kWG) {
                uint64_t a = 0, b = 0;
                for (uint32_t it = 0;; ++it) {
                    a = __hip_atomic_load(&ws->cand_t[t][0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    b = __hip_atomic_load(&ws->cand_t[t][1], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    if ((uint32_t)(a >> 32) == H.epoch && (uint32_t)(b >> 32) == H.epoch) break;
                    if (it >= kSpinLimit || ((it & 1023) == 1023 && ld_agent(&ws->abort) != 0)) {
                        __hip_atomic_fetch_or(&ws->abort, FLEET_MOE_ABORT_STEP_WAIT,
                                              __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        break;
                    }
                    __builtin_amdgcn_s_sleep(1);
                }
                S.av[t] = __uint_as_float((uint32_t)a);
                S.ai[t] = (int)(uint32_t)b;
            }
            __syncthreads();
            argmax256(S.av, S.ai);
            if (t == 0) {
                if (H.token_out) *H.token_out = S.ai[0];
                if (H.token_next) *H.token_next = S.ai[0];
                if (H.pos_advance) *H.pos_advance += 1;
            }
        }
    }
}

}  // namespace attn
}  // namespace fleet_moe
