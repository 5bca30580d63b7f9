// Device helpers shared by the MoE kernels (gfx950, wave64).
//
// Numerics contract (the CPU oracle follows the same one):
//   * bf16 rounding is round-to-nearest-even on the fp32 bit pattern;
//   * reductions whose result must be reproducible bit for bit (RMSNorm mean of
//     squares, router logits, softmax) run in fp64 and are rounded once to fp32;
//   * every bf16 GEMV result is the exact dot product rounded once to fp32
//     and then to bf16: an fp32 evaluation is accepted when a rigorous error
//     bound proves its bf16 rounding equal to the exact one (certify_bf16),
//     and the exact fp64 sum of the exact products is used otherwise.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fleet_moe.h"

namespace fleet_moe {

// The workitem id, opaque to the compiler at each use: in the whole-step
// kernel every stage derives its lane and wave indices afresh, instead of the
// compiler hoisting them out of the layer loop and keeping them in registers
// across every stage (which made that kernel spill).
__device__ __forceinline__ int fm_tid() {
    int t = (int)__builtin_amdgcn_workitem_id_x();
    asm volatile("" : "+v"(t));
    return t;
}

// Loads through global-memory pointers. A pointer read from memory (the
// whole-step kernel's layer table) rather than taken from a kernel argument
// has no known address space, and the compiler would emit flat loads for it,
// which also count against the LDS wait counter: every LDS wait would then
// wait for the weight stream too. Loading through an address_space(1)
// pointer emits global loads whatever the pointer's origin.
template <class T>
using gmem_ptr = const __attribute__((address_space(1))) T*;
template <class T>
__device__ __forceinline__ T ld_global(const T* p) {
    return *(gmem_ptr<T>)p;
}
// (uint2 through a 64-bit load: the vector type's copy constructor takes a
// generic reference and would turn the load back into a flat one)
__device__ __forceinline__ uint2 ld_global_u2(const void* p, int i) {
    const uint64_t v = ld_global(reinterpret_cast<const uint64_t*>(p) + i);
    return make_uint2((uint32_t)v, (uint32_t)(v >> 32));
}
template <class T>
__device__ __forceinline__ void st_global(T* p, T v) {
    *(__attribute__((address_space(1))) T*)p = v;
}

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
    return __builtin_nontemporal_load((gmem_ptr<u32x4>)p);
}

__device__ __forceinline__ float bf_lo(uint32_t v) { return __uint_as_float(v << 16); }
__device__ __forceinline__ float bf_hi(uint32_t v) { return __uint_as_float(v & 0xffff0000u); }

__device__ __forceinline__ uint32_t bf16_bits(float f) {
    const uint32_t u = __float_as_uint(f);
    return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}
__device__ __forceinline__ float bf16r(float f) { return __uint_as_float(bf16_bits(f) << 16); }

// bf16 pair dot with fp32 accumulation (v_dot2c_f32_bf16):
// acc + a.lo * b.lo + a.hi * b.hi. The products of two bf16 values are exact.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float acc) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                           __builtin_bit_cast(bf16x2_t, b), acc, false);
}
// 8-element dot of two 16-byte bf16 chunks through four dot2 steps.
__device__ __forceinline__ float dot8_d2(const u32x4& w, const u32x4& x, float acc) {
    acc = dot2(w.x, x.x, acc);
    acc = dot2(w.y, x.y, acc);
    acc = dot2(w.z, x.z, acc);
    acc = dot2(w.w, x.w, acc);
    return acc;
}

// Exactly rounded dot products. Every product of two bf16 values is exact in
// fp32 (8-bit significands), and an fp64 sum of such products is exact as
// long as the terms span at most 53 bits (for these operands always, up to
// values far below anything that reaches an fp32 result), so the fp64 total
// does not depend on the order of the additions and one rounding to fp32
// gives the correctly rounded fp32 dot product. The decode path evaluates
// every weight GEMV this way, so its results do not depend on how the rows
// are split over lanes, waves or workgroups.
__device__ __forceinline__ double dot8_x(const u32x4& w, const u32x4& x, double acc) {
    acc += (double)(bf_lo(w.x) * bf_lo(x.x));
    acc += (double)(bf_hi(w.x) * bf_hi(x.x));
    acc += (double)(bf_lo(w.y) * bf_lo(x.y));
    acc += (double)(bf_hi(w.y) * bf_hi(x.y));
    acc += (double)(bf_lo(w.z) * bf_lo(x.z));
    acc += (double)(bf_hi(w.z) * bf_hi(x.z));
    acc += (double)(bf_lo(w.w) * bf_lo(x.w));
    acc += (double)(bf_hi(w.w) * bf_hi(x.w));
    return acc;
}

// bf16 weights against fp32 values (8 + 24 significand bits: the product is
// exact in fp64 and rounded once into the fp64 sum).
__device__ __forceinline__ double dot8_xf(const u32x4& w, const float* x, double acc) {
    acc = fma((double)bf_lo(w.x), (double)x[0], acc);
    acc = fma((double)bf_hi(w.x), (double)x[1], acc);
    acc = fma((double)bf_lo(w.y), (double)x[2], acc);
    acc = fma((double)bf_hi(w.y), (double)x[3], acc);
    acc = fma((double)bf_lo(w.z), (double)x[4], acc);
    acc = fma((double)bf_hi(w.z), (double)x[5], acc);
    acc = fma((double)bf_lo(w.w), (double)x[6], acc);
    acc = fma((double)bf_hi(w.w), (double)x[7], acc);
    return acc;
}

// Certified fast path for exactly rounded bf16 results. A dot product of
// bf16 operands evaluated in fp32 (v_dot2 chains, a fixed summation tree)
// differs from the exact value s by at most
//   E = gamma_d * sum |w_i x_i| <= gamma_d * ||w||_2 * ||x||_2,
// gamma_d = d u / (1 - d u), d the largest number of roundings on any path
// from a product to the result, u = 2^-23 (one ulp per rounding, whatever
// rounding v_dot2 uses internally, two roundings per v_dot2). With lo / hi
// the computed value minus / plus E widened by two of its ulps (so the
// fp32 subtraction and addition cannot round inwards), every s in [lo, hi]
// has fp32(s) in [lo, hi]; bf16 rounding is monotone, so when lo and hi
// round to the same bf16, that value is bf16(fp32(s)) -- the exactly rounded
// result -- and `out` receives it. Otherwise (a result near a bf16 rounding
// boundary, non-finite values) the caller evaluates the exact dot product.
// w2 is the computed sum of w_i^2 and xnorm the computed ||x||_2; the factor
// 1 + 2^-10 covers their own rounding, the square root's and the bound's,
// and 2^-100 (1 + ||w|| + xnorm) any flush of values below 2^-126.
__device__ __forceinline__ float cert_gamma(int depth) {
    const float du = (float)depth * 1.1920929e-7f;            // d * 2^-23
    return du / (1.0f - du) * 1.0009766f;                     // * (1 + 2^-10)
}
__device__ __forceinline__ bool certify_bf16(float a, float w2, float xnorm, float gamma,
                                             float& out) {
    const float wn = __builtin_sqrtf(fmaxf(w2, 0.f));
    const float e = gamma * wn * xnorm + fabsf(a) * 2.3841858e-7f +
                    7.8886091e-31f * (1.0f + wn + xnorm);
    const float lo = a - e, hi = a + e;
    const uint32_t bl = bf16_bits(lo), bh = bf16_bits(hi);
    if (bl == bh && __builtin_isfinite(lo) && __builtin_isfinite(hi)) {
        out = __uint_as_float(bl << 16);
        return true;
    }
    return false;
}

// Pairwise sum of N values in a fixed tree of depth ceil(log2 N).
template <int N>
__device__ __forceinline__ float tree_sum(const float (&v)[N]) {
    if constexpr (N == 1) {
        return v[0];
    } else {
        constexpr int H = (N + 1) / 2;
        float a[H];
#pragma unroll
        for (int i = 0; i < H; ++i) a[i] = (2 * i + 1 < N) ? v[2 * i] + v[2 * i + 1] : v[2 * i];
        return tree_sum<H>(a);
    }
}
constexpr int tree_depth(int n) { return n <= 1 ? 0 : 1 + tree_depth((n + 1) / 2); }

// Wave reductions with DPP row operations (a few cycles each, no LDS
// round trip): xor-1 and xor-2 quad permutes, the half-row and row mirrors
// leave every lane of a 16-lane row holding the row sum, and the four row
// sums are added in a fixed order through v_readlane. Every lane returns the
// same value and the order of additions never changes, so results are
// bitwise reproducible.
// Every control used (quad permutes, row mirrors, row rotates) gives each
// lane a source inside its row, so no lane reads an "old" value: the move has
// none (bound_ctrl), and no register has to be cleared before it.
#define FLEET_DPP(v, ctrl) __builtin_amdgcn_mov_dpp((v), (ctrl), 0xF, 0xF, true)

__device__ __forceinline__ float wave_sum(float v) {
    v += __int_as_float(FLEET_DPP(__float_as_int(v), 0xB1));   // quad_perm [1,0,3,2]
    v += __int_as_float(FLEET_DPP(__float_as_int(v), 0x4E));   // quad_perm [2,3,0,1]
    v += __int_as_float(FLEET_DPP(__float_as_int(v), 0x141));  // row_half_mirror
    v += __int_as_float(FLEET_DPP(__float_as_int(v), 0x140));  // row_mirror
    const int b = __float_as_int(v);
    return (__int_as_float(__builtin_amdgcn_readlane(b, 0)) +
            __int_as_float(__builtin_amdgcn_readlane(b, 16))) +
           (__int_as_float(__builtin_amdgcn_readlane(b, 32)) +
            __int_as_float(__builtin_amdgcn_readlane(b, 48)));
}

// Sum of lane l and lane l ^ 16 (permlane16_swap), then of l and l ^ 32
// (permlane32_swap): the swap's two results hold both rows, so their sum is
// the pair sum in every lane.
__device__ __forceinline__ float xor16_sum(float v) {
    const auto s = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v),
                                                    false, false);
    return __uint_as_float(s[0]) + __uint_as_float(s[1]);
}
__device__ __forceinline__ float xor32_sum(float v) {
    const auto s = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v),
                                                    false, false);
    return __uint_as_float(s[0]) + __uint_as_float(s[1]);
}

// N wave sums at once (N = 1, 2, 4, 8 or 16): lane l returns the sum over
// all 64 lanes of v[l % N] (wave_msum below maps sums to lanes differently).
// Each of the first log2 N levels halves the values a lane holds: it keeps
// the half its lane bit k selects and adds the partner's copy of that half,
// the partner being lane ^ 1, lane ^ 2 (quad permutes), then lane + 4 and
// lane + 8 within the row of 16 (row rotates; the partner always has the
// opposite bit k and the same lower bits, and the rotations cover every lane
// of the row once). The remaining levels add the single value the same way,
// then across rows and halves. N sums cost about 3N + 10 instructions
// instead of N full reductions, and each result is a binary tree of 63 fp32
// additions, six roundings deep. For N >= 8 every lane holding a value gets
// the same tree; for N <= 4 the single-value level on the rotate by 4 pairs
// lanes asymmetrically (lane l takes (a_l + a_l-4) + (a_l-8 + a_l-12), lane
// l + 4 takes (a_l+4 + a_l) + (a_l-4 + a_l-8)), so lanes holding the same sum
// may differ in its last bit: a branch on a result must follow one lane's
// value (__ballot / readlane), never each lane's own.
template <int K, int N>
__device__ __forceinline__ void nsum_level(float (&v)[N], int lane) {
    constexpr int kCtrl = K == 0 ? 0xB1 : K == 1 ? 0x4E : K == 2 ? 0x124 : 0x128;
    constexpr int n = N >> K;                 // values held entering level K
    if constexpr (n > 1) {
        const bool bit = (lane >> K) & 1;
#pragma unroll
        for (int i = 0; i < n / 2; ++i) {
            const float keep = bit ? v[2 * i + 1] : v[2 * i];
            const float send = bit ? v[2 * i] : v[2 * i + 1];
            v[i] = keep + __int_as_float(FLEET_DPP(__float_as_int(send), kCtrl));
        }
    } else {
        v[0] += __int_as_float(FLEET_DPP(__float_as_int(v[0]), kCtrl));
    }
}
template <int N>
__device__ __forceinline__ float wave_nsum(float (&v)[N]) {
    static_assert(N == 1 || N == 2 || N == 4 || N == 8 || N == 16, "N sums, N a power of 2 <= 16");
    const int lane = fm_tid() & 63;
    nsum_level<0>(v, lane);
    nsum_level<1>(v, lane);
    nsum_level<2>(v, lane);
    nsum_level<3>(v, lane);
    return xor32_sum(xor16_sum(v[0]));
}

template <int kCtrl>
__device__ __forceinline__ double dpp64(double v) {
    const long long b = __double_as_longlong(v);
    const int lo = FLEET_DPP((int)(b & 0xffffffffll), kCtrl);
    const int hi = FLEET_DPP((int)(b >> 32), kCtrl);
    return __longlong_as_double(((long long)hi << 32) | (unsigned int)lo);
}
__device__ __forceinline__ double readlane64(double v, int lane) {
    const long long b = __double_as_longlong(v);
    const int lo = __builtin_amdgcn_readlane((int)(b & 0xffffffffll), lane);
    const int hi = __builtin_amdgcn_readlane((int)(b >> 32), lane);
    return __longlong_as_double(((long long)hi << 32) | (unsigned int)lo);
}
__device__ __forceinline__ double wave_sum64(double v) {
    v += dpp64<0xB1>(v);
    v += dpp64<0x4E>(v);
    v += dpp64<0x141>(v);
    v += dpp64<0x140>(v);
    return (readlane64(v, 0) + readlane64(v, 16)) + (readlane64(v, 32) + readlane64(v, 48));
}

// Value of lane 0 in every lane (all lanes must be active).
__device__ __forceinline__ int wave_bcast(int v) { return __builtin_amdgcn_readfirstlane(v); }

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

// Buffer resource over a device buffer (raw, 32-bit byte offsets).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, 0x7fffffff, 0x00020000);
}
// 16-byte device-scope (sc1) load: sees the latest values written by any CU
// with device-scope stores, whatever this CU's caches hold.
__device__ __forceinline__ u32x4 ld_dev16(__amdgpu_buffer_rsrc_t r, int byte_off) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 16);
}

// Multi-value wave reduction: N values per lane (N a power of two <= 64) are
// summed over the 64 lanes in six exchange steps, lane L with lane L ^ a_k for
// a = {1, 2, 7, 15, 16, 32} (DPP quad_perm x2, row_half_mirror, row_mirror,
// then permlane16 / permlane32 swaps). In each of the first log2(N) steps a lane keeps
// half of its values (the upper half when parity(L & f_k) = 1, f = {5, 6, 12,
// 8, 16, 32}, the dual basis of a) and adds its partner's copy of that half;
// the remaining steps add the single value. On return v[0] of every lane holds
// the wave total of value msum_index<N>(L); the lanes sharing an index hold
// bitwise equal totals (each addition pairs the same two operands). Cost:
// about 1.5 N + 6 DPP adds, against 11 N for N separate wave sums.
template <int K>
__device__ __forceinline__ float msum_xchg(float x) {
    if constexpr (K == 0) return __int_as_float(FLEET_DPP(__float_as_int(x), 0xB1));
    else if constexpr (K == 1) return __int_as_float(FLEET_DPP(__float_as_int(x), 0x4E));
    else if constexpr (K == 2) return __int_as_float(FLEET_DPP(__float_as_int(x), 0x141));
    else if constexpr (K == 3) return __int_as_float(FLEET_DPP(__float_as_int(x), 0x140));
    else if constexpr (K == 4)
        return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(x), 0x401F));
    else
        return __int_as_float(__builtin_amdgcn_ds_bpermute(
            (int)(((fm_tid() & (kLanes - 1)) ^ 32u) << 2), __float_as_int(x)));
}
constexpr int kMsumDual[6] = {5, 6, 12, 8, 16, 32};

// x plus its step-K partner's x (the cross-row steps through permlane swaps).
template <int K>
__device__ __forceinline__ float msum_pair(float x) {
    if constexpr (K == 4) return xor16_sum(x);
    else if constexpr (K == 5) return xor32_sum(x);
    else return x + msum_xchg<K>(x);
}

template <int K, int LEN, int N>
__device__ __forceinline__ void msum_step(float (&v)[N]) {
    if constexpr (K < 6) {
        if constexpr (LEN > 1) {
            const bool up = __builtin_popcount((fm_tid() & (kLanes - 1)) & kMsumDual[K]) & 1;
#pragma unroll
            for (int j = 0; j < LEN / 2; ++j) {
                const float lo = msum_pair<K>(v[j]);
                const float hi = msum_pair<K>(v[j + LEN / 2]);
                v[j] = up ? hi : lo;
            }
            msum_step<K + 1, LEN / 2, N>(v);
        } else {
            v[0] = msum_pair<K>(v[0]);
            msum_step<K + 1, 1, N>(v);
        }
    }
}

template <int N>
__device__ __forceinline__ float wave_msum(float (&v)[N]) {
    static_assert(N >= 1 && N <= 64 && (N & (N - 1)) == 0, "N is a power of two <= 64");
    msum_step<0, N, N>(v);
    return v[0];
}

template <int N>
__device__ __forceinline__ int msum_index(int lane) {
    int idx = 0;
#pragma unroll
    for (int k = 0; (1 << k) < N; ++k)
        idx = (idx << 1) | (__builtin_popcount(lane & kMsumDual[k]) & 1);
    return idx;
}

// Softmax over one logit per lane (lanes >= n are padding) and greedy top-k
// with ties to the lowest index, for one whole wave, entirely in registers:
//   z = fp32(logit + bias), m = max z, e = exp(z - m) in fp64,
//   p = fp32(e / sum e) (sum in the fixed DPP order),
//   then k passes of: the wave max of p (exact in any order), a ballot of the
//   lanes holding it, the lowest such lane wins the slot and drops out.
// Selection rule of select_experts_from (src/kernels/fleet_kernel.hip:
// 469-494: highest p, equal p to the lower index, unnormalised weights).
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, __int_as_float(FLEET_DPP(__float_as_int(v), 0xB1)));
    v = fmaxf(v, __int_as_float(FLEET_DPP(__float_as_int(v), 0x4E)));
    v = fmaxf(v, __int_as_float(FLEET_DPP(__float_as_int(v), 0x141)));
    v = fmaxf(v, __int_as_float(FLEET_DPP(__float_as_int(v), 0x140)));
    const int b = __float_as_int(v);
    return fmaxf(fmaxf(__int_as_float(__builtin_amdgcn_readlane(b, 0)),
                       __int_as_float(__builtin_amdgcn_readlane(b, 16))),
                 fmaxf(__int_as_float(__builtin_amdgcn_readlane(b, 32)),
                       __int_as_float(__builtin_amdgcn_readlane(b, 48))));
}

__device__ inline void wave_softmax_topk(float logit, int n, int k, float scaling,
                                         int* ids_out, float* w_out, const float* bias) {
    const int lane = fm_tid() & (kLanes - 1);
    const bool valid = lane < n;
    const float z = valid ? (bias ? logit + bias[lane] : logit) : -INFINITY;
    const float m = wave_max(z);
    const double e = valid ? exp((double)z - (double)m) : 0.0;
    const double sum = wave_sum64(e);
    const float p = valid ? (float)(e / sum) : -INFINITY;
    float q = p;
    for (int j = 0; j < k; ++j) {
        const float best = wave_max(q);
        const unsigned long long hit = __ballot(q == best);
        const int sel = (int)__builtin_ctzll(hit);     // lowest lane holding the max
        if (lane == 0) {
            ids_out[j] = sel;
            w_out[j] = best * scaling;
        }
        if (lane == sel) q = -INFINITY;
    }
}

// ---------------------------------------------------------------- residual exchange
// The whole-step kernel (fleet_decode_step) hands the residual x (bf16-valued
// fp32) from stage to stage as tagged words, tag | bf16 bits, in kXCopies
// copies of kHidden words: every workgroup reads all of x (workgroup w polls
// copy w % kXCopies, so each line sees 32 pollers instead of 256), and each
// writer publishes its rows to every copy.
constexpr int kXCopies = 8;

// Polls this thread's four words x[4 tid .. 4 tid + 3] of the copy at `base`
// (512 threads cover the 2048) until all four carry `tag`; returns them as
// fp32. A wait that runs out sets `bit` in *abort and returns what it read.
__device__ inline float4 poll_x4(const uint32_t* base, uint32_t tag, uint32_t* abort,
                                 uint32_t bit) {
    const __amdgpu_buffer_rsrc_t r = rsrc(base);
    for (uint32_t it = 0;; ++it) {
        const u32x4 a = ld_dev16(r, 16 * (int)fm_tid());
        const bool ok = ((a.x & 0xffff0000u) == tag) & ((a.y & 0xffff0000u) == tag) &
                        ((a.z & 0xffff0000u) == tag) & ((a.w & 0xffff0000u) == tag);
        const bool done = __all(ok);
        if (done || it >= kSpinLimit || ((it & 1023) == 1023 && ld_agent(abort) != 0)) {
            if (!done && (fm_tid() & (kLanes - 1)) == 0)
                __hip_atomic_fetch_or(abort, bit, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            return make_float4(__uint_as_float(a.x << 16), __uint_as_float(a.y << 16),
                               __uint_as_float(a.z << 16), __uint_as_float(a.w << 16));
        }
        __builtin_amdgcn_s_sleep(1);
    }
}

// Row `row` of x (a bf16 value) into every copy at `xout`.
__device__ __forceinline__ void publish_x(uint32_t* xout, int row, float v, uint32_t tag) {
    const uint32_t w = tag | bf16_bits(v);
#pragma unroll
    for (int c = 0; c < kXCopies; ++c) st_agent(xout + c * kHidden + row, w);
}

}  // namespace fleet_moe
