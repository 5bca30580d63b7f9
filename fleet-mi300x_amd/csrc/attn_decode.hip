// The attention half of a DeepSeek-V2-Lite decoder layer (absorbed MLA), the
// embedding and the lm_head + argmax, at batch 1: with the dense and MoE FFN
// kernels they make the full 27-layer decode step.
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
// One layer is five launches on the caller's stream (each reads what the
// previous one wrote; the kernel boundary orders them):
//   qkv      256 workgroups: RMSNorm(x) and the 3648 rows of [q_proj ; kv_a]
//   prep     17 workgroups: per head q_c = W_UK^T q_nope (8 waves x 16 rows of
//            W_UK, 1 KB row loads, summed through LDS) and RoPE(q_pe); the 17th
//            normalises c, rotates k_pe and writes the cache row at pos
//   mla      16 heads x 64-position chunks: the chunk's 64 scores (a wave per
//            8 positions, rows held in registers), then its fp64 softmax
//            partial (max, sum of exp, sum exp * c) from the same registers
//   combine  16 heads x 8: merge the chunks into o_c, then 16 of the head's 128
//            outputs of W_UV o_c, bf16
//   oproj    256 workgroups: 8 rows of o_proj each, bf16, residual add
// The position can come from the host (an argument) or from device memory
// (pos_dev), so a whole decode step can be captured once in a HIP graph and
// replayed: the argmax kernel then advances *pos_dev itself. A device
// position outside [0, max_pos) raises FLEET_MOE_ABORT_POSITION and the layer
// does nothing past the check; a token outside the vocabulary raises
// FLEET_MOE_ABORT_TOKEN in the embedding, which then writes zeros.
//
// Cache layout [max_pos][512 + 64] bf16 per layer: c after kv_a_layernorm,
// then k_pe after RoPE in DeepseekV2's reordered basis. RoPE tables (cos, sin
// [max_pos][64] fp32) are the caller's.
#include <stddef.h>

#include <cmath>

#include "moe_common.h"

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
constexpr int kPosChunk = 64;                            // positions per mla workgroup
constexpr int kMaxPos = 4096;
constexpr int kMaxChunks = kMaxPos / kPosChunk;          // 64
constexpr int kVocab = 102400;
constexpr int kWG = 256;
constexpr int kThreads = 512;
constexpr int kWaves = kThreads / kLanes;
constexpr int kPerWave = kPosChunk / kWaves;             // 8 positions per wave in mla
constexpr int kUkRows = kNope / kWaves;                  // 16 W_UK rows per wave in prep

struct Workspace {
    uint32_t epoch;                            // unused by these kernels
    uint32_t pad0;
    uint32_t abort;                            // offset 8: sticky status
    uint32_t pad1[61];
    float qkv[kQkvRows];                       // bf16-valued
    float qc[kHeads][kLora];                   // absorbed queries
    float qpe[kHeads][kRope];                  // rotated, bf16-valued
    double part_m[kHeads][kMaxChunks];         // chunk partials of the softmax, fp64
    double part_l[kHeads][kMaxChunks];
    double part_o[kHeads][kMaxChunks][kLora];
    uint16_t out[kHeads * kV];                 // bf16 head outputs
    float cand_v[kWG];                         // lm_head: best logit per workgroup
    int32_t cand_i[kWG];
};
static_assert(offsetof(Workspace, abort) == 8, "status word offset");
static_assert(offsetof(Workspace, qkv) % 16 == 0, "16-byte aligned arrays");
static_assert(offsetof(Workspace, out) % 16 == 0, "head outputs are read with 16-byte loads");

struct Pos {
    const int32_t* dev;   // device position, or null: use `host`
    int32_t host;
    int32_t max_pos;
};

__device__ __forceinline__ int read_pos(const Pos& p) { return p.dev ? *p.dev : p.host; }
__device__ __forceinline__ bool pos_ok(const Pos& p, int pos) { return pos >= 0 && pos < p.max_pos; }

__device__ __forceinline__ void raise(Workspace* ws, uint32_t bit) {
    __hip_atomic_fetch_or(&ws->abort, bit, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// RMSNorm of a 2048-vector held 4 per thread (512 threads), the arithmetic of
// the MoE decode kernel (fp64 sum of squares, correctly rounded sqrt and
// division, two bf16 roundings); writes the bf16 result as packed pairs.
__device__ void norm2048(const float* x, const uint16_t* gamma, float eps, uint32_t* xb,
                         double* red) {
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & (kLanes - 1);
    const float4 xv = reinterpret_cast<const float4*>(x)[tid];
    const uint2 gb = gamma ? reinterpret_cast<const uint2*>(gamma)[tid]
                           : make_uint2(0x3f803f80u, 0x3f803f80u);
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
    __syncthreads();
}

__device__ __forceinline__ void load_row(const uint16_t* W, int64_t row, u32x4 (&w)[4]) {
    const int lane = threadIdx.x & (kLanes - 1);
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

// Rows first, first + stride, ... (< end) of a K = 2048 matrix against the
// packed bf16 vector xq; each wave keeps its next row in flight while it
// reduces the current one. f(row, value) receives every wave total.
template <typename F>
__device__ __forceinline__ void gemv_rows2048(const uint16_t* W, int first, int stride, int end,
                                              const u32x4 (&xq)[4], F f) {
    if (first >= end) return;
    u32x4 w[4], wn[4];
    load_row(W, first, w);
    for (int row = first; row < end; row += stride) {
        const int nxt = row + stride;
        if (nxt < end) load_row(W, nxt, wn);
        f(row, dot_row(w, xq));
#pragma unroll
        for (int m = 0; m < 4; ++m) w[m] = wn[m];
    }
}

// ---------------------------------------------------------------- qkv
// Row r of [q_proj ; kv_a] goes to workgroup r % 256, wave (r / 256) % 8.
__global__ __launch_bounds__(kThreads, 1) void qkv_kernel(const float* x, const uint16_t* norm,
                                                          const uint16_t* W, float eps,
                                                          Workspace* ws) {
    __shared__ alignas(16) uint32_t xb[kHidden / 2];
    __shared__ double red[kWaves];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & (kLanes - 1);
    norm2048(x, norm, eps, xb, red);
    u32x4 xq[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) xq[m] = reinterpret_cast<const u32x4*>(xb)[lane + kLanes * m];
    gemv_rows2048(W, blockIdx.x + kWG * wave, kWG * kWaves, kQkvRows, xq,
                  [&](int row, float a) {
                      if (lane == 0) ws->qkv[row] = bf16r(a);
                  });
}

// DeepseekV2 RoPE of 64 bf16-valued inputs v: reordered basis y = [v0, v2, ..,
// v62, v1, v3, .., v63]; out[i] = y[i] cos[i] - y[i+32] sin[i] (i < 32),
// y[i] cos[i] + y[i-32] sin[i] (i >= 32), two products and a sum, unfused, as
// the fp32 reference computes them; rounded to bf16. Returns out[i].
// Contraction is off for these three operations (HIP compiles with
// -ffp-contract=fast, and its __fmul_rn / __fadd_rn carry that flag into the
// inlined code): a fused multiply-add rounds twice instead of three times and
// moves about one result in 2^16 to the neighbouring bf16 value.
__device__ __forceinline__ float rope_one(const float* v, const float* cs, const float* sn, int i) {
#pragma clang fp contract(off)
    const int half = kRope / 2;
    const float y = i < half ? v[2 * i] : v[2 * (i - half) + 1];
    const float r = i < half ? -v[2 * i + 1] : v[2 * (i - half)];
    const float a = y * cs[i];
    const float b = r * sn[i];
    return bf16r(a + b);
}

// ---------------------------------------------------------------- prep
// blockIdx.x < 16: head h's absorbed query and rotated q_pe;
// blockIdx.x == 16: the new cache row.
__global__ __launch_bounds__(kThreads, 1) void prep_kernel(const uint16_t* kv_b,
                                                           const uint16_t* kv_a_norm,
                                                           const float* rope_cos,
                                                           const float* rope_sin, Pos P,
                                                           uint16_t* cache, float eps,
                                                           Workspace* ws) {
    __shared__ float v[kLora + kRope];
    __shared__ double part[kWaves][kLora];
    __shared__ double red[kWaves];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & (kLanes - 1);
    const int pos = read_pos(P);
    if (!pos_ok(P, pos)) {
        if (blockIdx.x == kHeads && tid == 0) raise(ws, FLEET_MOE_ABORT_POSITION);
        return;
    }
    const float* cs = rope_cos + (int64_t)pos * kRope;
    const float* sn = rope_sin + (int64_t)pos * kRope;
    if (blockIdx.x < kHeads) {
        const int h = blockIdx.x;
        const u32x4* wuk = reinterpret_cast<const u32x4*>(kv_b + (int64_t)h * kKvbRowsPerHead * kLora);
        u32x4 w[kUkRows];
#pragma unroll
        for (int r = 0; r < kUkRows; ++r)
            w[r] = ld_stream(wuk + (int64_t)(kUkRows * wave + r) * (kLora / kChunk) + lane);
        if (tid < kNope + kRope) v[tid] = ws->qkv[h * (kNope + kRope) + tid];
        __syncthreads();
        // lane holds columns 8 lane .. 8 lane + 7 of this wave's 16 rows; q_nope
        // is bf16-valued, so every product is exact in fp32 and the fp64 sums
        // are exact
        double acc[8] = {0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0};
#pragma unroll
        for (int r = 0; r < kUkRows; ++r) {
            const float q = v[kUkRows * wave + r];
            const uint32_t ww[4] = {w[r].x, w[r].y, w[r].z, w[r].w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                acc[2 * j] += (double)(q * bf_lo(ww[j]));
                acc[2 * j + 1] += (double)(q * bf_hi(ww[j]));
            }
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) part[wave][8 * lane + j] = acc[j];
        __syncthreads();
        double s = 0.0;
#pragma unroll
        for (int w8 = 0; w8 < kWaves; ++w8) s += part[w8][tid];
        ws->qc[h][tid] = (float)s;
        if (tid < kRope) ws->qpe[h][tid] = rope_one(v + kNope, cs, sn, tid);
        return;
    }
    // c = rms_norm(kv_a[:512], kv_a_norm) (two bf16 roundings), k_pe = RoPE(kv_a[512:])
    const float* kva = ws->qkv + kQDim;
    const float c = kva[tid];
    double ss = (double)c * c;
    ss = wave_sum64(ss);
    if (lane == 0) red[wave] = ss;
    if (tid < kRope) v[tid] = kva[kLora + tid];
    __syncthreads();
    double ssq = 0.0;
#pragma unroll
    for (int w8 = 0; w8 < kWaves; ++w8) ssq += red[w8];
    const float var = (float)(ssq / (double)kLora);
    const float inv = __fdiv_rn(1.0f, sqrt_rn(var + eps));
    const float g = kv_a_norm ? __uint_as_float((uint32_t)kv_a_norm[tid] << 16) : 1.0f;
    const float cn = bf16r(bf16r(c * inv) * g);
    uint16_t* row = cache + (int64_t)pos * kRowElems;
    row[tid] = (uint16_t)bf16_bits(cn);
    if (tid < kRope) row[kLora + tid] = (uint16_t)bf16_bits(rope_one(v, cs, sn, tid));
}

// ---------------------------------------------------------------- mla
// Workgroup (h, k): positions [64 k, min(64 k + 64, pos + 1)). Wave w holds
// positions 64 k + w + 8 j (j < 8) in registers (lane: c[8 lane .. 8 lane + 7]
// and k_pe[lane]). In fp64: the scores s = scale * (q_c . c + q_pe . k_pe),
// and the chunk partial m = max s, l = sum exp(s - m), o = sum exp(s - m) c.
__global__ __launch_bounds__(kThreads, 1) void mla_kernel(const uint16_t* cache, Pos P,
                                                          double scale, Workspace* ws) {
    __shared__ alignas(16) float qc[kLora];
    __shared__ float qpe[kRope];
    __shared__ double s[kPosChunk];
    __shared__ double part[kWaves][kLora];
    const int h = blockIdx.x, k = blockIdx.y;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & (kLanes - 1);
    const int pos = read_pos(P);
    if (!pos_ok(P, pos)) return;
    const int t0 = k * kPosChunk;
    if (t0 > pos) return;
    const int n = min(kPosChunk, pos + 1 - t0);
    u32x4 c8[kPerWave];
    float kp[kPerWave];
#pragma unroll
    for (int j = 0; j < kPerWave; ++j) {
        const int i = min(wave + kWaves * j, n - 1);          // clamped: always a written row
        const uint16_t* row = cache + (int64_t)(t0 + i) * kRowElems;
        c8[j] = reinterpret_cast<const u32x4*>(row)[lane];
        kp[j] = __uint_as_float((uint32_t)row[kLora + lane] << 16);
    }
    qc[tid] = ws->qc[h][tid];
    if (tid < kRope) qpe[tid] = ws->qpe[h][tid];
    __syncthreads();
    const float qp = qpe[lane];
#pragma unroll
    for (int j = 0; j < kPerWave; ++j) {
        double a = dot8_xf(c8[j], qc + 8 * lane, 0.0);
        a += (double)(kp[j] * qp);                             // bf16 x bf16: exact
        a = wave_sum64(a);
        if (lane == 0) {
            const int i = wave + kWaves * j;
            s[i] = i < n ? a * scale : -INFINITY;
        }
    }
    __syncthreads();
    double m = -INFINITY;
    for (int i = 0; i < n; ++i) m = fmax(m, s[i]);
    double o[8] = {0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0};
#pragma unroll
    for (int j = 0; j < kPerWave; ++j) {
        const int i = wave + kWaves * j;
        const double e = i < n ? exp(s[i] - m) : 0.0;
        const uint32_t cw[4] = {c8[j].x, c8[j].y, c8[j].z, c8[j].w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            o[2 * q] = fma(e, (double)bf_lo(cw[q]), o[2 * q]);
            o[2 * q + 1] = fma(e, (double)bf_hi(cw[q]), o[2 * q + 1]);
        }
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) part[wave][8 * lane + j] = o[j];
    __syncthreads();
    double acc = 0.0;
#pragma unroll
    for (int w8 = 0; w8 < kWaves; ++w8) acc += part[w8][tid];
    ws->part_o[h][k][tid] = acc;
    if (tid == 0) {
        double l = 0.0;
        for (int i = 0; i < n; ++i) l += exp(s[i] - m);
        ws->part_m[h][k] = m;
        ws->part_l[h][k] = l;
    }
}

// ---------------------------------------------------------------- combine
// Workgroup (h, g): the head's chunks merged into o_c (512, all threads), then
// outputs 16 g .. 16 g + 15 of W_UV o_c (a wave per two rows), bf16.
__global__ __launch_bounds__(kThreads, 1) void combine_kernel(const uint16_t* kv_b, Pos P,
                                                              Workspace* ws) {
    __shared__ alignas(16) float oc[kLora];
    const int h = blockIdx.x, g = blockIdx.y;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & (kLanes - 1);
    const int pos = read_pos(P);
    if (!pos_ok(P, pos)) return;
    const int n_chunks = pos / kPosChunk + 1;
    double M = -INFINITY;
    for (int k = 0; k < n_chunks; ++k) M = fmax(M, ws->part_m[h][k]);
    double L = 0.0, o = 0.0;
    for (int k = 0; k < n_chunks; ++k) {
        const double f = exp(ws->part_m[h][k] - M);
        L = fma(f, ws->part_l[h][k], L);
        o = fma(f, ws->part_o[h][k][tid], o);
    }
    oc[tid] = (float)(o / L);                                 // o_c, rounded once
    __syncthreads();
    const uint16_t* wuv = kv_b + ((int64_t)h * kKvbRowsPerHead + kNope) * kLora;
#pragma unroll
    for (int r = 0; r < 2; ++r) {
        const int dv = 16 * g + 2 * wave + r;
        const u32x4 w8 = reinterpret_cast<const u32x4*>(wuv + (int64_t)dv * kLora)[lane];
        const float a = (float)wave_sum64(dot8_xf(w8, oc + 8 * lane, 0.0));
        if (lane == 0) ws->out[h * kV + dv] = (uint16_t)bf16_bits(a);
    }
}

// ---------------------------------------------------------------- oproj
// Workgroup w: rows 8 w .. 8 w + 7, one per wave; x_out = bf16(x + bf16(o_proj . out)).
// Each output element is read from x and written to x_out by the same lane,
// so x_out may alias x.
__global__ __launch_bounds__(kThreads, 1) void oproj_kernel(const uint16_t* W, const float* x,
                                                            float* x_out, const Workspace* ws) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & (kLanes - 1);
    const int n = 8 * blockIdx.x + wave;
    u32x4 w[4], xq[4];
    load_row(W, n, w);
#pragma unroll
    for (int m = 0; m < 4; ++m) xq[m] = reinterpret_cast<const u32x4*>(ws->out)[lane + kLanes * m];
    const float a = dot_row(w, xq);
    if (lane == 0) x_out[n] = bf16r(x[n] + bf16r(a));
}

// ---------------------------------------------------------------- embed / lm_head / argmax
__global__ __launch_bounds__(kThreads, 1) void embed_kernel(const uint16_t* E, const int32_t* token,
                                                            float* x, Workspace* ws) {
    const int t = *token;
    const int i = threadIdx.x;
    if (t < 0 || t >= kVocab) {
        reinterpret_cast<float4*>(x)[i] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (i == 0) raise(ws, FLEET_MOE_ABORT_TOKEN);
        return;
    }
    const uint2 b = reinterpret_cast<const uint2*>(E + (int64_t)t * kHidden)[i];
    reinterpret_cast<float4*>(x)[i] = make_float4(bf_lo(b.x), bf_hi(b.x), bf_lo(b.y), bf_hi(b.y));
}

// Workgroup w: rows w + 256 j (400 of them); logits bf16; its best (max,
// lowest index on ties) goes to the candidate arrays.
__global__ __launch_bounds__(kThreads, 1) void lmhead_kernel(const float* x, const uint16_t* norm,
                                                             const uint16_t* W, float eps,
                                                             float* logits, Workspace* ws) {
    __shared__ alignas(16) uint32_t xb[kHidden / 2];
    __shared__ double red[kWaves];
    __shared__ float bv_s[kWaves];
    __shared__ int bi_s[kWaves];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & (kLanes - 1);
    norm2048(x, norm, eps, xb, red);
    u32x4 xq[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) xq[m] = reinterpret_cast<const u32x4*>(xb)[lane + kLanes * m];
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    gemv_rows2048(W, blockIdx.x + kWG * wave, kWG * kWaves, kVocab, xq, [&](int row, float a) {
        const float v = bf16r(a);
        if (logits && lane == 0) logits[row] = v;
        if (v > bv || (v == bv && row < bi)) {
            bv = v;
            bi = row;
        }
    });
    if (lane == 0) {
        bv_s[wave] = bv;
        bi_s[wave] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w8 = 1; w8 < kWaves; ++w8)
            if (bv_s[w8] > bv || (bv_s[w8] == bv && bi_s[w8] < bi)) {
                bv = bv_s[w8];
                bi = bi_s[w8];
            }
        ws->cand_v[blockIdx.x] = bv;
        ws->cand_i[blockIdx.x] = bi;
    }
}

__global__ __launch_bounds__(kWG, 1) void argmax_kernel(const Workspace* ws, int32_t* token_out,
                                                        int32_t* token_next, int32_t* pos_advance) {
    __shared__ float v[kWG];
    __shared__ int ix[kWG];
    const int t = threadIdx.x;
    v[t] = ws->cand_v[t];
    ix[t] = ws->cand_i[t];
    __syncthreads();
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
    if (t == 0) {
        if (token_out) *token_out = ix[0];
        if (token_next) *token_next = ix[0];
        if (pos_advance) *pos_advance += 1;
    }
}

}  // namespace attn
}  // namespace fleet_moe

using namespace fleet_moe;

int fleet_moe_check_dims(const fleet_moe_dims* d);
int fleet_moe_check_device(int min_cus);

static bool aligned(const void* p, size_t a) { return ((uintptr_t)p % a) == 0; }

extern "C" size_t fleet_attn_workspace_bytes(const fleet_moe_dims* dims) {
    if (fleet_moe_check_dims(dims) != 0) return 0;
    return (sizeof(attn::Workspace) + 255) & ~(size_t)255;
}

extern "C" int fleet_attn_decode(const fleet_attn_layer* layer, const float* x, float* x_out,
                                 uint16_t* cache, int32_t max_pos, int32_t pos,
                                 const int32_t* pos_dev, const float* rope_cos,
                                 const float* rope_sin, void* workspace, size_t workspace_bytes,
                                 const fleet_moe_dims* dims, hipStream_t stream) {
    if (!layer || !dims) return FLEET_MOE_ERR_ARG;
    if (int e = fleet_moe_check_dims(dims)) return e;
    if (!layer->qkv || !layer->kv_b || !layer->o_proj || !x || !x_out || !cache || !rope_cos ||
        !rope_sin || !workspace)
        return FLEET_MOE_ERR_ARG;
    if (max_pos < 1 || max_pos > attn::kMaxPos) return FLEET_MOE_ERR_ARG;
    if (!pos_dev && (pos < 0 || pos >= max_pos)) return FLEET_MOE_ERR_ARG;
    if (!aligned(layer->qkv, 16) || !aligned(layer->kv_b, 16) || !aligned(layer->o_proj, 16) ||
        !aligned(x, 16) || !aligned(x_out, 16) || !aligned(cache, 16) ||
        !aligned(workspace, 256) || (layer->norm_in && !aligned(layer->norm_in, 8)) ||
        (layer->kv_a_norm && !aligned(layer->kv_a_norm, 2)) || (pos_dev && !aligned(pos_dev, 4)) ||
        !aligned(rope_cos, 4) || !aligned(rope_sin, 4))
        return FLEET_MOE_ERR_ARG;
    if (workspace_bytes < sizeof(attn::Workspace)) return FLEET_MOE_ERR_WORKSPACE;
    if (int e = fleet_moe_check_device(attn::kWG)) return e;
    auto* ws = static_cast<attn::Workspace*>(workspace);
    const float eps = dims->rms_eps;
    const attn::Pos P = {pos_dev, pos, max_pos};
    // with a device position the grid covers every chunk of max_pos (chunks
    // past the position return at once)
    const int span = pos_dev ? max_pos : pos + 1;
    const int n_chunks = (span + attn::kPosChunk - 1) / attn::kPosChunk;
    // (qk_nope + qk_rope)^-0.5 * mscale(40, 0.707)^2 (src/host/reference_decode.py:
    // 78-83, 197-203), in double
    const double m = 0.1 * 0.707 * std::log(40.0) + 1.0;
    const double scale = std::pow(192.0, -0.5) * m * m;
    hipLaunchKernelGGL(attn::qkv_kernel, dim3(attn::kWG), dim3(attn::kThreads), 0, stream, x,
                       layer->norm_in, layer->qkv, eps, ws);
    hipLaunchKernelGGL(attn::prep_kernel, dim3(attn::kHeads + 1), dim3(attn::kThreads), 0, stream,
                       layer->kv_b, layer->kv_a_norm, rope_cos, rope_sin, P, cache, eps, ws);
    hipLaunchKernelGGL(attn::mla_kernel, dim3(attn::kHeads, n_chunks), dim3(attn::kThreads), 0,
                       stream, cache, P, scale, ws);
    hipLaunchKernelGGL(attn::combine_kernel, dim3(attn::kHeads, attn::kV / 16),
                       dim3(attn::kThreads), 0, stream, layer->kv_b, P, ws);
    hipLaunchKernelGGL(attn::oproj_kernel, dim3(kHidden / 8), dim3(attn::kThreads), 0, stream,
                       layer->o_proj, x, x_out, ws);
    return (int)hipGetLastError();
}

extern "C" int fleet_embed(const uint16_t* embed, const int32_t* token, float* x, void* workspace,
                           size_t workspace_bytes, hipStream_t stream) {
    if (!embed || !token || !x || !workspace || !aligned(embed, 16) || !aligned(x, 16) ||
        !aligned(token, 4) || !aligned(workspace, 256))
        return FLEET_MOE_ERR_ARG;
    if (workspace_bytes < sizeof(attn::Workspace)) return FLEET_MOE_ERR_WORKSPACE;
    hipLaunchKernelGGL(attn::embed_kernel, dim3(1), dim3(kHidden / 4), 0, stream, embed, token, x,
                       static_cast<attn::Workspace*>(workspace));
    return (int)hipGetLastError();
}

extern "C" int fleet_lm_head_argmax(const float* x, const uint16_t* final_norm,
                                    const uint16_t* lm_head, float* logits, int32_t* token_out,
                                    int32_t* token_next, int32_t* pos_advance, void* workspace,
                                    size_t workspace_bytes, const fleet_moe_dims* dims,
                                    hipStream_t stream) {
    if (int e = fleet_moe_check_dims(dims)) return e;
    if (!x || !lm_head || !workspace || !aligned(x, 16) || !aligned(lm_head, 16) ||
        !aligned(workspace, 256) || (logits && !aligned(logits, 4)) ||
        (final_norm && !aligned(final_norm, 8)) || (token_out && !aligned(token_out, 4)) ||
        (token_next && !aligned(token_next, 4)) || (pos_advance && !aligned(pos_advance, 4)))
        return FLEET_MOE_ERR_ARG;
    if (workspace_bytes < sizeof(attn::Workspace)) return FLEET_MOE_ERR_WORKSPACE;
    if (int e = fleet_moe_check_device(attn::kWG)) return e;
    auto* ws = static_cast<attn::Workspace*>(workspace);
    hipLaunchKernelGGL(attn::lmhead_kernel, dim3(attn::kWG), dim3(attn::kThreads), 0, stream, x,
                       final_norm, lm_head, dims->rms_eps, logits, ws);
    hipLaunchKernelGGL(attn::argmax_kernel, dim3(1), dim3(attn::kWG), 0, stream, ws, token_out,
                       token_next, pos_advance);
    return (int)hipGetLastError();
}
