// Multi-token grouped-expert MoE step (config: T tokens, each routed to 6 of
// 64 experts, plus the shared expert on every token).
//
// The reference has no kernel for this (it is batch-1 only); the semantics are
// HF DeepseekV2MoE.moe_infer (reference/modeling_deepseek.py:591-664): count
// tokens per expert, permute the (token, slot) entries so each expert's rows
// are contiguous, run each expert's SwiGLU on its rows, un-permute and combine
// per token with the rounding of src/host/reference_decode.py:280-287.
//
// Four launches on the caller's stream:
//   1. permute   - one workgroup: per-expert counts, offsets, and the stable
//                  position of every (token, slot) entry; per-expert work tiles.
//   2. gate/up   - every selected expert's interleaved gate/up rows in tiles
//                  of 16 rows x up to 64 tokens: bf16 MFMA (16x16x32) when the
//                  expert holds >= kMfmaMin tokens, a register-streamed GEMV
//                  over the expert's few tokens below that. h is bf16.
//   3. down      - same tiling over the 2048 down rows; the epilogue applies
//                  bf16(w * bf16(d)) per entry (shared: bf16(d)).
//   4. combine   - out[t] = bf16(bf16(sum_k part[t,k]) + shared[t]), k order.
// Weights stream once per (expert, 64-token group); activations come from L2.
#include <stddef.h>

#include "moe_common.h"

namespace fleet_moe {
namespace grouped {

constexpr int kMaxTokens = 256;
constexpr int kMaxEntries = kMaxTokens * kTopK;     // 1536
constexpr int kTileRows = 16;
constexpr int kGroup = 64;                          // tokens per weight pass (4 MFMA tiles)
constexpr int kGuTiles = 2 * kInter / kTileRows;    // 176 tiles of routed gate/up
constexpr int kSgTiles = 2 * kSharedInter / kTileRows;   // 352 tiles of shared gate/up
constexpr int kDnTiles = kHidden / kTileRows;       // 128 tiles of down rows
constexpr int kMfmaMin = 16;                        // tokens per expert for the MFMA path
constexpr int kWaves = 8;
constexpr int kThreads = kWaves * kLanes;
constexpr int kGrid = 256;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// Workspace. Header words match the decode workspace (status at offset 8).
struct Header {
    uint32_t epoch, exits, abort, n_tokens;
    uint32_t n_items_gu, n_items_dn, pad[58];
    int32_t cnt[kRouted];        // tokens per expert
    int32_t off[kRouted + 1];    // exclusive scan of cnt
    int32_t gu_base[kRouted + 2];   // first gate/up item of expert e; [64] = shared
    int32_t dn_base[kRouted + 2];
    int32_t pad2[1];
    int32_t ent_at[kMaxEntries]; // sorted position -> flat entry (t * 6 + k)
    int32_t pos_of[kMaxEntries]; // flat entry -> sorted position
};

struct Layout {
    size_t header, h_routed, h_shared, part, part_shared, total;
};

__host__ __device__ inline size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

__host__ __device__ inline Layout layout(int max_tokens) {
    Layout L;
    L.header = 0;
    L.h_routed = align256(sizeof(Header));
    L.h_shared = L.h_routed + align256((size_t)max_tokens * kTopK * kInter * 2);
    L.part = L.h_shared + align256((size_t)max_tokens * kSharedInter * 2);
    L.part_shared = L.part + align256((size_t)max_tokens * kTopK * kHidden * 2);
    L.total = L.part_shared + align256((size_t)max_tokens * kHidden * 2);
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
    uint16_t* h_routed;        // bf16 [6T][I], sorted positions
    uint16_t* h_shared;        // bf16 [T][SI]
    uint16_t* part;            // bf16 [6T][H], sorted positions
    uint16_t* part_shared;     // bf16 [T][H]
    int T;
};

__device__ __forceinline__ int groups_of(int n) { return (n + kGroup - 1) / kGroup; }

// ---------------------------------------------------------------- 1. permute
// Lane e of wave 0 scans all entries in flat order and numbers the ones routed
// to expert e: positions are stable (flat order within an expert), which is
// the order of a stable argsort of the flat ids (moe_infer's `argsort`).
__global__ __launch_bounds__(kLanes) void permute_kernel(Params P) {
    __shared__ int s_ids[kMaxEntries];
    const int lane = threadIdx.x;
    const int N = P.T * kTopK;
    Header* H = P.hdr;
    for (int i = lane; i < N; i += kLanes) s_ids[i] = min(max(P.ids[i], 0), kRouted - 1);
    __syncthreads();
    int c = 0;
    for (int i = 0; i < N; ++i) c += s_ids[i] == lane;
    // exclusive scan over the 64 lanes (Hillis-Steele with shuffles)
    int incl = c;
#pragma unroll
    for (int d = 1; d < kLanes; d <<= 1) {
        const int o = __shfl_up(incl, d, kLanes);
        if (lane >= d) incl += o;
    }
    const int off = incl - c;
    H->cnt[lane] = c;
    H->off[lane] = off;
    if (lane == kLanes - 1) H->off[kRouted] = incl;
    int run = off;
    for (int i = 0; i < N; ++i) {
        if (s_ids[i] == lane) {
            H->ent_at[run] = i;
            H->pos_of[i] = run;
            ++run;
        }
    }
    // work tiles: gate/up and down items per expert, shared last
    const int g = c > 0 ? groups_of(c) : 0;
    int gu = g * kGuTiles, dn = g * kDnTiles;
    int gi = gu, di = dn;
#pragma unroll
    for (int d = 1; d < kLanes; d <<= 1) {
        const int o1 = __shfl_up(gi, d, kLanes);
        const int o2 = __shfl_up(di, d, kLanes);
        if (lane >= d) { gi += o1; di += o2; }
    }
    H->gu_base[lane] = gi - gu;
    H->dn_base[lane] = di - dn;
    if (lane == kLanes - 1) {
        const int gs = groups_of(P.T);
        H->gu_base[kRouted] = gi;
        H->dn_base[kRouted] = di;
        H->gu_base[kRouted + 1] = gi + gs * kSgTiles;
        H->dn_base[kRouted + 1] = di + gs * kDnTiles;
        H->n_items_gu = gi + gs * kSgTiles;
        H->n_items_dn = di + gs * kDnTiles;
        H->n_tokens = P.T;
    }
}

// Which expert (64 = shared) item `it` belongs to, given bases[0..65].
__device__ __forceinline__ int find_unit(const int32_t* base, int it) {
    int lo = 0, hi = kRouted;      // base[lo] <= it < base[hi + 1]
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (base[mid] <= it) lo = mid; else hi = mid - 1;
    }
    return lo;
}

__device__ __forceinline__ f32x4 mfma16(const u32x4& a, const u32x4& b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

// One tile: rows [r0, r0 + 16) of a row-major bf16 matrix W (leading dim K)
// times the B columns of up to 4 x 16 tokens, where token column j of tile tt
// reads activation row act + rowidx[16 tt + j] * act_ld (K bf16 values).
// acc[tt] receives D[i][j] with i = 4 (lane / 16) + v, j = lane % 16.
template <int K>
__device__ __forceinline__ void mfma_tile(const uint16_t* W, int r0, const uint16_t* act,
                                          int act_ld, const int* rowidx, int m, f32x4 (&acc)[4]) {
    const int lane = threadIdx.x & (kLanes - 1);
    const int r = lane & 15, kq = lane >> 4;
    const u32x4* wrow = reinterpret_cast<const u32x4*>(W + (int64_t)(r0 + r) * K) + kq;
    const int nt = (m + 15) >> 4;
    const u32x4* arow[4];
    bool live[4];
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
        const int j = 16 * tt + r;
        live[tt] = j < m;
        arow[tt] = reinterpret_cast<const u32x4*>(act + (int64_t)(live[tt] ? rowidx[j] : 0) * act_ld) + kq;
        acc[tt] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    constexpr int kSteps = K / 32;
    constexpr int kU = (kSteps % 8 == 0) ? 8 : 4;
    static_assert(kSteps % kU == 0, "K unroll");
    for (int s0 = 0; s0 < kSteps; s0 += kU) {
        u32x4 a[kU];
#pragma unroll
        for (int u = 0; u < kU; ++u) a[u] = ld_stream(wrow + 4 * (s0 + u));
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) {
            if (tt < nt) {
#pragma unroll
                for (int u = 0; u < kU; ++u) {
                    const u32x4 b = live[tt] ? arow[tt][4 * (s0 + u)] : u32x4{0u, 0u, 0u, 0u};
                    acc[tt] = mfma16(a[u], b, acc[tt]);
                }
            }
        }
    }
}

// ---------------------------------------------------------------- 2. gate/up
__global__ __launch_bounds__(kThreads) void gate_up_kernel(Params P) {
    __shared__ int s_tok[kWaves][kGroup];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & (kLanes - 1);
    const Header* H = P.hdr;
    const int n_items = H->n_items_gu;
    for (int it = blockIdx.x * kWaves + wave; it < n_items; it += gridDim.x * kWaves) {
        const int e = find_unit(H->gu_base, it);
        const int local = it - H->gu_base[e];
        const bool shared = e == kRouted;
        const int tiles = shared ? kSgTiles : kGuTiles;
        const int grp = local / tiles, tile = local - grp * tiles;
        const int n_tok = shared ? P.T : H->cnt[e];
        const int p0 = shared ? kGroup * grp : H->off[e] + kGroup * grp;
        const int m = min(kGroup, n_tok - kGroup * grp);
        // activation rows of this group: token ids in sorted order
        if (lane < m) s_tok[wave][lane] = shared ? p0 + lane : H->ent_at[p0 + lane] / kTopK;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
        const uint16_t* W = shared ? P.shared
                                   : P.experts + (int64_t)e * P.expert_stride;
        f32x4 acc[4];
        mfma_tile<kHidden>(W, kTileRows * tile, P.x, kHidden, s_tok[wave], m, acc);
        // D rows 4q+v: pair (tile*8 + 2q + v/2), v even = gate, odd = up.
        const int q = lane >> 4, j = lane & 15;
        const int inter = shared ? kSharedInter : kInter;
        uint16_t* hb = shared ? P.h_shared : P.h_routed;
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) {
            const int jj = 16 * tt + j;
            if (jj < m) {
                const int row = shared ? p0 + jj : p0 + jj;   // token (shared) or sorted position
                const int pair = 8 * tile + 2 * q;
                const float h0 = bf16r(bf16r(silu_rn(bf16r(acc[tt][0]))) * bf16r(acc[tt][1]));
                const float h1 = bf16r(bf16r(silu_rn(bf16r(acc[tt][2]))) * bf16r(acc[tt][3]));
                const uint32_t packed = bf16_bits(h0) | (bf16_bits(h1) << 16);
                *reinterpret_cast<uint32_t*>(hb + (int64_t)row * inter + pair) = packed;
            }
        }
    }
}

// ---------------------------------------------------------------- 3. down
__global__ __launch_bounds__(kThreads) void down_kernel(Params P) {
    __shared__ int s_row[kWaves][kGroup];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & (kLanes - 1);
    const Header* H = P.hdr;
    const int n_items = H->n_items_dn;
    for (int it = blockIdx.x * kWaves + wave; it < n_items; it += gridDim.x * kWaves) {
        const int e = find_unit(H->dn_base, it);
        const int local = it - H->dn_base[e];
        const bool shared = e == kRouted;
        const int grp = local / kDnTiles, tile = local - grp * kDnTiles;
        const int n_tok = shared ? P.T : H->cnt[e];
        const int p0 = shared ? kGroup * grp : H->off[e] + kGroup * grp;
        const int m = min(kGroup, n_tok - kGroup * grp);
        if (lane < m) s_row[wave][lane] = p0 + lane;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
        f32x4 acc[4];
        if (shared) {
            mfma_tile<kSharedInter>(P.shared + (int64_t)2 * kSharedInter * kHidden,
                                    kTileRows * tile, P.h_shared, kSharedInter, s_row[wave], m,
                                    acc);
        } else {
            mfma_tile<kInter>(P.experts + (int64_t)e * P.expert_stride +
                                  (int64_t)2 * kInter * kHidden,
                              kTileRows * tile, P.h_routed, kInter, s_row[wave], m, acc);
        }
        const int q = lane >> 4, j = lane & 15;
        const int n0 = kTileRows * tile + 4 * q;
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) {
            const int jj = 16 * tt + j;
            if (jj < m) {
                const int pos = p0 + jj;
                uint32_t b[4];
                if (shared) {
#pragma unroll
                    for (int v = 0; v < 4; ++v) b[v] = bf16_bits(acc[tt][v]);
                } else {
                    const float w = P.weights[H->ent_at[pos]];
#pragma unroll
                    for (int v = 0; v < 4; ++v) b[v] = bf16_bits(w * bf16r(acc[tt][v]));
                }
                uint16_t* dst = (shared ? P.part_shared : P.part) + (int64_t)pos * kHidden + n0;
                *reinterpret_cast<uint2*>(dst) = make_uint2(b[0] | (b[1] << 16), b[2] | (b[3] << 16));
            }
        }
    }
}

// ---------------------------------------------------------------- 4. combine
__global__ __launch_bounds__(256) void combine_kernel(Params P) {
    const Header* H = P.hdr;
    const int t = blockIdx.x;
    int pos[kTopK];
#pragma unroll
    for (int k = 0; k < kTopK; ++k) pos[k] = H->pos_of[t * kTopK + k];
    for (int n = threadIdx.x; n < kHidden; n += blockDim.x) {
        float y = 0.f;
#pragma unroll
        for (int k = 0; k < kTopK; ++k)
            y += __uint_as_float((uint32_t)P.part[(int64_t)pos[k] * kHidden + n] << 16);
        const float s = __uint_as_float((uint32_t)P.part_shared[(int64_t)t * kHidden + n] << 16);
        P.out[(int64_t)t * kHidden + n] = (uint16_t)bf16_bits(bf16r(y) + s);
    }
}

}  // namespace grouped
}  // namespace fleet_moe

using namespace fleet_moe;

int fleet_moe_check_dims(const fleet_moe_dims* d);
int fleet_moe_check_device(int min_cus);

static bool aligned(const void* p, size_t a) { return ((uintptr_t)p % a) == 0; }

extern "C" size_t fleet_moe_grouped_workspace_bytes(const fleet_moe_dims* dims, int32_t max_tokens) {
    (void)dims;
    if (max_tokens < 1 || max_tokens > grouped::kMaxTokens) return 0;
    return grouped::layout(max_tokens).total;
}

extern "C" int fleet_moe_grouped(const fleet_moe_layer* layer, int32_t n_tokens,
                                 const int32_t* ids, const float* weights,
                                 const uint16_t* x_norm, uint16_t* out, void* workspace,
                                 size_t workspace_bytes, const fleet_moe_dims* dims,
                                 hipStream_t stream) {
    if (!layer || !dims) return FLEET_MOE_ERR_ARG;
    if (int e = fleet_moe_check_dims(dims)) return e;
    if (!layer->experts || !layer->shared || !ids || !weights || !x_norm || !out || !workspace)
        return FLEET_MOE_ERR_ARG;
    if (n_tokens < 1 || n_tokens > grouped::kMaxTokens) return FLEET_MOE_ERR_ARG;
    if (!aligned(layer->experts, 16) || !aligned(layer->shared, 16) || !aligned(x_norm, 16) ||
        !aligned(out, 4) || !aligned(ids, 4) || !aligned(weights, 4) || !aligned(workspace, 256))
        return FLEET_MOE_ERR_ARG;
    if (layer->expert_stride < kExpertStride || layer->expert_stride % kChunk != 0)
        return FLEET_MOE_ERR_DIMS;
    // The workspace is laid out for the max_tokens it was sized for; recover it.
    int max_tokens = 0;
    for (int t = grouped::kMaxTokens; t >= 1; --t)
        if (grouped::layout(t).total <= workspace_bytes) { max_tokens = t; break; }
    if (max_tokens < n_tokens) return FLEET_MOE_ERR_WORKSPACE;
    if (int e = fleet_moe_check_device(1)) return e;

    const grouped::Layout L = grouped::layout(max_tokens);
    char* ws = static_cast<char*>(workspace);
    grouped::Params P;
    P.experts = layer->experts;
    P.shared = layer->shared;
    P.expert_stride = layer->expert_stride;
    P.ids = ids;
    P.weights = weights;
    P.x = x_norm;
    P.out = out;
    P.hdr = reinterpret_cast<grouped::Header*>(ws + L.header);
    P.h_routed = reinterpret_cast<uint16_t*>(ws + L.h_routed);
    P.h_shared = reinterpret_cast<uint16_t*>(ws + L.h_shared);
    P.part = reinterpret_cast<uint16_t*>(ws + L.part);
    P.part_shared = reinterpret_cast<uint16_t*>(ws + L.part_shared);
    P.T = n_tokens;
    hipLaunchKernelGGL(grouped::permute_kernel, dim3(1), dim3(kLanes), 0, stream, P);
    hipLaunchKernelGGL(grouped::gate_up_kernel, dim3(grouped::kGrid), dim3(grouped::kThreads), 0,
                       stream, P);
    hipLaunchKernelGGL(grouped::down_kernel, dim3(grouped::kGrid), dim3(grouped::kThreads), 0,
                       stream, P);
    hipLaunchKernelGGL(grouped::combine_kernel, dim3(n_tokens), dim3(256), 0, stream, P);
    return (int)hipGetLastError();
}
