// Launches of the attention half of a decoder layer, the embedding and the
// lm_head + argmax (the device code is attn_body.h) and their C entry points.
#include "attn_body.h"

namespace fleet_moe {
namespace attn {

__global__ __launch_bounds__(kThreads, 1) void attn_layer_kernel(Params P) {
    __shared__ Lds L;
    u32x4 pre[8];
    attn_layer<false>(P, L, pre, false, [] {});
}

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

__global__ __launch_bounds__(kThreads, 1) void lmhead_kernel(HeadParams H) {
    __shared__ HeadLds S;
    lmhead_body<false>(H, S);
}

__global__ __launch_bounds__(kWG, 1) void argmax_kernel(const Workspace* ws, int32_t* token_out,
                                                        int32_t* token_next, int32_t* pos_advance) {
    __shared__ float v[kWG];
    __shared__ int ix[kWG];
    const int t = threadIdx.x;
    v[t] = ws->cand_v[t];
    ix[t] = ws->cand_i[t];
    __syncthreads();
    argmax256(v, ix);
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
int fleet_moe_check_resident(const void* fn, int threads, int grid);

static bool aligned(const void* p, size_t a) { return ((uintptr_t)p % a) == 0; }

#if FLEET_ATTN_TRACE
static unsigned long long* g_attn_trace = nullptr;
extern "C" void fleet_attn_debug_set_trace(void* p) { g_attn_trace = (unsigned long long*)p; }
#endif

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
    if (int e = fleet_moe_check_resident(reinterpret_cast<const void*>(&attn::attn_layer_kernel),
                                         attn::kThreads, attn::kWG))
        return e;
    attn::Params P{};
    P.x = x;
    P.x_out = x_out;
    P.norm_in = layer->norm_in;
    P.qkv = layer->qkv;
    P.kv_a_norm = layer->kv_a_norm;
    P.kv_b = layer->kv_b;
    P.o_proj = layer->o_proj;
    P.cache = cache;
    P.cos = rope_cos;
    P.sin = rope_sin;
    P.pos_dev = pos_dev;
    P.pos_host = pos;
    P.max_pos = max_pos;
    // (qk_nope + qk_rope)^-0.5 * mscale(40, 0.707)^2 (src/host/reference_decode.py:
    // 78-83, 197-203), in double
    const double m = 0.1 * 0.707 * std::log(40.0) + 1.0;
    P.scale = std::pow(192.0, -0.5) * m * m;
    P.eps = dims->rms_eps;
    P.ws = static_cast<attn::Workspace*>(workspace);
#if FLEET_ATTN_TRACE
    P.trace = g_attn_trace;
#endif
    hipLaunchKernelGGL(attn::attn_layer_kernel, dim3(attn::kWG), dim3(attn::kThreads), 0, stream,
                       P);
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
    attn::HeadParams H{};
    H.x = x;
    H.norm = final_norm;
    H.W = lm_head;
    H.eps = dims->rms_eps;
    H.logits = logits;
    H.ws = ws;
    hipLaunchKernelGGL(attn::lmhead_kernel, dim3(attn::kWG), dim3(attn::kThreads), 0, stream, H);
    hipLaunchKernelGGL(attn::argmax_kernel, dim3(1), dim3(attn::kWG), 0, stream, ws, token_out,
                       token_next, pos_advance);
    return (int)hipGetLastError();
}
