// One greedy decode step of the whole model in ONE launch: embedding, every
// decoder layer (the absorbed-MLA attention half, then the dense or MoE FFN
// half), the final RMSNorm, lm_head and the argmax, with the token and the
// position in device memory, so a decode loop is one launch per token (or one
// graph node).
//
// The stages are the device code of the per-layer launches (attn_body.h,
// moe_body.h, dense_body.h) run back to back by the same 256 workgroups (one
// per CU, 8 waves each). What a launch boundary used to do between them is
// done by the data itself: every stage publishes its residual rows as tagged
// words (tag | bf16 bits) in an exchange buffer, and the next stage polls the
// whole residual before it starts, so no workgroup runs ahead on a stale
// input. Two exchange buffers alternate (attention outputs, FFN outputs).
// Every stage's cross-workgroup words carry a call count unique to the
// (step, layer), derived from the call counts read once at the start: the
// attention, MoE and dense workspaces are reused by every layer, and a word a
// stage polls is always rewritten by that stage, so it is at most one stage
// old. Reuse is safe because every stage ends with an all-to-all exchange:
// a workgroup can only write a stage's words after every workgroup has
// published the previous stage's residual, which it does after its last read
// of those words. Workgroup 0 advances the call counts at the very end, after
// the argmax, which needed every workgroup's lm_head candidate.
#include "attn_body.h"
#include "dense_body.h"
#include "moe_body.h"

#ifndef FLEET_STEP_TRACE
#define FLEET_STEP_TRACE 0
#endif

namespace fleet_moe {
namespace step {

constexpr int kWG = 256;
constexpr int kThreads = 512;
constexpr int kMaxLayers = FLEET_STEP_MAX_LAYERS;
// Residual exchange tags advance by kTagStride per step. A step has stages
// 1 .. 2 n_layers (and the lm_head reads stage 2 n_layers), so the stride must
// exceed every stage number: a buffer polled at stage s of step k then holds
// either stage s - 2 of step k or the last stage of its parity of step k - 1,
// and neither can carry step k's tag for stage s - 1 (with a stride of 64, a
// 33-layer step's stage 2 read step k - 1's stage 65 as current).
constexpr uint32_t kTagStride = 256;
static_assert(kTagStride >= 2 * kMaxLayers + 2, "a step's stages must fit in its tag stride");
static_assert(65536 % kTagStride == 0, "16-bit tags: consecutive steps never share a tag");
static_assert(attn::kWG == kWG && decode::kWG == kWG && dense::kWG == kWG, "one grid");
static_assert(attn::kThreads == kThreads && decode::kThreads == kThreads &&
                  dense::kThreads == kThreads,
              "one workgroup shape");

struct Workspace {
    uint32_t epoch;                           // steps completed
    uint32_t pad0;
    uint32_t abort;                           // offset 8: sticky status
    uint32_t pad1[61];
    uint32_t x[2][kXCopies][kHidden];         // residual exchange: [0] attention, [1] FFN outputs
};
static_assert(offsetof(Workspace, abort) == 8, "status word offset");
static_assert(offsetof(Workspace, x) % 16 == 0, "x is read with 16-byte loads");

// Byte offsets of the four workspaces inside the caller's one buffer.
constexpr size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }
constexpr size_t kOffAttn = 0;
constexpr size_t kOffMoe = kOffAttn + align256(sizeof(attn::Workspace));
constexpr size_t kOffDense = kOffMoe + align256(sizeof(decode::Workspace));
constexpr size_t kOffStep = kOffDense + align256(sizeof(dense::Workspace));
constexpr size_t kBytes = kOffStep + align256(sizeof(Workspace));

struct Params {
    const fleet_step_layer* layers;   // device table
    int32_t n_layers;
    int32_t max_pos;
    const uint16_t* embed;
    const uint16_t* final_norm;
    const uint16_t* lm_head;
    const float* cos;
    const float* sin;
    const int32_t* token;
    int32_t* token_out;
    int32_t* token_next;
    int32_t* pos_dev;
    const float* x_in;         // the FFN column's input (kFull false)
    float* x_out;
    float* logits;
    double scale;
    float eps;
    float scaling;
    attn::Workspace* aws;
    decode::Workspace* mws;
    dense::Workspace* dws;
    Workspace* sws;
#if FLEET_STEP_TRACE
    unsigned long long* trace;     // [2 n_layers + 2][kWG] stage-end stamps, or null
    unsigned long long* trace_a;   // the attention stage trace of layer trace_layer
    unsigned long long* trace_m;   // its FFN stage trace
    int trace_layer;
#endif
};

union Lds {
    attn::Lds a;
    decode::Lds m;
    dense::Lds d;
    attn::HeadLds h;
};

// A word written by an earlier launch, read through the scalar cache (which
// every launch starts with invalidated): a uniform value in SGPRs, its wait
// independent of the vector loads in flight.
template <class T>
__device__ __forceinline__ T ld_launch_const(const T* p) {
    return *(const __attribute__((address_space(4))) T*)p;
}

constexpr int kLayerWords = sizeof(fleet_step_layer) / 8;
static_assert(sizeof(fleet_step_layer) % 8 == 0, "the layer table is copied in 8-byte words");
static_assert(kMaxLayers * kLayerWords <= 2 * kThreads, "two table words per thread at most");

// kFull: the decode step (embed, attention and FFN of every layer, lm_head,
// argmax). Otherwise the FFN column: the FFN stage of every layer of the table
// on S.x_in, the last one's output in S.x_out (no attention, no position).
template <bool kFull>
__global__ __launch_bounds__(kThreads, 1) void step_kernel(Params S) {
    __shared__ Lds L;
    // The layer table, copied into LDS once per launch: read from global
    // memory at each stage, a stage's weight pointers would arrive about a
    // microsecond after the stage starts, and every weight load waits for them.
    __shared__ uint64_t tbl_words[kMaxLayers * kLayerWords];
    const int wg = blockIdx.x, tid = fm_tid();
    {
        const uint64_t* src = reinterpret_cast<const uint64_t*>(S.layers);
        const int n = S.n_layers * kLayerWords;
        const uint64_t a = tid < n ? ld_global(src + tid) : 0ull;
        const uint64_t b = tid + kThreads < n ? ld_global(src + tid + kThreads) : 0ull;
        if (tid < n) tbl_words[tid] = a;
        if (tid + kThreads < n) tbl_words[tid + kThreads] = b;
    }
    const fleet_step_layer* tbl = reinterpret_cast<const fleet_step_layer*>(tbl_words);
    int pos = 0, token = 0;
    if constexpr (kFull) {
        pos = ld_launch_const(S.pos_dev);
        token = ld_launch_const(S.token);
        if (pos < 0 || pos >= S.max_pos || token < 0 || token >= attn::kVocab) {
            if (wg == 0 && tid == 0)
                attn::raise(S.aws, (pos < 0 || pos >= S.max_pos) ? FLEET_MOE_ABORT_POSITION
                                                                 : FLEET_MOE_ABORT_TOKEN);
            return;
        }
    }
    // the call counts, written by the previous launch (plain loads: current
    // after the launch boundary)
    const uint32_t ea = kFull ? ld_launch_const(&S.aws->epoch) : 0u;
    const uint32_t em = ld_launch_const(&S.mws->epoch), ed = ld_launch_const(&S.dws->epoch),
                   es = ld_launch_const(&S.sws->epoch);
    // exchange tags: kTagStride per step, one per stage
    const uint32_t sbase = (es + 1u) * kTagStride;
    auto xtag = [&](int stage) { return ((sbase + (uint32_t)stage) & 0xffffu) << 16; };
    uint32_t* xbuf[2] = {&S.sws->x[0][0][0], &S.sws->x[1][0][0]};
    int n_moe = 0, n_dense = 0;
#if FLEET_STEP_TRACE
#define STEP_TRACE(k) \
    do { if (S.trace && tid == 0) S.trace[(size_t)(k) * kWG + wg] = __builtin_amdgcn_s_memrealtime(); } while (0)
#else
#define STEP_TRACE(k) do {} while (0)
#endif
    __syncthreads();                          // the table
    STEP_TRACE(0);
    // stage numbering: the decode step's attention of layer i is stage 2i + 1
    // and its FFN 2i + 2; the column's FFN of layer i is stage i + 1. Stage s
    // publishes into xbuf[s % 2] with tag xtag(s) and reads stage s - 1's.
    // A stage issues the next stage's first loads (an attention's first rows,
    // a MoE stage's first shared pair per streaming wave) into `pre` once its
    // own last wait is done, and the next stage starts on them (pre_in).
    u32x4 pre[8];
    bool pre_in = false;
    for (int i = 0; i < S.n_layers; ++i) {
        const fleet_step_layer& ly = tbl[i];
        const bool last = i == S.n_layers - 1;
        if constexpr (kFull) {
            const int st = 2 * i + 1;
            attn::Params A{};
            A.norm_in = ly.attn.norm_in;
            A.qkv = ly.attn.qkv;
            A.kv_a_norm = ly.attn.kv_a_norm;
            A.kv_b = ly.attn.kv_b;
            A.o_proj = ly.attn.o_proj;
            A.cache = ly.cache;
            A.cos = S.cos;
            A.sin = S.sin;
            A.pos_host = pos;
            A.max_pos = S.max_pos;
            A.scale = S.scale;
            A.eps = S.eps;
            A.ws = S.aws;
            A.epoch = ea + 1u + (uint32_t)i;
            A.xin = i == 0 ? nullptr : xbuf[(st - 1) % 2];
            A.xin_row = i == 0 ? S.embed + (int64_t)token * kHidden : nullptr;
            A.xin_tag = xtag(st - 1);
            A.xout = xbuf[st % 2];
            A.xout_tag = xtag(st);
#if FLEET_STEP_TRACE && FLEET_ATTN_TRACE
            A.trace = i == S.trace_layer ? S.trace_a : nullptr;
#endif
            // the FFN of this layer follows: its first pair
            auto next = [&]() {
                if (ly.dense) dense::issue_first_pair(ly.dense, pre);
                else decode::issue_first_pair(ly.moe.shared, pre);
            };
            attn::attn_layer<true>(A, L.a, pre, pre_in, next);
            pre_in = true;
            __syncthreads();
            STEP_TRACE(st);
        }
        const int st = kFull ? 2 * i + 2 : i + 1;
        const bool first = !kFull && i == 0;
        // the next stage: the attention of layer i + 1 (decode step) or its
        // FFN (column); after the last layer nothing (the buffer is cleared,
        // so that no path leaves it holding older values)
        const fleet_step_layer* nl = last ? nullptr : &tbl[i + 1];
        auto next = [&]() {
            if (!nl) {
#pragma unroll
                for (int m = 0; m < 8; ++m) pre[m] = u32x4{0u, 0u, 0u, 0u};
            } else if constexpr (kFull) {
                attn::issue_first_rows(nl->attn.qkv, pre);
            } else if (nl->dense) {
                dense::issue_first_pair(nl->dense, pre);
            } else {
                decode::issue_first_pair(nl->moe.shared, pre);
            }
        };
        if (ly.dense) {
            dense::Params D{};
            D.norm = ly.moe.norm;
            D.w = ly.dense;
            D.x_out = last ? S.x_out : nullptr;
            D.ws = S.dws;
            D.eps = S.eps;
            D.epoch = ed + 1u + (uint32_t)n_dense++;
            D.xin = first ? nullptr : xbuf[(st - 1) % 2];
            D.xin_f32 = first ? S.x_in : nullptr;
            D.xin_tag = xtag(st - 1);
            D.xout = xbuf[st % 2];
            D.xout_tag = xtag(st);
            dense::dense_layer<true>(D, L.d, pre, pre_in, next);
        } else {
            decode::Params M{};
            M.norm = ly.moe.norm;
            M.router = reinterpret_cast<const u32x4*>(ly.moe.router);
            M.experts = ly.moe.experts;
            M.shared = ly.moe.shared;
            M.x_out = last ? S.x_out : nullptr;
            M.ws = S.mws;
            M.expert_stride = ly.moe.expert_stride;
            M.eps = S.eps;
            M.scaling = S.scaling;
            M.epoch = em + 1u + (uint32_t)n_moe++;
            M.xin = first ? nullptr : xbuf[(st - 1) % 2];
            M.xin_f32 = first ? S.x_in : nullptr;
            M.xin_tag = xtag(st - 1);
            M.xout = xbuf[st % 2];
            M.xout_tag = xtag(st);
            M.router_first = !kFull;
#if FLEET_STEP_TRACE && FLEET_MOE_TRACE
            M.trace = i == S.trace_layer ? S.trace_m : nullptr;
#endif
            decode::moe_layer<true>(M, L.m, pre, pre_in, next);
        }
        pre_in = true;
        __syncthreads();
        STEP_TRACE(st);
    }
    if constexpr (kFull) {
        attn::HeadParams H{};
        H.norm = S.final_norm;
        H.W = S.lm_head;
        H.eps = S.eps;
        H.logits = S.logits;
        H.ws = S.aws;
        H.xin = xbuf[(2 * S.n_layers) % 2];
        H.xin_tag = xtag(2 * S.n_layers);
        H.epoch = es + 1u;
        H.token_out = S.token_out;
        H.token_next = S.token_next;
        H.pos_advance = S.pos_dev;
        attn::lmhead_body<true>(H, L.h);
        STEP_TRACE(2 * S.n_layers + 1);
    } else if (S.n_layers == 1) {
        // A one-layer column writes only xbuf[1]. Stamp xbuf[0] with this
        // step's stage-0 tag, which no stage polls, so that neither buffer
        // ever holds words older than the previous step (a 16-bit tag comes
        // back every 65536 / kTagStride steps).
        const int g = wg * kThreads + tid;
        if (g < kXCopies * kHidden) st_agent(xbuf[0] + g, xtag(0));
    }
    // workgroup 0 advances the call counts: the argmax (decode step) or the
    // last FFN stage's h exchange (column) needed every workgroup, so every
    // workgroup has read them
    if (wg == 0 && tid == 0) {
        if constexpr (kFull) st_agent(&S.aws->epoch, ea + (uint32_t)S.n_layers);
        st_agent(&S.mws->epoch, em + (uint32_t)n_moe);
        st_agent(&S.dws->epoch, ed + (uint32_t)n_dense);
        st_agent(&S.sws->epoch, es + 1u);
    }
}

}  // namespace step
}  // namespace fleet_moe

using namespace fleet_moe;

int fleet_moe_check_dims(const fleet_moe_dims* d);
int fleet_moe_check_resident(const void* fn, int threads, int grid);

static bool aligned(const void* p, size_t a) { return ((uintptr_t)p % a) == 0; }

#if FLEET_STEP_TRACE
static unsigned long long *g_step_trace, *g_step_trace_a, *g_step_trace_m;
static int g_step_trace_layer = -1;
extern "C" void fleet_step_debug_set_trace(void* t, void* a, void* m, int layer) {
    g_step_trace = (unsigned long long*)t;
    g_step_trace_a = (unsigned long long*)a;
    g_step_trace_m = (unsigned long long*)m;
    g_step_trace_layer = layer;
}
#endif

extern "C" size_t fleet_decode_step_workspace_bytes(const fleet_moe_dims* dims) {
    if (!dims || fleet_moe_check_dims(dims) != 0) return 0;
    return step::kBytes;
}

extern "C" int fleet_decode_step(const fleet_step_model* model, const int32_t* token,
                                 int32_t* token_out, int32_t* token_next, int32_t* pos_dev,
                                 float* x_out, float* logits, void* workspace,
                                 size_t workspace_bytes, const fleet_moe_dims* dims,
                                 hipStream_t stream) {
    if (!model || !dims) return FLEET_MOE_ERR_ARG;
    if (int e = fleet_moe_check_dims(dims)) return e;
    if (!model->layers || model->n_layers < 1 || model->n_layers > step::kMaxLayers ||
        !model->embed || !model->lm_head || !model->rope_cos || !model->rope_sin ||
        model->max_pos < 1 || model->max_pos > attn::kMaxPos || !token || !pos_dev ||
        !workspace)
        return FLEET_MOE_ERR_ARG;
    if (!aligned(model->layers, 8) || !aligned(model->embed, 16) || !aligned(model->lm_head, 16) ||
        (model->final_norm && !aligned(model->final_norm, 8)) || !aligned(model->rope_cos, 4) ||
        !aligned(model->rope_sin, 4) || !aligned(token, 4) || !aligned(pos_dev, 4) ||
        (token_out && !aligned(token_out, 4)) || (token_next && !aligned(token_next, 4)) ||
        (x_out && !aligned(x_out, 4)) || (logits && !aligned(logits, 4)) ||
        !aligned(workspace, 256))
        return FLEET_MOE_ERR_ARG;
    if (workspace_bytes < step::kBytes) return FLEET_MOE_ERR_WORKSPACE;
    if (int e = fleet_moe_check_resident(reinterpret_cast<const void*>(&step::step_kernel<true>),
                                         step::kThreads, step::kWG))
        return e;
    uint8_t* w = static_cast<uint8_t*>(workspace);
    step::Params S{};
    S.layers = model->layers;
    S.n_layers = model->n_layers;
    S.max_pos = model->max_pos;
    S.embed = model->embed;
    S.final_norm = model->final_norm;
    S.lm_head = model->lm_head;
    S.cos = model->rope_cos;
    S.sin = model->rope_sin;
    S.token = token;
    S.token_out = token_out;
    S.token_next = token_next;
    S.pos_dev = pos_dev;
    S.x_out = x_out;
    S.logits = logits;
    // (qk_nope + qk_rope)^-0.5 * mscale(40, 0.707)^2 (src/host/reference_decode.py:
    // 78-83, 197-203), in double
    const double m = 0.1 * 0.707 * std::log(40.0) + 1.0;
    S.scale = std::pow(192.0, -0.5) * m * m;
    S.eps = dims->rms_eps;
    S.scaling = dims->routed_scaling;
    S.aws = reinterpret_cast<attn::Workspace*>(w + step::kOffAttn);
    S.mws = reinterpret_cast<decode::Workspace*>(w + step::kOffMoe);
    S.dws = reinterpret_cast<dense::Workspace*>(w + step::kOffDense);
    S.sws = reinterpret_cast<step::Workspace*>(w + step::kOffStep);
#if FLEET_STEP_TRACE
    S.trace = g_step_trace;
    S.trace_a = g_step_trace_a;
    S.trace_m = g_step_trace_m;
    S.trace_layer = g_step_trace_layer;
#endif
    hipLaunchKernelGGL(step::step_kernel<true>, dim3(step::kWG), dim3(step::kThreads), 0, stream,
                       S);
    return (int)hipGetLastError();
}

extern "C" int fleet_ffn_column(const fleet_step_layer* layers, int32_t n_layers, const float* x,
                                float* x_out, void* workspace, size_t workspace_bytes,
                                const fleet_moe_dims* dims, hipStream_t stream) {
    if (!dims) return FLEET_MOE_ERR_ARG;
    if (int e = fleet_moe_check_dims(dims)) return e;
    if (!layers || n_layers < 1 || n_layers > step::kMaxLayers || !x || !x_out || !workspace)
        return FLEET_MOE_ERR_ARG;
    if (!aligned(layers, 8) || !aligned(x, 16) || !aligned(x_out, 4) || !aligned(workspace, 256))
        return FLEET_MOE_ERR_ARG;
    if (workspace_bytes < step::kBytes) return FLEET_MOE_ERR_WORKSPACE;
    if (int e = fleet_moe_check_resident(reinterpret_cast<const void*>(&step::step_kernel<false>),
                                         step::kThreads, step::kWG))
        return e;
    uint8_t* w = static_cast<uint8_t*>(workspace);
    step::Params S{};
    S.layers = layers;
    S.n_layers = n_layers;
    S.x_in = x;
    S.x_out = x_out;
    S.eps = dims->rms_eps;
    S.scaling = dims->routed_scaling;
    S.aws = reinterpret_cast<attn::Workspace*>(w + step::kOffAttn);
    S.mws = reinterpret_cast<decode::Workspace*>(w + step::kOffMoe);
    S.dws = reinterpret_cast<dense::Workspace*>(w + step::kOffDense);
    S.sws = reinterpret_cast<step::Workspace*>(w + step::kOffStep);
#if FLEET_STEP_TRACE
    S.trace = g_step_trace;
    S.trace_a = g_step_trace_a;
    S.trace_m = g_step_trace_m;
    S.trace_layer = g_step_trace_layer;
#endif
    hipLaunchKernelGGL(step::step_kernel<false>, dim3(step::kWG), dim3(step::kThreads), 0, stream,
                       S);
    return (int)hipGetLastError();
}

extern "C" int fleet_decode_step_status(const void* workspace, uint32_t* status,
                                        hipStream_t stream) {
    if (!workspace || !status || !aligned(workspace, 256)) return FLEET_MOE_ERR_ARG;
    uint32_t v[4] = {0u, 0u, 0u, 0u};
    const size_t offs[4] = {step::kOffAttn, step::kOffMoe, step::kOffDense, step::kOffStep};
    const char* w = static_cast<const char*>(workspace);
    for (int i = 0; i < 4; ++i) {
        hipError_t e = hipMemcpyAsync(&v[i], w + offs[i] + 8, sizeof(uint32_t),
                                      hipMemcpyDeviceToHost, stream);
        if (e != hipSuccess) return (int)e;
    }
    if (hipError_t e = hipStreamSynchronize(stream)) return (int)e;
    *status = v[0] | v[1] | v[2] | v[3];
    return 0;
}
