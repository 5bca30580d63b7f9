/*
 * fleet_moe.h -- C ABI of the MI355X (gfx950) batch-1 MoE decode path for
 * DeepSeek-V2-Lite: router + greedy top-k, routed SwiGLU experts, the fused
 * shared expert, the weighted combine, and the multi-token grouped product.
 *
 * Conventions (match the reference launcher's, src/host/fleet_launch.hip:55-63,
 * 612-644, and its task-body ABI, src/kernels/fleet_kernel.hip:1057-1078):
 *   - every entry point returns 0 on success, a hipError_t value when a HIP
 *     call fails, or a FLEET_MOE_ERR_* code (>= 10000) for a rejected argument;
 *   - nothing here allocates: the caller owns every buffer (weights, inputs,
 *     outputs, workspace) as device memory, and passes plain device pointers;
 *   - work is enqueued on `stream` and is asynchronous; inputs are read-only;
 *   - a workspace must be zero-filled once before its first use and may then
 *     be reused by any number of calls that are ordered on one stream; two
 *     calls that overlap in time must not share a workspace;
 *   - weights use the reference's packed layout (src/host/pack_weights.py:
 *     41-54, 71-83, 125-146): bf16 bit patterns (uint16_t), experts as
 *     n_routed blocks of `expert_stride` elements [gate/up interleaved
 *     (2*I rows of H) | down (H rows of I)], the merged shared expert as
 *     [gate/up interleaved (2*SI rows of H) | down (H rows of SI)], SI =
 *     n_shared * I. Tensor bases must be 16-byte aligned (the packer aligns
 *     every tensor to 256 bytes).
 * The kernels are built for the DeepSeek-V2-Lite shape (hidden 2048,
 * moe_inter 1408, 64 routed experts, top-6, 2 shared experts); other shapes
 * are rejected with FLEET_MOE_ERR_DIMS.
 */
#ifndef FLEET_MOE_H
#define FLEET_MOE_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FLEET_MOE_ERR_DIMS 10001      /* shape other than the supported one  */
#define FLEET_MOE_ERR_ARG 10002       /* null or misaligned pointer, bad count */
#define FLEET_MOE_ERR_WORKSPACE 10003 /* workspace smaller than required      */
#define FLEET_MOE_ERR_DEVICE 10004    /* device is not gfx950 / too few CUs   */
#define FLEET_MOE_ERR_CAPACITY 10005  /* more tokens than the static scratch holds */
#define FLEET_MOE_ERR_CAPTURE 10006   /* first call on a device made under graph capture */

/* Model scalars, the MoE subset of ModelDims (src/runtime/fleet_types.h:33-39)
 * and of the packed manifest's scalars (src/host/pack_weights.py:153-184). */
typedef struct fleet_moe_dims {
    int32_t hidden;        /* 2048 */
    int32_t moe_inter;     /* 1408 */
    int32_t n_routed;      /* 64   */
    int32_t n_shared;      /* 2: the shared expert has n_shared*moe_inter rows */
    int32_t top_k;         /* 6    */
    float routed_scaling;  /* 1.0  */
    float rms_eps;         /* 1e-6 */
} fleet_moe_dims;

/* One MoE layer's weights: the per-layer pointer tables of Weights
 * (src/runtime/fleet_types.h:44-59: layer_norm_post, layer_router,
 * layer_experts, layer_shared, expert_stride). */
typedef struct fleet_moe_layer {
    const uint16_t* norm;     /* post-attention RMSNorm weight bf16[hidden]; NULL = unit */
    const uint16_t* router;   /* bf16[n_routed][hidden] ("L{i}.router") */
    const uint16_t* experts;  /* n_routed blocks ("L{i}.experts") */
    int64_t expert_stride;    /* elements between experts: 3*hidden*moe_inter */
    const uint16_t* shared;   /* merged shared expert block ("L{i}.shared") */
} fleet_moe_layer;

/* Router logits and greedy top-k for n_tokens rows of x_norm.
 * Replaces the router GEMV of task_norm_router (src/kernels/fleet_kernel.hip:
 * 433-435) and select_experts_from (:469-494); semantics of
 * src/host/reference_decode.py:271-278 and HF MoEGate.forward
 * (reference/modeling_deepseek.py:420-467):
 *   logits = W_router . x_norm (fp32; evaluated exactly and rounded once),
 *   p = softmax(logits + logit_bias), ids = the top_k largest p in decreasing
 *   order, ties to the lowest index, weights = p[ids] * routed_scaling.
 * x_norm: fp32[n_tokens][hidden] (bf16-valued); logit_bias: fp32[n_routed]
 * or NULL; logits: fp32[n_tokens][n_routed] or NULL; ids: int32[n_tokens]
 * [top_k]; weights: fp32[n_tokens][top_k]. 1 <= n_tokens <= 65535. */
int fleet_moe_router_topk(const uint16_t* router, const float* x_norm, int32_t n_tokens,
                          const float* logit_bias, float* logits, int32_t* ids,
                          float* weights, const fleet_moe_dims* dims, hipStream_t stream);

/* The residual fold of the NORM_ROUTER prologue (stage_residual_f32,
 * src/kernels/fleet_kernel.hip:107-144, called at :405-425): the post-
 * attention residual x[1] = bf16(x[0] + bf16(p_0 + ... + p_{n-1})) from the
 * layer input and o_proj's n K-split fp32 partials (Activations.oproj_partial,
 * [n][hidden], n = 8 in the reference), the partials added in fp32 in index
 * order. fleet_moe_layer_decode takes that x[1] as its input; a graph whose
 * o_proj writes x[1] itself (OPROJ_ROW_SPLIT) needs no fold.
 * x, x_out: fp32[hidden] (may be equal); 1 <= n_partials <= 64. */
int fleet_moe_residual_fold(const float* x, const float* partials, int32_t n_partials,
                            float* x_out, const fleet_moe_dims* dims, hipStream_t stream);

/* Workspace bytes fleet_moe_layer_decode needs. */
size_t fleet_moe_layer_workspace_bytes(const fleet_moe_dims* dims);

/* One batch-1 MoE layer: x_out = bf16(x + moe(rms_norm(x))).
 * Replaces, for one token, the NORM_ROUTER (kind 4), EXPERT_GATE_UP (5) and
 * EXPERT_DOWN (6) task bodies and the expert-partial fold (src/kernels/
 * fleet_kernel.hip:398-456, 469-500, 826-889, 146-201; src/kernels/expert.h:
 * 45-116); semantics of src/host/reference_decode.py:294-302 (rms_norm, moe,
 * residual add) with the selection rule above.
 * x: fp32[hidden]; x_out: fp32[hidden] (may equal x); moe_out: bf16[hidden]
 * (the MoE output before the residual add) or NULL; ids: int32[top_k] or
 * NULL; weights: fp32[top_k] or NULL. One launch of 256 workgroups (one per
 * CU) that hand data to each other through the workspace, so all of them must
 * be resident at once: the entry point checks once per device that the device
 * has >= 256 CUs and that one workgroup of the kernel fits on a CU
 * (FLEET_MOE_ERR_DEVICE otherwise); a wait that still runs past its bound
 * (other work holding CUs) sets FLEET_MOE_ABORT_UNIT_WAIT or _ROUTER_WAIT. */
int fleet_moe_layer_decode(const fleet_moe_layer* layer, const float* x, float* x_out,
                           uint16_t* moe_out, int32_t* ids, float* weights,
                           void* workspace, size_t workspace_bytes,
                           const fleet_moe_dims* dims, hipStream_t stream);

/* Workspace bytes fleet_moe_dense_decode needs (dense_inter = 10944). */
size_t fleet_moe_dense_workspace_bytes(const fleet_moe_dims* dims, int32_t dense_inter);

/* Batch-1 dense SwiGLU layer (DeepSeek-V2-Lite layer 0, first_k_dense = 1):
 * x_out = bf16(x + mlp(rms_norm(x))), mlp(v) = down(bf16(bf16(silu(bf16(gate v)))
 * * bf16(up v))). Replaces the layer's NORM_ROUTER prologue and the
 * DENSE_GATE_UP (8) / DENSE_DOWN (9) task bodies (src/kernels/fleet_kernel.hip:
 * 891-903; src/host/taskgraph.py:444-474); semantics of src/host/
 * reference_decode.py:290-302 (dense_mlp, residual add).
 * norm: post-attention RMSNorm weight bf16[hidden] or NULL (unit); w: the
 * packed "L0.dense" block, [2*dense_inter][hidden] gate/up interleaved then
 * [hidden][dense_inter] down (src/host/pack_weights.py:143-146); x, x_out:
 * fp32[hidden] (may be equal); mlp_out: bf16[hidden] or NULL. One launch over
 * every CU. */
int fleet_moe_dense_decode(const uint16_t* norm, const uint16_t* w, int32_t dense_inter,
                           const float* x, float* x_out, uint16_t* mlp_out, void* workspace,
                           size_t workspace_bytes, const fleet_moe_dims* dims,
                           hipStream_t stream);

/* Workspace bytes fleet_moe_grouped needs for up to max_tokens tokens. */
size_t fleet_moe_grouped_workspace_bytes(const fleet_moe_dims* dims, int32_t max_tokens);

/* Multi-token grouped-expert product for one layer (no reference kernel; HF
 * DeepseekV2MoE.forward + moe_infer, reference/modeling_deepseek.py:568-664):
 * tokens are grouped by expert, every selected expert runs its SwiGLU over
 * its tokens (VALU GEMV for an expert holding <= 8 tokens, bf16 MFMA above
 * that), and out[t] = bf16(bf16(sum_k bf16(w[t][k] * E_{ids[t][k]}(x[t]))) +
 * shared(x[t])), the per-token combine of src/host/reference_decode.py:
 * 280-287, so grouped(T) equals T batch-1 MoE outputs up to fp32 summation
 * order. One launch over every CU (256 workgroups resident at once) for
 * n_tokens <= 8, two (gate/up, then down + combine) above that.
 * x_norm: bf16[n_tokens][hidden]; ids: int32[n_tokens][top_k] (each in
 * [0, n_routed), distinct per token; an id outside that range is clamped into
 * it and raises FLEET_MOE_ABORT_BAD_ID); weights: fp32[n_tokens][top_k];
 * out: bf16[n_tokens][hidden]. 1 <= n_tokens <= max_tokens of the workspace
 * (max_tokens <= 256). Workspace words carry a 32-bit call count; the call
 * numbered 2^32 - 1 clears them and restarts the count, so a workspace never
 * needs to be zero-filled again. */
int fleet_moe_grouped(const fleet_moe_layer* layer, int32_t n_tokens, const int32_t* ids,
                      const float* weights, const uint16_t* x_norm, uint16_t* out,
                      void* workspace, size_t workspace_bytes, const fleet_moe_dims* dims,
                      hipStream_t stream);

/* fleet_moe_grouped without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). No counterpart in the reference.
 * Same kernels, arguments and results as fleet_moe_grouped, but the workspace
 * is a static device array inside this library (FLEET_MOE_NOALLOC_SCRATCH_BYTES
 * per device, held until the process ends), laid out for at most
 * FLEET_MOE_NOALLOC_MAX_TOKENS tokens; n_tokens above that returns
 * FLEET_MOE_ERR_CAPACITY. Nothing is allocated by any call. The first call on
 * a device looks up that device's copy of the array and zero-fills it (a fill
 * kernel on `stream`, then a stream synchronize): it must not be made under
 * graph capture (FLEET_MOE_ERR_CAPTURE); later calls may be captured.
 * status: device uint32 that receives the step's FLEET_MOE_ABORT_* bits (0 =
 * healthy); the array's status word is cleared at the same time, so every
 * call reports its own. Every call on a device shares that device's array:
 * calls that overlap in time on one device (two streams, two host threads
 * without ordering) race and give unspecified results; order them on one
 * stream. */
#define FLEET_MOE_NOALLOC_MAX_TOKENS 64
#define FLEET_MOE_NOALLOC_SCRATCH_BYTES 7574528
int fleet_moe_grouped_noalloc(const fleet_moe_layer* layer, int32_t n_tokens,
                              const int32_t* ids, const float* weights, const uint16_t* x_norm,
                              uint16_t* out, uint32_t* status, const fleet_moe_dims* dims,
                              hipStream_t stream);

/* ------------------------------------------------------------------------
 * The rest of a decoder layer and of the decode step (absorbed MLA attention,
 * embedding, lm_head + argmax), so that the full 27-layer batch-1 decode runs
 * on this library: per token, embed, then per layer fleet_attn_decode and
 * fleet_moe_dense_decode / fleet_moe_layer_decode, then fleet_lm_head_argmax.
 * Fixed shape: 16 heads, kv_lora 512, qk_nope 128, qk_rope 64, v_head 128,
 * vocab 102400, max_pos <= 4096. */

/* One layer's attention weights: the per-layer pointer tables of Weights
 * (src/runtime/fleet_types.h:44-59: layer_norm_in, layer_qkv,
 * layer_kv_a_norm, layer_kv_b, layer_o_proj), i.e. the manifest tensors
 * "L{i}.norm_in", "L{i}.qkv" ([q_proj (3072) ; kv_a_proj_with_mqa (576)]
 * rows of hidden), "L{i}.kv_a_norm", "L{i}.kv_b" ([16 * 256][512]),
 * "L{i}.o_proj" ([hidden][2048]) (src/host/pack_weights.py:113-121). */
typedef struct fleet_attn_layer {
    const uint16_t* norm_in;    /* bf16[hidden] or NULL (unit) */
    const uint16_t* qkv;        /* bf16[3648][hidden] */
    const uint16_t* kv_a_norm;  /* bf16[512] or NULL (unit) */
    const uint16_t* kv_b;       /* bf16[4096][512] */
    const uint16_t* o_proj;     /* bf16[hidden][2048] */
} fleet_attn_layer;

/* Workspace bytes fleet_attn_decode, fleet_embed and fleet_lm_head_argmax
 * need (one workspace serves all three; about 2.4 MB). */
size_t fleet_attn_workspace_bytes(const fleet_moe_dims* dims);

/* The attention half of one decoder layer at one position:
 * x_out = bf16(x + o_proj(mla(rms_norm(x, norm_in)))). Replaces the
 * QKV_FUSED (kind 0), Q_ABSORB (14), ATTENTION (1), MERGE_UV (2) and O_PROJ
 * (3) task bodies (src/kernels/fleet_kernel.hip:647-660, 675-704, 706-803,
 * 805-830; src/kernels/attention.h:62-93, 171-222, 230-350, 358-420);
 * semantics of src/host/reference_decode.py:210-256 (attention_absorbed) and
 * :294-298 (the residual add). Writes this layer's cache row at the position
 * (c after kv_a_layernorm, then k_pe after RoPE, 576 bf16) and attends over
 * rows 0..position of `cache` ([max_pos][576] bf16: KVCache.data of one
 * layer, src/runtime/fleet_types.h:107-111). rope_cos / rope_sin:
 * fp32[max_pos][64] YaRN tables (the reference's act.cos / act.sin,
 * src/host/fleet_launch.hip:186-218). x, x_out: fp32[hidden] (may be equal).
 * The position is `pos` (0 <= pos < max_pos <= 4096, checked here) or, when
 * pos_dev is not NULL, the device int32 *pos_dev read by the kernels, so one
 * captured graph serves every step; a device position outside [0, max_pos)
 * sets FLEET_MOE_ABORT_POSITION in the workspace status and leaves x_out
 * unspecified. One launch of 256 workgroups on `stream`, all resident at once
 * (their stages hand data to each other through the workspace; a stage that
 * waits past its bound sets FLEET_MOE_ABORT_ATTN_WAIT). */
int fleet_attn_decode(const fleet_attn_layer* layer, const float* x, float* x_out,
                      uint16_t* cache, int32_t max_pos, int32_t pos, const int32_t* pos_dev,
                      const float* rope_cos, const float* rope_sin, void* workspace,
                      size_t workspace_bytes, const fleet_moe_dims* dims, hipStream_t stream);

/* ------------------------------------------------------------------------
 * The whole decode step in one launch (no separate counterpart in the
 * reference, whose persistent kernel runs a step's task graph in one launch:
 * src/kernels/fleet_kernel.hip:933-1040, driven by src/host/fleet_launch.hip).
 * Same arithmetic as embed, then per layer fleet_attn_decode and
 * fleet_moe_dense_decode / fleet_moe_layer_decode, then fleet_lm_head_argmax:
 * every result equals that sequence's bit for bit. */

/* One decoder layer: its attention weights, its FFN (the dense SwiGLU blob
 * "L{i}.dense" when dense is not NULL, with moe.norm as its post-attention
 * norm and the other moe fields unused; else the MoE layer moe) and its KV
 * cache (bf16 [max_pos][576]). */
typedef struct fleet_step_layer {
    fleet_attn_layer attn;
    fleet_moe_layer moe;
    const uint16_t* dense;
    uint16_t* cache;
} fleet_step_layer;

/* Most layers a fleet_decode_step / fleet_ffn_column layer table may hold. */
#define FLEET_STEP_MAX_LAYERS 64

/* The model: layers is a DEVICE array of n_layers (<= FLEET_STEP_MAX_LAYERS)
 * entries, which the kernel reads; embed, lm_head bf16 [102400][hidden];
 * final_norm bf16[hidden] or NULL; rope_cos / rope_sin fp32 [max_pos][64],
 * max_pos <= 4096. */
typedef struct fleet_step_model {
    const fleet_step_layer* layers;
    int32_t n_layers;
    int32_t max_pos;
    const uint16_t* embed;
    const uint16_t* final_norm;
    const uint16_t* lm_head;
    const float* rope_cos;
    const float* rope_sin;
} fleet_step_model;

/* Workspace bytes fleet_decode_step needs (one buffer; about 2.8 MB). */
size_t fleet_decode_step_workspace_bytes(const fleet_moe_dims* dims);

/* One greedy step at position *pos_dev for the token *token (device int32s):
 * x = embed[token], every layer (attention half, then FFN half), then
 * token = argmax(bf16(lm_head . rms_norm(x, final_norm))) (lowest index on
 * ties) into *token_out and *token_next (either may be NULL; token_next may
 * equal token, feeding the next step), and *pos_dev += 1. x_out: fp32[hidden]
 * receives the final residual, or NULL; logits: fp32[102400] or NULL. One
 * launch of 256 workgroups (one per CU), all resident at once (checked as for
 * fleet_moe_layer_decode). A position outside [0, max_pos) or a token outside
 * the vocabulary sets FLEET_MOE_ABORT_POSITION / _TOKEN and the step does
 * nothing else; a stage whose input never arrives sets
 * FLEET_MOE_ABORT_STEP_WAIT (or its stage's wait bit). Calls on one workspace
 * must be ordered on one stream. */
int fleet_decode_step(const fleet_step_model* model, const int32_t* token, int32_t* token_out,
                      int32_t* token_next, int32_t* pos_dev, float* x_out, float* logits,
                      void* workspace, size_t workspace_bytes, const fleet_moe_dims* dims,
                      hipStream_t stream);

/* The FLEET_MOE_ABORT_* bits recorded in a fleet_decode_step workspace (the
 * OR over its stages), read synchronously on `stream`. */
int fleet_decode_step_status(const void* workspace, uint32_t* status, hipStream_t stream);

/* The FFN half of every layer of the table chained on x in ONE launch (the
 * benchmark's config 3, reference_decode.py:294-302 without the attention
 * half): x_out = ffn_{n-1}(... ffn_0(x)), each x' = bf16(x + ffn(rms_norm(x)))
 * with the layer's dense or MoE FFN; equal bit for bit to chaining
 * fleet_moe_dense_decode / fleet_moe_layer_decode. layers: DEVICE array
 * (only the FFN fields are read); x, x_out: fp32[hidden] (may be equal);
 * workspace: as fleet_decode_step's (status: fleet_decode_step_status). */
int fleet_ffn_column(const fleet_step_layer* layers, int32_t n_layers, const float* x,
                     float* x_out, void* workspace, size_t workspace_bytes,
                     const fleet_moe_dims* dims, hipStream_t stream);

/* x = embed[*token] as fp32 (the EMBED task, src/kernels/fleet_kernel.hip:
 * 68-78). token: a device int32, so a decode loop can feed the previous
 * step's argmax without a host round trip; a token outside [0, 102400) sets
 * FLEET_MOE_ABORT_TOKEN in the (attention) workspace status and x = 0. */
int fleet_embed(const uint16_t* embed, const int32_t* token, float* x, void* workspace,
                size_t workspace_bytes, hipStream_t stream);

/* Greedy next token: logits = bf16(lm_head . rms_norm(x, final_norm)), token
 * = argmax with ties to the lowest index. Replaces the LM_HEAD (11) and
 * ARGMAX (12) task bodies (src/kernels/fleet_kernel.hip:905-920, 509-585);
 * semantics of HF's bf16 lm_head and torch.argmax as src/host/
 * reference_run.py:99-105 picks the greedy token. logits: fp32[102400]
 * (bf16-valued) or NULL; token_out, token_next: device int32 or NULL (both
 * receive the token; token_next is the input of the next fleet_embed, NULL
 * under teacher forcing); pos_advance: device int32 incremented by one after
 * the pick (the pos_dev of the next step) or NULL. Two launches. */
int fleet_lm_head_argmax(const float* x, const uint16_t* final_norm, const uint16_t* lm_head,
                         float* logits, int32_t* token_out, int32_t* token_next,
                         int32_t* pos_advance, void* workspace, size_t workspace_bytes,
                         const fleet_moe_dims* dims, hipStream_t stream);

/* Copies the workspace's sticky status word to *status (0 = healthy; a
 * nonzero value names a bounded wait that expired, see FLEET_MOE_ABORT_*),
 * synchronising `stream`. The reference's equivalent is the sticky rt.abort
 * word (src/runtime/fleet_runtime.h:194-198, 287-293). */
int fleet_moe_workspace_status(const void* workspace, uint32_t* status, hipStream_t stream);

#define FLEET_MOE_ABORT_ROUTER_WAIT 0x1u  /* router logits never published  */
#define FLEET_MOE_ABORT_UNIT_WAIT 0x2u    /* an expert unit never completed */
#define FLEET_MOE_ABORT_GROUP_WAIT 0x4u   /* grouped step phase never completed */
#define FLEET_MOE_ABORT_POSITION 0x8u     /* device position outside [0, max_pos) */
#define FLEET_MOE_ABORT_TOKEN 0x10u       /* device token outside the vocabulary */
#define FLEET_MOE_ABORT_ATTN_WAIT 0x20u   /* an attention stage never completed */
#define FLEET_MOE_ABORT_BAD_ID 0x40u      /* grouped: an expert id outside [0, n_routed)
                                             was clamped into range (output unspecified) */
#define FLEET_MOE_ABORT_STEP_WAIT 0x80u   /* fleet_decode_step: a stage's input residual
                                             (or an lm_head candidate) never arrived */

/* Diagnostic: reads `bytes` of device memory with the weight-streaming load
 * pattern of the kernels above (16-byte non-temporal loads, 1 KB per wave
 * instruction) and nothing else. Gives the achievable HBM read rate, and is
 * the known-size kernel against which rocprofv3 FETCH_SIZE is calibrated.
 * The reference's equivalent is bench/microbench.hip section (c),
 * gemv_stream (:422-447). bytes must be a multiple of 4096; sink: a device
 * uint32 that is written only if the XOR of the data is 0x9e3779b9. */
int fleet_moe_stream_read(const void* buf, size_t bytes, uint32_t* sink, hipStream_t stream);

/* Human-readable text for a return code of this library. */
const char* fleet_moe_error_string(int code);

/* ABI version of this header (major * 100 + minor). */
int fleet_moe_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* FLEET_MOE_H */
