"""CPU oracle for the batch-1 DeepSeek-V2-Lite MoE decode path.

TEST INFRASTRUCTURE ONLY. This module is the checker the HIP path is compared
against; it is imported by `tests/`, by `__graft_entry__.smoke()` and by the
`cpu_baseline` leg of `bench.py`, and by nothing the product ships. The
product path (the `fleet_moe` package and `libfleet_moe.so`) never calls it.

It restates, in plain NumPy, the task semantics of the reference's
`src/host/reference_decode.py` (cited per function below) together with the
selection rule of the reference kernel (`src/kernels/fleet_kernel.hip`) and
the multi-token semantics of HF's `DeepseekV2MoE.moe_infer`
(`reference/modeling_deepseek.py:591-664`). All citations are relative to the
reference repository root.

Arithmetic choices, each one the exact value the reference's fp32 arithmetic
approximates (the reference leaves the rounding of these reductions to
OpenBLAS / numpy and is therefore only defined up to a few fp32 ulps):

* the RMSNorm mean of squares, the router dot products and the softmax are
  evaluated in fp64 and rounded once to fp32. Every router product is a
  product of two bf16 values, so these sums are exact to ~1e-16 relative and
  independent of summation order, which makes the routed expert ids a
  deterministic function of the inputs (the GPU path computes them the same
  way, so ids compare bit-exactly);
* SiLU is evaluated in fp64 and rounded to fp32 before the bf16 rounding;
* every other GEMV (expert gate / up / down, the dense MLP, q / kv_a, the
  absorbed query, W_UV, o_proj, lm_head) is evaluated as each dot product's
  exact value rounded once to fp32 (`mv_exact`): the value every fp32
  summation order -- the reference's NumPy/OpenBLAS one included --
  approximates to within a few fp32 ulps. The attention softmax and its
  weighted sum of cache rows are evaluated in fp64 and o_c is rounded once.
  The GPU decode path evaluates them the same way, so its batch-1 outputs
  compare bit for bit; the multi-token grouped kernel (bf16 MFMA, fp32
  accumulation) is compared at bf16 tolerance (rel 1e-2).

Parity status of each function (how it is pinned) is listed in
`tests/test_oracle.py`; every function here is pinned by at least one check
that does not retype its formula.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np

# DeepSeek-V2-Lite shapes (reference/dsv2lite_config.json).
HIDDEN = 2048
MOE_INTER = 1408
N_ROUTED = 64
N_SHARED = 2
TOP_K = 6
RMS_EPS = 1e-6
ROUTED_SCALING = 1.0


# ---------------------------------------------------------------- bf16

def bf16_round(x) -> np.ndarray:
    """Round fp32 to the nearest bf16, ties to even, returned as fp32.

    Restates reference_decode.py:37-48 (the same add-0x7FFF-plus-odd-bit RNE
    formula on the fp32 bit pattern). Finite inputs only.
    """
    x = np.array(x, dtype=np.float32)
    u = x.view(np.uint32)
    r = (u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) & np.uint32(0xFFFF0000)
    return r.astype(np.uint32).view(np.float32)


def bf16_bits(x) -> np.ndarray:
    """bf16 bit patterns (uint16) of the RNE rounding of fp32 `x`."""
    return (bf16_round(x).view(np.uint32) >> np.uint32(16)).astype(np.uint16)


def bf16_to_f32(bits) -> np.ndarray:
    """Widen bf16 bit patterns (uint16) to fp32 exactly."""
    b = np.asarray(bits, dtype=np.uint16)
    return (b.astype(np.uint32) << np.uint32(16)).view(np.float32)


# ---------------------------------------------------------------- a1 residual fold

def residual_fold(x, partials) -> np.ndarray:
    """The post-attention residual x[1] = bf16(x[0] + bf16(sum of o_proj's
    K-split fp32 partials)), the partials added in fp32 one after the other in
    index order (the non-coherent path of stage_residual_f32,
    src/kernels/fleet_kernel.hip:107-144: acc = p[0]; acc += p[x] for x = 1..7;
    then the two roundings). x: fp32 [H]; partials: fp32 [n][H]."""
    p = np.asarray(partials, np.float32)
    acc = p[0].copy()
    for q in p[1:]:
        acc = (acc + q).astype(np.float32)
    return bf16_round(np.asarray(x, np.float32) + bf16_round(acc))


# ---------------------------------------------------------------- a1 RMSNorm

def rms_norm(x, gamma=None, eps: float = RMS_EPS) -> np.ndarray:
    """DeepseekV2RMSNorm with HF's two bf16 roundings.

    reference_decode.py:51-65 (bf16=True) and fleet_kernel.hip:83-96:
    y = bf16(bf16(x * (1 / sqrt(mean(x^2) + eps))) * gamma).
    The mean of squares is the fp64 sum rounded once to fp32; `1/sqrt` are
    single fp32 operations (correctly rounded, as NumPy computes them).
    `gamma=None` is the unit weight. Works on [..., H].
    """
    x32 = np.asarray(x, dtype=np.float32)
    h = x32.shape[-1]
    ssq = np.sum(x32.astype(np.float64) ** 2, axis=-1, keepdims=True)
    var = (ssq / h).astype(np.float32)
    inv = np.float32(1.0) / np.sqrt(var + np.float32(eps))
    y = bf16_round(x32 * inv)
    g = np.float32(1.0) if gamma is None else np.asarray(gamma, dtype=np.float32)
    return bf16_round(y * g)


# ---------------------------------------------------------------- a2 router

def router_logits(w_router, x_n) -> np.ndarray:
    """fp32 router logits = W_g @ x_n.

    reference_decode.py:271 (`w.gate_weight @ x_n`, fp32) and HF
    modeling_deepseek.py:424-426 (F.linear in fp32). Evaluated in fp64 and
    rounded once to fp32 (see module docstring). Accepts x_n of shape [H] or
    [T, H]; returns [E] or [T, E].
    """
    w64 = np.asarray(w_router, dtype=np.float32).astype(np.float64)
    x64 = np.asarray(x_n, dtype=np.float32).astype(np.float64)
    return (x64 @ w64.T).astype(np.float32)


# ---------------------------------------------------------------- a3 top-k

def softmax(logits) -> np.ndarray:
    """Softmax over the last axis: reference_decode.py:72-75, in fp64 then fp32."""
    l64 = np.asarray(logits, dtype=np.float32).astype(np.float64)
    m = np.max(l64, axis=-1, keepdims=True)
    e = np.exp(l64 - m)
    return (e / np.sum(e, axis=-1, keepdims=True)).astype(np.float32)


def topk_lowest_index(scores, k: int):
    """Greedy top-k with ties to the lowest index, in selection order.

    The reference kernel's rule (fleet_kernel.hip:469-494: k passes of an
    argmax in which an equal score with a smaller index wins); the NumPy
    reference's `np.argpartition` (reference_decode.py:273) selects the same
    set but leaves tie order unspecified, and HF's `torch.topk(sorted=False)`
    (modeling_deepseek.py:436-438) likewise. Returns (ids int32[..., k],
    values fp32[..., k]) ordered by decreasing score.
    """
    s = np.asarray(scores, dtype=np.float32)
    # lexsort sorts by the last key first: primary -score, secondary index.
    idx = np.arange(s.shape[-1])
    if s.ndim == 1:
        order = np.lexsort((idx, -s))[:k]
        return order.astype(np.int32), s[order]
    ids = np.stack([np.lexsort((idx, -row))[:k] for row in s]).astype(np.int32)
    return ids, np.take_along_axis(s, ids, axis=-1)


def route(w_router, x_n, top_k: int = TOP_K, routed_scaling: float = ROUTED_SCALING,
          logit_bias=None):
    """Router + softmax + greedy top-k, unnormalised weights x scaling.

    reference_decode.py:271-278 with norm_topk_prob=False; `logit_bias`
    (optional fp32 [E]) is added to the logits before the softmax, which is
    how the skewed-load benchmark of the grouped step biases routing.
    Returns (logits, ids, weights).
    """
    logits = router_logits(w_router, x_n)
    z = logits if logit_bias is None else (logits + np.asarray(logit_bias, np.float32))
    p = softmax(z)
    ids, pv = topk_lowest_index(p, top_k)
    return logits, ids, (pv * np.float32(routed_scaling)).astype(np.float32)


# ---------------------------------------------------------------- exact GEMV

def mv_exact(W, x, chunk_elems: int = 1 << 24) -> np.ndarray:
    """x @ W.T with every dot product's exact value rounded once to fp32.

    W [N, K] (fp32 of bf16 values, or bf16 bits as uint16), x [..., K] (bf16
    or fp32 values). Products of these operands are exact in fp64 (at most
    8 + 24 significand bits) and their fp64 sum is exact up to terms 2^53
    below the largest partial sum, far below what can move an fp32 rounding,
    so the result does not depend on the summation order. Rows are widened
    chunk by chunk to bound memory.
    """
    W = np.asarray(W)
    x64 = np.asarray(x, np.float32).astype(np.float64)
    n, k = W.shape
    out = np.empty(x64.shape[:-1] + (n,), np.float32)
    step = max(1, chunk_elems // max(k, 1))
    for r0 in range(0, n, step):
        blk = W[r0: r0 + step]
        blk = bf16_to_f32(blk) if blk.dtype == np.uint16 else blk
        out[..., r0: r0 + step] = (x64 @ blk.astype(np.float64).T).astype(np.float32)
    return out


# ---------------------------------------------------------------- a5/a6 SwiGLU

def silu(x) -> np.ndarray:
    """x / (1 + exp(-x)) (reference_decode.py:68-69), fp64 then fp32."""
    x64 = np.asarray(x, dtype=np.float32).astype(np.float64)
    return (x64 / (1.0 + np.exp(-x64))).astype(np.float32)


def swiglu_h(gate, up, x_n) -> np.ndarray:
    """h = bf16(bf16(silu(bf16(gate x))) * bf16(up x)), exactly rounded GEMVs.

    reference_decode.py:263-264 and the epilogue of gemv.h:537-542.
    gate/up: [I, H] fp32 (bf16-valued); x_n: [H] or [T, H].
    """
    g = bf16_round(mv_exact(gate, x_n))
    u = bf16_round(mv_exact(up, x_n))
    return bf16_round(bf16_round(silu(g)) * u)


def down_proj(down, h) -> np.ndarray:
    """bf16(down @ h), exactly rounded GEMV: reference_decode.py:265."""
    return bf16_round(mv_exact(down, h))


def mlp_unit(gate, up, down, x_n) -> np.ndarray:
    """One SwiGLU expert with HF's bf16 roundings: reference_decode.py:259-265."""
    return down_proj(down, swiglu_h(gate, up, x_n))


# ---------------------------------------------------------------- a4 packed layout

@dataclass
class PackedLayer:
    """One MoE layer in the reference's packed-weight layout.

    pack_weights.py:125-142: `router` is [E][H] bf16; `experts` is E blocks of
    `expert_stride` elements, each the gate/up rows interleaved
    [g0, u0, g1, u1, ...] ([2I][H]) followed by down ([H][I]); `shared` is the
    interleaved gate/up of the merged shared expert ([2*SI][H]) followed by its
    down ([H][SI]), SI = n_shared * I. Arrays hold bf16 bit patterns (uint16).
    `norm` is the post-attention RMSNorm weight (bf16 bits) or None for unit.
    """
    router: np.ndarray
    experts: np.ndarray
    shared: np.ndarray
    expert_stride: int
    hidden: int = HIDDEN
    moe_inter: int = MOE_INTER
    n_shared: int = N_SHARED
    norm: np.ndarray | None = None
    cache: dict = field(default_factory=dict, repr=False)

    @property
    def shared_inter(self) -> int:
        return self.n_shared * self.moe_inter

    def router_f32(self) -> np.ndarray:
        return bf16_to_f32(self.router).reshape(-1, self.hidden)

    def gamma_f32(self):
        return None if self.norm is None else bf16_to_f32(self.norm)

    def expert_f32(self, e: int):
        """(gate [I,H], up [I,H], down [H,I]) of routed expert e, fp32.

        Addressing as expert.h:52-59: base = experts + e * stride,
        down = base + 2 * I * H.
        """
        if int(e) in self.cache:
            return self.cache[int(e)]
        H, I = self.hidden, self.moe_inter
        base = int(e) * self.expert_stride
        gu = bf16_to_f32(self.experts[base: base + 2 * I * H]).reshape(2 * I, H)
        dn = bf16_to_f32(self.experts[base + 2 * I * H: base + 3 * I * H]).reshape(H, I)
        return np.ascontiguousarray(gu[0::2]), np.ascontiguousarray(gu[1::2]), dn

    def shared_f32(self):
        """(gate [SI,H], up [SI,H], down [H,SI]) of the merged shared expert."""
        if "shared" in self.cache:
            return self.cache["shared"]
        H, SI = self.hidden, self.shared_inter
        gu = bf16_to_f32(self.shared[: 2 * SI * H]).reshape(2 * SI, H)
        dn = bf16_to_f32(self.shared[2 * SI * H: 3 * SI * H]).reshape(H, SI)
        return np.ascontiguousarray(gu[0::2]), np.ascontiguousarray(gu[1::2]), dn

    def widen(self, experts=None) -> None:
        """Pre-widen experts (all if None) and the shared expert to fp32 and
        keep them, so repeated oracle calls skip the bf16 -> fp32 conversion
        (the reference's LayerWeights hold fp32 arrays, reference_decode.py:
        139-163)."""
        n = self.experts.size // self.expert_stride
        for e in (range(n) if experts is None else experts):
            if int(e) not in self.cache:
                self.cache[int(e)] = self.expert_f32(int(e))
        if "shared" not in self.cache:
            self.cache["shared"] = self.shared_f32()


def resolve_unit(layer: PackedLayer, slot: int, ids, weights):
    """Map a descriptor routing slot to (gate_up, down, down_ld, weight, rows).

    Restates expert.h:45-71 on flat uint16 arrays: slot k >= 0 is routed
    expert ids[k] (base + id * stride, down after the 2*I*H gate/up block,
    ld = I, weight = weights[k]); slot -1/-2 is half h of the shared expert
    (gate/up rows [h*I, (h+1)*I) at element offset h*2*I*H, down columns
    [h*I, (h+1)*I) of every row at offset 2*SI*H + h*I, ld = SI, weight 1).
    Returns flat views plus the row count, like the device pointers.
    """
    H, I, SI = layer.hidden, layer.moe_inter, layer.shared_inter
    if slot >= 0:
        base = int(ids[slot]) * layer.expert_stride
        gate_up = layer.experts[base: base + 2 * I * H]
        down = layer.experts[base + 2 * I * H: base + layer.expert_stride]
        return gate_up, down, I, float(weights[slot]), I
    half = -slot - 1
    rows = SI // 2
    gate_up = layer.shared[half * 2 * rows * H: (half + 1) * 2 * rows * H]
    down = layer.shared[2 * SI * H + half * rows:]
    return gate_up, down, SI, 1.0, rows


def unit_forward(gate_up, down, ld: int, weight: float, rows: int, x_n, hidden: int):
    """One unit of the 8-unit split: bf16(weight * bf16(down_n . h)) per row n,
    the unit arithmetic of gemv.h (gate_up epilogue :537-542, EPI_BF16 :244)."""
    gu = bf16_to_f32(gate_up).reshape(2 * rows, hidden)
    h = swiglu_h(gu[0::2], gu[1::2], x_n)
    d = bf16_to_f32(np.asarray(down)[: (hidden - 1) * ld + rows])
    idx = np.arange(hidden)[:, None] * ld + np.arange(rows)[None, :]
    return bf16_round(np.float32(weight) * down_proj(d[idx], h))


# ---------------------------------------------------------------- a7 combine

def combine(routed_terms, shared_out) -> np.ndarray:
    """moe = bf16(bf16(sum_k t_k) + shared), t_k = bf16(w_k * E_k(x_n)).

    reference_decode.py:280-287; the fp32 sum runs over k in selection order
    (the reference runs it in argpartition order; the terms are bf16 values
    whose fp32 sum is exact unless their exponents differ by more than 16).
    """
    y = np.zeros_like(np.asarray(shared_out, np.float32))
    for t in routed_terms:
        y = (y + np.asarray(t, np.float32)).astype(np.float32)
    return bf16_round(bf16_round(y) + np.asarray(shared_out, np.float32))


def moe(layer: PackedLayer, x_n, top_k: int = TOP_K,
        routed_scaling: float = ROUTED_SCALING, logit_bias=None) -> dict:
    """Router + top-k routed experts + shared expert for one token.

    reference_decode.py:268-287 (`moe`) with the lowest-index tie rule.
    Returns dict(logits, ids, weights, out) with out the bf16-valued fp32 [H].
    """
    x_n = np.asarray(x_n, np.float32)
    logits, ids, ws = route(layer.router_f32(), x_n, top_k, routed_scaling, logit_bias)
    terms = []
    for k, e in enumerate(ids):
        g, u, d = layer.expert_f32(int(e))
        terms.append(bf16_round(ws[k] * mlp_unit(g, u, d, x_n)))
    sg, su, sd = layer.shared_f32()
    out = combine(terms, mlp_unit(sg, su, sd, x_n))
    return {"logits": logits, "ids": ids, "weights": ws, "out": out}


def moe_layer(layer: PackedLayer, x, top_k: int = TOP_K,
              routed_scaling: float = ROUTED_SCALING, eps: float = RMS_EPS) -> dict:
    """The MoE half of a decoder layer: x' = bf16(x + moe(rms_norm(x))).

    reference_decode.py:301-302 (post-attention norm, MoE, bf16 residual add).
    Returns dict(x_n, logits, ids, weights, out, x_out).
    """
    x = np.asarray(x, np.float32)
    x_n = rms_norm(x, layer.gamma_f32(), eps)
    r = moe(layer, x_n, top_k, routed_scaling)
    r["x_n"] = x_n
    r["x_out"] = bf16_round(x + r["out"])
    return r


def moe_layer_fp32(layer: PackedLayer, x, top_k: int = TOP_K,
                   routed_scaling: float = ROUTED_SCALING, eps: float = RMS_EPS) -> dict:
    """The MoE half of a decoder layer in the reference's own arithmetic: the
    CPU path the benchmark times beside the GPU, not a checker.

    reference_decode.py:262-287, 301-302 as written: fp32 NumPy/BLAS matmuls
    for the router and every expert GEMV, SiLU x / (1 + exp(-x)) and the
    softmax in fp32, bf16 rounding points as there, routed terms summed in
    fp32 in selection order; the top-k set uses the lowest-index tie rule
    (the reference's argpartition picks the same set and leaves the order of
    equal scores unspecified). Experts come from layer.expert_f32 (pre-widened
    by layer.widen(), as the reference's LayerWeights are fp32). Outputs agree
    with moe_layer within bf16 tolerance (tests/test_oracle.py); ids agree
    unless a 6th/7th-place gap is below fp32 resolution.
    """
    R = bf16_round
    x = np.asarray(x, np.float32)
    x_n = rms_norm(x, layer.gamma_f32(), eps)
    logits = (layer.cache.get("router32") if "router32" in layer.cache
              else layer.cache.setdefault("router32", layer.router_f32())) @ x_n
    m = np.max(logits)
    e = np.exp(logits - m)
    scores = (e / np.sum(e)).astype(np.float32)
    ids, pv = topk_lowest_index(scores, top_k)
    ws = (pv * np.float32(routed_scaling)).astype(np.float32)

    def mlp(g, u, d):
        a = R(g @ x_n)
        h = R(R(a / (np.float32(1.0) + np.exp(-a, dtype=np.float32))) * R(u @ x_n))
        return R(d @ h)

    y = np.zeros_like(x_n)
    for k, eid in enumerate(ids):
        y = y + R(ws[k] * mlp(*layer.expert_f32(int(eid))))
    out = R(R(y) + mlp(*layer.shared_f32()))
    return {"x_n": x_n, "logits": logits, "ids": ids, "weights": ws, "out": out,
            "x_out": R(x + out)}


def dense_layer(gate, up, down, x, gamma=None, eps: float = RMS_EPS) -> dict:
    """A dense decoder layer's FFN half: x' = bf16(x + mlp(rms_norm(x))).

    reference_decode.py:290-291 (dense_mlp = mlp_unit at the dense width) and
    :301-302 (post-attention norm, bf16 residual add); gate/up [I][H], down
    [H][I] as fp32 arrays of bf16 values. Returns dict(x_n, out, x_out).
    """
    x = np.asarray(x, np.float32)
    x_n = rms_norm(x, gamma, eps)
    out = mlp_unit(gate, up, down, x_n)
    return {"x_n": x_n, "out": out, "x_out": bf16_round(x + out)}


# ---------------------------------------------------------------- a8 grouped

def moe_grouped(layer: PackedLayer, x_n, ids, weights, combine_rule: str = "decode") -> dict:
    """Multi-token MoE product with HF `moe_infer` data movement.

    modeling_deepseek.py:591-664: count tokens per expert (cnts.scatter_),
    argsort the flat (token, slot) ids, gather sorted_tokens = x[idxs // k],
    run each expert's SwiGLU on its contiguous rows, scatter back
    new_x[idxs] = outs, then combine per token; shared expert on every token
    (modeling_deepseek.py:586-587).

    combine_rule "decode": reference_decode.py:283-287 per token (bf16 of each
    weighted expert output, fp32 sum in slot order, bf16, + bf16 shared) --
    the rule the batch-1 path uses, so grouped(T) equals T batch-1 calls.
    combine_rule "hf": moe_infer's `.type(fp32).mul_(w).sum(1).type(bf16)`
    then the bf16 add of the shared output.
    x_n: [T, H] bf16-valued; ids int [T, k]; weights fp32 [T, k].
    Returns dict(out [T,H], tokens_per_expert [E], order (argsort) [T*k]).
    """
    x_n = np.asarray(x_n, np.float32)
    ids = np.asarray(ids, np.int64)
    ws = np.asarray(weights, np.float32)
    T, k = ids.shape
    E = layer.experts.size // layer.expert_stride
    cnts = np.zeros((T, E), np.int64)
    np.put_along_axis(cnts, ids, 1, axis=1)
    tokens_per_expert = cnts.sum(axis=0)
    flat = ids.reshape(-1)
    order = np.argsort(flat, kind="stable")
    sorted_tokens = x_n[order // k]
    outs = np.empty((T * k, layer.hidden), np.float32)
    start = 0
    for e in range(E):
        n = int(tokens_per_expert[e])
        if n == 0:
            continue
        g, u, d = layer.expert_f32(e)
        outs[start: start + n] = mlp_unit(g, u, d, sorted_tokens[start: start + n])
        start += n
    new_x = np.empty_like(outs)
    new_x[order] = outs
    per_slot = new_x.reshape(T, k, layer.hidden)
    sg, su, sd = layer.shared_f32()
    shared = mlp_unit(sg, su, sd, x_n)
    if combine_rule == "decode":
        out = np.stack([combine([bf16_round(ws[t, j] * per_slot[t, j]) for j in range(k)],
                                shared[t]) for t in range(T)])
    elif combine_rule == "hf":
        y = np.zeros((T, layer.hidden), np.float32)
        for j in range(k):
            y = (y + per_slot[:, j] * ws[:, j: j + 1]).astype(np.float32)
        out = bf16_round(bf16_round(y) + shared)
    else:
        raise ValueError(f"unknown combine_rule {combine_rule!r}")
    return {"out": out, "tokens_per_expert": tokens_per_expert, "order": order}


# ---------------------------------------------------------------- a9 byte model

def moe_bytes(hidden: int = HIDDEN, moe_inter: int = MOE_INTER, top_k: int = TOP_K,
              n_shared: int = N_SHARED, n_routed: int = N_ROUTED, distinct=None) -> dict:
    """Algorithmic bytes of one MoE layer per token (bf16 weights).

    model_analysis.py:92-99: each selected routed expert streams
    3 * H * I * 2 bytes, the shared expert 3 * H * (n_shared * I) * 2, the
    router E * H * 2. `distinct` overrides the routed count (grouped step).
    """
    per_expert = 3 * hidden * moe_inter * 2
    shared = 3 * hidden * n_shared * moe_inter * 2
    router = n_routed * hidden * 2
    n = top_k if distinct is None else int(distinct)
    return {"expert": per_expert, "shared": shared, "router": router,
            "selected": n * per_expert + shared}


# ---------------------------------------------------------------- full decode (config 4)
# The attention half of a decoder layer, the embedding and the lm_head, so the
# 27-layer decode can be checked end to end. Shapes of DeepSeek-V2-Lite
# (reference/dsv2lite_config.json); RoPE is YaRN as that config states it
# (theta 1e4, factor 40, original context 4096, beta 32 / 1, mscale 0.707 on
# both sides).

HEADS = 16
KV_LORA = 512
QK_NOPE = 128
QK_ROPE = 64
V_HEAD = 128
VOCAB = 102400
ROPE_THETA = 1e4
ROPE_FACTOR = 40.0
ROPE_ORIG_MAX = 4096
BETA_FAST, BETA_SLOW = 32.0, 1.0
MSCALE = MSCALE_ALL_DIM = 0.707


def yarn_mscale(scale: float, m: float) -> float:
    """reference_decode.py:78-82 (HF yarn_get_mscale)."""
    return 1.0 if scale <= 1 else 0.1 * m * math.log(scale) + 1.0


def rope_tables(max_pos: int, dim: int = QK_ROPE, base: float = ROPE_THETA,
                scale: float = ROPE_FACTOR, original_max: int = ROPE_ORIG_MAX,
                beta_fast: float = BETA_FAST, beta_slow: float = BETA_SLOW,
                mscale: float = MSCALE, mscale_all_dim: float = MSCALE_ALL_DIM):
    """cos, sin [max_pos][dim] fp32: DeepseekV2YarnRotaryEmbedding's cache
    (reference_decode.py:85-117): inverse frequencies blended between the
    extrapolated and the interpolated ones by a linear ramp over the
    correction range, angles t * inv_freq duplicated over both halves, times
    mscale(scale, mscale) / mscale(scale, mscale_all_dim)."""
    def corr_dim(rot):
        return (dim * math.log(original_max / (rot * 2 * math.pi))) / (2 * math.log(base))
    lo = max(math.floor(corr_dim(beta_fast)), 0)
    hi = min(math.ceil(corr_dim(beta_slow)), dim - 1)
    if lo == hi:
        hi += 0.001
    half = np.arange(0, dim, 2, dtype=np.float32)
    extra = 1.0 / (base ** (half / dim))
    inter = 1.0 / (scale * base ** (half / dim))
    ramp = np.clip((np.arange(dim // 2, dtype=np.float32) - lo) / (hi - lo), 0, 1)
    keep = 1.0 - ramp                     # weight of the extrapolated frequency
    inv_freq = inter * (1 - keep) + extra * keep
    t = np.arange(max_pos, dtype=np.float32)
    ang = np.outer(t, inv_freq)
    emb = np.concatenate([ang, ang], axis=-1)
    m = yarn_mscale(scale, mscale) / yarn_mscale(scale, mscale_all_dim)
    return (np.cos(emb) * m).astype(np.float32), (np.sin(emb) * m).astype(np.float32)


def apply_rope(x, cos, sin) -> np.ndarray:
    """DeepseekV2 RoPE (reference_decode.py:120-134): reorder [x0, x1, ..., x63]
    to [x0, x2, ..., x62, x1, x3, ..., x63], then x * cos + rotate_half(x) * sin
    with rotate_half(v) = [-v[32:], v[:32]]. The result stays in the reordered
    basis (that is what HF caches and what the queries meet)."""
    x = np.asarray(x, np.float32)
    d = x.shape[-1]
    y = np.concatenate([x[..., 0::2], x[..., 1::2]], axis=-1)
    rot = np.concatenate([-y[..., d // 2:], y[..., :d // 2]], axis=-1)
    return (y * cos + rot * sin).astype(np.float32)


def softmax_scale() -> float:
    """reference_decode.py:191-197: (qk_nope + qk_rope)^-0.5 * mscale_all_dim^2."""
    m = yarn_mscale(ROPE_FACTOR, MSCALE_ALL_DIM)
    return (QK_NOPE + QK_ROPE) ** -0.5 * m * m


@dataclass
class AttnLayer:
    """One layer's attention tensors in the packed layout (bf16 bits):
    norm_in [H], qkv [(heads*(nope+rope)) + kv_lora + rope][H] (q_proj rows
    then kv_a_proj_with_mqa rows), kv_a_norm [kv_lora], kv_b
    [heads*(nope+v)][kv_lora], o_proj [H][heads*v] (pack_weights.py:113-121)."""
    norm_in: np.ndarray
    qkv: np.ndarray
    kv_a_norm: np.ndarray
    kv_b: np.ndarray
    o_proj: np.ndarray
    heads: int = HEADS
    cache_f32: dict = field(default_factory=dict, repr=False)

    def f32(self, name):
        if name not in self.cache_f32:
            self.cache_f32[name] = bf16_to_f32(getattr(self, name))
        return self.cache_f32[name]


def attention(w: AttnLayer, x, cache, pos: int, cos, sin, eps: float = RMS_EPS) -> dict:
    """Absorbed-MLA decode step (reference_decode.py:210-256), bf16 rounding
    points as there: q and kv_a bf16, c after kv_a_layernorm and k_pe after
    RoPE bf16 (written to cache[pos]), q_c fp32, the 2048 head outputs bf16,
    o_proj bf16. Every GEMV is exactly rounded (mv_exact); the scores, the
    softmax and its weighted sum of c are evaluated in fp64 and o_c is
    rounded once to fp32 (the reference's fp32 values, each to within a few
    ulps). cache: fp32 [max_pos][576], rows < pos filled. Returns dict(out,
    q_c, scores, row)."""
    H = w.heads
    L, Dk, Dr, Dv = KV_LORA, QK_NOPE, QK_ROPE, V_HEAD
    hidden = np.asarray(x).shape[-1]
    x_n = rms_norm(x, bf16_to_f32(w.norm_in), eps)
    qkv = bf16_round(mv_exact(w.f32("qkv").reshape(-1, hidden), x_n))
    q = qkv[: H * (Dk + Dr)].reshape(H, Dk + Dr)
    kv_a = qkv[H * (Dk + Dr):]
    c_new = rms_norm(kv_a[:L], bf16_to_f32(w.kv_a_norm), eps)
    k_pe = bf16_round(apply_rope(kv_a[L:], cos[pos], sin[pos]))
    q_pe = bf16_round(apply_rope(q[:, Dk:], cos[pos], sin[pos]))
    cache[pos, :L] = c_new
    cache[pos, L:] = k_pe
    rows = cache[: pos + 1].astype(np.float64)           # [c ; k_pe] per position
    kv_b = w.f32("kv_b").reshape(H * (Dk + Dv), L)
    scale = softmax_scale()
    out = np.empty(H * Dv, np.float32)
    qcs, scs, ocs = [], [], []
    for h in range(H):
        w_uk = kv_b[h * (Dk + Dv): h * (Dk + Dv) + Dk]
        w_uv = kv_b[h * (Dk + Dv) + Dk: (h + 1) * (Dk + Dv)]
        q_c = mv_exact(w_uk.T, q[h, :Dk])
        s = (rows @ np.concatenate([q_c, q_pe[h]]).astype(np.float64)) * scale
        e = np.exp(s - s.max())
        o_c = ((e @ rows[:, :L]) / e.sum()).astype(np.float32)
        out[h * Dv:(h + 1) * Dv] = bf16_round(mv_exact(w_uv, o_c))
        qcs.append(q_c)
        scs.append(s)
        ocs.append(o_c)
    o = bf16_round(mv_exact(w.f32("o_proj").reshape(hidden, H * Dv), out))
    return {"out": o, "q_c": np.array(qcs), "scores": np.array(scs),
            "row": cache[pos].copy(), "qkv": qkv, "o_c": np.array(ocs), "heads": out,
            "q_pe": q_pe}


def lm_head_argmax(x, final_norm, lm_head, eps: float = RMS_EPS) -> dict:
    """Final RMSNorm, logits = bf16(lm_head . x_n) (fleet_kernel.hip:915-920,
    EPI_BF16; exactly rounded GEMV), next token = the largest logit, lowest
    index on ties (the argmax rule of fleet_kernel.hip:509-585)."""
    x_n = rms_norm(x, None if final_norm is None else bf16_to_f32(final_norm), eps)
    logits = bf16_round(mv_exact(np.asarray(lm_head).reshape(-1, x_n.shape[-1]), x_n))
    best = float(logits.max())
    tok = int(np.flatnonzero(logits == best)[0])
    second = float(np.max(np.where(np.arange(logits.size) == tok, -np.inf, logits)))
    return {"logits": logits, "token": tok, "margin": best - second}


@dataclass
class DenseFfn:
    """A dense layer's FFN (pack_weights.py:143-146, unpacked): gate, up
    [I][H] and down [H][I] as fp32 arrays of bf16 values; norm is the
    post-attention RMSNorm weight (bf16 bits) or None."""
    gate: np.ndarray
    up: np.ndarray
    down: np.ndarray
    norm: np.ndarray | None = None


def decoder_layer(attn_w: AttnLayer, ffn, x, cache, pos: int, cos, sin,
                  eps: float = RMS_EPS) -> dict:
    """One decoder layer, reference_decode.py:294-302: x1 = bf16(x + attn(x)),
    then x2 = bf16(x1 + ffn(rms_norm(x1, norm_post))) with the MoE of
    `moe_layer` (ffn a PackedLayer) or the dense MLP (ffn a DenseFfn).
    Appends cache[pos]. Returns dict(x_attn, x_out, ids)."""
    a = attention(attn_w, x, cache, pos, cos, sin, eps)
    x1 = bf16_round(np.asarray(x, np.float32) + a["out"])
    if isinstance(ffn, DenseFfn):
        g = None if ffn.norm is None else bf16_to_f32(ffn.norm)
        r = dense_layer(ffn.gate, ffn.up, ffn.down, x1, g, eps)
        ids = None
    else:
        r = moe_layer(ffn, x1, eps=eps)
        ids = r["ids"]
    return {"x_attn": x1, "x_out": r["x_out"], "ids": ids}


@dataclass
class DecodeModel:
    """The whole decoder for `decode_step`: embed / lm_head bf16 bits
    [vocab][H] (lm_head may be pre-widened fp32), final_norm bf16 bits or
    None, and per layer an AttnLayer and a PackedLayer or DenseFfn."""
    embed: np.ndarray
    final_norm: np.ndarray | None
    lm_head: np.ndarray
    attn: list
    ffn: list


def decode_step(model: DecodeModel, token: int, pos: int, caches, cos, sin,
                eps: float = RMS_EPS) -> dict:
    """One greedy step at position `pos`: x = embed[token] (fp32 of the bf16
    row, fleet_kernel.hip:68-78), every decoder_layer, then lm_head_argmax.
    caches: per layer fp32 [max_pos][576], row pos appended. Returns
    dict(token, margin, logits, x per layer output)."""
    hidden = model.attn[0].norm_in.size
    x = bf16_to_f32(model.embed.reshape(-1, hidden)[int(token)])
    xs = []
    for i, (aw, fw) in enumerate(zip(model.attn, model.ffn)):
        x = decoder_layer(aw, fw, x, caches[i], pos, cos, sin, eps)["x_out"]
        xs.append(x)
    r = lm_head_argmax(x, model.final_norm, model.lm_head, eps)
    r["xs"] = xs
    return r
