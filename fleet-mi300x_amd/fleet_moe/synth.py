"""Seeded synthetic MoE weights and inputs (no checkpoint exists offline).

Every tensor is drawn from its own stream, keyed by (seed, layer, kind,
index) through NumPy's SeedSequence, so one expert can be regenerated
without drawing the other 63. Weights are N(0, 0.02^2) in fp32 rounded to
bf16 (round to nearest even); hidden inputs are N(0, 1).
"""
from __future__ import annotations

from concurrent.futures import ThreadPoolExecutor

import numpy as np

from .layout import DSV2_LITE, Layout, MoeDims, moe_layout, view_u16

STD = 0.02

# tensor kinds of the key
ROUTER, EXPERT_GATE, EXPERT_UP, EXPERT_DOWN, SHARED_GATE, SHARED_UP, SHARED_DOWN, HIDDEN, ZIPF = range(9)


def rng_for(seed: int, layer: int, kind: int, index: int = 0) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(np.random.SeedSequence([seed, layer, kind, index])))


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bit patterns, round to nearest even (finite inputs)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    return ((u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)).astype(np.uint16)


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def normal_bf16(seed: int, layer: int, kind: int, index: int, shape, std: float = STD) -> np.ndarray:
    g = rng_for(seed, layer, kind, index)
    return bf16_bits(g.standard_normal(shape, dtype=np.float32) * np.float32(std))


def fill_expert(block: np.ndarray, seed: int, layer: int, e: int, dims: MoeDims) -> None:
    """Write routed expert e into its packed block (uint16 [expert_stride])."""
    H, I = dims.hidden, dims.moe_inter
    gu = block[: 2 * I * H].reshape(2 * I, H)
    gu[0::2] = normal_bf16(seed, layer, EXPERT_GATE, e, (I, H))
    gu[1::2] = normal_bf16(seed, layer, EXPERT_UP, e, (I, H))
    block[2 * I * H: 3 * I * H] = normal_bf16(seed, layer, EXPERT_DOWN, e, (H * I,))


def fill_shared(block: np.ndarray, seed: int, layer: int, dims: MoeDims) -> None:
    H, SI = dims.hidden, dims.shared_inter
    gu = block[: 2 * SI * H].reshape(2 * SI, H)
    gu[0::2] = normal_bf16(seed, layer, SHARED_GATE, 0, (SI, H))
    gu[1::2] = normal_bf16(seed, layer, SHARED_UP, 0, (SI, H))
    block[2 * SI * H: 3 * SI * H] = normal_bf16(seed, layer, SHARED_DOWN, 0, (H * SI,))


def moe_layer_blob(seed: int = 0, layer: int = 1, dims: MoeDims = DSV2_LITE,
                   threads: int = 8, lay: Layout | None = None) -> tuple[np.ndarray, Layout]:
    """One MoE layer in the packed layout: (uint8 blob, layout). The
    post-attention norm weight is unit (bf16 1.0), as in the benchmark configs."""
    lay = lay or moe_layout(dims, layers=(layer,))
    blob = np.zeros(lay.nbytes, dtype=np.uint8)
    t = lay.tensors
    if f"L{layer}.norm_post" in t:
        view_u16(blob, t[f"L{layer}.norm_post"])[:] = bf16_bits(np.ones(dims.hidden, np.float32))
    view_u16(blob, t[f"L{layer}.router"])[:] = normal_bf16(
        seed, layer, ROUTER, 0, (dims.n_routed * dims.hidden,))
    experts = view_u16(blob, t[f"L{layer}.experts"]).reshape(dims.n_routed, dims.expert_stride)
    with ThreadPoolExecutor(max(1, threads)) as ex:
        list(ex.map(lambda e: fill_expert(experts[e], seed, layer, e, dims), range(dims.n_routed)))
    fill_shared(view_u16(blob, t[f"L{layer}.shared"]), seed, layer, dims)
    return blob, lay


def hidden_inputs(seed: int, n: int, hidden: int = 2048, layer: int = 0) -> np.ndarray:
    """n seeded N(0,1) hidden vectors, fp32 [n, hidden]."""
    return rng_for(seed, layer, HIDDEN, 0).standard_normal((n, hidden), dtype=np.float32)


def zipf_logit_bias(seed: int, n_routed: int = 64, s: float = 1.1) -> np.ndarray:
    """log p_e with p_e proportional to rank(e)^-s over a seeded permutation of
    the experts: the skewed-load prior of the grouped benchmark."""
    perm = rng_for(seed, 0, ZIPF, 0).permutation(n_routed)
    rank = np.empty(n_routed, np.int64)
    rank[perm] = np.arange(1, n_routed + 1)
    p = rank.astype(np.float64) ** -s
    p /= p.sum()
    return np.log(p).astype(np.float32)
