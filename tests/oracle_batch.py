"""The oracle's MoE layer over a batch of tokens, for tests that check many
GPU outputs at once. Test infrastructure, like the oracle it composes."""
from __future__ import annotations

import numpy as np

from oracle import moe_oracle as orc


def moe_layer_batched(pl, x) -> dict:
    """orc.moe_layer over a batch of tokens [T, H], composed from the same
    oracle functions: one routing call, the shared expert as one batch, each
    routed expert once over the tokens that selected it (its exactly rounded
    GEMVs do not depend on the batching), the combine in selection order."""
    x = np.asarray(x, np.float32)
    x_n = orc.rms_norm(x, pl.gamma_f32())
    _, ids, ws = orc.route(pl.router_f32(), x_n)
    shared = orc.mlp_unit(*pl.shared_f32(), x_n)
    e_out = np.zeros(ids.shape + (x.shape[1],), np.float32)
    for e in np.unique(ids):
        t, k = np.nonzero(ids == e)
        e_out[t, k] = orc.mlp_unit(*pl.expert_f32(int(e)), x_n[t])
    terms = [orc.bf16_round(ws[:, k:k + 1] * e_out[:, k]) for k in range(ids.shape[1])]
    out = orc.combine(terms, shared)
    return {"ids": ids, "weights": ws, "out": out, "x_out": orc.bf16_round(x + out)}
