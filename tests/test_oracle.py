"""Pins the CPU oracle (oracle/moe_oracle.py) before it is trusted as the
checker of the HIP path.

The reference holds no committed numeric golden vectors for the MoE path
(its MoE tests compute their expectations inside the test), so each oracle
function is pinned here by checks that do not retype its formula:

| oracle function      | pinned by                                                      |
|----------------------|----------------------------------------------------------------|
| bf16_round/bits      | torch's fp32->bf16 cast (library), hand-picked tie cases        |
| rms_norm             | torch HF-style RMSNorm in bf16 (DeepseekV2RMSNorm semantics);   |
|                      | fp64 closed form; scale invariance; a one-rounding sabotage     |
| router_logits        | fp64 matmul of the bf16 operands; torch F.linear fp32           |
| softmax              | scipy.special.softmax                                           |
| topk_lowest_index    | brute force over (-p, index); all-equal, planted-tie and        |
|                      | permutation cases; torch.topk set on distinct scores            |
| silu / mlp_unit      | torch bf16 nn.Linear + F.silu (HF DeepseekV2MLP rounding        |
|                      | points); zero weights; one-hot input selects a column           |
| moe / moe_layer      | torch restatement of HF MoEGate + moe_infer + shared expert     |
|                      | (reference tolerance bf16 rel 3e-2, ids set-equal); the 8-unit  |
|                      | split of expert.h on the packed layout (reference test          |
|                      | test_expert_addressing.py: ids exact, rel <= 1e-2) with its     |
|                      | old-offset sabotage (must fail)                                 |
| resolve_unit         | gathering via slot pointers reproduces experts[id] / shared     |
|                      | halves; sabotaged offsets are detected                          |
| moe_grouped          | grouped(T) == stack of per-token moe (rel 1e-2); brute force at |
|                      | tiny T; tokens_per_expert sums to k*T; HF combine rule agrees   |
| moe_bytes            | the byte counts of model_analysis.py:92-99 at the real shape    |
"""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import moe_oracle as orc

R = orc.bf16_round


def rel_err(got, want) -> float:
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    return float(np.max(np.abs(got - want)) / max(np.max(np.abs(want)), 1e-30))


def t_bf16(a) -> torch.Tensor:
    return torch.from_numpy(np.asarray(a, np.float32)).to(torch.bfloat16)


# ---------------------------------------------------------------- bf16

def test_bf16_round_matches_torch_cast():
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(100_000).astype(np.float32) * 10.0 ** rng.integers(-30, 30, 100_000),
                        np.float32([0.0, -0.0, 1.0, -1.0, 3.4e38, 1e-40, -1e-42])]).astype(np.float32)
    want = torch.from_numpy(x).to(torch.bfloat16).to(torch.float32).numpy()
    np.testing.assert_array_equal(R(x).view(np.uint32), want.view(np.uint32))


def test_bf16_round_ties_to_even():
    # 1 + 2^-8 is exactly halfway between bf16 1.0 and 1 + 2^-7: ties to even (1.0)
    assert R(np.float32(1 + 2 ** -8)) == np.float32(1.0)
    # 1 + 3 * 2^-8 is halfway between 1 + 2^-7 (odd) and 1 + 2^-6 (even)
    assert R(np.float32(1 + 3 * 2 ** -8)) == np.float32(1 + 2 ** -6)
    assert R(np.float32(1 + 2 ** -8 + 2 ** -20)) == np.float32(1 + 2 ** -7)
    bits = orc.bf16_bits(np.float32([1.0, -2.0]))
    np.testing.assert_array_equal(orc.bf16_to_f32(bits), [1.0, -2.0])


# ---------------------------------------------------------------- a1 RMSNorm

def hf_rmsnorm_bf16(x: np.ndarray, gamma: np.ndarray, eps: float) -> np.ndarray:
    """DeepseekV2RMSNorm run by torch in bf16 (modeling_deepseek.py RMSNorm:
    fp32 variance, x * rsqrt, cast to bf16, times the bf16 weight)."""
    h = torch.from_numpy(x.astype(np.float32))
    var = h.pow(2).mean(-1, keepdim=True)
    h = h * torch.rsqrt(var + eps)
    return (t_bf16(gamma) * h.to(torch.bfloat16)).to(torch.float32).numpy()


def test_residual_fold_order_and_roundings():
    """residual_fold = bf16(x + bf16(p_0 + ... + p_7)), fp32 adds in index
    order (stage_residual_f32, fleet_kernel.hip:107-144). Planted cases, each
    failing one plausible mistake."""
    z = np.zeros(2048, np.float32)

    def fold1(x0, ps):
        parts = np.zeros((8, 2048), np.float32)
        for i, v in enumerate(ps):
            parts[i, 0] = v
        x = z.copy()
        x[0] = x0
        return float(orc.residual_fold(x, parts)[0])
    # index order: 1e8 + 1 rounds to 1e8 in fp32, so the 1 survives only after
    # the cancellation (a pairwise or reversed order gives 0 here)
    assert fold1(0.0, [1e8, 1.0, -1e8, 1.0]) == 1.0
    assert fold1(0.0, [1.0, 1e8, -1e8]) == 0.0
    # the inner bf16 rounding: bf16(2^-8 + 2^-16) = 2^-8, then 1 + 2^-8 is a
    # tie that rounds to even (1.0); without it the sum rounds up
    assert fold1(1.0, [2.0 ** -8 + 2.0 ** -16]) == 1.0
    # the outer rounding: 1 + 2^-10 is not a bf16 value
    assert fold1(1.0, [2.0 ** -10]) == 1.0
    # exactly representable values: the fold is the plain sum
    rng = np.random.default_rng(0)
    x = rng.integers(-64, 64, 2048).astype(np.float32)
    parts = rng.integers(-16, 16, (8, 2048)).astype(np.float32)
    np.testing.assert_array_equal(orc.residual_fold(x, parts), x + parts.sum(0))


def test_rms_norm_matches_torch_hf_module():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((64, 2048)).astype(np.float32)
    gamma = R(1.0 + 0.1 * rng.standard_normal(2048).astype(np.float32))
    got = orc.rms_norm(x, gamma)
    want = hf_rmsnorm_bf16(x, gamma, 1e-6)
    # rsqrt vs 1/sqrt and the mean's rounding differ in the last fp32 bits, so
    # a bf16 rounding may flip: allow 1 bf16 ulp on a handful of elements.
    ulp = np.abs(got.view(np.int32) - want.view(np.int32)) >> 16
    assert ulp.max() <= 1
    assert np.mean(ulp != 0) < 1e-3


def test_rms_norm_closed_form_and_invariants():
    rng = np.random.default_rng(2)
    x = rng.standard_normal(2048).astype(np.float32)
    y = orc.rms_norm(x)
    ideal = x.astype(np.float64) / np.sqrt(np.mean(x.astype(np.float64) ** 2) + 1e-6)
    assert np.max(np.abs(y - ideal) / (np.abs(ideal) + 1e-12)) <= 2 ** -8
    # scale invariance up to eps and the bf16 rounding of the scale
    np.testing.assert_allclose(orc.rms_norm(4.0 * x), y, rtol=2 ** -7)
    # zero input stays zero (var = 0, inv = 1/sqrt(eps))
    assert not np.any(orc.rms_norm(np.zeros(2048, np.float32)))


def test_rms_norm_two_roundings_sabotage():
    """A one-rounding RMSNorm (gamma applied before the first bf16 cast) must
    disagree with the oracle somewhere for a non-unit gamma."""
    rng = np.random.default_rng(3)
    x = rng.standard_normal((16, 2048)).astype(np.float32)
    gamma = R(1.0 + 0.3 * rng.standard_normal(2048).astype(np.float32))
    var = (np.sum(x.astype(np.float64) ** 2, -1, keepdims=True) / 2048).astype(np.float32)
    one_rounding = R(x * (np.float32(1) / np.sqrt(var + np.float32(1e-6))) * gamma)
    assert np.any(one_rounding != orc.rms_norm(x, gamma))


# ---------------------------------------------------------------- a2 router

def test_router_logits_exact_against_fp64():
    rng = np.random.default_rng(4)
    w = R(0.02 * rng.standard_normal((64, 2048)).astype(np.float32))
    xn = orc.rms_norm(rng.standard_normal((8, 2048)).astype(np.float32))
    got = orc.router_logits(w, xn)
    exact = xn.astype(np.float64) @ w.astype(np.float64).T
    # one rounding of an (almost) exact sum: within half an fp32 ulp
    assert np.all(np.abs(got - exact) <= np.spacing(np.abs(got).astype(np.float32)) * 0.5 + 1e-30)
    # and within fp32 accumulation noise of torch's fp32 F.linear (HF gate)
    tl = F.linear(torch.from_numpy(xn), torch.from_numpy(w)).numpy()
    assert np.max(np.abs(got - tl)) < 1e-5
    # a transposed operand is caught
    assert np.max(np.abs(orc.router_logits(w[:, ::-1], xn) - got)) > 1e-2


# ---------------------------------------------------------------- a3 softmax + top-k

def test_softmax_matches_scipy():
    from scipy.special import softmax as sp_softmax
    rng = np.random.default_rng(5)
    z = (3 * rng.standard_normal((10, 64))).astype(np.float32)
    np.testing.assert_allclose(orc.softmax(z), sp_softmax(z.astype(np.float64), axis=-1), rtol=1e-6)
    np.testing.assert_allclose(orc.softmax(z).sum(-1), 1.0, rtol=1e-6)


def brute_topk(p: np.ndarray, k: int):
    order = sorted(range(len(p)), key=lambda e: (-float(p[e]), e))[:k]
    return np.array(order, np.int32)


def test_topk_brute_force_and_special_cases():
    rng = np.random.default_rng(6)
    for _ in range(200):
        # coarse values force many ties
        p = rng.integers(0, 8, 64).astype(np.float32) / 8
        ids, vals = orc.topk_lowest_index(p, 6)
        np.testing.assert_array_equal(ids, brute_topk(p, 6))
        np.testing.assert_array_equal(vals, p[ids])
    # all equal -> 0..5
    ids, _ = orc.topk_lowest_index(np.full(64, 1 / 64, np.float32), 6)
    np.testing.assert_array_equal(ids, np.arange(6))
    # planted tie at rank 6: indices 40 and 7 tie for the last slot -> 7 wins
    p = np.zeros(64, np.float32)
    p[[3, 9, 11, 20, 33]] = [0.9, 0.8, 0.7, 0.6, 0.5]
    p[[40, 7]] = 0.25
    ids, _ = orc.topk_lowest_index(p, 6)
    np.testing.assert_array_equal(ids, [3, 9, 11, 20, 33, 7])
    # permuting the experts permutes the answer
    q = rng.permutation(64)
    s = rng.random(64).astype(np.float32)
    ids_s, _ = orc.topk_lowest_index(s, 6)
    ids_q, _ = orc.topk_lowest_index(s[q], 6)
    np.testing.assert_array_equal(q[ids_q], ids_s)
    # same set as torch.topk on distinct scores
    tv, ti = torch.topk(torch.from_numpy(s), 6, sorted=False)
    assert set(ti.tolist()) == set(ids_s.tolist())


def test_route_weights_unnormalised_and_scaled():
    rng = np.random.default_rng(7)
    w = R(0.02 * rng.standard_normal((64, 2048)).astype(np.float32))
    xn = orc.rms_norm(rng.standard_normal(2048).astype(np.float32))
    logits, ids, ws = orc.route(w, xn, 6, 2.5)
    p = orc.softmax(logits)
    np.testing.assert_array_equal(ws, (p[ids] * np.float32(2.5)).astype(np.float32))
    assert ws.sum() < 2.5   # not renormalised


# ---------------------------------------------------------------- a5/a6 SwiGLU

def hf_mlp_bf16(gate, up, down, x) -> np.ndarray:
    """DeepseekV2MLP in bf16 with torch CPU kernels: down(silu(gate x) * up x)."""
    xb = t_bf16(x)
    g = F.linear(xb, t_bf16(gate))
    u = F.linear(xb, t_bf16(up))
    return F.linear(F.silu(g) * u, t_bf16(down)).to(torch.float32).numpy()


def test_mlp_unit_matches_torch_bf16_module():
    rng = np.random.default_rng(8)
    H, I = 2048, 1408
    gate = R(0.02 * rng.standard_normal((I, H)).astype(np.float32))
    up = R(0.02 * rng.standard_normal((I, H)).astype(np.float32))
    down = R(0.02 * rng.standard_normal((H, I)).astype(np.float32))
    x = orc.rms_norm(rng.standard_normal((4, H)).astype(np.float32))
    got = orc.mlp_unit(gate, up, down, x)
    want = hf_mlp_bf16(gate, up, down, x)
    assert rel_err(got, want) <= 1e-2
    # most elements agree exactly (differences come from fp32 sum order only)
    assert np.mean(got == want) > 0.9
    # 1-D input equals the row of the 2-D result
    np.testing.assert_allclose(orc.mlp_unit(gate, up, down, x[1]), got[1], rtol=1e-2, atol=1e-6)


def test_mlp_unit_special_cases():
    rng = np.random.default_rng(9)
    H, I = 64, 16
    gate = R(rng.standard_normal((I, H)).astype(np.float32))
    up = R(rng.standard_normal((I, H)).astype(np.float32))
    down = R(rng.standard_normal((H, I)).astype(np.float32))
    assert not np.any(orc.mlp_unit(np.zeros_like(gate), up, down, np.ones(H, np.float32)))
    # one-hot x selects column c: g = gate[:, c], u = up[:, c]
    c = 17
    x = np.zeros(H, np.float32)
    x[c] = 1.0
    h = R(R(orc.silu(gate[:, c])) * up[:, c])
    np.testing.assert_array_equal(orc.swiglu_h(gate, up, x), h)
    # silu closed form at a few points
    np.testing.assert_allclose(orc.silu(np.float32([0.0, 1.0, -2.0])),
                               [0.0, 1 / (1 + np.exp(-1)), -2 / (1 + np.exp(2))], rtol=1e-7)


def test_dense_layer_matches_torch_hf_decoder_ffn_half():
    """Dense layer 0: torch runs DeepseekV2RMSNorm, DeepseekV2MLP at the dense
    width and the bf16 residual add of DeepseekV2DecoderLayer; the oracle's
    dense_layer must agree to bf16 tolerance, element-exact on most."""
    rng = np.random.default_rng(12)
    H, I = 2048, 10944
    gate = R(0.02 * rng.standard_normal((I, H)).astype(np.float32))
    up = R(0.02 * rng.standard_normal((I, H)).astype(np.float32))
    down = R(0.02 * rng.standard_normal((H, I)).astype(np.float32))
    gamma = R(1.0 + 0.1 * rng.standard_normal(H).astype(np.float32))
    x = R(rng.standard_normal((2, H)).astype(np.float32))
    got = orc.dense_layer(gate, up, down, x, gamma)
    xn = hf_rmsnorm_bf16(x, gamma, 1e-6)
    out = hf_mlp_bf16(gate, up, down, xn)
    want = (t_bf16(x) + t_bf16(out)).to(torch.float32).numpy()
    assert rel_err(got["out"], out) <= 1e-2
    assert rel_err(got["x_out"], want) <= 1e-2
    assert np.mean(got["x_out"] == want) > 0.95
    # zero weights leave the residual stream unchanged
    z = orc.dense_layer(np.zeros_like(gate), up, down, x[0], gamma)
    np.testing.assert_array_equal(z["x_out"], x[0])


# ---------------------------------------------------------------- a4 packed layout

def pack_tiny(rng, H, I, E, n_shared, std):
    """Independent restatement of pack_weights.py:126-142 for test layers."""
    f = lambda *s: R((std * rng.standard_normal(s)).astype(np.float32))  # noqa: E731
    gate, up, down = f(E, I, H), f(E, I, H), f(E, H, I)
    SI = n_shared * I
    sg, su, sd = f(SI, H), f(SI, H), f(H, SI)
    blocks = []
    for e in range(E):
        gu = np.empty((2 * I, H), np.float32)
        gu[0::2], gu[1::2] = gate[e], up[e]
        blocks.append(np.concatenate([gu.reshape(-1), down[e].reshape(-1)]))
    sgu = np.empty((2 * SI, H), np.float32)
    sgu[0::2], sgu[1::2] = sg, su
    router = f(E, H)
    layer = orc.PackedLayer(router=orc.bf16_bits(router), experts=orc.bf16_bits(np.concatenate(blocks)),
                            shared=orc.bf16_bits(np.concatenate([sgu.reshape(-1), sd.reshape(-1)])),
                            expert_stride=3 * H * I, hidden=H, moe_inter=I, n_shared=n_shared)
    return layer, dict(router=router, gate=gate, up=up, down=down, sg=sg, su=su, sd=sd)


def test_packed_layout_addressing():
    rng = np.random.default_rng(10)
    layer, w = pack_tiny(rng, 64, 16, 8, 2, 0.08)
    for e in range(8):
        g, u, d = layer.expert_f32(e)
        np.testing.assert_array_equal(g, w["gate"][e])
        np.testing.assert_array_equal(u, w["up"][e])
        np.testing.assert_array_equal(d, w["down"][e])
    sg, su, sd = layer.shared_f32()
    np.testing.assert_array_equal(sg, w["sg"])
    np.testing.assert_array_equal(sd, w["sd"])
    # slot pointers (expert.h resolve_unit): routed slot -> experts[id]
    ids, ws = np.array([5, 2, 7, 0, 1, 3]), np.full(6, 0.5, np.float32)
    gu, dn, ld, wt, rows = orc.resolve_unit(layer, 2, ids, ws)
    np.testing.assert_array_equal(orc.bf16_to_f32(gu).reshape(32, 64)[0::2], w["gate"][7])
    assert ld == 16 and rows == 16 and wt == 0.5
    # shared half 1 -> gate/up rows [16, 32) and down columns [16, 32)
    gu, dn, ld, wt, rows = orc.resolve_unit(layer, -2, ids, ws)
    np.testing.assert_array_equal(orc.bf16_to_f32(gu).reshape(32, 64)[1::2], w["su"][16:32])
    dcols = orc.bf16_to_f32(dn)[np.arange(64)[:, None] * ld + np.arange(16)[None, :]]
    np.testing.assert_array_equal(dcols, w["sd"][:, 16:32])
    assert ld == 32 and wt == 1.0


def moe_phase_8units(layer, x, x_n, ids, ws, old_bug=False):
    """The reference kernel's 8-unit phase: 6 routed slots + 2 shared halves,
    each bf16(weight * bf16(down . h)), summed in fixed fp32 order, then the
    bf16 residual fold (fleet_kernel.hip:146-201)."""
    H = layer.hidden
    acc = np.zeros(H, np.float32)
    for xcd in range(8):
        slot = xcd if xcd < 6 else -(xcd - 6 + 1)
        gu, dn, ld, wt, rows = orc.resolve_unit(layer, slot, ids, ws)
        if old_bug and slot < 0:   # the offsets before the reference's review: no x2, ld = rows
            half = -slot - 1
            gu = layer.shared[half * rows * H: half * rows * H + 2 * rows * H]
            ld = rows
        acc = (acc + orc.unit_forward(gu, dn, ld, wt, rows, x_n, H)).astype(np.float32)
    return R(x + R(acc))


def test_moe_eight_unit_split_matches_oracle_and_sabotage_fails():
    """Mirror of the reference's tests/test_expert_addressing.py scenario:
    hidden 64, inter 16, 8 routed, top-6, rng(7), weights R(N(0, 0.08)),
    post-norm gamma = 1 + f."""
    rng = np.random.default_rng(7)
    layer, _ = pack_tiny(rng, 64, 16, 8, 2, 0.08)
    gamma = R(R(0.08 * rng.standard_normal(64).astype(np.float32)) + 1.0)
    layer.norm = orc.bf16_bits(gamma)
    for trial in range(3):
        x = R((0.5 * rng.standard_normal(64)).astype(np.float32))
        r = orc.moe_layer(layer, x, top_k=6)
        got = moe_phase_8units(layer, x, r["x_n"], r["ids"], r["weights"])
        p = orc.softmax(orc.router_logits(layer.router_f32(), r["x_n"]))
        assert sorted(r["ids"].tolist()) == sorted(np.argpartition(-p, 5)[:6].tolist())
        assert rel_err(got, r["x_out"]) <= 1e-2
        if trial == 0:
            bad = moe_phase_8units(layer, x, r["x_n"], r["ids"], r["weights"], old_bug=True)
            assert rel_err(bad, r["x_out"]) > 1e-2


# ---------------------------------------------------------------- a7/a8 vs HF semantics

def hf_moe_bf16(layer: orc.PackedLayer, x_n: np.ndarray, top_k: int, scaling: float):
    """Torch restatement of HF DeepseekV2MoE.forward in bf16 (MoEGate in fp32,
    moe_infer's permute / per-expert MLP / un-permute / fp32 weighted sum,
    then + shared_experts(identity)), modeling_deepseek.py:420-467, 568-664."""
    E = layer.experts.size // layer.expert_stride
    xb = t_bf16(x_n)
    logits = F.linear(xb.float(), torch.from_numpy(layer.router_f32()))
    scores = logits.softmax(-1, dtype=torch.float32)
    tw, ti = torch.topk(scores, top_k, dim=-1, sorted=False)
    tw = tw * scaling
    cnts = torch.zeros((ti.shape[0], E), dtype=torch.int64).scatter_(1, ti, 1)
    tpe = cnts.sum(0).tolist()
    idxs = ti.view(-1).argsort()
    sorted_tokens = xb[idxs // top_k]
    outs, start = [], 0
    for e, n in enumerate(tpe):
        if n == 0:
            continue
        g, u, d = layer.expert_f32(e)
        tok = sorted_tokens[start: start + n]
        outs.append(F.linear(F.silu(F.linear(tok, t_bf16(g))) * F.linear(tok, t_bf16(u)), t_bf16(d)))
        start += n
    outs = torch.cat(outs)
    new_x = torch.empty_like(outs)
    new_x[idxs] = outs
    y = (new_x.view(*ti.shape, -1).float().mul_(tw.unsqueeze(-1)).sum(1)).to(torch.bfloat16)
    sg, su, sd = layer.shared_f32()
    shared = F.linear(F.silu(F.linear(xb, t_bf16(sg))) * F.linear(xb, t_bf16(su)), t_bf16(sd))
    return (y + shared).float().numpy(), ti.numpy()


def test_moe_matches_torch_hf_semantics_tiny():
    rng = np.random.default_rng(11)
    layer, _ = pack_tiny(rng, 64, 32, 8, 2, 0.08)
    x_n = orc.rms_norm((0.5 * rng.standard_normal((6, 64))).astype(np.float32))
    want, ti = hf_moe_bf16(layer, x_n, top_k=2, scaling=1.0)
    for t in range(6):
        r = orc.moe(layer, x_n[t], top_k=2)
        assert set(r["ids"].tolist()) == set(ti[t].tolist())
        assert rel_err(r["out"], want[t]) <= 3e-2     # reference test's bf16 tolerance


def test_moe_matches_torch_hf_semantics_full_shape(full_layer):
    _, _, pl = full_layer
    rng = np.random.default_rng(12)
    x_n = orc.rms_norm(rng.standard_normal((2, 2048)).astype(np.float32))
    want, ti = hf_moe_bf16(pl, x_n, top_k=6, scaling=1.0)
    for t in range(2):
        r = orc.moe(pl, x_n[t])
        assert set(r["ids"].tolist()) == set(ti[t].tolist())
        assert rel_err(r["out"], want[t]) <= 1e-2


def test_moe_layer_fp32_reference_arithmetic_agrees(full_layer):
    """The fp32 restatement the CPU baseline times (the reference's own BLAS
    arithmetic) selects the same experts as the exact oracle and agrees with
    it, and with the torch restatement of HF, within bf16 tolerance."""
    _, _, pl = full_layer
    rng = np.random.default_rng(14)
    x = rng.standard_normal((3, 2048)).astype(np.float32)
    want_hf, ti = hf_moe_bf16(pl, orc.rms_norm(x), top_k=6, scaling=1.0)
    for t in range(3):
        r = orc.moe_layer_fp32(pl, x[t])
        e = orc.moe_layer(pl, x[t])
        np.testing.assert_array_equal(r["ids"], e["ids"])
        assert set(r["ids"].tolist()) == set(ti[t].tolist())
        assert rel_err(r["out"], e["out"]) <= 1e-2
        assert rel_err(r["out"], want_hf[t]) <= 1e-2
        assert rel_err(r["x_out"], e["x_out"]) <= 1e-2


def test_batched_moe_layer_equals_the_per_token_oracle(full_layer):
    """tests/oracle_batch.py (the GPU tests' checker over many tokens) gives
    the per-token oracle's ids, weights and layer outputs bit for bit; with
    two slots' weights exchanged (a plausible batching slip) it does not."""
    from oracle_batch import moe_layer_batched
    _, _, pl = full_layer
    rng = np.random.default_rng(15)
    x = orc.bf16_round(rng.standard_normal((12, 2048)).astype(np.float32))
    got = moe_layer_batched(pl, x)
    for t in range(12):
        e = orc.moe_layer(pl, x[t])
        np.testing.assert_array_equal(got["ids"][t], e["ids"])
        np.testing.assert_array_equal(got["weights"][t].view(np.uint32), e["weights"].view(np.uint32))
        np.testing.assert_array_equal(got["x_out"][t].view(np.uint32), e["x_out"].view(np.uint32))
    # planted mistake: slots 0 and 1 take each other's weights
    real = orc.route

    def swapped(*a, **k):
        logits, ids, ws = real(*a, **k)
        return logits, ids, ws[..., [1, 0, 2, 3, 4, 5]]
    try:
        orc.route = swapped
        bad = moe_layer_batched(pl, x)
    finally:
        orc.route = real
    assert not np.array_equal(bad["x_out"].view(np.uint32), got["x_out"].view(np.uint32))


def test_moe_grouped_equals_per_token_and_hf_rule():
    rng = np.random.default_rng(13)
    layer, _ = pack_tiny(rng, 64, 16, 8, 2, 0.08)
    T = 9
    x_n = orc.rms_norm((0.5 * rng.standard_normal((T, 64))).astype(np.float32))
    _, ids, ws = orc.route(layer.router_f32(), x_n, 6)
    g = orc.moe_grouped(layer, x_n, ids, ws)
    assert int(g["tokens_per_expert"].sum()) == 6 * T
    for t in range(T):
        want = orc.moe(layer, x_n[t], 6)["out"]
        assert rel_err(g["out"][t], want) <= 1e-2
    gh = orc.moe_grouped(layer, x_n, ids, ws, combine_rule="hf")
    assert rel_err(gh["out"], g["out"]) <= 1e-2
    # brute force at T = 2: every (token, slot) computed directly
    for t in range(2):
        terms = []
        for k in range(6):
            gg, uu, dd = layer.expert_f32(ids[t, k])
            terms.append(R(ws[t, k] * orc.mlp_unit(gg, uu, dd, x_n[t])))
        sg, su, sd = layer.shared_f32()
        want = orc.combine(terms, orc.mlp_unit(sg, su, sd, x_n[t]))
        assert rel_err(g["out"][t], want) <= 1e-2


def test_combine_invariants():
    rng = np.random.default_rng(14)
    terms = [R(0.01 * rng.standard_normal(2048).astype(np.float32)) for _ in range(6)]
    shared = R(0.05 * rng.standard_normal(2048).astype(np.float32))
    base = orc.combine(terms, shared)
    perm = orc.combine(terms[::-1], shared)
    # permuting the k order moves results by at most one bf16 ulp
    assert np.max(np.abs(base.view(np.int32) - perm.view(np.int32)) >> 16) <= 1
    # a zero-weight expert (term 0) removes it
    np.testing.assert_array_equal(orc.combine([np.zeros(2048, np.float32)] + terms[1:], shared),
                                  orc.combine(terms[1:], shared))


def test_moe_bytes_match_model_analysis():
    b = orc.moe_bytes()
    assert b["expert"] == 17_301_504
    assert b["shared"] == 34_603_008
    assert b["router"] == 262_144
    assert b["selected"] == 138_412_032


def _f32_nearest(q) -> np.float32:
    """The fp32 nearest to the rational q (ties to even), by exact comparison."""
    from fractions import Fraction
    f = np.float32(float(q))
    lo, hi = np.nextafter(f, np.float32(-np.inf)), np.nextafter(f, np.float32(np.inf))
    best = min((lo, f, hi), key=lambda c: (abs(Fraction(float(c)) - q),
                                           int(np.array(c).view(np.uint32)) & 1))
    return np.float32(best)


def test_mv_exact_is_the_correctly_rounded_dot_product():
    """mv_exact against exact rational arithmetic: random bf16 rows, bf16 x
    fp32 rows, and a planted cancellation whose fp32 value depends on the
    summation order; and within a few fp32 ulps of a plain fp32 product (the
    reference's NumPy evaluation)."""
    from fractions import Fraction
    rng = np.random.default_rng(9)
    W = orc.bf16_round(0.02 * rng.standard_normal((6, 2048)).astype(np.float32))
    xb = orc.bf16_round(rng.standard_normal(2048).astype(np.float32))
    xf = rng.standard_normal(2048).astype(np.float32)
    for x in (xb, xf):
        got = orc.mv_exact(W, x)
        for r in range(W.shape[0]):
            q = sum(Fraction(float(a)) * Fraction(float(b)) for a, b in zip(W[r], x))
            assert got[r] == _f32_nearest(q)
        f32 = (W @ x).astype(np.float32)
        mag = np.abs(W).astype(np.float64) @ np.abs(x).astype(np.float64)
        assert np.all(np.abs(f32.astype(np.float64) - got) <= 64 * 2.0 ** -24 * mag)
    # 1 + 2^-24 + 2^-24 - 1: fp32 left to right loses both small terms, the
    # exact value is 2^-23
    w = np.array([[1.0, 2.0 ** -24, 2.0 ** -24, -1.0]], np.float32)
    x = np.ones(4, np.float32)
    assert orc.mv_exact(w, x)[0] == np.float32(2.0 ** -23)
    acc = np.float32(0)
    for a in w[0]:
        acc = np.float32(acc + a)
    assert acc == 0.0
    # uint16 bf16 bits and batched x give the same values
    np.testing.assert_array_equal(orc.mv_exact(orc.bf16_bits(W), xb), orc.mv_exact(W, xb))
    np.testing.assert_array_equal(orc.mv_exact(W, np.stack([xb, xf]))[1], orc.mv_exact(W, xf))
