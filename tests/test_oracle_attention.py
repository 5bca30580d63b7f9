"""Pins for the oracle's attention half, embedding-free lm_head and RoPE
(config 4), each against an independent formulation rather than the same
formula retyped:

* RoPE: DeepseekV2's reorder + rotate_half equals a complex rotation of the
  adjacent pairs (x[2i], x[2i+1]) by angle t * inv_freq[i], written to slots
  i and i + 32;
* YaRN tables: with factor 1 they are plain RoPE (theta^(-2i/d)); at factor
  40 the blend keeps the high frequencies, divides the low ones by 40, and the
  magnitude factor is 1 (mscale == mscale_all_dim);
* absorbed MLA: equals materialised per-head K = [W_UK c ; k_pe],
  V = W_UV c attention in fp64 (the algebraic identity of
  reference_decode.py:19-25);
* lm_head: bf16 logits, argmax with the lowest index on ties."""
from __future__ import annotations

import math

import numpy as np
import pytest

from oracle import moe_oracle as orc


def test_rope_is_a_complex_rotation_of_adjacent_pairs():
    rng = np.random.default_rng(0)
    cos, sin = orc.rope_tables(64, scale=1.0)       # plain RoPE
    x = rng.standard_normal((5, 64)).astype(np.float32)
    for pos in (0, 1, 7, 63):
        got = orc.apply_rope(x, cos[pos], sin[pos])
        inv = 1e4 ** (-np.arange(0, 64, 2) / 64.0)
        z = (x[:, 0::2] + 1j * x[:, 1::2]) * np.exp(1j * pos * inv)
        want = np.concatenate([z.real, z.imag], axis=-1)
        np.testing.assert_allclose(got, want, rtol=2e-5, atol=2e-5)
    # position 0 is a pure reorder
    np.testing.assert_array_equal(orc.apply_rope(x, cos[0], sin[0]),
                                  np.concatenate([x[:, 0::2], x[:, 1::2]], -1))


def test_yarn_tables_limits_and_magnitude():
    c1, s1 = orc.rope_tables(32, scale=1.0)
    inv = (1.0 / (1e4 ** (np.arange(0, 64, 2, dtype=np.float32) / 64))).astype(np.float32)
    ang = np.outer(np.arange(32, dtype=np.float32), inv)
    np.testing.assert_allclose(c1[:, :32], np.cos(ang), rtol=1e-6, atol=1e-6)
    np.testing.assert_array_equal(c1[:, :32], c1[:, 32:])
    c, s = orc.rope_tables(4096)
    # mscale(40, 0.707) / mscale(40, 0.707) = 1: unit-magnitude rotations
    np.testing.assert_allclose(c ** 2 + s ** 2, 1.0, atol=2e-6)
    # the effective frequency of each pair, read back from position 1
    f = np.arctan2(s[1, :32], c[1, :32])
    assert abs(f[0] - 1.0) < 1e-6                       # fastest pair: extrapolated, 1 rad/pos
    np.testing.assert_allclose(f[-1], inv[-1] / 40.0, rtol=1e-4)   # slowest: interpolated
    assert np.all(np.diff(f) < 0)
    # softmax scale: 192^-0.5 * (0.1 * 0.707 * ln 40 + 1)^2
    m = 0.1 * 0.707 * math.log(40) + 1
    assert orc.softmax_scale() == pytest.approx(192 ** -0.5 * m * m, rel=1e-12)


def _random_attn(rng, heads=2, hidden=256):
    L, Dk, Dr, Dv = orc.KV_LORA, orc.QK_NOPE, orc.QK_ROPE, orc.V_HEAD
    rows = heads * (Dk + Dr) + L + Dr
    bits = lambda a: orc.bf16_bits(a.astype(np.float32))
    return orc.AttnLayer(
        norm_in=bits(1 + 0.1 * rng.standard_normal(hidden)),
        qkv=bits(0.05 * rng.standard_normal((rows, hidden))),
        kv_a_norm=bits(1 + 0.1 * rng.standard_normal(L)),
        kv_b=bits(0.05 * rng.standard_normal((heads * (Dk + Dv), L))),
        o_proj=bits(0.05 * rng.standard_normal((hidden, heads * Dv))),
        heads=heads)


def test_absorbed_attention_equals_materialised_kv():
    rng = np.random.default_rng(1)
    heads, hidden = 2, 256
    w = _random_attn(rng, heads, hidden)
    cos, sin = orc.rope_tables(16)
    cache = np.zeros((16, orc.KV_LORA + orc.QK_ROPE), np.float32)
    cache[:9] = orc.bf16_round(rng.standard_normal((9, cache.shape[1])).astype(np.float32))
    x = orc.bf16_round(rng.standard_normal(hidden).astype(np.float32))
    pos = 9
    r = orc.attention(w, x, cache, pos, cos, sin)
    # materialised K, V per head in fp64 from the same cache rows and query
    L, Dk, Dr, Dv = orc.KV_LORA, orc.QK_NOPE, orc.QK_ROPE, orc.V_HEAD
    x_n = orc.rms_norm(x, orc.bf16_to_f32(w.norm_in))
    qkv = orc.bf16_round(orc.bf16_to_f32(w.qkv).reshape(-1, hidden) @ x_n)
    q = qkv[: heads * (Dk + Dr)].reshape(heads, Dk + Dr).astype(np.float64)
    q_pe = orc.bf16_round(orc.apply_rope(q[:, Dk:].astype(np.float32), cos[pos], sin[pos]))
    C = cache[: pos + 1, :L].astype(np.float64)
    KP = cache[: pos + 1, L:].astype(np.float64)
    kv_b = orc.bf16_to_f32(w.kv_b).reshape(heads * (Dk + Dv), L).astype(np.float64)
    outs = []
    for h in range(heads):
        wk = kv_b[h * (Dk + Dv): h * (Dk + Dv) + Dk]
        wv = kv_b[h * (Dk + Dv) + Dk: (h + 1) * (Dk + Dv)]
        K = np.concatenate([C @ wk.T, KP], axis=1)          # [S, Dk + Dr]
        V = C @ wv.T                                         # [S, Dv]
        qh = np.concatenate([q[h, :Dk], q_pe[h]])
        s = K @ qh * orc.softmax_scale()
        np.testing.assert_allclose(r["scores"][h], s, rtol=1e-4, atol=1e-4)
        p = np.exp(s - s.max())
        outs.append((p / p.sum()) @ V)
    o = orc.bf16_round(orc.bf16_to_f32(w.o_proj).reshape(hidden, -1)
                       @ orc.bf16_round(np.concatenate(outs).astype(np.float32)))
    assert np.max(np.abs(r["out"] - o)) <= 1e-2 * np.max(np.abs(o))
    # the appended cache row: c = rms_norm(kv_a[:512]), k_pe = RoPE(kv_a[512:])
    np.testing.assert_array_equal(r["row"][:L], orc.rms_norm(qkv[heads * (Dk + Dr):][:L],
                                                             orc.bf16_to_f32(w.kv_a_norm)))
    np.testing.assert_array_equal(cache[pos], r["row"])


def test_lm_head_argmax_lowest_index_and_bf16_logits():
    rng = np.random.default_rng(2)
    W = orc.bf16_round(rng.standard_normal((50, 8)).astype(np.float32))
    x = orc.bf16_round(rng.standard_normal(8).astype(np.float32))
    r = orc.lm_head_argmax(x, None, W)
    xn = orc.rms_norm(x)
    np.testing.assert_array_equal(r["logits"], orc.bf16_round(W @ xn))
    assert r["token"] == int(np.argmax(r["logits"]))       # numpy: first maximum
    W2 = np.vstack([W, W[[r["token"]]]])                    # duplicate the best row at the end
    r2 = orc.lm_head_argmax(x, None, W2)
    assert r2["token"] == r["token"] and r2["margin"] == 0.0


def _zero_like(w: orc.AttnLayer) -> orc.AttnLayer:
    return orc.AttnLayer(norm_in=w.norm_in, qkv=w.qkv, kv_a_norm=w.kv_a_norm, kv_b=w.kv_b,
                         o_proj=np.zeros_like(w.o_proj), heads=w.heads)


def test_decoder_layer_composition_special_cases():
    """o_proj = 0 makes the attention half the identity, so the layer is the
    FFN half alone; a zero FFN makes the layer the attention half alone."""
    rng = np.random.default_rng(3)
    heads, hidden, inter = 2, 256, 64
    w = _random_attn(rng, heads, hidden)
    cos, sin = orc.rope_tables(8)
    x = orc.bf16_round(rng.standard_normal(hidden).astype(np.float32))
    g = orc.bf16_round(0.05 * rng.standard_normal((inter, hidden)).astype(np.float32))
    u = orc.bf16_round(0.05 * rng.standard_normal((inter, hidden)).astype(np.float32))
    d = orc.bf16_round(0.05 * rng.standard_normal((hidden, inter)).astype(np.float32))
    ffn = orc.DenseFfn(g, u, d)
    cache = np.zeros((8, orc.KV_LORA + orc.QK_ROPE), np.float32)
    r = orc.decoder_layer(_zero_like(w), ffn, x, cache, 0, cos, sin)
    np.testing.assert_array_equal(r["x_attn"], x)
    np.testing.assert_array_equal(r["x_out"], orc.dense_layer(g, u, d, x)["x_out"])
    zero = orc.DenseFfn(np.zeros_like(g), np.zeros_like(u), np.zeros_like(d))
    cache2 = np.zeros_like(cache)
    r2 = orc.decoder_layer(w, zero, x, cache2, 0, cos, sin)
    a = orc.attention(w, x, np.zeros_like(cache), 0, cos, sin)["out"]
    np.testing.assert_array_equal(r2["x_out"], orc.bf16_round(x + a))
    np.testing.assert_array_equal(r2["x_attn"], r2["x_out"])


def test_decode_step_reads_the_token_row_and_picks_it_back():
    """With one-hot embedding rows, lm_head = embed and a layer that adds
    nothing, the step maps every token to itself: the embedding is indexed by
    row and the logits are lm_head rows."""
    rng = np.random.default_rng(4)
    heads, hidden, vocab, inter = 2, 256, 40, 32
    w = _zero_like(_random_attn(rng, heads, hidden))
    zero = orc.DenseFfn(np.zeros((inter, hidden), np.float32),
                        np.zeros((inter, hidden), np.float32),
                        np.zeros((hidden, inter), np.float32))
    E = np.zeros((vocab, hidden), np.float32)
    E[np.arange(vocab), rng.permutation(hidden)[:vocab]] = 1.0
    model = orc.DecodeModel(embed=orc.bf16_bits(E), final_norm=None, lm_head=orc.bf16_bits(E),
                            attn=[w], ffn=[zero])
    cos, sin = orc.rope_tables(4)
    for tok in (0, 7, vocab - 1):
        caches = [np.zeros((4, orc.KV_LORA + orc.QK_ROPE), np.float32)]
        r = orc.decode_step(model, tok, 0, caches, cos, sin)
        assert r["token"] == tok and r["margin"] == pytest.approx(hidden ** 0.5, rel=1e-2)
