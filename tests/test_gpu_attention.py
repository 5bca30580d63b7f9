"""GPU parity of the attention half of a decoder layer (fleet_attn_decode),
the embedding (fleet_embed) and lm_head + argmax (fleet_lm_head_argmax)
against the CPU oracle, at the DeepSeek-V2-Lite shape (16 heads, kv_lora 512,
qk_nope 128, qk_rope 64, v_head 128, hidden 2048, vocab 102400).

Each attention call is teacher-forced: the oracle gets the same input x and
the same cache rows. Every dot product on both sides is the exact value
rounded once, so the checks are bit for bit:
* the q / kv_a GEMV;
* everything downstream of it recomputed by the oracle from the GPU's own
  q / kv_a: the appended cache row (kv_a_layernorm, RoPE of k_pe), the
  rotated q_pe and the absorbed query q_c;
* the layer output x_out = bf16(x + o_proj(...)) (also within bf16 tolerance,
  rel 1e-2, as the north star states it).
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from fleet_moe import _lib, ops, rope  # noqa: E402
from fleet_moe.layout import DSV2_LITE  # noqa: E402
from oracle import moe_oracle as orc  # noqa: E402

H, NH, L, DK, DR, DV, V = 2048, 16, 512, 128, 64, 128, 102400
QKV_ROWS = NH * (DK + DR) + L + DR
MAX_POS = 1100
WS_QKV = 256                                   # byte offsets of workspace arrays
WS_QC = WS_QKV + 4 * QKV_ROWS
WS_QPE = WS_QC + 4 * NH * L


def say(msg: str) -> None:
    print(f"[gpu] {msg}", flush=True)


def rel_err(got, want) -> float:
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    return float(np.max(np.abs(got - want)) / max(np.max(np.abs(want)), 1e-30))


def bits(a) -> np.ndarray:
    return orc.bf16_bits(np.asarray(a, np.float32))


def dev16(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).cuda()


def ws_f32(dec: ops.AttnDecoder, off: int, n: int) -> np.ndarray:
    return dec.workspace[off: off + 4 * n].view(torch.float32).cpu().numpy()


@pytest.fixture(scope="module")
def attn_setup():
    rng = np.random.default_rng(11)
    w = orc.AttnLayer(
        norm_in=bits(1 + 0.1 * rng.standard_normal(H, dtype=np.float32)),
        qkv=bits(0.02 * rng.standard_normal((QKV_ROWS, H), dtype=np.float32)),
        kv_a_norm=bits(1 + 0.1 * rng.standard_normal(L, dtype=np.float32)),
        kv_b=bits(0.02 * rng.standard_normal((NH * (DK + DV), L), dtype=np.float32)),
        o_proj=bits(0.02 * rng.standard_normal((H, NH * DV), dtype=np.float32)))
    d = {k: dev16(getattr(w, k)) for k in ("norm_in", "qkv", "kv_a_norm", "kv_b", "o_proj")}
    layer = _lib.FleetAttnLayer(*(d[k].data_ptr() for k in
                                  ("norm_in", "qkv", "kv_a_norm", "kv_b", "o_proj")))
    cos, sin = rope.yarn_tables(MAX_POS)
    # cache rows as a decode would leave them: normalised c, rotated k_pe
    cache = orc.bf16_round(rng.standard_normal((MAX_POS, L + DR), dtype=np.float32))
    return {"w": w, "dev": d, "layer": layer, "cos": cos, "sin": sin,
            "cos_d": torch.from_numpy(cos).cuda(), "sin_d": torch.from_numpy(sin).cuda(),
            "cache": cache, "rng": rng}


def _x(rng) -> np.ndarray:
    # a residual stream after a few layers: bf16 values of rms ~ 0.5
    return orc.bf16_round(0.5 * rng.standard_normal(H, dtype=np.float32))


def test_attention_layer_matches_oracle(attn_setup):
    S = attn_setup
    w, rng, cos, sin = S["w"], S["rng"], S["cos"], S["sin"]
    host_cache = S["cache"].copy()
    cache_d = dev16(bits(host_cache))
    dec = ops.AttnDecoder(DSV2_LITE)
    qkv_w = orc.bf16_to_f32(w.qkv)
    for pos in (0, 1, 63, 64, 65, 200, 1023, MAX_POS - 1):
        say(f"attention pos {pos}")
        x = _x(rng)
        xd = torch.from_numpy(x).cuda()
        yd = torch.empty_like(xd)
        dec.attn_into(S["layer"], xd, yd, cache_d, pos, None, S["cos_d"], S["sin_d"])
        torch.cuda.synchronize()
        assert dec.status() == 0
        g_qkv = ws_f32(dec, WS_QKV, QKV_ROWS)
        g_qc = ws_f32(dec, WS_QC, NH * L).reshape(NH, L)
        g_qpe = ws_f32(dec, WS_QPE, NH * DR).reshape(NH, DR)
        g_row = orc.bf16_to_f32(cache_d[pos].cpu().numpy().view(np.uint16))
        # q / kv_a GEMV
        x_n = orc.rms_norm(x, orc.bf16_to_f32(w.norm_in))
        want_qkv = orc.bf16_round(orc.mv_exact(qkv_w, x_n))
        np.testing.assert_array_equal(g_qkv.view(np.uint32), want_qkv.view(np.uint32),
                                      err_msg="q / kv_a")
        # downstream of the GPU's own q / kv_a: bit for bit
        kv_a = g_qkv[NH * (DK + DR):]
        np.testing.assert_array_equal(
            g_row[:L], orc.rms_norm(kv_a[:L], orc.bf16_to_f32(w.kv_a_norm)), err_msg="c row")
        np.testing.assert_array_equal(
            g_row[L:], orc.bf16_round(orc.apply_rope(kv_a[L:], cos[pos], sin[pos])),
            err_msg="k_pe row")
        q = g_qkv[: NH * (DK + DR)].reshape(NH, DK + DR)
        np.testing.assert_array_equal(
            g_qpe, orc.bf16_round(orc.apply_rope(q[:, DK:], cos[pos], sin[pos])), err_msg="q_pe")
        kv_b = orc.bf16_to_f32(w.kv_b).reshape(NH, DK + DV, L)
        want_qc = np.einsum("hd,hdl->hl", q[:, :DK].astype(np.float64),
                            kv_b[:, :DK].astype(np.float64)).astype(np.float32)
        np.testing.assert_array_equal(g_qc.view(np.uint32), want_qc.view(np.uint32),
                                      err_msg="q_c")
        # the layer output, oracle teacher-forced on the same cache rows
        r = orc.attention(w, x, host_cache, pos, cos, sin)
        host_cache[pos] = g_row                      # keep both caches identical
        want = orc.bf16_round(x + r["out"])
        got = yd.cpu().numpy()
        assert rel_err(got, want) <= 1e-2, f"pos {pos}"
        np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32),
                                      err_msg=f"pos {pos}: layer output")


def test_attention_layer_matches_oracle_past_one_batch(attn_setup):
    """Positions whose chunks need more than one batch of S3 rows: a chunk is
    ceil((pos + 1) / 16) positions, a batch 8 waves x 9 rows = 72, so from
    position 1152 on the S3 loop reloads cache rows inside the loop. Up to the
    last position a 4096-row cache allows. The layer output is bit-exact."""
    S = attn_setup
    w, rng = S["w"], S["rng"]
    max_pos = 4096
    cos, sin = rope.yarn_tables(max_pos)
    cos_d, sin_d = torch.from_numpy(cos).cuda(), torch.from_numpy(sin).cuda()
    host_cache = orc.bf16_round(rng.standard_normal((max_pos, L + DR), dtype=np.float32))
    cache_d = dev16(bits(host_cache))
    dec = ops.AttnDecoder(DSV2_LITE)
    for pos in (1151, 1152, 1153, 1300, 2047, 3000, max_pos - 1):
        batches = -(-(-(-(pos + 1) // 16)) // 72)
        say(f"attention pos {pos} ({batches} S3 batches)")
        x = _x(rng)
        xd = torch.from_numpy(x).cuda()
        yd = torch.empty_like(xd)
        dec.attn_into(S["layer"], xd, yd, cache_d, pos, None, cos_d, sin_d)
        torch.cuda.synchronize()
        assert dec.status() == 0
        g_row = orc.bf16_to_f32(cache_d[pos].cpu().numpy().view(np.uint16))
        r = orc.attention(w, x, host_cache, pos, cos, sin)
        np.testing.assert_array_equal(g_row.view(np.uint32), r["row"].view(np.uint32),
                                      err_msg=f"pos {pos}: cache row")
        host_cache[pos] = g_row
        want = orc.bf16_round(x + r["out"])
        got = yd.cpu().numpy()
        np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32),
                                      err_msg=f"pos {pos}: layer output")


def test_attention_layer_matches_oracle_at_64_positions(attn_setup):
    """64 positions over a 4096-row cache, in a seeded random order (8 of them
    at the chunking's edges: the first positions, where chunks hold one row and
    some hold none, a last chunk of one row, one and several S3 batches): cache
    row and layer output bit-exact at each, every call seeing the rows the
    calls before it wrote."""
    S = attn_setup
    w = S["w"]
    rng = np.random.default_rng(23)
    max_pos = 4096
    cos, sin = rope.yarn_tables(max_pos)
    cos_d, sin_d = torch.from_numpy(cos).cuda(), torch.from_numpy(sin).cuda()
    host_cache = orc.bf16_round(rng.standard_normal((max_pos, L + DR), dtype=np.float32))
    cache_d = dev16(bits(host_cache))
    dec = ops.AttnDecoder(DSV2_LITE)
    edges = [0, 14, 15, 16, 255, 1151, 2048, max_pos - 1]
    rest = rng.choice(np.setdiff1d(np.arange(max_pos), edges), 56, replace=False)
    order = rng.permutation(np.concatenate([edges, rest]))
    for i, pos in enumerate(order.tolist()):
        if i % 16 == 0:
            say(f"attention, positions {i}..{i + 15} of 64")
        x = _x(rng)
        xd = torch.from_numpy(x).cuda()
        yd = torch.empty_like(xd)
        dec.attn_into(S["layer"], xd, yd, cache_d, pos, None, cos_d, sin_d)
        torch.cuda.synchronize()
        g_row = orc.bf16_to_f32(cache_d[pos].cpu().numpy().view(np.uint16))
        r = orc.attention(w, x, host_cache, pos, cos, sin)
        np.testing.assert_array_equal(g_row.view(np.uint32), r["row"].view(np.uint32),
                                      err_msg=f"pos {pos}: cache row")
        host_cache[pos] = g_row
        want = orc.bf16_round(x + r["out"])
        np.testing.assert_array_equal(yd.cpu().numpy().view(np.uint32), want.view(np.uint32),
                                      err_msg=f"pos {pos}: layer output")
    assert dec.status() == 0


def test_attention_in_place_and_device_position_and_graph(attn_setup):
    """x_out may alias x; a device position gives the same bits as the host
    position; a captured graph replays at the positions the device holds."""
    S = attn_setup
    rng = S["rng"]
    cache0 = dev16(bits(S["cache"]))
    dec = ops.AttnDecoder(DSV2_LITE)
    x = torch.from_numpy(_x(rng)).cuda()
    positions = (5, 64, 700)
    want = []
    for p in positions:
        c = cache0.clone()
        y = torch.empty_like(x)
        dec.attn_into(S["layer"], x, y, c, p, None, S["cos_d"], S["sin_d"])
        want.append((y.clone(), c[p].clone()))
    torch.cuda.synchronize()
    say("device position, in place")
    pos_d = torch.zeros(1, dtype=torch.int32, device="cuda")
    for p, (wy, wrow) in zip(positions, want):
        c = cache0.clone()
        y = x.clone()
        pos_d.fill_(p)
        dec.attn_into(S["layer"], y, y, c, 0, pos_d, S["cos_d"], S["sin_d"])
        torch.cuda.synchronize()
        assert torch.equal(y, wy) and torch.equal(c[p], wrow), f"pos {p}"
    say("graph replay")
    c = cache0.clone()
    y = torch.empty_like(x)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            dec.attn_into(S["layer"], x, y, c, 0, pos_d, S["cos_d"], S["sin_d"], stream=s)
    torch.cuda.current_stream().wait_stream(s)
    for rep in range(2):
        for p, (wy, wrow) in zip(positions, want):
            c.copy_(cache0)
            pos_d.fill_(p)
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(y, wy) and torch.equal(c[p], wrow), f"replay {rep} pos {p}"
    assert dec.status() == 0


def test_attention_tags_cannot_alias_after_65536_calls(attn_setup):
    """Published words carry the low 16 bits of the call count. A call at a
    short position leaves chunks without positions; those chunks must still
    publish (neutral partials), or a later call whose 16-bit tag equals the
    one their stale words carry could merge them. The workspace's call count
    is set from the host to stand in for 65,535 intervening calls, so call C
    has call A's tag; A and C attend with different inputs (so A's partials
    differ from C's), and C must still equal the oracle bit for bit."""
    S = attn_setup
    w, rng, cos, sin = S["w"], S["rng"], S["cos"], S["sin"]
    host_cache = S["cache"].copy()
    cache_d = dev16(bits(host_cache))
    dec = ops.AttnDecoder(DSV2_LITE)
    pos_long, pos_short = 1055, 3

    def call(x, pos):
        xd = torch.from_numpy(x).cuda()
        yd = torch.empty_like(xd)
        dec.attn_into(S["layer"], xd, yd, cache_d, pos, None, S["cos_d"], S["sin_d"])
        torch.cuda.synchronize()
        assert dec.status() == 0
        host_cache[pos] = orc.bf16_to_f32(cache_d[pos].cpu().numpy().view(np.uint16))
        return yd.cpu().numpy()

    say("tag wrap: call A at 1055, call B at 3")
    call(_x(rng), pos_long)                     # call 1: every chunk's words get tag 1
    call(_x(rng), pos_short)                    # call 2: chunks 4..15 hold no positions
    head = np.array([65536, (65536 * 256) & 0xFFFFFFFF], np.uint32)   # call count, exits
    dec.workspace[:8].copy_(torch.from_numpy(head.view(np.uint8)).cuda())
    say("tag wrap: call C at 1055 with call A's tag")
    x = _x(rng)
    want_cache = host_cache.copy()
    got = call(x, pos_long)                     # call 65537: tag 1 again
    r = orc.attention(w, x, want_cache, pos_long, cos, sin)
    want = orc.bf16_round(x + r["out"])
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32),
                                  err_msg="call with a wrapped tag")
    assert dec.workspace[:4].view(torch.int32).item() == 65537


def test_attention_position_checks(attn_setup):
    S = attn_setup
    dec = ops.AttnDecoder(DSV2_LITE)
    x = torch.zeros(H, dtype=torch.float32, device="cuda")
    c = torch.zeros((64, L + DR), dtype=torch.int16, device="cuda")
    with pytest.raises(_lib.FleetMoeError):
        dec.attn_into(S["layer"], x, x, c, 64, None, S["cos_d"], S["sin_d"])
    pos_d = torch.tensor([64], dtype=torch.int32, device="cuda")
    dec.attn_into(S["layer"], x, x, c, 0, pos_d, S["cos_d"], S["sin_d"])
    assert dec.status() & _lib.ABORT_POSITION
    assert int(torch.count_nonzero(c)) == 0             # nothing written


def test_embed_and_token_check():
    rng = np.random.default_rng(5)
    E = bits(0.02 * rng.standard_normal((V, H), dtype=np.float32))
    Ed = dev16(E)
    dec = ops.AttnDecoder(DSV2_LITE)
    x = torch.empty(H, dtype=torch.float32, device="cuda")
    for t in (0, 1, 4097, V - 1):
        dec.embed_into(Ed.data_ptr(), torch.tensor([t], dtype=torch.int32, device="cuda"), x)
        np.testing.assert_array_equal(x.cpu().numpy(), orc.bf16_to_f32(E[t]))
    assert dec.status() == 0
    dec.embed_into(Ed.data_ptr(), torch.tensor([V], dtype=torch.int32, device="cuda"), x)
    assert dec.status() & _lib.ABORT_TOKEN
    assert int(torch.count_nonzero(x)) == 0


def test_lm_head_argmax_matches_oracle():
    rng = np.random.default_rng(6)
    W = bits(0.02 * rng.standard_normal((V, H), dtype=np.float32))
    fn = bits(1 + 0.1 * rng.standard_normal(H, dtype=np.float32))
    Wd, fnd = dev16(W), dev16(fn)
    Wf = orc.bf16_to_f32(W)
    dec = ops.AttnDecoder(DSV2_LITE)
    logits = torch.empty(V, dtype=torch.float32, device="cuda")
    tok = torch.full((1,), -1, dtype=torch.int32, device="cuda")
    nxt = torch.full((1,), -1, dtype=torch.int32, device="cuda")
    pos = torch.tensor([7], dtype=torch.int32, device="cuda")
    for trial in range(3):
        x = orc.bf16_round(rng.standard_normal(H, dtype=np.float32))
        say(f"lm_head trial {trial}")
        dec.lm_head_into(torch.from_numpy(x).cuda(), fnd.data_ptr(), Wd.data_ptr(), logits,
                         tok, nxt, pos)
        torch.cuda.synchronize()
        r = orc.lm_head_argmax(x, fn, Wf)
        g = logits.cpu().numpy()
        np.testing.assert_array_equal(g.view(np.uint32), r["logits"].view(np.uint32))
        t = int(tok.item())
        assert t == int(nxt.item()) == int(np.flatnonzero(g == g.max())[0]) == r["token"]
    assert int(pos.item()) == 10
    # a planted tie: a copy of the best row at a lower index wins
    best = int(tok.item())
    lower = best // 2
    W2 = Wd.clone()
    W2[lower] = Wd[best]
    dec.lm_head_into(torch.from_numpy(x).cuda(), fnd.data_ptr(), W2.data_ptr(), None, tok)
    torch.cuda.synchronize()
    assert int(tok.item()) == lower
    assert dec.status() == 0


def test_rope_bit_exact_over_many_positions(attn_setup):
    """q_pe and the cached k_pe equal the oracle's three-rounding RoPE
    (products and sum each rounded to fp32, then bf16) at 400 positions x 16
    heads: a fused multiply-add in the kernel would move about one element in
    2^16 (an expected 6 of these 435,200) to the neighbouring bf16 value."""
    S = attn_setup
    rng, cos, sin = S["rng"], S["cos"], S["sin"]
    cache_d = dev16(bits(S["cache"]))
    dec = ops.AttnDecoder(DSV2_LITE)
    x = torch.empty(H, dtype=torch.float32, device="cuda")
    y = torch.empty_like(x)
    bad = 0
    for pos in range(0, MAX_POS, MAX_POS // 400 + 1):
        x.copy_(torch.from_numpy(_x(rng)))
        dec.attn_into(S["layer"], x, y, cache_d, pos, None, S["cos_d"], S["sin_d"])
        g_qkv = ws_f32(dec, WS_QKV, QKV_ROWS)
        g_qpe = ws_f32(dec, WS_QPE, NH * DR).reshape(NH, DR)
        g_kpe = orc.bf16_to_f32(cache_d[pos, L:].cpu().numpy().view(np.uint16))
        q = g_qkv[: NH * (DK + DR)].reshape(NH, DK + DR)
        bad += int(np.sum(g_qpe != orc.bf16_round(orc.apply_rope(q[:, DK:], cos[pos], sin[pos]))))
        kv_pe = g_qkv[NH * (DK + DR) + L:]
        bad += int(np.sum(g_kpe != orc.bf16_round(orc.apply_rope(kv_pe, cos[pos], sin[pos]))))
    assert bad == 0
