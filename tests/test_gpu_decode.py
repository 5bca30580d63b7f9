"""GPU parity of the batch-1 path through the C ABI: router + top-k, and the
full MoE layer decode, against the CPU oracle on the same seeded inputs.

Bar: routed expert ids bit-exact (ties to the lowest
index); layer outputs within bf16 tolerance, max|got - want| / max|want|
<= 1e-2 (fp32 accumulation). The router logits are expected bit-exact too
(both sides round an fp64 sum of exact bf16 x bf16 products once)."""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from fleet_moe import ops, synth  # noqa: E402
from fleet_moe.layout import DSV2_LITE  # noqa: E402
from oracle import moe_oracle as orc  # noqa: E402

REL_TOL = 1e-2


def say(msg: str) -> None:
    print(f"[gpu] {msg}", flush=True)


def rel_err(got, want) -> float:
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    return float(np.max(np.abs(got - want)) / max(np.max(np.abs(want)), 1e-30))


@pytest.fixture(scope="module")
def dev(full_layer):
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    blob, lay, pl = full_layer
    say("upload layer (1.14 GB)")
    layer = ops.DeviceLayer.from_host(blob, lay, 1, DSV2_LITE, device="cuda")
    torch.cuda.synchronize()
    return layer, pl


def test_router_topk_bit_exact(dev):
    layer, pl = dev
    x = synth.hidden_inputs(1, 256)
    xn = orc.rms_norm(x)
    say("router_topk T=256")
    logits, ids, ws = ops.route(layer, torch.from_numpy(xn).cuda())
    torch.cuda.synchronize()
    want_l, want_ids, want_w = orc.route(pl.router_f32(), xn)
    np.testing.assert_array_equal(logits.cpu().numpy().view(np.uint32), want_l.view(np.uint32))
    np.testing.assert_array_equal(ids.cpu().numpy(), want_ids)
    np.testing.assert_array_equal(ws.cpu().numpy().view(np.uint32), want_w.view(np.uint32))


def test_router_ties_and_bias(dev):
    layer, pl = dev
    # zero input -> all logits 0 -> all p equal -> ids 0..5, weights 1/64
    say("router_topk zero input")
    _, ids, ws = ops.route(layer, torch.zeros((3, 2048), dtype=torch.float32, device="cuda"))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(ids.cpu().numpy(), np.tile(np.arange(6), (3, 1)))
    np.testing.assert_allclose(ws.cpu().numpy(), 1 / 64, rtol=1e-6)
    # Zipf-biased routing (grouped benchmark prior)
    bias = synth.zipf_logit_bias(0)
    xn = orc.rms_norm(synth.hidden_inputs(2, 64))
    say("router_topk zipf bias T=64")
    logits, ids, ws = ops.route(layer, torch.from_numpy(xn).cuda(), torch.from_numpy(bias).cuda())
    torch.cuda.synchronize()
    want_l, want_ids, want_w = orc.route(pl.router_f32(), xn, logit_bias=bias)
    np.testing.assert_array_equal(ids.cpu().numpy(), want_ids)
    np.testing.assert_array_equal(ws.cpu().numpy().view(np.uint32), want_w.view(np.uint32))


def test_decode_matches_oracle(dev):
    layer, pl = dev
    dec = ops.LayerDecoder(DSV2_LITE)
    x = synth.hidden_inputs(0, 24)
    pl.widen()
    exact = []
    for t in range(x.shape[0]):
        say(f"decode token {t}")
        r = dec.decode(layer, torch.from_numpy(x[t]).cuda())
        torch.cuda.synchronize()
        want = orc.moe_layer(pl, x[t])
        np.testing.assert_array_equal(r["ids"].cpu().numpy(), want["ids"], err_msg=f"token {t}")
        np.testing.assert_array_equal(r["weights"].cpu().numpy().view(np.uint32),
                                      want["weights"].view(np.uint32), err_msg=f"token {t}")
        got = r["x_out"].cpu().numpy()
        assert rel_err(got, want["x_out"]) <= REL_TOL, f"token {t}"
        moe = ops.bf16_bits_to_f32(r["moe_out"]).cpu().numpy()
        assert rel_err(moe, want["out"]) <= REL_TOL, f"token {t}"
        exact.append(np.mean(got == want["x_out"]))
    assert dec.status() == 0
    # only fp32 accumulation order differs: nearly every element is identical
    assert float(np.mean(exact)) > 0.98, f"bit-exact fraction {np.mean(exact):.4f}"


def test_decode_routing_1000_tokens_covers_all_experts(dev):
    """Config 1: 1,000 seeded bf16 N(0,1) tokens one at a time; every routed id
    bit-exact; over the 1,000 tokens all 64 experts are selected."""
    layer, pl = dev
    dec = ops.LayerDecoder(DSV2_LITE)
    x = orc.bf16_round(synth.hidden_inputs(0, 1000))
    xd = torch.from_numpy(x).cuda()
    outs = torch.empty((1000, 2048), dtype=torch.float32, device="cuda")
    ids = torch.empty((1000, 6), dtype=torch.int32, device="cuda")
    ws = torch.empty((1000, 6), dtype=torch.float32, device="cuda")
    say("decode 1000 tokens")
    for t in range(1000):
        dec.decode_into(layer, xd[t], outs[t], None, ids[t], ws[t])
    torch.cuda.synchronize()
    assert dec.status() == 0
    want_ids = orc.route(pl.router_f32(), orc.rms_norm(x))[1]
    got_ids = ids.cpu().numpy()
    np.testing.assert_array_equal(got_ids, want_ids)
    assert len(np.unique(got_ids)) == 64
    # spot-check outputs of a few tokens against the oracle
    pl.widen()
    o = outs.cpu().numpy()
    for t in (0, 499, 999):
        assert rel_err(o[t], orc.moe_layer(pl, x[t])["x_out"]) <= REL_TOL


def test_decode_in_place_repeatable_and_zero_input(dev):
    layer, pl = dev
    dec = ops.LayerDecoder(DSV2_LITE)
    x = torch.from_numpy(synth.hidden_inputs(3, 1)[0]).cuda()
    say("decode determinism")
    a = dec.decode(layer, x)
    b = dec.decode(layer, x)
    torch.cuda.synchronize()
    assert torch.equal(a["x_out"], b["x_out"]) and torch.equal(a["moe_out"], b["moe_out"])
    # in place: x_out aliases x
    say("decode in place")
    y = x.clone()
    dec.decode_into(layer, y, y)
    torch.cuda.synchronize()
    assert torch.equal(y, a["x_out"])
    # zero input: norm 0, logits 0 -> ids 0..5, all expert outputs 0
    say("decode zero input")
    z = dec.decode(layer, torch.zeros(2048, dtype=torch.float32, device="cuda"))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(z["ids"].cpu().numpy(), np.arange(6))
    assert not torch.any(z["x_out"] != 0)
    assert dec.status() == 0
