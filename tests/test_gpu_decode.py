"""GPU parity of the batch-1 path through the C ABI: router + top-k, and the
full MoE layer decode, against the CPU oracle on the same seeded inputs.

Bar: routed expert ids bit-exact (ties to the lowest
index); layer outputs within bf16 tolerance, max|got - want| / max|want|
<= 1e-2. Both sides evaluate every dot product as its exact value rounded
once (the oracle in fp64; the kernels in fp32 where an error bound proves the
bf16 rounding, in fp64 otherwise), so the router logits, routing weights and
layer outputs are checked bit for bit as well."""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from fleet_moe import ops, synth  # noqa: E402
from fleet_moe.layout import DSV2_LITE  # noqa: E402
from oracle import moe_oracle as orc  # noqa: E402
from oracle_batch import moe_layer_batched  # noqa: E402

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
        np.testing.assert_array_equal(moe.view(np.uint32), want["out"].view(np.uint32),
                                      err_msg=f"token {t}: MoE output bits")
        np.testing.assert_array_equal(got.view(np.uint32), want["x_out"].view(np.uint32),
                                      err_msg=f"token {t}: layer output bits")
    assert dec.status() == 0
    say(f"bit-exact fraction {np.mean(exact):.6f}")


def test_decode_routing_1000_tokens_covers_all_experts(dev):
    """Config 1: 1,000 seeded bf16 N(0,1) tokens one at a time; every routed
    id, routing weight and layer output bit-exact; over the 1,000 tokens all
    64 experts are selected."""
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
    # every token's layer output and routing weights, bit for bit (about 7
    # million certified GEMV results, of which the fp64 fallback takes a few
    # percent): the oracle over the batch
    pl.widen()
    say("oracle over the 1000 tokens (batched)")
    want = moe_layer_batched(pl, x)
    np.testing.assert_array_equal(want["ids"], want_ids)
    np.testing.assert_array_equal(ws.cpu().numpy().view(np.uint32), want["weights"].view(np.uint32))
    o = outs.cpu().numpy()
    assert rel_err(o, want["x_out"]) <= REL_TOL
    bad = np.argwhere(o.view(np.uint32) != want["x_out"].view(np.uint32))
    assert bad.size == 0, (f"{len(bad)} elements differ, first (token, row) {bad[:4].tolist()}: "
                           f"got {o[tuple(bad[0])]} want {want['x_out'][tuple(bad[0])]}")


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


class _RouterSwap:
    """A DeviceLayer with its router pointer replaced (duck-typed for
    LayerDecoder.decode_into, which only asks for c_layer())."""

    def __init__(self, base, router_dev):
        self.base, self.router_dev = base, router_dev

    def c_layer(self):
        cl = self.base.c_layer()
        cl.router = self.router_dev.data_ptr()
        return cl


def test_decode_exact_tie_takes_the_exact_routing_path(dev):
    """Copy the router row of the 6th-ranked expert over the 7th-ranked one:
    the two logits are then exactly equal, the kernel's local selection cannot
    separate them (gap 0 < the error bound), so it must fall back to the
    exact logits and break the tie to the lower index, as the oracle does."""
    import dataclasses
    layer, pl = dev
    pl.widen()
    dec = ops.LayerDecoder(DSV2_LITE)
    cases = 0
    for seed in (50, 51, 52):
        x = synth.hidden_inputs(seed, 1)[0]
        want0 = orc.moe_layer(pl, x)
        order = np.lexsort((np.arange(64), -want0["logits"].astype(np.float64)))
        e6, e7 = int(order[5]), int(order[6])
        router = pl.router.reshape(64, -1).copy()
        router[e7] = router[e6]
        pl2 = dataclasses.replace(pl, router=router.reshape(pl.router.shape))
        want = orc.moe_layer(pl2, x)
        lo = want["logits"]
        assert lo[e6] == lo[e7]
        assert min(e6, e7) in want["ids"] and max(e6, e7) not in want["ids"]
        rdev = torch.from_numpy(router.view(np.int16).reshape(-1)).cuda()
        say(f"decode exact tie seed={seed} experts {e6}/{e7}")
        got = dec.decode(_RouterSwap(layer, rdev), torch.from_numpy(x).cuda())
        torch.cuda.synchronize()
        np.testing.assert_array_equal(got["ids"].cpu().numpy(), want["ids"])
        np.testing.assert_array_equal(got["weights"].cpu().numpy().view(np.uint32),
                                      want["weights"].view(np.uint32))
        got_x = got["x_out"].cpu().numpy()
        assert rel_err(got_x, want["x_out"]) <= REL_TOL
        np.testing.assert_array_equal(got_x.view(np.uint32), want["x_out"].view(np.uint32),
                                      err_msg=f"tie seed {seed}: layer output bits")
        cases += 1
    assert cases == 3 and dec.status() == 0


def test_decode_graph_replay_matches_eager(dev):
    """Four decode launches captured in one HIP graph and replayed three times,
    with eager launches on the same workspace in between: every replay equals
    the eager result bit for bit (the workspace is never memset; the call
    epoch lives in it)."""
    layer, _ = dev
    dec = ops.LayerDecoder(DSV2_LITE)
    n = 4
    x = torch.from_numpy(orc.bf16_round(synth.hidden_inputs(60, n))).cuda()
    ref = torch.empty_like(x)
    ref_ids = torch.empty((n, 6), dtype=torch.int32, device="cuda")
    for t in range(n):
        dec.decode_into(layer, x[t], ref[t], ids=ref_ids[t])
    out = torch.empty_like(x)
    ids = torch.empty_like(ref_ids)
    say("graph capture of 4 decode launches")
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            for t in range(n):
                dec.decode_into(layer, x[t], out[t], ids=ids[t])
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    extra = torch.from_numpy(synth.hidden_inputs(61, 1)[0]).cuda()
    for rep in range(3):
        out.fill_(float("nan"))
        ids.fill_(-1)
        torch.cuda.synchronize()
        say(f"graph replay {rep}")
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref) and torch.equal(ids, ref_ids), f"replay {rep}"
        dec.decode(layer, extra)          # eager work on the same workspace between replays
        torch.cuda.synchronize()
    assert dec.status() == 0
