"""GPU parity of the multi-token grouped-expert step through the C ABI.

Config 2: T in {4, 16, 64} tokens (bf16 N(0,1) hidden, normed), routing
biased by the seeded Zipf(1.1) prior; outputs within bf16 tolerance
(rel 1e-2) of the oracle's moe_grouped (moe_infer data movement, per-token
combine of reference_decode.moe), and grouped(T) equal to T batch-1 outputs.
The multi-token semantics have no reference test with T > 1, so they are
pinned by that invariant (see tests/test_oracle.py)."""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from fleet_moe import ops, synth  # noqa: E402
from fleet_moe.layout import DSV2_LITE  # noqa: E402
from oracle import moe_oracle as orc  # noqa: E402


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
    say("upload layer")
    layer = ops.DeviceLayer.from_host(blob, lay, 1, DSV2_LITE, device="cuda")
    pl.widen()
    return layer, pl


@pytest.mark.parametrize("T", [1, 4, 16, 64])
def test_grouped_matches_oracle(dev, T):
    layer, pl = dev
    runner = ops.GroupedRunner(64, DSV2_LITE)
    bias = synth.zipf_logit_bias(0)
    xn = orc.rms_norm(synth.hidden_inputs(10 + T, T))
    _, ids, ws = orc.route(pl.router_f32(), xn, logit_bias=bias)
    say(f"grouped T={T} distinct={len(np.unique(ids))}")
    out = runner.run(layer, torch.from_numpy(orc.bf16_bits(xn).view(np.int16)).cuda(),
                     torch.from_numpy(ids).cuda(), torch.from_numpy(ws).cuda())
    torch.cuda.synchronize()
    got = ops.bf16_bits_to_f32(out).cpu().numpy()
    want = orc.moe_grouped(pl, xn, ids, ws)["out"]
    assert rel_err(got, want) <= 1e-2
    # MFMA and NumPy sum in different orders; most elements still agree exactly
    assert np.mean(got == want) > 0.95
    assert runner.status() == 0


@pytest.mark.parametrize("T", [8, 9, 256])
def test_grouped_edges_uniform_routing(dev, T):
    """Unbiased routing at the edges of the launch plans: T = 8 (the largest
    single-launch step), T = 9 (the smallest two-launch step, the first with
    MFMA-eligible units) and T = 256 (the largest step: every expert an MFMA
    unit, the shared expert four 64-token passes)."""
    layer, pl = dev
    runner = ops.GroupedRunner(T, DSV2_LITE)
    xn = orc.rms_norm(synth.hidden_inputs(50 + T, T))
    _, ids, ws = orc.route(pl.router_f32(), xn)
    say(f"grouped edge T={T} distinct={len(np.unique(ids))}")
    out = runner.run(layer, torch.from_numpy(orc.bf16_bits(xn).view(np.int16)).cuda(),
                     torch.from_numpy(ids).cuda(), torch.from_numpy(ws).cuda())
    torch.cuda.synchronize()
    got = ops.bf16_bits_to_f32(out).cpu().numpy()
    want = orc.moe_grouped(pl, xn, ids, ws)["out"]
    assert rel_err(got, want) <= 1e-2
    assert np.mean(got == want) > 0.95
    assert runner.status() == 0


def test_grouped_equals_batch1_decode(dev):
    """grouped(T) == T batch-1 MoE outputs (decode kernel's moe_out)."""
    layer, pl = dev
    T = 8
    x = synth.hidden_inputs(21, T)
    xn = orc.rms_norm(x)
    dec = ops.LayerDecoder(DSV2_LITE)
    runner = ops.GroupedRunner(T, DSV2_LITE)
    outs, idl, wl = [], [], []
    say("batch-1 decode x8")
    for t in range(T):
        r = dec.decode(layer, torch.from_numpy(x[t]).cuda())
        outs.append(ops.bf16_bits_to_f32(r["moe_out"]))
        idl.append(r["ids"])
        wl.append(r["weights"])
    ids = torch.stack(idl)
    ws = torch.stack(wl)
    say("grouped T=8 with the decode routing")
    g = runner.run(layer, torch.from_numpy(orc.bf16_bits(xn).view(np.int16)).cuda(), ids, ws)
    torch.cuda.synchronize()
    got = ops.bf16_bits_to_f32(g).cpu().numpy()
    want = torch.stack(outs).cpu().numpy()
    assert rel_err(got, want) <= 1e-2
    assert np.mean(got == want) > 0.95


def test_grouped_hot_expert_over_64_tokens(dev):
    """Every token routed to the same 6 experts, T = 96 > one 64-token group."""
    layer, pl = dev
    T = 96
    runner = ops.GroupedRunner(T, DSV2_LITE)
    xn = orc.rms_norm(synth.hidden_inputs(30, T))
    ids = np.tile(np.array([5, 17, 3, 60, 0, 41], np.int32), (T, 1))
    ws = np.full((T, 6), 0.125, np.float32)
    say("grouped T=96 hot experts")
    out = runner.run(layer, torch.from_numpy(orc.bf16_bits(xn).view(np.int16)).cuda(),
                     torch.from_numpy(ids).cuda(), torch.from_numpy(ws).cuda())
    torch.cuda.synchronize()
    got = ops.bf16_bits_to_f32(out).cpu().numpy()
    want = orc.moe_grouped(pl, xn, ids, ws)["out"]
    assert rel_err(got, want) <= 1e-2


def test_grouped_workspace_reuse_across_token_counts(dev):
    """One workspace, calls of T = 64, 4, 16, 1, 64 in a row: words left by a
    larger earlier call are never taken for the current call's (each call's
    words carry its own call count), so every result matches the oracle."""
    layer, pl = dev
    runner = ops.GroupedRunner(64, DSV2_LITE)
    bias = synth.zipf_logit_bias(1)
    for n, T in enumerate((64, 4, 16, 1, 64)):
        xn = orc.rms_norm(synth.hidden_inputs(70 + n, T))
        _, ids, ws = orc.route(pl.router_f32(), xn, logit_bias=bias)
        say(f"grouped reuse call {n} T={T}")
        out = runner.run(layer, torch.from_numpy(orc.bf16_bits(xn).view(np.int16)).cuda(),
                         torch.from_numpy(ids).cuda(), torch.from_numpy(ws).cuda())
        torch.cuda.synchronize()
        got = ops.bf16_bits_to_f32(out).cpu().numpy()
        want = orc.moe_grouped(pl, xn, ids, ws)["out"]
        assert rel_err(got, want) <= 1e-2, f"call {n} T={T}"
    assert runner.status() == 0


def test_grouped_out_of_range_ids_raise_the_status_bit(dev):
    """An id outside [0, 64) is clamped (the addresses stay in bounds) and
    reported through FLEET_MOE_ABORT_BAD_ID; a valid call reports nothing."""
    layer, pl = dev
    from fleet_moe import _lib
    T = 4
    xn = orc.rms_norm(synth.hidden_inputs(90, T))
    _, ids, ws = orc.route(pl.router_f32(), xn)
    x = torch.from_numpy(orc.bf16_bits(xn).view(np.int16)).cuda()
    runner = ops.GroupedRunner(T, DSV2_LITE)
    say("grouped valid ids")
    runner.run(layer, x, torch.from_numpy(ids).cuda(), torch.from_numpy(ws).cuda())
    torch.cuda.synchronize()
    assert runner.status() == 0
    bad = ids.copy()
    bad[2, 3] = 64
    bad[0, 0] = -1
    say("grouped ids out of range")
    runner.run(layer, x, torch.from_numpy(bad).cuda(), torch.from_numpy(ws).cuda())
    torch.cuda.synchronize()
    assert runner.status() == _lib.ABORT_BAD_ID


def test_grouped_call_count_wrap_restarts_a_clean_workspace(dev):
    """Workspace words carry a 32-bit call count. The header is seeded from the
    host as if 2^32 - 3 calls had run; the call numbered 2^32 - 1 clears the
    tagged words and restarts the count at 0, so the calls on either side of
    the wrap give the same outputs as a fresh workspace, bit for bit."""
    layer, pl = dev
    T_max = 64
    runner = ops.GroupedRunner(T_max, DSV2_LITE)
    fresh = ops.GroupedRunner(T_max, DSV2_LITE)
    start = 0xFFFFFFFD          # header words: call count, exit count (256 per call)
    head0 = np.array([start, (start * 256) & 0xFFFFFFFF], np.uint32)
    runner.workspace[:8].copy_(torch.from_numpy(head0.view(np.uint8)).cuda())
    bias = synth.zipf_logit_bias(3)
    for n, T in enumerate((16, 4, 64, 9, 4)):
        xn = orc.rms_norm(synth.hidden_inputs(110 + n, T))
        _, ids, ws = orc.route(pl.router_f32(), xn, logit_bias=bias)
        x = torch.from_numpy(orc.bf16_bits(xn).view(np.int16)).cuda()
        idt, wst = torch.from_numpy(ids).cuda(), torch.from_numpy(ws).cuda()
        say(f"grouped wrap call {n} (count {(start + 1 + n) & 0xFFFFFFFF:#x}) T={T}")
        got = runner.run(layer, x, idt, wst)
        want = fresh.run(layer, x, idt, wst)
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"call {n} T={T}"
        head = runner.workspace[:8].cpu().numpy().view(np.uint32).tolist()
        if n == 0:
            assert head == [start + 1, ((start + 1) * 256) & 0xFFFFFFFF]
        else:           # the call numbered 2^32 - 1 (n = 1) restarted the count at 0
            assert head == [n - 1, 256 * (n - 1)]
    assert runner.status() == 0
