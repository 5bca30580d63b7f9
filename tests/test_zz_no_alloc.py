"""GPU test of fleet_moe_grouped_noalloc, the grouped step that allocates
nothing (its workspace is a static device array inside the library).

Called through the C ABI, its outputs must be bit-equal to fleet_moe_grouped's
(same kernels, same inputs, a caller workspace) on consecutive calls whose
token counts shrink, so words a larger call left in the shared static array
are never taken for a smaller call's; every call reports status 0. A call
captured in a HIP graph (the callers it is for) and replayed between other
calls on the same static array gives the same bits and status on every
replay."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from fleet_moe import _lib, ops, synth  # noqa: E402
from fleet_moe.layout import DSV2_LITE  # noqa: E402
from oracle import moe_oracle as orc  # noqa: E402


def say(msg: str) -> None:
    print(f"[gpu] {msg}", flush=True)


@pytest.fixture(scope="module")
def dev(full_layer):
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    blob, lay, pl = full_layer
    say("upload layer")
    layer = ops.DeviceLayer.from_host(blob, lay, 1, DSV2_LITE, device="cuda")
    return layer, pl


def _inputs(pl, seed: int, T: int):
    xn = orc.rms_norm(synth.hidden_inputs(seed, T))
    _, ids, ws = orc.route(pl.router_f32(), xn, logit_bias=synth.zipf_logit_bias(seed))
    return (torch.from_numpy(orc.bf16_bits(xn).view(np.int16)).cuda(),
            torch.from_numpy(ids).cuda(), torch.from_numpy(ws).cuda())


def _noalloc_into(layer, x, ids, ws, out, status):
    lib = _lib.load()
    cl = layer.c_layer()
    dims = ops.c_dims(DSV2_LITE)
    rc = lib.fleet_moe_grouped_noalloc(ctypes.byref(cl), x.shape[0], ids.data_ptr(),
                                       ws.data_ptr(), x.data_ptr(), out.data_ptr(),
                                       status.data_ptr(), ctypes.byref(dims), ops._stream())
    _lib.check(rc, "fleet_moe_grouped_noalloc")


def _noalloc(layer, x, ids, ws):
    T = x.shape[0]
    out = torch.full((T, DSV2_LITE.hidden), -1, dtype=torch.int16, device="cuda")
    status = torch.full((1,), 0x7fffffff, dtype=torch.int32, device="cuda")
    _noalloc_into(layer, x, ids, ws, out, status)
    return out, status


def test_noalloc_equals_workspace_entry_point_on_shrinking_calls(dev):
    layer, pl = dev
    runner = ops.GroupedRunner(_lib.NOALLOC_MAX_TOKENS, DSV2_LITE)
    for n, T in enumerate((64, 16, 4, 64, 9)):
        x, ids, ws = _inputs(pl, 200 + n, T)
        say(f"noalloc call {n} T={T}")
        got, status = _noalloc(layer, x, ids, ws)
        want = runner.run(layer, x, ids, ws)
        torch.cuda.synchronize()
        assert int(status.item()) == 0, f"call {n} T={T}: status {int(status.item()):#x}"
        assert runner.status() == 0
        assert torch.equal(got, want), f"call {n} T={T}: outputs differ"
    # and the second call's inputs against the oracle, to the grouped path's
    # own bar
    x, ids, ws = _inputs(pl, 201, 16)
    got, _ = _noalloc(layer, x, ids, ws)
    torch.cuda.synchronize()
    xn = ops.bf16_bits_to_f32(x).cpu().numpy()
    want = orc.moe_grouped(pl, xn, ids.cpu().numpy(), ws.cpu().numpy())["out"]
    g = ops.bf16_bits_to_f32(got).cpu().numpy()
    assert np.max(np.abs(g - want)) / np.max(np.abs(want)) <= 1e-2


def test_noalloc_captured_in_a_graph_replays_bit_equal(dev):
    """One noalloc call (T = 16, two launches) captured in a HIP graph after
    eager calls have set the array up; three replays, each followed by eager
    noalloc calls of other sizes on the same array: every replay's output
    equals fleet_moe_grouped's bit for bit and reports status 0."""
    layer, pl = dev
    runner = ops.GroupedRunner(_lib.NOALLOC_MAX_TOKENS, DSV2_LITE)
    x, ids, ws = _inputs(pl, 400, 16)
    want = runner.run(layer, x, ids, ws)
    _noalloc(layer, x, ids, ws)                   # not the first call on the device
    out = torch.empty((16, DSV2_LITE.hidden), dtype=torch.int16, device="cuda")
    status = torch.empty((1,), dtype=torch.int32, device="cuda")
    torch.cuda.synchronize()
    say("graph capture of one noalloc call")
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            _noalloc_into(layer, x, ids, ws, out, status)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    others = [_inputs(pl, 401 + k, T) for k, T in enumerate((64, 4, 9))]
    for rep in range(3):
        out.fill_(-1)
        status.fill_(0x7fffffff)
        torch.cuda.synchronize()
        say(f"graph replay {rep}")
        g.replay()
        torch.cuda.synchronize()
        assert int(status.item()) == 0, f"replay {rep}: status {int(status.item()):#x}"
        assert torch.equal(out, want), f"replay {rep}: outputs differ"
        xo, io, wo = others[rep]
        got_o, st_o = _noalloc(layer, xo, io, wo)     # eager work on the same array
        want_o = runner.run(layer, xo, io, wo)
        torch.cuda.synchronize()
        assert int(st_o.item()) == 0 and torch.equal(got_o, want_o), f"eager after {rep}"
    assert runner.status() == 0


def test_noalloc_rejects_more_tokens_than_the_scratch_holds(dev):
    layer, pl = dev
    T = _lib.NOALLOC_MAX_TOKENS + 1
    x, ids, ws = _inputs(pl, 300, T)
    with pytest.raises(_lib.FleetMoeError) as e:
        _noalloc(layer, x, ids, ws)
    assert e.value.code == _lib.ERR_CAPACITY
