"""GPU test of fleet_moe_grouped_noalloc, the grouped step that allocates
nothing (its workspace is a static device array inside the library).

Called through the C ABI, its outputs must be bit-equal to fleet_moe_grouped's
(same kernels, same inputs, a caller workspace) on consecutive calls whose
token counts shrink, so words a larger call left in the shared static array
are never taken for a smaller call's; every call reports status 0."""
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


def _noalloc(layer, x, ids, ws):
    lib = _lib.load()
    T = x.shape[0]
    out = torch.full((T, DSV2_LITE.hidden), -1, dtype=torch.int16, device="cuda")
    status = torch.full((1,), 0x7fffffff, dtype=torch.int32, device="cuda")
    cl = layer.c_layer()
    dims = ops.c_dims(DSV2_LITE)
    rc = lib.fleet_moe_grouped_noalloc(ctypes.byref(cl), T, ids.data_ptr(), ws.data_ptr(),
                                       x.data_ptr(), out.data_ptr(), status.data_ptr(),
                                       ctypes.byref(dims), ops._stream())
    _lib.check(rc, "fleet_moe_grouped_noalloc")
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
    # and the first two against the oracle, to the grouped path's own bar
    x, ids, ws = _inputs(pl, 201, 16)
    got, _ = _noalloc(layer, x, ids, ws)
    torch.cuda.synchronize()
    xn = ops.bf16_bits_to_f32(x).cpu().numpy()
    want = orc.moe_grouped(pl, xn, ids.cpu().numpy(), ws.cpu().numpy())["out"]
    g = ops.bf16_bits_to_f32(got).cpu().numpy()
    assert np.max(np.abs(g - want)) / np.max(np.abs(want)) <= 1e-2


def test_noalloc_rejects_more_tokens_than_the_scratch_holds(dev):
    layer, pl = dev
    T = _lib.NOALLOC_MAX_TOKENS + 1
    x, ids, ws = _inputs(pl, 300, T)
    with pytest.raises(_lib.FleetMoeError) as e:
        _noalloc(layer, x, ids, ws)
    assert e.value.code == _lib.ERR_CAPACITY
