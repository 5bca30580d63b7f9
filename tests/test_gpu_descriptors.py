"""A task graph's MoE layers run through the descriptor adapter on the GPU:
plan() of a graph with two MoE layers (the reference's shape,
taskgraph.py:366-441), executed by MoeSteps through fleet_moe_layer_decode,
gives the same residual stream, bit for bit, as two direct decode calls."""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from fleet_moe import descriptors as D, ops, synth  # noqa: E402
from fleet_moe.layout import DSV2_LITE  # noqa: E402


def test_graph_moe_layers_run_through_the_library(full_layer):
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    blob, lay, _ = full_layer
    print("[gpu] upload layer", flush=True)
    layer = ops.DeviceLayer.from_host(blob, lay, 1, DSV2_LITE, device="cuda")
    K = D.TaskKind
    g = [D.Descriptor(K.O_PROJ, 1, 0, signal_event=0)]
    m1, done1 = D.moe_layer_descriptors(1, wait_event=0, first_event=1)
    g += m1 + [D.Descriptor(K.QKV_FUSED, 2, 0, wait_event=done1, signal_event=done1 + 1,
                            flags=D.Flags.FOLD_PARTIALS)]
    m2, done2 = D.moe_layer_descriptors(2, wait_event=done1 + 1, first_event=done1 + 2)
    g += m2 + [D.Descriptor(K.LM_HEAD, -1, 0, wait_event=done2, flags=D.Flags.FOLD_PARTIALS)]
    steps = D.plan(D.unpack_all(D.pack_all(g)))
    dec = ops.LayerDecoder(DSV2_LITE)
    runner = D.MoeSteps(steps, {1: layer, 2: layer}, dec)
    x0 = torch.from_numpy(synth.hidden_inputs(90, 1)[0]).cuda()
    x = x0.clone()
    segs = []
    print("[gpu] descriptor plan: 2 MoE calls", flush=True)
    runner.run(x, segment_runner=segs.append)
    ref = x0.clone()
    dec2 = ops.LayerDecoder(DSV2_LITE)
    dec2.decode_into(layer, ref, ref)
    dec2.decode_into(layer, ref, ref)
    torch.cuda.synchronize()
    assert len(segs) == 3
    assert torch.equal(x, ref)
    assert not torch.equal(x, x0)
    assert dec.status() == 0
