"""The descriptor adapter on the GPU, driven by graphs the reference emitted
(tests/golden/taskgraph/, written by src/host/taskgraph.py --emit for a
3-layer DeepSeek-V2-Lite config: dense layer 0, MoE layers 1 and 2).

plan() cuts each graph into runtime segments and two MoE calls; MoeSteps runs
the calls through the library (fleet_moe_residual_fold, then
fleet_moe_layer_decode in place on x[1]). The segments belong to the
reference's runtime, which is not part of this library: a stand-in plays its
part on the residual buffers (Activations.x[0], x[1], oproj_partial), as the
reference's tasks leave them -- o_proj's eight fp32 partials before each MoE
layer (or, for --oproj-row-split, x[1] written directly), and the next
QKV_FUSED prologue publishing x[0] = x[1]. The result is checked bit for bit
against the oracle chained the same way: x[1] = residual_fold(x[0],
partials), then oracle.moe_layer, per layer. Also checked: the fold kernel
alone against oracle.residual_fold."""
from __future__ import annotations

import gzip
from pathlib import Path

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from fleet_moe import descriptors as D, ops, synth  # noqa: E402
from fleet_moe.layout import DSV2_LITE, view_u16  # noqa: E402
from oracle import moe_oracle as orc  # noqa: E402

FIX = Path(__file__).resolve().parent / "golden" / "taskgraph"
H = 2048


def say(msg: str) -> None:
    print(f"[gpu] {msg}", flush=True)


def load(name):
    descs = D.unpack_all(gzip.decompress((FIX / f"{name}.bin.gz").read_bytes()))
    events = D.parse_events(gzip.decompress((FIX / f"{name}.events.txt.gz").read_bytes()).decode())
    return descs, events


@pytest.fixture(scope="module")
def two_layers(full_layer):
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    blob1, lay1, pl1 = full_layer
    say("draw MoE layer 2")
    blob2, lay2 = synth.moe_layer_blob(seed=0, layer=2, dims=DSV2_LITE)
    t = lay2.tensors
    pl2 = orc.PackedLayer(router=view_u16(blob2, t["L2.router"]),
                          experts=view_u16(blob2, t["L2.experts"]),
                          shared=view_u16(blob2, t["L2.shared"]),
                          expert_stride=DSV2_LITE.expert_stride,
                          norm=view_u16(blob2, t["L2.norm_post"]))
    say("upload MoE layers 1 and 2")
    dev = {1: ops.DeviceLayer.from_host(blob1, lay1, 1, DSV2_LITE, device="cuda"),
           2: ops.DeviceLayer.from_host(blob2, lay2, 2, DSV2_LITE, device="cuda")}
    return dev, {1: pl1, 2: pl2}


def test_residual_fold_matches_oracle():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    rng = np.random.default_rng(4)
    for n in (8, 1, 3):
        x = orc.bf16_round(rng.standard_normal(H, dtype=np.float32))
        parts = (0.3 * rng.standard_normal((n, H))).astype(np.float32)
        # planted cases at element 0..2: index order, the two roundings
        if n == 8:
            parts[:, :3] = 0.0
            parts[:4, 0] = [1e8, 1.0, -1e8, 1.0]
            x[1], parts[0, 1] = 1.0, 2.0 ** -8 + 2.0 ** -16
            x[2], parts[0, 2] = 1.0, 2.0 ** -10
        xd, pd = torch.from_numpy(x).cuda(), torch.from_numpy(parts).cuda()
        out = torch.empty_like(xd)
        ops.residual_fold(xd, pd, out)
        ops.residual_fold(xd, pd, xd)          # in place
        torch.cuda.synchronize()
        want = orc.residual_fold(x, parts)
        np.testing.assert_array_equal(out.cpu().numpy().view(np.uint32), want.view(np.uint32))
        np.testing.assert_array_equal(xd.cpu().numpy().view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("name", ["default", "local_fold", "oproj_row_split", "topk_published",
                                  "split_workers_18"])
def test_reference_graph_moe_layers_match_the_chained_oracle(two_layers, name):
    dev, pls = two_layers
    descs, events = load(name)
    steps = D.plan(descs, events=events)
    calls = [s for s in steps if isinstance(s, D.MoeCall)]
    assert [c.layer for c in calls] == [1, 2]
    row_split = name == "oproj_row_split"
    assert all(c.fold_oproj == (not row_split) for c in calls)
    rng = np.random.default_rng(17)
    x_layer1 = orc.bf16_round(rng.standard_normal(H, dtype=np.float32))
    partials = {L: (0.2 * rng.standard_normal((8, H))).astype(np.float32) for L in (1, 2)}
    x0 = torch.zeros(H, dtype=torch.float32, device="cuda")     # Activations.x[0]
    x1 = torch.zeros(H, dtype=torch.float32, device="cuda")     # Activations.x[1]
    op = torch.zeros((8, H), dtype=torch.float32, device="cuda")  # oproj_partial
    seen = []

    def runtime_stand_in(seg: D.Segment):
        k = len(seen)
        seen.append(seg)
        if k == 0:                 # embed, dense layer 0, layer 1's attention
            x0.copy_(torch.from_numpy(x_layer1))
        elif k == 1:               # layer 2's QKV_FUSED prologue publishes x[0] = x[1]
            x0.copy_(x1)
        else:                      # LM_HEAD reads x[1]
            return
        L = k + 1
        op.copy_(torch.from_numpy(partials[L]))
        if row_split:              # o_proj's residual epilogue writes x[1] itself
            x1.copy_(torch.from_numpy(orc.residual_fold(x0.cpu().numpy(), partials[L])))

    dec = ops.LayerDecoder(DSV2_LITE)
    say(f"graph {name}: {len(descs)} descriptors, {len(steps)} steps")
    D.MoeSteps(steps, dev, dec).run(x0, x1, op, segment_runner=runtime_stand_in)
    torch.cuda.synchronize()
    assert len(seen) == 3 and dec.status() == 0
    x = x_layer1
    for L in (1, 2):
        mid = orc.residual_fold(x, partials[L])
        x = orc.moe_layer(pls[L], mid)["x_out"]
    np.testing.assert_array_equal(x1.cpu().numpy().view(np.uint32), x.view(np.uint32))
