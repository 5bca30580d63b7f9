"""The dense layer (fleet_moe_dense_decode, and the same stage inside the
one-launch fleet_ffn_column) on many inputs, bit for bit against the oracle.

Its down rows are K = 10944 dot products, certified in fp32 or evaluated
exactly in fp64; the certificate is near its bound for about one row in ten.
Every lane of a wave must then take the same branch: when lanes decided
alone (their fp32 sums can differ in the last bit), the fp64 fallback ran
with part of the wave masked off and returned a wrong value for about one row
in 80,000. 512 inputs (a million rows) make such a row all but certain to
show; the oracle evaluates them as one batch of fp64 GEMMs."""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from fleet_moe import layout as lay_mod, ops, synth_gpu  # noqa: E402
from fleet_moe.layout import DSV2_LITE  # noqa: E402
from oracle import moe_oracle as orc  # noqa: E402

H, DI = 2048, 10944
N_INPUTS, N_FUSED = 512, 64


def say(msg: str) -> None:
    print(f"[gpu] {msg}", flush=True)


@pytest.fixture(scope="module")
def dense_column():
    lay = lay_mod.column_layout(DSV2_LITE, n_layers=1)
    blob = torch.empty(lay.nbytes, dtype=torch.uint8, device="cuda")
    synth_gpu.fill_column(blob, lay, seed=5)
    g = torch.Generator(device="cuda").manual_seed(13)
    t = lay.tensors["L0.norm_post"]
    gamma = 1.0 + 0.1 * torch.randn(t.nbytes // 2, generator=g, device="cuda")
    blob.view(torch.int16)[t.offset // 2:(t.offset + t.nbytes) // 2] = \
        gamma.to(torch.bfloat16).view(torch.int16)
    torch.cuda.synchronize()
    col = ops.FfnColumn(blob, lay, DSV2_LITE)
    w = blob[lay.tensors["L0.dense"].offset:][: lay.tensors["L0.dense"].nbytes]
    blk = orc.bf16_to_f32(w.view(torch.int16).cpu().numpy().view(np.uint16))
    gu = blk[: 2 * DI * H].reshape(2 * DI, H)
    norm = blob[t.offset: t.offset + t.nbytes].view(torch.int16).cpu().numpy().view(np.uint16)
    return col, (np.ascontiguousarray(gu[0::2]), np.ascontiguousarray(gu[1::2]),
                 blk[2 * DI * H:].reshape(H, DI), orc.bf16_to_f32(norm))


def inputs(n: int) -> np.ndarray:
    rng = np.random.default_rng(21)
    scale = rng.choice([0.3, 1.0, 3.0], size=(n, 1)).astype(np.float32)
    return orc.bf16_round(scale * rng.standard_normal((n, H), dtype=np.float32))


def test_dense_layer_is_bit_exact_over_512_inputs(dense_column):
    col, (gate, up, down, gamma) = dense_column
    x = inputs(N_INPUTS)
    xd = torch.from_numpy(x).cuda()
    yd = torch.empty_like(xd)
    say(f"dense layer on {N_INPUTS} inputs (separate launches)")
    for i in range(N_INPUTS):
        col.layer_into(0, xd[i], yd[i])
    torch.cuda.synchronize()
    assert col.status() == 0
    say("oracle (batched fp64 GEMMs)")
    want = orc.dense_layer(gate, up, down, x, gamma)["x_out"]
    got = yd.cpu().numpy()
    bad = np.argwhere(got.view(np.uint32) != want.view(np.uint32))
    assert bad.size == 0, (f"{len(bad)} elements differ, first (input, row) {bad[:4].tolist()}: "
                           f"got {got[tuple(bad[0])]} want {want[tuple(bad[0])]}")
    say(f"fused column stage on {N_FUSED} of them (fleet_ffn_column, one layer)")
    for i in range(N_FUSED):
        xi = xd[i].clone()
        col.run_into(xi)
        yd[i] = xi
    torch.cuda.synchronize()
    assert col.status() == 0
    np.testing.assert_array_equal(yd[:N_FUSED].cpu().numpy().view(np.uint32),
                                  want[:N_FUSED].view(np.uint32))
