"""GPU parity of the stacked FFN column (config 3): the dense layer 0
(fleet_moe_dense_decode) and MoE layers (fleet_moe_layer_decode) chained at
batch 1 over weights drawn on the device, against the CPU oracle layer by
layer. Each layer is checked teacher-forced (the oracle gets the GPU's input
of that layer), so routing is compared bit for bit at every layer: ids,
weights and layer outputs bit-equal (every GEMV on the path rounds each dot
product's exact value once, as the oracle does)."""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from fleet_moe import layout as lay_mod, ops, synth, synth_gpu  # noqa: E402
from fleet_moe.layout import DSV2_LITE  # noqa: E402
from oracle import moe_oracle as orc  # noqa: E402

H, I, DI = 2048, 1408, 10944


def say(msg: str) -> None:
    print(f"[gpu] {msg}", flush=True)


def rel_err(got, want) -> float:
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    return float(np.max(np.abs(got - want)) / max(np.max(np.abs(want)), 1e-30))


def same(got, want, what: str) -> None:
    """Bit-equal fp32 arrays (the message gives the size of any difference)."""
    got, want = np.asarray(got, np.float32), np.asarray(want, np.float32)
    eq = got.view(np.uint32) == want.view(np.uint32)
    assert eq.all(), f"{what}: {np.mean(eq):.4f} bit-equal, rel err {rel_err(got, want):.2e}"


def fetch(col, name, start=0, count=None) -> np.ndarray:
    t = col.layout.tensors[name]
    n = t.nbytes // 2 if count is None else count
    w = col.blob[t.offset + 2 * start: t.offset + 2 * (start + n)].view(torch.int16)
    return w.cpu().numpy().view(np.uint16)


def check_dense(col, i, x_in, x_out):
    blk = orc.bf16_to_f32(fetch(col, f"L{i}.dense"))
    gu = blk[: 2 * DI * H].reshape(2 * DI, H)
    dn = blk[2 * DI * H:].reshape(H, DI)
    gamma = orc.bf16_to_f32(fetch(col, f"L{i}.norm_post"))
    want = orc.dense_layer(gu[0::2], gu[1::2], dn, x_in, gamma)["x_out"]
    same(x_out, want, f"layer {i}")


def check_moe(col, i, x_in, x_out, ids, ws):
    pl = orc.PackedLayer(router=fetch(col, f"L{i}.router"), experts=np.zeros(0, np.uint16),
                         shared=fetch(col, f"L{i}.shared"), expert_stride=3 * H * I,
                         norm=fetch(col, f"L{i}.norm_post"))
    want_ids = orc.route(pl.router_f32(), orc.rms_norm(x_in, pl.gamma_f32()))[1]
    for e in want_ids:
        blk = orc.bf16_to_f32(fetch(col, f"L{i}.experts", int(e) * 3 * H * I, 3 * H * I))
        gu = blk[: 2 * I * H].reshape(2 * I, H)
        pl.cache[int(e)] = (gu[0::2].copy(), gu[1::2].copy(), blk[2 * I * H:].reshape(H, I))
    r = orc.moe_layer(pl, x_in)
    np.testing.assert_array_equal(ids, r["ids"], err_msg=f"layer {i}")
    np.testing.assert_array_equal(ws.view(np.uint32), r["weights"].view(np.uint32))
    same(x_out, r["x_out"], f"layer {i}")


def run_and_check(col, x0: np.ndarray, layers):
    x = torch.from_numpy(x0).cuda()
    y = torch.empty_like(x)
    ids = torch.empty(6, dtype=torch.int32, device="cuda")
    ws = torch.empty(6, dtype=torch.float32, device="cuda")
    for i in range(col.n_layers):
        if i < col.first_k_dense:
            col.layer_into(i, x, y)
        else:
            col.decoder.decode_into(col.moe[i], x, y, ids=ids, weights=ws)
        if i in layers:
            torch.cuda.synchronize()
            say(f"check layer {i}")
            xi, yo = x.cpu().numpy(), y.cpu().numpy()
            if i < col.first_k_dense:
                check_dense(col, i, xi, yo)
            else:
                check_moe(col, i, xi, yo, ids.cpu().numpy(), ws.cpu().numpy())
        x, y = y, x
    torch.cuda.synchronize()
    assert col.status() == 0
    return x.cpu().numpy()


def build(n_layers, seed):
    lay = lay_mod.column_layout(DSV2_LITE, n_layers=n_layers)
    say(f"fill column: {n_layers} layers, {lay.nbytes / 1e9:.1f} GB")
    blob = torch.empty(lay.nbytes, dtype=torch.uint8, device="cuda")
    synth_gpu.fill_column(blob, lay, seed)
    torch.cuda.synchronize()
    return ops.FfnColumn(blob, lay, DSV2_LITE)


def test_column_four_layers_teacher_forced():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    col = build(4, seed=3)
    x0 = orc.bf16_round(synth.hidden_inputs(40, 1)[0])
    out = run_and_check(col, x0, layers={0, 1, 2, 3})
    # run_into (in place, no allocation, one launch: fleet_ffn_column) gives
    # the same stream, bit for bit, on every call
    assert col.fused
    for _ in range(3):
        x = torch.from_numpy(x0).cuda()
        col.run_into(x)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(x.cpu().numpy(), out)
    assert col.status() == 0
    del col
    torch.cuda.empty_cache()


def test_column_full_27_layers():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    col = build(27, seed=0)
    x0 = orc.bf16_round(synth.hidden_inputs(41, 1)[0])
    out = run_and_check(col, x0, layers={0, 1, 26})
    assert np.all(np.isfinite(out))
    # the 27 layers in one launch (fleet_ffn_column): the same output bit for bit
    x = torch.from_numpy(x0).cuda()
    col.run_into(x)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(x.cpu().numpy(), out)
    assert col.status() == 0
    del col
    torch.cuda.empty_cache()
