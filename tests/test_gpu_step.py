"""The whole decode step in one launch (fleet_decode_step) against the same
step as separate launches (embed, per layer fleet_attn_decode and the dense or
MoE launch, lm_head + argmax): every final residual, every cache row and every
pick equal bit for bit, eagerly and from a captured graph replayed several
times with other work between the replays.

A 4-layer model (dense layer 0, MoE layers 1-3) with non-unit RMSNorm weights
on every norm (norm_in, kv_a_norm, norm_post, final_norm), so every weight
the fused stages read is exercised; 24 teacher-forced steps from position 0,
then 8 greedy steps. The same comparison runs on 33- and 64-layer tables that
reuse those weights, so the residual exchange's tags are exercised at every
depth where a step has more than 64 stages."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from fleet_moe import _lib, layout as lay_mod, ops, synth_gpu  # noqa: E402
from fleet_moe.layout import DSV2_LITE  # noqa: E402

LAYERS, PROMPT, GEN = 4, 24, 8


def say(msg: str) -> None:
    print(f"[gpu] {msg}", flush=True)


@pytest.fixture(scope="module")
def model():
    lay = lay_mod.model_layout(DSV2_LITE, n_layers=LAYERS)
    blob = torch.empty(lay.nbytes, dtype=torch.uint8, device="cuda")
    say(f"drawing {lay.nbytes / 1e9:.1f} GB of weights")
    synth_gpu.fill_model(blob, lay, seed=3)
    g = torch.Generator(device="cuda").manual_seed(11)
    words = blob.view(torch.int16)
    names = ["final_norm"] + [f"L{i}.{n}" for i in range(LAYERS)
                              for n in ("norm_in", "kv_a_norm", "norm_post")]
    for name in names:
        t = lay.tensors[name]
        gamma = 1.0 + 0.1 * torch.randn(t.nbytes // 2, generator=g, device="cuda")
        words[t.offset // 2:(t.offset + t.nbytes) // 2] = gamma.to(torch.bfloat16).view(torch.int16)
    torch.cuda.synchronize()
    return blob, lay


def run(dec: ops.Decoder, prompt: torch.Tensor, use_graph: bool, n_prompt: int = PROMPT,
        n_gen: int = GEN):
    """n_prompt teacher-forced steps from position 0, then n_gen greedy
    steps; per step the final residual and the pick, then the cache."""
    dec.reset(0)
    xs, picks = [], []

    def one():
        if use_graph:
            dec.graph.replay()
        else:
            dec.enqueue_step()
        xs.append(dec.x.clone())
        picks.append(dec.token_out.clone())

    for p in range(n_prompt):
        dec.token.copy_(prompt[p:p + 1])
        one()
    dec.token.copy_(dec.token_out)
    for _ in range(n_gen):
        one()
    torch.cuda.synchronize()
    return (torch.stack(xs).view(torch.int32).cpu(), torch.cat(picks).cpu(),
            dec.cache[:, :n_prompt + n_gen].cpu())


def test_fused_step_equals_separate_launches(model):
    blob, lay = model
    prompt = torch.from_numpy(
        np.random.default_rng(5).integers(0, lay_mod.VOCAB, PROMPT).astype(np.int32)).cuda()
    sep = ops.Decoder(blob, lay, DSV2_LITE, max_pos=64, fused=False)
    fused = ops.Decoder(blob, lay, DSV2_LITE, max_pos=64, fused=True)
    say("separate launches, eager")
    x0, p0, c0 = run(sep, prompt, use_graph=False)
    say("one launch per step, eager")
    x1, p1, c1 = run(fused, prompt, use_graph=False)
    assert sep.status() == 0 and fused.status() == 0
    assert torch.equal(x0, x1), "final residuals differ"
    assert torch.equal(c0, c1), "KV caches differ"
    assert torch.equal(p0, p1), "picks differ"
    say(f"picks {p1.tolist()}")
    say("one launch per step, graph replays (three passes, other work between them)")
    fused.capture()
    for rep in range(3):
        xg, pg, cg = run(fused, prompt, use_graph=True)
        assert torch.equal(x0, xg) and torch.equal(c0, cg) and torch.equal(p0, pg), rep
        sep.enqueue_step()
        torch.cuda.synchronize()
    assert fused.status() == 0
    say(f"{PROMPT + GEN} fused steps equal the separate launches bit for bit")


def aliased_layout(lay, n_layers: int):
    """A layout of n_layers whose layer i reads the drawn layer i (i < LAYERS)
    or MoE layer 1 + (i - 1) % (LAYERS - 1): deep tables without more
    weights. Every layer keeps its own KV cache."""
    fake = lay_mod.Layout(tensors=dict(lay.tensors), scalars=dict(lay.scalars), pos=lay.pos)
    for i in range(LAYERS, n_layers):
        src = 1 + (i - 1) % (LAYERS - 1)
        for name, t in lay.tensors.items():
            if name.startswith(f"L{src}."):
                fake.tensors[f"L{i}." + name.split(".", 1)[1]] = t
    fake.scalars["layers"] = n_layers
    return fake


@pytest.mark.parametrize("n_layers", [33, 64])
def test_fused_step_equals_separate_launches_on_deep_tables(model, n_layers):
    """33 layers is the smallest table whose stages (2n + 1 > 64) outran the
    old per-step tag stride: the first stages of a step then took the
    previous step's residual as current. 64 is the bound."""
    blob, lay = model
    deep = aliased_layout(lay, n_layers)
    prompt = torch.from_numpy(
        np.random.default_rng(6).integers(0, lay_mod.VOCAB, 6).astype(np.int32)).cuda()
    sep = ops.Decoder(blob, deep, DSV2_LITE, max_pos=16, fused=False)
    fused = ops.Decoder(blob, deep, DSV2_LITE, max_pos=16, fused=True)
    say(f"{n_layers} layers: separate launches, then one launch per step")
    x0, p0, c0 = run(sep, prompt, use_graph=False, n_prompt=6, n_gen=4)
    x1, p1, c1 = run(fused, prompt, use_graph=False, n_prompt=6, n_gen=4)
    assert sep.status() == 0 and fused.status() == 0
    assert torch.equal(x0, x1), "final residuals differ"
    assert torch.equal(c0, c1), "KV caches differ"
    assert torch.equal(p0, p1), "picks differ"
    say(f"picks {p1.tolist()}")


def test_fused_step_equals_separate_launches_at_long_positions(model):
    """Steps from position 2300 over a seeded cache, where every attention
    chunk needs several batches of S3 rows: one launch per step equals the
    separate launches bit for bit."""
    blob, lay = model
    g = torch.Generator(device="cuda").manual_seed(12)
    prompt = torch.from_numpy(
        np.random.default_rng(8).integers(0, lay_mod.VOCAB, 4).astype(np.int32)).cuda()
    outs = []
    for fused in (False, True):
        dec = ops.Decoder(blob, lay, DSV2_LITE, max_pos=2400, fused=fused)
        dec.cache.copy_((0.5 * torch.randn(dec.cache.shape, generator=g.manual_seed(12),
                                           device="cuda")).to(torch.bfloat16).view(torch.int16))
        dec.reset(2300)
        xs, picks = [], []
        for p in range(4):
            dec.token.copy_(prompt[p:p + 1])
            dec.enqueue_step()
            xs.append(dec.x.clone())
            picks.append(dec.token_out.clone())
        torch.cuda.synchronize()
        assert dec.status() == 0
        outs.append((torch.stack(xs).view(torch.int32).cpu(), torch.cat(picks).cpu(),
                     dec.cache[:, 2300:2304].cpu()))
    say(f"fused at 2300..2303 equal: {[torch.equal(a, b) for a, b in zip(*outs)]}")
    for a, b in zip(*outs):
        assert torch.equal(a, b)


def test_fused_step_rejects_a_bad_position_without_running(model):
    """A device position outside [0, max_pos) raises FLEET_MOE_ABORT_POSITION
    and the step does nothing (the cache and the position are untouched)."""
    blob, lay = model
    dec = ops.Decoder(blob, lay, DSV2_LITE, max_pos=64, fused=True)
    dec.reset(64)
    before = dec.cache.clone()
    dec.enqueue_step()
    torch.cuda.synchronize()
    assert dec.status() & _lib.ABORT_POSITION
    assert int(dec.pos.item()) == 64
    assert torch.equal(before, dec.cache)


def test_fused_step_entry_point_rejects_bad_arguments(model):
    blob, lay = model
    dec = ops.Decoder(blob, lay, DSV2_LITE, max_pos=64, fused=True)
    lib = _lib.load()
    dims = ops.c_dims(DSV2_LITE)
    bad = _lib.FleetStepModel(dec.step_model.layers, 0, 64, dec.step_model.embed, None,
                              dec.step_model.lm_head, dec.step_model.rope_cos,
                              dec.step_model.rope_sin)
    rc = lib.fleet_decode_step(ctypes.byref(bad), dec.token.data_ptr(), None, None,
                               dec.pos.data_ptr(), None, None, dec.step_ws.data_ptr(),
                               dec.step_ws.numel(), ctypes.byref(dims), None)
    assert rc == _lib.ERR_ARG
    rc = lib.fleet_decode_step(ctypes.byref(dec.step_model), dec.token.data_ptr(), None, None,
                               dec.pos.data_ptr(), None, None, dec.step_ws.data_ptr(),
                               dec.step_ws.numel() - 256, ctypes.byref(dims), None)
    assert rc == _lib.ERR_WORKSPACE
