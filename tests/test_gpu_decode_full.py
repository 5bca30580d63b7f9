"""Config 4 parity: the full 27-layer DeepSeek-V2-Lite-shape model (weights
N(0, 0.02^2) drawn on the device, dense layer 0, MoE layers 1-26, absorbed
MLA, vocabulary 102400) decodes 32 greedy tokens after a 1024-token seeded
uniform prompt, and the tokens equal the CPU oracle's.

The GPU runs the whole thing as the benchmark does (graph replays, token and
position on the device). The oracle decodes from the GPU's prefilled KV cache
(a NumPy prefill of 1024 positions x 27 layers would take most of an hour):
it recomputes the last prompt step itself, which re-derives cache row 1023 of
every layer and the first pick, then runs the 32 greedy steps on its own
state. The routed experts a step needs are read back from the device as the
oracle asks for them.

The prefill itself is checked teacher-forced at sampled positions (0, 255,
511, 1023): those steps run eagerly, layer by layer, recording every layer's
input and its residual after attention, and for all 27 layers the oracle,
given the GPU's input and the GPU's cache rows before the position, must
reproduce bit for bit the appended cache row and the attention half (at every
sampled position) and the FFN half (dense or MoE; at positions 0 and 1023)."""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from fleet_moe import layout as lay_mod, ops, rope, synth_gpu  # noqa: E402
from fleet_moe.layout import DSV2_LITE  # noqa: E402
from oracle import moe_oracle as orc  # noqa: E402

H, I, DI, V = 2048, 1408, 10944, 102400
LAYERS, PROMPT, GEN = 27, 1024, 32


def say(msg: str) -> None:
    print(f"[gpu] {msg}", flush=True)


def rel_err(got, want) -> float:
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    return float(np.max(np.abs(got - want)) / max(np.max(np.abs(want)), 1e-30))


class _Fetch:
    def __init__(self, dec: ops.Decoder):
        self.dec = dec

    def __call__(self, name: str, start: int = 0, count: int | None = None) -> np.ndarray:
        t = self.dec.layout.tensors[name]
        n = t.nbytes // 2 if count is None else count
        w = self.dec.blob[t.offset + 2 * start: t.offset + 2 * (start + n)]
        return w.view(torch.int16).cpu().numpy().view(np.uint16)


class DeviceMoeLayer(orc.PackedLayer):
    """An oracle MoE layer whose routed experts stay on the device: each one
    the oracle asks for is read back and widened (not kept, so the host holds
    one layer's selection at a time)."""

    def __init__(self, fetch: _Fetch, i: int):
        super().__init__(router=fetch(f"L{i}.router"), experts=np.zeros(0, np.uint16),
                         shared=fetch(f"L{i}.shared"), expert_stride=3 * H * I,
                         norm=fetch(f"L{i}.norm_post"))
        self._fetch, self._i = fetch, i

    def expert_f32(self, e: int):
        blk = orc.bf16_to_f32(self._fetch(f"L{self._i}.experts", int(e) * 3 * H * I, 3 * H * I))
        gu = blk[: 2 * I * H].reshape(2 * I, H)
        return (np.ascontiguousarray(gu[0::2]), np.ascontiguousarray(gu[1::2]),
                blk[2 * I * H:].reshape(H, I))


def oracle_model(dec: ops.Decoder) -> orc.DecodeModel:
    f = _Fetch(dec)
    attn, ffn = [], []
    for i in range(dec.n_layers):
        attn.append(orc.AttnLayer(norm_in=f(f"L{i}.norm_in"), qkv=f(f"L{i}.qkv"),
                                  kv_a_norm=f(f"L{i}.kv_a_norm"), kv_b=f(f"L{i}.kv_b"),
                                  o_proj=f(f"L{i}.o_proj")))
        if f"L{i}.dense" in dec.layout.tensors:
            blk = orc.bf16_to_f32(f(f"L{i}.dense"))
            gu = blk[: 2 * DI * H].reshape(2 * DI, H)
            ffn.append(orc.DenseFfn(np.ascontiguousarray(gu[0::2]), np.ascontiguousarray(gu[1::2]),
                                    blk[2 * DI * H:].reshape(H, DI), norm=f(f"L{i}.norm_post")))
        else:
            ffn.append(DeviceMoeLayer(f, i))
        attn[-1].f32("qkv"), attn[-1].f32("kv_b"), attn[-1].f32("o_proj")
    return orc.DecodeModel(embed=f("embed").reshape(V, H), final_norm=f("final_norm"),
                           lm_head=orc.bf16_to_f32(f("lm_head")), attn=attn, ffn=ffn)


SAMPLED = (0, 255, 511, PROMPT - 1)
FFN_SAMPLED = (0, PROMPT - 1)


def eager_step_recording(dec: ops.Decoder):
    """One decode step launched layer by layer (the kernels a graph replay
    runs, in the same order), recording each layer's input and its residual
    after the attention half. Returns fp32 [layers + 1][H] inputs (the last
    one: the final residual) and [layers][H] mid residuals, on the host."""
    x = dec.x
    ins, mids = [], []
    dec.attn.embed_into(dec._addr("embed"), dec.token, x)
    for i in range(dec.n_layers):
        ins.append(x.clone())
        dec.attn.attn_into(dec.attn_layers[i], x, x, dec.cache[i], 0, dec.pos, dec.cos, dec.sin)
        mids.append(x.clone())
        dec.ffn.layer_into(i, x, x)
    ins.append(x.clone())
    dec.attn.lm_head_into(x, dec._addr("final_norm"), dec._addr("lm_head"), None, dec.token_out,
                          dec.token, dec.pos)
    return torch.stack(ins).cpu().numpy(), torch.stack(mids).cpu().numpy()


def check_prefill_teacher_forced(m: orc.DecodeModel, g_cache, records, cos, sin):
    """Bit-exact teacher-forced checks of the recorded prefill steps."""
    for p, (ins, mids) in records.items():
        for i in range(LAYERS):
            cache = np.zeros((p + 1, 576), np.float32)
            cache[:p] = orc.bf16_to_f32(g_cache[i, :p])
            a = orc.attention(m.attn[i], ins[i], cache, p, cos, sin)
            g_row = orc.bf16_to_f32(g_cache[i, p])
            np.testing.assert_array_equal(g_row.view(np.uint32), a["row"].view(np.uint32),
                                          err_msg=f"cache row {p} of layer {i}")
            x1 = orc.bf16_round(ins[i] + a["out"])
            np.testing.assert_array_equal(mids[i].view(np.uint32), x1.view(np.uint32),
                                          err_msg=f"attention half, layer {i} pos {p}")
            if p in FFN_SAMPLED:
                f = m.ffn[i]
                if isinstance(f, orc.DenseFfn):
                    want = orc.dense_layer(f.gate, f.up, f.down, mids[i],
                                           orc.bf16_to_f32(f.norm))["x_out"]
                else:
                    want = orc.moe_layer(f, mids[i])["x_out"]
                np.testing.assert_array_equal(ins[i + 1].view(np.uint32), want.view(np.uint32),
                                              err_msg=f"FFN half, layer {i} pos {p}")
        say(f"prefill position {p}: cache rows, attention"
            f"{' and FFN' if p in FFN_SAMPLED else ''} of all {LAYERS} layers bit-exact")


@pytest.mark.timeout(900)
def test_full_decode_32_greedy_tokens_match_oracle():
    lay = lay_mod.model_layout(DSV2_LITE, n_layers=LAYERS)
    blob = torch.empty(lay.nbytes, dtype=torch.uint8, device="cuda")
    say(f"drawing {lay.nbytes / 1e9:.1f} GB of weights")
    synth_gpu.fill_model(blob, lay, seed=0)
    max_pos = PROMPT + GEN
    dec = ops.Decoder(blob, lay, DSV2_LITE, max_pos=max_pos)
    prompt = np.random.default_rng(0).integers(0, V, PROMPT).astype(np.int32)
    dec.capture()
    say("gpu prefill (graph replays; eager and recorded at the sampled positions)")
    prompt_d = torch.from_numpy(prompt).cuda()
    dec.reset(0)
    records = {}
    for p in range(PROMPT):
        dec.token.copy_(prompt_d[p:p + 1])
        if p in SAMPLED:
            records[p] = eager_step_recording(dec)
        else:
            dec.step()
    tok0 = int(dec.token_out.item())
    g_cache = dec.cache[:, :PROMPT].cpu().numpy().view(np.uint16)
    say("gpu generate")
    toks = dec.generate(GEN).cpu().numpy()
    assert dec.status() == 0
    got = [tok0] + [int(t) for t in toks]
    say(f"gpu tokens {got}")

    say("oracle weights")
    m = oracle_model(dec)
    cos, sin = rope.yarn_tables(max_pos)
    check_prefill_teacher_forced(m, g_cache, records, cos, sin)
    caches = []
    for i in range(LAYERS):
        c = np.zeros((max_pos, 576), np.float32)
        c[:PROMPT] = orc.bf16_to_f32(g_cache[i])
        caches.append(c)
    row_prev = [c[PROMPT - 1].copy() for c in caches]
    r = orc.decode_step(m, int(prompt[-1]), PROMPT - 1, caches, cos, sin)
    worst = max(rel_err(caches[i][PROMPT - 1], row_prev[i]) for i in range(LAYERS))
    say(f"cache row {PROMPT - 1} re-derived by the oracle: worst layer rel err {worst:.2e}")
    for i in range(LAYERS):
        np.testing.assert_array_equal(caches[i][PROMPT - 1].view(np.uint32),
                                      row_prev[i].view(np.uint32),
                                      err_msg=f"cache row {PROMPT - 1}, layer {i}")
    want, margins = [r["token"]], [r["margin"]]
    for j in range(GEN):
        r = orc.decode_step(m, want[-1], PROMPT + j, caches, cos, sin)
        want.append(r["token"])
        margins.append(r["margin"])
        say(f"oracle step {j}: token {r['token']} margin {r['margin']:.4f}")
    say(f"oracle tokens {want}")
    say(f"smallest top-2 margin {min(margins):.4f}")
    assert got == want
