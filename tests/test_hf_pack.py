"""The HF-checkpoint packer (fleet_moe.hf_pack) against the reference packer's
format (src/host/pack_weights.py:41-190), on a small synthetic checkpoint with
DeepSeek-V2-Lite's tensor names: two safetensors shards and their index, one
dense layer then two MoE layers, one tensor stored in fp32.

The expected blob is built here independently from the source tensors (each
tensor 256-byte aligned, in pack_weights.py's order, gate/up rows
interleaved, experts back to back), and the packed MoE layers are read back
through the oracle's own addressing (PackedLayer, expert.h:45-71)."""
from __future__ import annotations

import json

import numpy as np
import pytest

torch = pytest.importorskip("torch")
safetensors_torch = pytest.importorskip("safetensors.torch")

from fleet_moe import hf_pack, layout  # noqa: E402
from oracle import moe_oracle as orc  # noqa: E402

CFG = {
    "hidden_size": 64, "num_hidden_layers": 3, "first_k_dense_replace": 1,
    "moe_intermediate_size": 16, "intermediate_size": 48, "n_routed_experts": 4,
    "n_shared_experts": 2, "num_experts_per_tok": 2, "num_attention_heads": 2,
    "kv_lora_rank": 32, "qk_nope_head_dim": 16, "qk_rope_head_dim": 8, "v_head_dim": 16,
    "vocab_size": 100, "rms_norm_eps": 1e-06, "routed_scaling_factor": 1.0,
    "rope_theta": 10000, "max_position_embeddings": 163840,
    "rope_scaling": {"type": "yarn", "factor": 40, "original_max_position_embeddings": 4096,
                     "beta_fast": 32, "beta_slow": 1, "mscale": 0.707, "mscale_all_dim": 0.707},
}


def _tensors(rng) -> dict:
    H, L, I, D = 64, 32, 16, 48
    nh, nope, rope, v = 2, 16, 8, 16

    def t(*shape):
        return torch.from_numpy((0.05 * rng.standard_normal(shape)).astype(np.float32)
                                ).to(torch.bfloat16)
    out = {"model.embed_tokens.weight": t(100, H), "model.norm.weight": t(H),
           "lm_head.weight": t(100, H)}
    for i in range(3):
        p = f"model.layers.{i}."
        out.update({p + "input_layernorm.weight": t(H), p + "post_attention_layernorm.weight": t(H),
                    p + "self_attn.q_proj.weight": t(nh * (nope + rope), H),
                    p + "self_attn.kv_a_proj_with_mqa.weight": t(L + rope, H),
                    p + "self_attn.kv_a_layernorm.weight": t(L),
                    p + "self_attn.kv_b_proj.weight": t(nh * (nope + v), L),
                    p + "self_attn.o_proj.weight": t(H, nh * v)})
        if i == 0:
            out.update({p + "mlp.gate_proj.weight": t(D, H), p + "mlp.up_proj.weight": t(D, H),
                        p + "mlp.down_proj.weight": t(H, D)})
        else:
            out[p + "mlp.gate.weight"] = t(4, H)
            for e in range(4):
                out.update({p + f"mlp.experts.{e}.gate_proj.weight": t(I, H),
                            p + f"mlp.experts.{e}.up_proj.weight": t(I, H),
                            p + f"mlp.experts.{e}.down_proj.weight": t(H, I)})
            out.update({p + "mlp.shared_experts.gate_proj.weight": t(2 * I, H),
                        p + "mlp.shared_experts.up_proj.weight": t(2 * I, H),
                        p + "mlp.shared_experts.down_proj.weight": t(H, 2 * I)})
    # one tensor stored in fp32: the packer rounds it to bf16 like torch's cast
    out["model.layers.1.self_attn.o_proj.weight"] = torch.from_numpy(
        (0.05 * rng.standard_normal((H, nh * v))).astype(np.float32))
    return out


def _bits(t) -> np.ndarray:
    return t.to(torch.bfloat16).contiguous().view(torch.int16).numpy().view(np.uint16)


@pytest.fixture(scope="module")
def packed(tmp_path_factory):
    d = tmp_path_factory.mktemp("ckpt")
    rng = np.random.default_rng(3)
    ts = _tensors(rng)
    names = sorted(ts)
    shards = {"model-00001-of-00002.safetensors": names[::2],
              "model-00002-of-00002.safetensors": names[1::2]}
    wmap = {}
    for fn, ns in shards.items():
        safetensors_torch.save_file({n: ts[n].contiguous() for n in ns}, str(d / fn))
        wmap.update({n: fn for n in ns})
    (d / "model.safetensors.index.json").write_text(json.dumps({"weight_map": wmap}))
    (d / "config.json").write_text(json.dumps(CFG))
    out = d / "weights.bin"
    meta = hf_pack.pack_checkpoint(d, out, log=lambda *_: None)
    return ts, out, meta


def _expected(ts) -> tuple[bytes, list]:
    """The blob as pack_weights.py lays it out, from the source tensors."""
    order = [("embed", "model.embed_tokens.weight"), ("final_norm", "model.norm.weight"),
             ("lm_head", "lm_head.weight")]
    parts = [(n, _bits(ts[k]).reshape(-1)) for n, k in order]
    for i in range(3):
        p = f"model.layers.{i}."
        parts += [(f"L{i}.norm_in", _bits(ts[p + "input_layernorm.weight"])),
                  (f"L{i}.norm_post", _bits(ts[p + "post_attention_layernorm.weight"])),
                  (f"L{i}.qkv", np.concatenate([_bits(ts[p + "self_attn.q_proj.weight"]),
                                                _bits(ts[p + "self_attn.kv_a_proj_with_mqa.weight"])])),
                  (f"L{i}.kv_a_norm", _bits(ts[p + "self_attn.kv_a_layernorm.weight"])),
                  (f"L{i}.kv_b", _bits(ts[p + "self_attn.kv_b_proj.weight"])),
                  (f"L{i}.o_proj", _bits(ts[p + "self_attn.o_proj.weight"]))]

        def gu_block(g, u, dn):
            g, u = _bits(ts[g]), _bits(ts[u])
            inter = np.empty((2 * g.shape[0], g.shape[1]), np.uint16)
            for r in range(g.shape[0]):          # rows g0, u0, g1, u1, ...
                inter[2 * r], inter[2 * r + 1] = g[r], u[r]
            return np.concatenate([inter.reshape(-1), _bits(ts[dn]).reshape(-1)])
        if i == 0:
            parts.append((f"L{i}.dense", gu_block(p + "mlp.gate_proj.weight", p + "mlp.up_proj.weight",
                                                  p + "mlp.down_proj.weight")))
        else:
            parts.append((f"L{i}.router", _bits(ts[p + "mlp.gate.weight"])))
            parts.append((f"L{i}.experts", np.concatenate([
                gu_block(p + f"mlp.experts.{e}.gate_proj.weight", p + f"mlp.experts.{e}.up_proj.weight",
                         p + f"mlp.experts.{e}.down_proj.weight") for e in range(4)])))
            parts.append((f"L{i}.shared", gu_block(p + "mlp.shared_experts.gate_proj.weight",
                                                   p + "mlp.shared_experts.up_proj.weight",
                                                   p + "mlp.shared_experts.down_proj.weight")))
    blob, entries = bytearray(), []
    for name, a in parts:
        blob += b"\0" * ((-len(blob)) % 256)
        entries.append((name, len(blob), a.nbytes))
        blob += a.astype(np.uint16).tobytes()
    return bytes(blob), entries


def test_blob_is_the_reference_layout_byte_for_byte(packed):
    ts, out, meta = packed
    want, entries = _expected(ts)
    got = out.read_bytes()
    assert len(got) == len(want) == meta["bytes"]
    assert got == want
    assert [(n, t["offset"], t["bytes"]) for n, t in meta["tensors"].items()] == entries


def test_manifest_and_json_follow_pack_weights(packed):
    ts, out, meta = packed
    man = (out.parent / (out.name + ".manifest")).read_text().splitlines()
    scal = [ln for ln in man if ln.startswith("scalar ")]
    # pack_weights.py:155-185 key order; ints and floats only, in repr form
    assert [ln.split()[1] for ln in scal] == [
        "bytes", "expert_stride", "hidden", "layers", "first_k_dense", "moe_inter", "dense_inter",
        "n_routed", "n_shared", "top_k", "heads", "kv_lora", "qk_nope", "qk_rope", "v_head",
        "vocab", "rms_eps", "routed_scaling", "rope_theta", "rope_factor", "rope_original_max",
        "beta_fast", "beta_slow", "mscale", "mscale_all_dim"]
    sv = {ln.split()[1]: ln.split()[2] for ln in scal}
    assert sv["expert_stride"] == str(3 * 64 * 16) and sv["rms_eps"] == "1e-06"
    assert sv["rope_factor"] == "40.0" and sv["rope_original_max"] == "4096"
    assert sv["mscale_all_dim"] == "0.707" and sv["routed_scaling"] == "1.0"
    js = json.loads((out.parent / (out.name + ".json")).read_text())
    assert js["gate_up_layout"] == "interleaved [g0,u0,g1,u1,...]" and js["dtype"] == "bfloat16"
    assert js["tensors"]["L1.experts"]["shape"] == [4 * 3 * 64 * 16]
    assert js["tensors"]["L0.qkv"]["shape"] == [2 * 24 + 40, 64]
    # the manifest parses back into the layout the library addresses
    lay = layout.layout_from_manifest("\n".join(man))
    assert lay.scalars["expert_stride"] == 3 * 64 * 16
    assert {n: (e.offset, e.nbytes) for n, e in lay.tensors.items()} == \
        {n: (t["offset"], t["bytes"]) for n, t in meta["tensors"].items()}


def test_moe_layers_read_back_through_the_oracle_addressing(packed):
    ts, out, meta = packed
    lay = layout.layout_from_manifest((out.parent / (out.name + ".manifest")).read_text())
    blob = np.frombuffer(out.read_bytes(), dtype=np.uint8)
    f32 = lambda t: t.to(torch.bfloat16).float().numpy()          # noqa: E731
    for i in (1, 2):
        p = f"model.layers.{i}.mlp."
        pl = orc.PackedLayer(router=layout.view_u16(blob, lay.tensors[f"L{i}.router"]),
                             experts=layout.view_u16(blob, lay.tensors[f"L{i}.experts"]),
                             shared=layout.view_u16(blob, lay.tensors[f"L{i}.shared"]),
                             expert_stride=int(lay.scalars["expert_stride"]), hidden=64,
                             moe_inter=16, n_shared=2)
        np.testing.assert_array_equal(pl.router_f32(), f32(ts[p + "gate.weight"]))
        for e in range(4):
            g, u, dn = pl.expert_f32(e)
            np.testing.assert_array_equal(g, f32(ts[p + f"experts.{e}.gate_proj.weight"]))
            np.testing.assert_array_equal(u, f32(ts[p + f"experts.{e}.up_proj.weight"]))
            np.testing.assert_array_equal(dn, f32(ts[p + f"experts.{e}.down_proj.weight"]))
        sg, su, sd = pl.shared_f32()
        np.testing.assert_array_equal(sg, f32(ts[p + "shared_experts.gate_proj.weight"]))
        np.testing.assert_array_equal(sd, f32(ts[p + "shared_experts.down_proj.weight"]))
    # the fp32-stored tensor was rounded to bf16 exactly as torch casts it
    o = layout.view_u16(blob, lay.tensors["L1.o_proj"])
    np.testing.assert_array_equal(o, _bits(ts["model.layers.1.self_attn.o_proj.weight"]).reshape(-1))


def test_q_lora_checkpoint_is_refused(tmp_path):
    rng = np.random.default_rng(4)
    ts = _tensors(rng)
    ts["model.layers.0.self_attn.q_a_proj.weight"] = ts.pop("model.layers.0.self_attn.q_proj.weight")
    safetensors_torch.save_file({n: t.contiguous() for n, t in ts.items()},
                                str(tmp_path / "model.safetensors"))
    (tmp_path / "config.json").write_text(json.dumps(CFG))
    with pytest.raises(ValueError, match="q_proj"):
        hf_pack.pack_checkpoint(tmp_path, tmp_path / "w.bin", log=lambda *_: None)
