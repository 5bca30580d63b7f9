"""GPU parity through the drop-in file path: an HF DeepSeek-V2-Lite-shape
checkpoint directory (safetensors shards + config.json) is packed by
fleet_moe.hf_pack into the reference's blob + manifest format
(src/host/pack_weights.py:96-190), read back by layout.load_packed (the
launcher's manifest parse and upload, src/host/fleet_launch.hip:154-170,
583-600), and the kernels run on the tensors the manifest addresses.

The checkpoint has the full layer shapes (hidden 2048; a dense layer 0 of
width 10944; an MoE layer 1 with 64 experts of 1408 and the 2816-wide shared
expert; absorbed-MLA attention) and a small vocabulary. Every RMSNorm weight
(input_layernorm, post_attention_layernorm, kv_a_layernorm) is
1 + 0.1 N(0, 1) rounded to bf16, as in a real checkpoint, so the y = bf16(y * gamma)
step of reference_decode.py:51-65 runs with gamma != 1. Checked bit for bit
against the oracle: the MoE layer's routing, weights, MoE output and layer
output; the dense layer's MLP output and layer output; the attention half of
both layers. The dense and attention oracles take their weights from the
source tensors, not from the blob, so the packing is checked as well."""
from __future__ import annotations

import json

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
safetensors_torch = pytest.importorskip("safetensors.torch")

from fleet_moe import _lib, hf_pack, layout, ops, rope  # noqa: E402
from fleet_moe.layout import DSV2_LITE  # noqa: E402
from oracle import moe_oracle as orc  # noqa: E402

H, I, DI, E, VOCAB = 2048, 1408, 10944, 64, 256
NH, LORA, NOPE, ROPE_D, VH = 16, 512, 128, 64, 128
MAX_POS = 800

CFG = {
    "hidden_size": H, "num_hidden_layers": 2, "first_k_dense_replace": 1,
    "moe_intermediate_size": I, "intermediate_size": DI, "n_routed_experts": E,
    "n_shared_experts": 2, "num_experts_per_tok": 6, "num_attention_heads": NH,
    "kv_lora_rank": LORA, "qk_nope_head_dim": NOPE, "qk_rope_head_dim": ROPE_D,
    "v_head_dim": VH, "vocab_size": VOCAB, "rms_norm_eps": 1e-06,
    "routed_scaling_factor": 1.0, "rope_theta": 10000, "max_position_embeddings": 163840,
    "rope_scaling": {"type": "yarn", "factor": 40, "original_max_position_embeddings": 4096,
                     "beta_fast": 32, "beta_slow": 1, "mscale": 0.707, "mscale_all_dim": 0.707},
}


def say(msg: str) -> None:
    print(f"[gpu] {msg}", flush=True)


def u16(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


@pytest.fixture(scope="module")
def packed(tmp_path_factory):
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    d = tmp_path_factory.mktemp("hf_ckpt")
    g = torch.Generator().manual_seed(1234)

    def w(*shape, std=0.02):
        return (torch.randn(shape, generator=g) * std).to(torch.bfloat16)

    def gamma(n):
        return (1.0 + 0.1 * torch.randn(n, generator=g)).to(torch.bfloat16)

    say("write a 2-layer full-shape checkpoint")
    src = {"model.embed_tokens.weight": w(VOCAB, H), "model.norm.weight": gamma(H),
           "lm_head.weight": w(VOCAB, H)}
    for i in range(2):
        p = f"model.layers.{i}."
        src.update({p + "input_layernorm.weight": gamma(H),
                    p + "post_attention_layernorm.weight": gamma(H),
                    p + "self_attn.q_proj.weight": w(NH * (NOPE + ROPE_D), H),
                    p + "self_attn.kv_a_proj_with_mqa.weight": w(LORA + ROPE_D, H),
                    p + "self_attn.kv_a_layernorm.weight": gamma(LORA),
                    p + "self_attn.kv_b_proj.weight": w(NH * (NOPE + VH), LORA),
                    p + "self_attn.o_proj.weight": w(H, NH * VH)})
    p = "model.layers.0.mlp."
    src.update({p + "gate_proj.weight": w(DI, H), p + "up_proj.weight": w(DI, H),
                p + "down_proj.weight": w(H, DI)})
    shard0 = dict(src)
    p = "model.layers.1.mlp."
    moe = {p + "gate.weight": w(E, H),
           p + "shared_experts.gate_proj.weight": w(2 * I, H),
           p + "shared_experts.up_proj.weight": w(2 * I, H),
           p + "shared_experts.down_proj.weight": w(H, 2 * I)}
    for e in range(E):
        moe.update({p + f"experts.{e}.gate_proj.weight": w(I, H),
                    p + f"experts.{e}.up_proj.weight": w(I, H),
                    p + f"experts.{e}.down_proj.weight": w(H, I)})
    wmap = {}
    for fn, part in (("model-00001-of-00002.safetensors", shard0),
                     ("model-00002-of-00002.safetensors", moe)):
        safetensors_torch.save_file({k: v.contiguous() for k, v in part.items()}, str(d / fn))
        wmap.update({k: fn for k in part})
    del moe
    (d / "model.safetensors.index.json").write_text(json.dumps({"weight_map": wmap}))
    (d / "config.json").write_text(json.dumps(CFG))
    say("hf_pack.pack_checkpoint")
    out = d / "weights.bin"
    hf_pack.pack_checkpoint(d, out, log=lambda *_: None)
    for fn in set(wmap.values()):
        (d / fn).unlink()                       # only the blob is needed from here on
    say("layout.load_packed")
    blob, lay = layout.load_packed(out, device="cuda")
    host = np.memmap(out, dtype=np.uint8, mode="r")
    return {"src": {k: u16(v) for k, v in src.items()}, "blob": blob, "lay": lay, "host": host}


def host_u16(P, name: str) -> np.ndarray:
    t = P["lay"].tensors[name]
    return np.asarray(P["host"][t.offset: t.offset + t.nbytes]).view(np.uint16)


def addr(P, name: str) -> int:
    return P["blob"].data_ptr() + P["lay"].tensors[name].offset


def tokens(seed: int, n: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    return orc.bf16_round(rng.standard_normal((n, H), dtype=np.float32))


def test_manifest_scalars_round_trip(packed):
    s = packed["lay"].scalars
    assert (s["hidden"], s["moe_inter"], s["dense_inter"], s["n_routed"], s["top_k"]) == \
        (H, I, DI, E, 6)
    assert s["expert_stride"] == DSV2_LITE.expert_stride
    assert s["layers"] == 2 and s["first_k_dense"] == 1


def test_packed_moe_layer_with_nonunit_norm_bit_exact(packed):
    P = packed
    gam = host_u16(P, "L1.norm_post")
    assert np.any(gam != orc.bf16_bits(np.ones(H, np.float32))), "gamma must not be unit"
    pl = orc.PackedLayer(router=host_u16(P, "L1.router"), experts=host_u16(P, "L1.experts"),
                         shared=host_u16(P, "L1.shared"), expert_stride=DSV2_LITE.expert_stride,
                         norm=gam)
    layer = ops.DeviceLayer(P["blob"], P["lay"], 1, DSV2_LITE)
    assert layer.c_layer().norm is not None
    dec = ops.LayerDecoder(DSV2_LITE)
    for t, x in enumerate(tokens(5, 8)):
        say(f"packed MoE layer token {t}")
        r = dec.decode(layer, torch.from_numpy(x).cuda())
        torch.cuda.synchronize()
        want = orc.moe_layer(pl, x)
        np.testing.assert_array_equal(r["ids"].cpu().numpy(), want["ids"], err_msg=f"ids {t}")
        np.testing.assert_array_equal(r["weights"].cpu().numpy().view(np.uint32),
                                      want["weights"].view(np.uint32), err_msg=f"weights {t}")
        got_out = ops.bf16_bits_to_f32(r["moe_out"]).cpu().numpy()
        np.testing.assert_array_equal(got_out.view(np.uint32), want["out"].view(np.uint32),
                                      err_msg=f"moe_out {t}")
        np.testing.assert_array_equal(r["x_out"].cpu().numpy().view(np.uint32),
                                      want["x_out"].view(np.uint32), err_msg=f"x_out {t}")
    assert dec.status() == 0


def test_packed_dense_layer_with_nonunit_norm_bit_exact(packed):
    P = packed
    src = P["src"]
    p = "model.layers.0."
    gate = orc.bf16_to_f32(src[p + "mlp.gate_proj.weight"])
    up = orc.bf16_to_f32(src[p + "mlp.up_proj.weight"])
    down = orc.bf16_to_f32(src[p + "mlp.down_proj.weight"])
    gam = orc.bf16_to_f32(src[p + "post_attention_layernorm.weight"])
    dec = ops.DenseDecoder(DSV2_LITE, DI)
    x_out = torch.empty(H, dtype=torch.float32, device="cuda")
    mlp_out = torch.empty(H, dtype=torch.int16, device="cuda")
    for t, x in enumerate(tokens(6, 8)):
        say(f"packed dense layer token {t}")
        dec.decode_into(addr(P, "L0.norm_post"), addr(P, "L0.dense"),
                        torch.from_numpy(x).cuda(), x_out, mlp_out)
        torch.cuda.synchronize()
        want = orc.dense_layer(gate, up, down, x, gam)
        got_mlp = ops.bf16_bits_to_f32(mlp_out).cpu().numpy()
        np.testing.assert_array_equal(got_mlp.view(np.uint32), want["out"].view(np.uint32),
                                      err_msg=f"mlp_out {t}")
        np.testing.assert_array_equal(x_out.cpu().numpy().view(np.uint32),
                                      want["x_out"].view(np.uint32), err_msg=f"x_out {t}")
    assert dec.status() == 0


def test_packed_attention_with_nonunit_norms_bit_exact(packed):
    P = packed
    src = P["src"]
    cos, sin = rope.yarn_tables(MAX_POS, rope.RopeParams.from_scalars(P["lay"].scalars))
    cos_d, sin_d = torch.from_numpy(cos).cuda(), torch.from_numpy(sin).cuda()
    rng = np.random.default_rng(8)
    dec = ops.AttnDecoder(DSV2_LITE)
    for i in range(2):
        p = f"model.layers.{i}.self_attn."
        w = orc.AttnLayer(
            norm_in=src[f"model.layers.{i}.input_layernorm.weight"],
            qkv=np.concatenate([src[p + "q_proj.weight"], src[p + "kv_a_proj_with_mqa.weight"]]),
            kv_a_norm=src[p + "kv_a_layernorm.weight"], kv_b=src[p + "kv_b_proj.weight"],
            o_proj=src[p + "o_proj.weight"])
        layer = _lib.FleetAttnLayer(addr(P, f"L{i}.norm_in"), addr(P, f"L{i}.qkv"),
                                    addr(P, f"L{i}.kv_a_norm"), addr(P, f"L{i}.kv_b"),
                                    addr(P, f"L{i}.o_proj"))
        host_cache = orc.bf16_round(rng.standard_normal((MAX_POS, LORA + ROPE_D),
                                                        dtype=np.float32))
        cache_d = torch.from_numpy(orc.bf16_bits(host_cache).view(np.int16)).cuda()
        for pos in (0, 9, MAX_POS - 1):
            say(f"packed attention layer {i} pos {pos}")
            x = orc.bf16_round(0.5 * rng.standard_normal(H, dtype=np.float32))
            xd = torch.from_numpy(x).cuda()
            yd = torch.empty_like(xd)
            dec.attn_into(layer, xd, yd, cache_d, pos, None, cos_d, sin_d)
            torch.cuda.synchronize()
            r = orc.attention(w, x, host_cache, pos, cos, sin)
            want = orc.bf16_round(x + r["out"])
            np.testing.assert_array_equal(yd.cpu().numpy().view(np.uint32),
                                          want.view(np.uint32), err_msg=f"layer {i} pos {pos}")
            host_cache[pos] = orc.bf16_to_f32(cache_d[pos].cpu().numpy().view(np.uint16))
    assert dec.status() == 0
