"""Pack a local HF DeepSeek-V2-Lite checkpoint directory into the packed blob.

The reference builds its blob with `src/host/pack_weights.py:96-190`, which
instantiates the model through `transformers.from_pretrained` (remote code,
the whole model in host memory). This packer reads the checkpoint's own
files instead -- `config.json` and the `*.safetensors` shards named by
`model.safetensors.index.json` (or a single `model.safetensors`) -- one
tensor at a time, and writes the same three outputs byte for byte:

* `<out>`: one flat bf16 blob, every tensor 256-byte aligned, in the
  reference's order (embed, final_norm, lm_head, then per layer norm_in,
  norm_post, qkv = [q_proj ; kv_a_proj_with_mqa], kv_a_norm, kv_b, o_proj,
  then router, experts (64 blocks of [gate/up interleaved ; down]) and shared
  for an MoE layer, or dense for a dense one);
* `<out>.json`: the metadata dict (`pack_weights.py:155-185`, same keys and
  order);
* `<out>.manifest`: its `scalar` / `tensor` lines (`pack_weights.py:86-93`).

A layer is an MoE layer when the checkpoint holds its router
(`model.layers.{i}.mlp.gate.weight`), which is the reference's
`hasattr(mlp, "experts")` test. Tensors stored in another float dtype are
rounded to bf16 (round to nearest even, as torch's cast is), as the
reference's `to_bf16_u16` does. Peak host memory is one expert block plus
the largest single tensor.

    python -m fleet_moe.hf_pack --model ~/models/dsv2-lite-base --out build/weights.bin
"""
from __future__ import annotations

import argparse
import json
from pathlib import Path

import numpy as np

from .layout import ALIGN, interleave_gate_up


class CheckpointReader:
    """Tensors of a safetensors checkpoint directory by HF parameter name."""

    def __init__(self, model_dir: Path):
        self.dir = Path(model_dir)
        index = self.dir / "model.safetensors.index.json"
        if index.exists():
            self.weight_map = json.loads(index.read_text())["weight_map"]
        else:
            single = self.dir / "model.safetensors"
            if not single.exists():
                raise FileNotFoundError(f"{self.dir}: no model.safetensors(.index.json)")
            from safetensors import safe_open
            with safe_open(str(single), framework="pt") as f:
                self.weight_map = {k: single.name for k in f.keys()}
        self._open: dict = {}

    def __contains__(self, name: str) -> bool:
        return name in self.weight_map

    def bf16(self, name: str) -> np.ndarray:
        """The tensor as bf16 bit patterns (uint16), original shape."""
        import torch
        from safetensors import safe_open
        if name not in self.weight_map:
            raise KeyError(f"checkpoint has no tensor {name}")
        fn = self.weight_map[name]
        if fn not in self._open:
            self._open[fn] = safe_open(str(self.dir / fn), framework="pt")
        t = self._open[fn].get_tensor(name)
        if t.dtype != torch.bfloat16:
            t = t.to(torch.bfloat16)
        return t.contiguous().view(torch.int16).numpy().view(np.uint16)


class BlobWriter:
    """Appends bf16 tensors to one file, each 256-byte aligned; a tensor may
    be written in several consecutive parts (experts block by block)."""

    def __init__(self, path: Path):
        self.f = open(path, "wb")
        self.pos = 0
        self.offsets: dict[str, dict] = {}
        self._cur = None

    def begin(self, name: str, shape) -> None:
        pad = (-self.pos) % ALIGN
        if pad:
            self.f.write(b"\0" * pad)
            self.pos += pad
        self._cur = name
        self.offsets[name] = {"offset": self.pos, "shape": [int(s) for s in shape], "bytes": 0}

    def part(self, arr: np.ndarray) -> None:
        a = np.ascontiguousarray(arr, dtype=np.uint16)
        self.f.write(a.tobytes(order="C"))
        self.pos += a.nbytes
        self.offsets[self._cur]["bytes"] += int(a.nbytes)

    def write(self, name: str, arr: np.ndarray) -> None:
        self.begin(name, arr.shape)
        self.part(arr)

    def close(self) -> None:
        self.f.close()


def write_manifest(path: Path, meta: dict) -> None:
    """`scalar <name> <repr>` for every int/float entry in key order, then
    `tensor <name> <offset> <bytes>` (pack_weights.py:86-93)."""
    lines = []
    for k, v in meta.items():
        if isinstance(v, (int, float)) and not isinstance(v, bool):
            lines.append(f"scalar {k} {v!r}\n")
    for name, t in meta["tensors"].items():
        lines.append(f"tensor {name} {t['offset']} {t['bytes']}\n")
    Path(path).write_text("".join(lines))


def pack_checkpoint(model_dir, out, log=print) -> dict:
    """Pack `model_dir` into `out` (+ .json, .manifest). Returns the metadata."""
    model_dir, out = Path(model_dir), Path(out)
    cfg = json.loads((model_dir / "config.json").read_text())
    ck = CheckpointReader(model_dir)
    w = BlobWriter(out)

    def layer_key(i: int, rest: str) -> str:
        return f"model.layers.{i}.{rest}"

    w.write("embed", ck.bf16("model.embed_tokens.weight"))
    w.write("final_norm", ck.bf16("model.norm.weight"))
    w.write("lm_head", ck.bf16("lm_head.weight"))

    expert_strides = []
    n_layers = int(cfg["num_hidden_layers"])
    for i in range(n_layers):
        a = lambda rest: ck.bf16(layer_key(i, "self_attn." + rest))   # noqa: E731
        if layer_key(i, "self_attn.q_proj.weight") not in ck:
            raise ValueError(f"layer {i}: no q_proj (a q_lora checkpoint); the packed layout "
                             "holds DeepSeek-V2-Lite's direct q_proj")
        w.write(f"L{i}.norm_in", ck.bf16(layer_key(i, "input_layernorm.weight")))
        w.write(f"L{i}.norm_post", ck.bf16(layer_key(i, "post_attention_layernorm.weight")))
        w.write(f"L{i}.qkv", np.concatenate([a("q_proj.weight"),
                                             a("kv_a_proj_with_mqa.weight")], 0))
        w.write(f"L{i}.kv_a_norm", a("kv_a_layernorm.weight"))
        w.write(f"L{i}.kv_b", a("kv_b_proj.weight"))
        w.write(f"L{i}.o_proj", a("o_proj.weight"))
        m = lambda rest: ck.bf16(layer_key(i, "mlp." + rest))          # noqa: E731
        if layer_key(i, "mlp.gate.weight") in ck:
            w.write(f"L{i}.router", m("gate.weight"))
            n_exp = int(cfg["n_routed_experts"])
            stride = None
            w.begin(f"L{i}.experts", (0,))
            for e in range(n_exp):
                blk = np.concatenate([
                    interleave_gate_up(m(f"experts.{e}.gate_proj.weight"),
                                       m(f"experts.{e}.up_proj.weight")).reshape(-1),
                    m(f"experts.{e}.down_proj.weight").reshape(-1)])
                if stride is None:
                    stride = blk.size
                if blk.size != stride:
                    raise ValueError(f"layer {i} expert {e}: experts must be uniform")
                w.part(blk)
            w.offsets[f"L{i}.experts"]["shape"] = [n_exp * stride]
            expert_strides.append(int(stride))
            gu = interleave_gate_up(m("shared_experts.gate_proj.weight"),
                                    m("shared_experts.up_proj.weight"))
            w.write(f"L{i}.shared", np.concatenate(
                [gu.reshape(-1), m("shared_experts.down_proj.weight").reshape(-1)]))
        else:
            gu = interleave_gate_up(m("gate_proj.weight"), m("up_proj.weight"))
            w.write(f"L{i}.dense", np.concatenate([gu.reshape(-1),
                                                   m("down_proj.weight").reshape(-1)]))
        log(f"hf_pack: L{i} done ({'moe' if f'L{i}.router' in w.offsets else 'dense'}), "
            f"blob at {w.pos:,} bytes")
    w.close()
    if len(set(expert_strides)) > 1:
        raise ValueError(f"MoE layers disagree on the routed-expert block size "
                         f"(elements): {sorted(set(expert_strides))}")

    rs = cfg.get("rope_scaling") or {}
    meta = {
        "bytes": w.pos,
        "dtype": "bfloat16",
        "expert_stride": expert_strides[0] if expert_strides else 0,
        "hidden": cfg["hidden_size"],
        "layers": cfg["num_hidden_layers"],
        "first_k_dense": cfg["first_k_dense_replace"],
        "moe_inter": cfg["moe_intermediate_size"],
        "dense_inter": cfg["intermediate_size"],
        "n_routed": cfg["n_routed_experts"],
        "n_shared": cfg["n_shared_experts"],
        "top_k": cfg["num_experts_per_tok"],
        "heads": cfg["num_attention_heads"],
        "kv_lora": cfg["kv_lora_rank"],
        "qk_nope": cfg["qk_nope_head_dim"],
        "qk_rope": cfg["qk_rope_head_dim"],
        "v_head": cfg["v_head_dim"],
        "vocab": cfg["vocab_size"],
        "rms_eps": cfg["rms_norm_eps"],
        "routed_scaling": float(cfg.get("routed_scaling_factor", 1.0)),
        "rope_theta": float(cfg.get("rope_theta", 10000.0)),
        "rope_factor": float(rs.get("factor", 1.0)),
        "rope_original_max": int(rs.get("original_max_position_embeddings",
                                        cfg["max_position_embeddings"])),
        "beta_fast": float(rs.get("beta_fast", 32)),
        "beta_slow": float(rs.get("beta_slow", 1)),
        "mscale": float(rs.get("mscale", 1)),
        "mscale_all_dim": float(rs.get("mscale_all_dim", 0)),
        "gate_up_layout": "interleaved [g0,u0,g1,u1,...]",
        "tensors": w.offsets,
    }
    Path(str(out) + ".json").write_text(json.dumps(meta, indent=2))
    write_manifest(Path(str(out) + ".manifest"), meta)
    log(f"hf_pack: {w.pos:,} bytes of bf16 in {out}; metadata in {out}.json, "
        f"manifest in {out}.manifest")
    return meta


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--model", type=Path, required=True)
    ap.add_argument("--out", type=Path, default=Path("build/weights.bin"))
    a = ap.parse_args()
    a.out.parent.mkdir(parents=True, exist_ok=True)
    pack_checkpoint(a.model, a.out)


if __name__ == "__main__":
    main()
