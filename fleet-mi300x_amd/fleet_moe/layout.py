"""The reference's packed-weight layout and manifest, for the MoE tensors.

Layout contract (src/host/pack_weights.py:41-54, 71-83, 125-146): one flat
blob of bf16 values; every tensor starts on a 256-byte boundary;
`L{i}.router` is [n_routed][hidden]; `L{i}.experts` is n_routed contiguous
blocks of `expert_stride` = 3 * hidden * moe_inter elements, each block the
gate/up rows interleaved [g0, u0, g1, u1, ...] followed by down
[hidden][moe_inter]; `L{i}.shared` is the interleaved gate/up of the merged
shared expert followed by its down [hidden][n_shared * moe_inter];
`L{i}.norm_post` is the post-attention RMSNorm weight. The manifest is text,
`scalar <name> <repr>` lines then `tensor <name> <byte offset> <bytes>` lines
(pack_weights.py:86-93), which is the grammar the reference launcher parses
(src/host/fleet_launch.hip:154-170).

This module only computes offsets and packs NumPy arrays; moving the blob to
the GPU is the caller's business (fleet_moe.ops).
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

ALIGN = 256


@dataclass(frozen=True)
class MoeDims:
    """MoE shape and scalars (the manifest's scalars, pack_weights.py:153-184)."""
    hidden: int = 2048
    moe_inter: int = 1408
    n_routed: int = 64
    n_shared: int = 2
    top_k: int = 6
    routed_scaling: float = 1.0
    rms_eps: float = 1e-6

    @property
    def shared_inter(self) -> int:
        return self.n_shared * self.moe_inter

    @property
    def expert_stride(self) -> int:
        """Elements per routed expert block: gate/up (2*I*H) + down (H*I)."""
        return 3 * self.hidden * self.moe_inter

    @property
    def shared_elems(self) -> int:
        return 3 * self.hidden * self.shared_inter


DSV2_LITE = MoeDims()


@dataclass
class TensorEntry:
    name: str
    offset: int      # bytes from the blob base
    nbytes: int
    shape: tuple


@dataclass
class Layout:
    """Offsets of tensors in one blob, 256-byte aligned, in insertion order."""
    tensors: dict = field(default_factory=dict)
    scalars: dict = field(default_factory=dict)
    pos: int = 0

    def add(self, name: str, shape, itemsize: int = 2) -> TensorEntry:
        if name in self.tensors:
            raise ValueError(f"duplicate tensor {name}")
        self.pos += (-self.pos) % ALIGN
        n = int(np.prod(shape)) * itemsize
        e = TensorEntry(name, self.pos, n, tuple(int(s) for s in shape))
        self.tensors[name] = e
        self.pos += n
        return e

    @property
    def nbytes(self) -> int:
        return self.pos

    def manifest(self) -> str:
        """Manifest text in the reference's grammar (pack_weights.py:86-93)."""
        lines = []
        for k, v in self.scalars.items():
            if isinstance(v, (int, float)) and not isinstance(v, bool):
                lines.append(f"scalar {k} {v!r}\n")
        for name, t in self.tensors.items():
            lines.append(f"tensor {name} {t.offset} {t.nbytes}\n")
        return "".join(lines)


def parse_manifest(text: str):
    """Parse `scalar`/`tensor` lines (grammar of fleet_launch.hip:154-170).

    Returns (scalars: dict name -> int|float, tensors: dict name -> (offset,
    bytes)). Raises ValueError on a malformed line.
    """
    scalars, tensors = {}, {}
    for ln, line in enumerate(text.splitlines(), 1):
        parts = line.split()
        if not parts:
            continue
        if parts[0] == "scalar" and len(parts) == 3:
            v = parts[2]
            try:
                scalars[parts[1]] = int(v)
            except ValueError:
                scalars[parts[1]] = float(v)
        elif parts[0] == "tensor" and len(parts) == 4:
            tensors[parts[1]] = (int(parts[2]), int(parts[3]))
        else:
            raise ValueError(f"manifest line {ln}: {line!r}")
    return scalars, tensors


def layout_from_manifest(text: str) -> Layout:
    """A Layout from a manifest's text: the tensors at their recorded offsets
    (shape = flat bf16 elements; the manifest records bytes only) and the
    scalars, so a blob packed by the reference (or by hf_pack) is addressed
    exactly as the layouts built here."""
    scalars, tensors = parse_manifest(text)
    lay = Layout(scalars=dict(scalars))
    end = 0
    for name, (off, nbytes) in tensors.items():
        if off % ALIGN:
            raise ValueError(f"{name}: offset {off} is not {ALIGN}-byte aligned")
        lay.tensors[name] = TensorEntry(name, off, nbytes, (nbytes // 2,))
        end = max(end, off + nbytes)
    lay.pos = end
    return lay


def load_packed(path, device="cuda", chunk_bytes: int = 1 << 28):
    """Read a packed blob `path` (and `path`.manifest) into one uint8 device
    tensor, streaming the file in chunks so the host never holds it whole.
    Returns (blob tensor, Layout)."""
    import torch
    from pathlib import Path
    path = Path(path)
    lay = layout_from_manifest(Path(str(path) + ".manifest").read_text())
    size = path.stat().st_size
    if size < lay.nbytes:
        raise ValueError(f"{path}: {size} bytes, manifest needs {lay.nbytes}")
    blob = torch.empty(size, dtype=torch.uint8, device=device)
    mm = np.memmap(path, dtype=np.uint8, mode="r")
    for a in range(0, size, chunk_bytes):
        b = min(size, a + chunk_bytes)
        blob[a:b].copy_(torch.from_numpy(np.array(mm[a:b])))
    del mm
    return blob, lay


def moe_layout(dims: MoeDims = DSV2_LITE, layers=(1,), with_norm: bool = True) -> Layout:
    """Layout of the MoE tensors of `layers` (pack_weights.py:113-142 order:
    norm_post first, then router, experts, shared)."""
    lay = Layout()
    H = dims.hidden
    for i in layers:
        if with_norm:
            lay.add(f"L{i}.norm_post", (H,))
        lay.add(f"L{i}.router", (dims.n_routed, H))
        lay.add(f"L{i}.experts", (dims.n_routed * dims.expert_stride,))
        lay.add(f"L{i}.shared", (dims.shared_elems,))
    lay.scalars.update({
        "bytes": lay.nbytes, "expert_stride": dims.expert_stride, "hidden": H,
        "moe_inter": dims.moe_inter, "n_routed": dims.n_routed, "n_shared": dims.n_shared,
        "top_k": dims.top_k, "rms_eps": dims.rms_eps, "routed_scaling": float(dims.routed_scaling),
    })
    return lay


DENSE_INTER = 10944     # DeepSeek-V2-Lite intermediate_size (dense layer 0)


def column_layout(dims: MoeDims = DSV2_LITE, n_layers: int = 27, first_k_dense: int = 1,
                  dense_inter: int = DENSE_INTER) -> Layout:
    """The FFN tensors of a whole decoder stack in pack_weights.py:110-146
    order: per layer norm_post, then `L{i}.dense` (layers < first_k_dense:
    interleaved gate/up [2 I][H] then down [H][I]) or router, experts, shared."""
    lay = Layout()
    H = dims.hidden
    for i in range(n_layers):
        lay.add(f"L{i}.norm_post", (H,))
        if i < first_k_dense:
            lay.add(f"L{i}.dense", (3 * dense_inter * H,))
        else:
            lay.add(f"L{i}.router", (dims.n_routed, H))
            lay.add(f"L{i}.experts", (dims.n_routed * dims.expert_stride,))
            lay.add(f"L{i}.shared", (dims.shared_elems,))
    lay.scalars.update({
        "bytes": lay.nbytes, "expert_stride": dims.expert_stride, "hidden": H,
        "moe_inter": dims.moe_inter, "n_routed": dims.n_routed, "n_shared": dims.n_shared,
        "top_k": dims.top_k, "rms_eps": dims.rms_eps, "routed_scaling": float(dims.routed_scaling),
        "layers": n_layers, "first_k_dense": first_k_dense, "dense_inter": dense_inter,
    })
    return lay


VOCAB = 102400          # DeepSeek-V2-Lite vocab_size
ATTN_HEADS = 16
KV_LORA = 512
QK_NOPE = 128
QK_ROPE = 64
V_HEAD = 128
QKV_ROWS = ATTN_HEADS * (QK_NOPE + QK_ROPE) + KV_LORA + QK_ROPE    # 3648

# YaRN scalars of the manifest (pack_weights.py:171-181), DeepSeek-V2-Lite values
ROPE_SCALARS = {"rope_theta": 10000.0, "rope_factor": 40.0, "rope_original_max": 4096,
                "beta_fast": 32.0, "beta_slow": 1.0, "mscale": 0.707, "mscale_all_dim": 0.707}


def model_layout(dims: MoeDims = DSV2_LITE, n_layers: int = 27, first_k_dense: int = 1,
                 dense_inter: int = DENSE_INTER, vocab: int = VOCAB) -> Layout:
    """Every tensor of the decoder in pack_weights.py:106-146 order: embed,
    final_norm, lm_head, then per layer norm_in, norm_post, qkv (q_proj rows
    then kv_a_proj_with_mqa rows, [3648][H]), kv_a_norm [512], kv_b
    [16 * (128 + 128)][512], o_proj [H][16 * 128], then the FFN tensors as in
    column_layout."""
    lay = Layout()
    H = dims.hidden
    lay.add("embed", (vocab, H))
    lay.add("final_norm", (H,))
    lay.add("lm_head", (vocab, H))
    for i in range(n_layers):
        lay.add(f"L{i}.norm_in", (H,))
        lay.add(f"L{i}.norm_post", (H,))
        lay.add(f"L{i}.qkv", (QKV_ROWS, H))
        lay.add(f"L{i}.kv_a_norm", (KV_LORA,))
        lay.add(f"L{i}.kv_b", (ATTN_HEADS * (QK_NOPE + V_HEAD), KV_LORA))
        lay.add(f"L{i}.o_proj", (H, ATTN_HEADS * V_HEAD))
        if i < first_k_dense:
            lay.add(f"L{i}.dense", (3 * dense_inter * H,))
        else:
            lay.add(f"L{i}.router", (dims.n_routed, H))
            lay.add(f"L{i}.experts", (dims.n_routed * dims.expert_stride,))
            lay.add(f"L{i}.shared", (dims.shared_elems,))
    lay.scalars.update({
        "bytes": lay.nbytes, "expert_stride": dims.expert_stride, "hidden": H,
        "layers": n_layers, "first_k_dense": first_k_dense, "moe_inter": dims.moe_inter,
        "dense_inter": dense_inter, "n_routed": dims.n_routed, "n_shared": dims.n_shared,
        "top_k": dims.top_k, "heads": ATTN_HEADS, "kv_lora": KV_LORA, "qk_nope": QK_NOPE,
        "qk_rope": QK_ROPE, "v_head": V_HEAD, "vocab": vocab, "rms_eps": dims.rms_eps,
        "routed_scaling": float(dims.routed_scaling), **ROPE_SCALARS,
    })
    return lay


def dims_from_scalars(s: dict) -> MoeDims:
    """MoeDims from manifest scalars."""
    return MoeDims(hidden=int(s["hidden"]), moe_inter=int(s["moe_inter"]),
                   n_routed=int(s["n_routed"]), n_shared=int(s["n_shared"]),
                   top_k=int(s["top_k"]), routed_scaling=float(s.get("routed_scaling", 1.0)),
                   rms_eps=float(s.get("rms_eps", 1e-6)))


# ---------------------------------------------------------------- packing

def interleave_gate_up(gate: np.ndarray, up: np.ndarray) -> np.ndarray:
    """Rows [g0, u0, g1, u1, ...] (pack_weights.py:71-83)."""
    if gate.shape != up.shape:
        raise ValueError(f"gate {gate.shape} vs up {up.shape}")
    out = np.empty((2 * gate.shape[0], gate.shape[1]), dtype=gate.dtype)
    out[0::2] = gate
    out[1::2] = up
    return out


def pack_expert(gate: np.ndarray, up: np.ndarray, down: np.ndarray) -> np.ndarray:
    """One expert block: interleaved gate/up then down, flattened (uint16)."""
    return np.concatenate([interleave_gate_up(gate, up).reshape(-1), down.reshape(-1)])


def write_blob(blob: np.ndarray, entry: TensorEntry, arr: np.ndarray) -> None:
    """Copy bf16 bits `arr` into the uint8 blob at entry's offset."""
    a = np.ascontiguousarray(arr, dtype=np.uint16).reshape(-1)
    if a.nbytes != entry.nbytes:
        raise ValueError(f"{entry.name}: {a.nbytes} bytes, layout has {entry.nbytes}")
    blob[entry.offset: entry.offset + a.nbytes] = a.view(np.uint8)


def view_u16(blob: np.ndarray, entry: TensorEntry) -> np.ndarray:
    """uint16 view of one tensor of a uint8 blob."""
    return blob[entry.offset: entry.offset + entry.nbytes].view(np.uint16)
