"""Seeded synthetic weights generated on the device (benchmark / test data).

A full FFN column (27 layers, ~30 GB of bf16) is too slow to draw on the host,
so it is drawn on the GPU with torch's device generator, one stream per tensor
keyed by (seed, layer, kind, index): any expert can be regenerated alone, and
the same call on the same device and torch build gives the same bits. Values
are N(0, 0.02^2) rounded to bf16 (torch's round to nearest even); RMSNorm
weights are 1.0. A checker reads the weights it needs back from the device.
"""
from __future__ import annotations

import torch

from .layout import DSV2_LITE, Layout, MoeDims

STD = 0.02
ROUTER, EXPERT_GATE, EXPERT_UP, EXPERT_DOWN, SHARED_GATE, SHARED_UP, SHARED_DOWN, \
    DENSE_GATE, DENSE_UP, DENSE_DOWN, EMBED, LM_HEAD, QKV, KV_B, O_PROJ = range(15)


def _key(seed: int, layer: int, kind: int, index: int) -> int:
    """64-bit mix of the key (splitmix64 finaliser), torch seeds are < 2^63."""
    z = (seed * 0x9E3779B97F4A7C15 + layer * 0xBF58476D1CE4E5B9 + kind * 0x94D049BB133111EB
         + index * 0xD6E8FEB86659FD93 + 0x2545F4914F6CDD1D) & (2**64 - 1)
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & (2**64 - 1)
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & (2**64 - 1)
    return (z ^ (z >> 31)) & (2**63 - 1)


def _normal_bf16(shape, seed, layer, kind, index, device) -> torch.Tensor:
    g = torch.Generator(device=device)
    g.manual_seed(_key(seed, layer, kind, index))
    t = torch.randn(shape, generator=g, device=device, dtype=torch.float32)
    return (t * STD).to(torch.bfloat16).view(torch.int16)


def _fill_mlp(dst: torch.Tensor, inter: int, hidden: int, seed, layer, kinds, index, device):
    """dst: int16 [3 * inter * hidden], interleaved gate/up then down."""
    gu = dst[: 2 * inter * hidden].view(2 * inter, hidden)
    gu[0::2] = _normal_bf16((inter, hidden), seed, layer, kinds[0], index, device)
    gu[1::2] = _normal_bf16((inter, hidden), seed, layer, kinds[1], index, device)
    dst[2 * inter * hidden: 3 * inter * hidden] = _normal_bf16(
        (hidden * inter,), seed, layer, kinds[2], index, device)


def fill_column(blob: torch.Tensor, lay: Layout, seed: int = 0, dims: MoeDims = DSV2_LITE) -> None:
    """Write every FFN tensor of `lay` (fleet_moe.layout.column_layout) into
    the uint8 device tensor `blob`."""
    dev = blob.device
    H = dims.hidden
    words = blob.view(torch.int16)
    one = torch.tensor(1.0, dtype=torch.bfloat16).view(torch.int16).item()
    n_layers = int(lay.scalars.get("layers", 0))
    dense_inter = int(lay.scalars.get("dense_inter", 0))
    for i in range(n_layers):
        def view(name):
            t = lay.tensors[f"L{i}.{name}"]
            return words[t.offset // 2: (t.offset + t.nbytes) // 2]
        view("norm_post").fill_(one)
        if f"L{i}.dense" in lay.tensors:
            _fill_mlp(view("dense"), dense_inter, H, seed, i,
                      (DENSE_GATE, DENSE_UP, DENSE_DOWN), 0, dev)
            continue
        view("router")[:] = _normal_bf16((dims.n_routed * H,), seed, i, ROUTER, 0, dev)
        ex = view("experts").view(dims.n_routed, dims.expert_stride)
        for e in range(dims.n_routed):
            _fill_mlp(ex[e], dims.moe_inter, H, seed, i, (EXPERT_GATE, EXPERT_UP, EXPERT_DOWN),
                      e, dev)
        _fill_mlp(view("shared"), dims.shared_inter, H, seed, i,
                  (SHARED_GATE, SHARED_UP, SHARED_DOWN), 0, dev)


def fill_model(blob: torch.Tensor, lay: Layout, seed: int = 0, dims: MoeDims = DSV2_LITE) -> None:
    """Write every tensor of a whole-model layout (fleet_moe.layout.model_layout):
    the FFN tensors as fill_column does, then embed, lm_head and each layer's
    qkv, kv_b and o_proj drawn N(0, 0.02^2); final_norm, norm_in and kv_a_norm
    are 1.0 (HF's initial RMSNorm weight)."""
    fill_column(blob, lay, seed, dims)
    dev = blob.device
    words = blob.view(torch.int16)
    one = torch.tensor(1.0, dtype=torch.bfloat16).view(torch.int16).item()

    def view(name):
        t = lay.tensors[name]
        return words[t.offset // 2: (t.offset + t.nbytes) // 2]

    def draw(name, layer, kind):
        v = view(name)
        v[:] = _normal_bf16((v.numel(),), seed, layer, kind, 0, dev)

    draw("embed", -1, EMBED)
    draw("lm_head", -1, LM_HEAD)
    view("final_norm").fill_(one)
    for i in range(int(lay.scalars["layers"])):
        view(f"L{i}.norm_in").fill_(one)
        view(f"L{i}.kv_a_norm").fill_(one)
        draw(f"L{i}.qkv", i, QKV)
        draw(f"L{i}.kv_b", i, KV_B)
        draw(f"L{i}.o_proj", i, O_PROJ)
