"""Python host side of the MoE path: device buffers (PyTorch-ROCm tensors used
only as allocations) and thin calls into libfleet_moe.so.

Mirrors the reference's interface for this path: a packed layer is the
`L{i}.norm_post / router / experts / shared` tensors of one blob
(src/host/pack_weights.py), `decode_layer` is the MoE half of
`reference_decode.decoder_layer` (src/host/reference_decode.py:301-302) run
on the GPU, `moe` is `reference_decode.moe` (:268-287) for pre-normed
inputs, and `route` is its router + top-k (:271-278). Errors are raised as
`FleetMoeError` carrying the library's return code.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np
import torch

from . import _lib
from .layout import DSV2_LITE, Layout, MoeDims


def _stream(stream=None) -> int:
    s = torch.cuda.current_stream() if stream is None else stream
    return int(s.cuda_stream)


def c_dims(d: MoeDims) -> _lib.FleetMoeDims:
    return _lib.FleetMoeDims(d.hidden, d.moe_inter, d.n_routed, d.n_shared, d.top_k,
                             float(d.routed_scaling), float(d.rms_eps))


def _ptr(t) -> int | None:
    return None if t is None else int(t.data_ptr())


def _need(t: torch.Tensor, dtype, shape, name: str) -> None:
    if not t.is_cuda:
        raise ValueError(f"{name} must be a device tensor")
    if t.dtype != dtype or tuple(t.shape) != tuple(shape) or not t.is_contiguous():
        raise ValueError(f"{name}: expected contiguous {dtype} {tuple(shape)}, "
                         f"got {t.dtype} {tuple(t.shape)}")


@dataclass
class DeviceLayer:
    """One packed MoE layer resident in device memory."""
    blob: torch.Tensor          # uint8, the packed bytes
    layout: Layout
    layer: int
    dims: MoeDims = DSV2_LITE
    unit_norm: bool = False     # pass NULL for the norm weight (unit gamma)

    @classmethod
    def from_host(cls, blob: np.ndarray, layout: Layout, layer: int,
                  dims: MoeDims = DSV2_LITE, device="cuda", unit_norm: bool = False):
        t = torch.from_numpy(blob).to(device)
        return cls(t, layout, layer, dims, unit_norm)

    def _addr(self, name: str) -> int:
        return self.blob.data_ptr() + self.layout.tensors[f"L{self.layer}.{name}"].offset

    def c_layer(self) -> _lib.FleetMoeLayer:
        has_norm = f"L{self.layer}.norm_post" in self.layout.tensors and not self.unit_norm
        return _lib.FleetMoeLayer(self._addr("norm_post") if has_norm else None,
                                  self._addr("router"), self._addr("experts"),
                                  self.dims.expert_stride, self._addr("shared"))

    def router_u16(self) -> int:
        return self._addr("router")


def route(layer: DeviceLayer, x_norm: torch.Tensor, logit_bias: torch.Tensor | None = None,
          stream=None):
    """Router logits + greedy top-k for x_norm fp32 [T, H] (bf16-valued).
    Returns (logits fp32 [T, E], ids int32 [T, k], weights fp32 [T, k])."""
    d = layer.dims
    T = x_norm.shape[0]
    _need(x_norm, torch.float32, (T, d.hidden), "x_norm")
    if logit_bias is not None:
        _need(logit_bias, torch.float32, (d.n_routed,), "logit_bias")
    dev = x_norm.device
    logits = torch.empty((T, d.n_routed), dtype=torch.float32, device=dev)
    ids = torch.empty((T, d.top_k), dtype=torch.int32, device=dev)
    ws = torch.empty((T, d.top_k), dtype=torch.float32, device=dev)
    dims = c_dims(d)
    rc = _lib.load().fleet_moe_router_topk(layer.router_u16(), _ptr(x_norm), T, _ptr(logit_bias),
                                           _ptr(logits), _ptr(ids), _ptr(ws), ctypes.byref(dims),
                                           _stream(stream))
    _lib.check(rc, "fleet_moe_router_topk")
    return logits, ids, ws


class LayerDecoder:
    """Batch-1 MoE layer decode with its own persistent workspace.

    `decode(layer, x)` returns x_out = bf16(x + moe(rms_norm(x))) plus the
    bf16 MoE output and the routing. Calls on one decoder must be ordered on
    one stream (they share the workspace)."""

    def __init__(self, dims: MoeDims = DSV2_LITE, device="cuda"):
        self.dims = dims
        self._dims = c_dims(dims)
        n = _lib.load().fleet_moe_layer_workspace_bytes(ctypes.byref(self._dims))
        self.workspace = torch.zeros(n, dtype=torch.uint8, device=device)

    def decode_into(self, layer: DeviceLayer, x: torch.Tensor, x_out: torch.Tensor,
                    moe_out: torch.Tensor | None = None, ids: torch.Tensor | None = None,
                    weights: torch.Tensor | None = None, stream=None) -> None:
        """Enqueue one layer; no allocation, no synchronisation."""
        cl = layer.c_layer()
        rc = _lib.load().fleet_moe_layer_decode(
            ctypes.byref(cl), _ptr(x), _ptr(x_out), _ptr(moe_out), _ptr(ids), _ptr(weights),
            _ptr(self.workspace), self.workspace.numel(), ctypes.byref(self._dims),
            _stream(stream))
        _lib.check(rc, "fleet_moe_layer_decode")

    def decode(self, layer: DeviceLayer, x: torch.Tensor, stream=None) -> dict:
        d = self.dims
        _need(x, torch.float32, (d.hidden,), "x")
        dev = x.device
        out = {
            "x_out": torch.empty(d.hidden, dtype=torch.float32, device=dev),
            "moe_out": torch.empty(d.hidden, dtype=torch.int16, device=dev),
            "ids": torch.empty(d.top_k, dtype=torch.int32, device=dev),
            "weights": torch.empty(d.top_k, dtype=torch.float32, device=dev),
        }
        self.decode_into(layer, x, out["x_out"], out["moe_out"], out["ids"], out["weights"],
                         stream)
        return out

    def status(self, stream=None) -> int:
        v = ctypes.c_uint32(0)
        rc = _lib.load().fleet_moe_workspace_status(_ptr(self.workspace), ctypes.byref(v),
                                                    _stream(stream))
        _lib.check(rc, "fleet_moe_workspace_status")
        return int(v.value)


class GroupedRunner:
    """Multi-token grouped-expert product with its own workspace."""

    def __init__(self, max_tokens: int, dims: MoeDims = DSV2_LITE, device="cuda"):
        self.dims = dims
        self.max_tokens = int(max_tokens)
        self._dims = c_dims(dims)
        n = _lib.load().fleet_moe_grouped_workspace_bytes(ctypes.byref(self._dims),
                                                          self.max_tokens)
        self.workspace = torch.zeros(n, dtype=torch.uint8, device=device)

    def run_into(self, layer: DeviceLayer, x_norm_bf16: torch.Tensor, ids: torch.Tensor,
                 weights: torch.Tensor, out: torch.Tensor, stream=None) -> None:
        T = x_norm_bf16.shape[0]
        cl = layer.c_layer()
        rc = _lib.load().fleet_moe_grouped(
            ctypes.byref(cl), T, _ptr(ids), _ptr(weights), _ptr(x_norm_bf16), _ptr(out),
            _ptr(self.workspace), self.workspace.numel(), ctypes.byref(self._dims),
            _stream(stream))
        _lib.check(rc, "fleet_moe_grouped")

    def run(self, layer: DeviceLayer, x_norm_bf16: torch.Tensor, ids: torch.Tensor,
            weights: torch.Tensor, stream=None) -> torch.Tensor:
        d = self.dims
        T = x_norm_bf16.shape[0]
        _need(x_norm_bf16, torch.int16, (T, d.hidden), "x_norm (bf16 bits)")
        _need(ids, torch.int32, (T, d.top_k), "ids")
        _need(weights, torch.float32, (T, d.top_k), "weights")
        out = torch.empty((T, d.hidden), dtype=torch.int16, device=x_norm_bf16.device)
        self.run_into(layer, x_norm_bf16, ids, weights, out, stream)
        return out

    def status(self, stream=None) -> int:
        v = ctypes.c_uint32(0)
        rc = _lib.load().fleet_moe_workspace_status(_ptr(self.workspace), ctypes.byref(v),
                                                    _stream(stream))
        _lib.check(rc, "fleet_moe_workspace_status")
        return int(v.value)


def bf16_bits_to_f32(t: torch.Tensor) -> torch.Tensor:
    """Widen bf16 bit patterns held in an int16 tensor to fp32 (exact)."""
    return (t.to(torch.int32) & 0xFFFF).bitwise_left_shift(16).view(torch.float32)


def f32_to_bf16_bits(t: torch.Tensor) -> torch.Tensor:
    """fp32 -> bf16 bits (int16), round to nearest even (finite values)."""
    u = t.contiguous().view(torch.int32).to(torch.int64) & 0xFFFFFFFF
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF
    return (r - ((r >> 15) & 1) * 65536).to(torch.int16)


def moe(layer: DeviceLayer, x_norm: torch.Tensor, runner: GroupedRunner, stream=None) -> dict:
    """reference_decode.moe for pre-normed tokens x_norm fp32 [T, H]: route,
    then the grouped product. Returns dict(logits, ids, weights, out bf16 bits)."""
    logits, ids, ws = route(layer, x_norm, stream=stream)
    out = runner.run(layer, f32_to_bf16_bits(x_norm), ids, ws, stream)
    return {"logits": logits, "ids": ids, "weights": ws, "out": out}


class DenseDecoder:
    """Batch-1 dense SwiGLU layer (fleet_moe_dense_decode) with its own
    workspace: x_out = bf16(x + mlp(rms_norm(x)))."""

    def __init__(self, dims: MoeDims = DSV2_LITE, dense_inter: int = 10944, device="cuda"):
        self.dims = dims
        self.dense_inter = int(dense_inter)
        self._dims = c_dims(dims)
        n = _lib.load().fleet_moe_dense_workspace_bytes(ctypes.byref(self._dims),
                                                        self.dense_inter)
        if n == 0:
            raise ValueError(f"unsupported dense width {dense_inter}")
        self.workspace = torch.zeros(n, dtype=torch.uint8, device=device)

    def decode_into(self, norm_ptr: int | None, dense_ptr: int, x: torch.Tensor,
                    x_out: torch.Tensor, mlp_out: torch.Tensor | None = None, stream=None) -> None:
        rc = _lib.load().fleet_moe_dense_decode(
            norm_ptr, dense_ptr, self.dense_inter, _ptr(x), _ptr(x_out), _ptr(mlp_out),
            _ptr(self.workspace), self.workspace.numel(), ctypes.byref(self._dims),
            _stream(stream))
        _lib.check(rc, "fleet_moe_dense_decode")

    def status(self, stream=None) -> int:
        v = ctypes.c_uint32(0)
        rc = _lib.load().fleet_moe_workspace_status(_ptr(self.workspace), ctypes.byref(v),
                                                    _stream(stream))
        _lib.check(rc, "fleet_moe_workspace_status")
        return int(v.value)


class FfnColumn:
    """The FFN half of every decoder layer of a stack, chained at batch 1:
    x <- bf16(x + ffn_L(rms_norm_L(x))) for L = 0 .. layers-1, dense for
    L < first_k_dense, MoE after (the benchmark's config 3; reference_decode.py:
    294-302 without the attention half). `blob` is the packed uint8 device
    tensor of `layout` (fleet_moe.layout.column_layout)."""

    def __init__(self, blob: torch.Tensor, layout: Layout, dims: MoeDims = DSV2_LITE):
        self.blob, self.layout, self.dims = blob, layout, dims
        self.n_layers = int(layout.scalars["layers"])
        self.first_k_dense = int(layout.scalars["first_k_dense"])
        self.moe = {i: DeviceLayer(blob, layout, i, dims)
                    for i in range(self.first_k_dense, self.n_layers)}
        self.decoder = LayerDecoder(dims, device=blob.device)
        self.dense = DenseDecoder(dims, int(layout.scalars["dense_inter"]), device=blob.device)

    def _addr(self, name: str) -> int:
        return self.blob.data_ptr() + self.layout.tensors[name].offset

    def layer_into(self, i: int, x: torch.Tensor, x_out: torch.Tensor, stream=None) -> None:
        if i < self.first_k_dense:
            self.dense.decode_into(self._addr(f"L{i}.norm_post"), self._addr(f"L{i}.dense"),
                                   x, x_out, stream=stream)
        else:
            self.decoder.decode_into(self.moe[i], x, x_out, stream=stream)

    def run_into(self, x: torch.Tensor, stream=None) -> None:
        """All layers in place on x (fp32[hidden] on the device); no allocation."""
        for i in range(self.n_layers):
            self.layer_into(i, x, x, stream)

    def status(self) -> int:
        return self.decoder.status() | self.dense.status()
