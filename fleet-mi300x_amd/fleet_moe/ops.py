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


def residual_fold(x: torch.Tensor, partials: torch.Tensor, x_out: torch.Tensor,
                  dims: MoeDims = DSV2_LITE, stream=None) -> None:
    """x_out = bf16(x + bf16(sum of partials in index order)): the residual
    after attention from the layer input and o_proj's K-split fp32 partials
    [n][hidden] (the NORM_ROUTER prologue's fold). Enqueued, no allocation."""
    cd = c_dims(dims)
    rc = _lib.load().fleet_moe_residual_fold(_ptr(x), _ptr(partials), int(partials.shape[0]),
                                             _ptr(x_out), ctypes.byref(cd), _stream(stream))
    _lib.check(rc, "fleet_moe_residual_fold")


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

    def __init__(self, blob: torch.Tensor, layout: Layout, dims: MoeDims = DSV2_LITE,
                 fused: bool = True):
        self.blob, self.layout, self.dims = blob, layout, dims
        self.n_layers = int(layout.scalars["layers"])
        self.first_k_dense = int(layout.scalars["first_k_dense"])
        self.moe = {i: DeviceLayer(blob, layout, i, dims)
                    for i in range(self.first_k_dense, self.n_layers)}
        self.decoder = LayerDecoder(dims, device=blob.device)
        self.dense = DenseDecoder(dims, int(layout.scalars["dense_inter"]), device=blob.device)
        self.fused = bool(fused)
        if self.fused:
            lib = _lib.load()
            rows = (_lib.FleetStepLayer * self.n_layers)()
            for i in range(self.n_layers):
                if i < self.first_k_dense:
                    rows[i].moe = _lib.FleetMoeLayer(self._addr(f"L{i}.norm_post"), None, None, 0,
                                                     None)
                    rows[i].dense = self._addr(f"L{i}.dense")
                else:
                    rows[i].moe = self.moe[i].c_layer()
            raw = bytes(memoryview(rows).cast("B"))
            self.table = torch.frombuffer(bytearray(raw), dtype=torch.uint8).to(blob.device)
            n = lib.fleet_decode_step_workspace_bytes(ctypes.byref(self.decoder._dims))
            self.step_ws = torch.zeros(n, dtype=torch.uint8, device=blob.device)

    def _addr(self, name: str) -> int:
        return self.blob.data_ptr() + self.layout.tensors[name].offset

    def layer_into(self, i: int, x: torch.Tensor, x_out: torch.Tensor, stream=None) -> None:
        if i < self.first_k_dense:
            self.dense.decode_into(self._addr(f"L{i}.norm_post"), self._addr(f"L{i}.dense"),
                                   x, x_out, stream=stream)
        else:
            self.decoder.decode_into(self.moe[i], x, x_out, stream=stream)

    def run_into(self, x: torch.Tensor, stream=None) -> None:
        """All layers in place on x (fp32[hidden] on the device); no allocation.
        fused: one launch (fleet_ffn_column); else one launch per layer."""
        if self.fused:
            rc = _lib.load().fleet_ffn_column(
                self.table.data_ptr(), self.n_layers, _ptr(x), _ptr(x), _ptr(self.step_ws),
                self.step_ws.numel(), ctypes.byref(self.decoder._dims), _stream(stream))
            _lib.check(rc, "fleet_ffn_column")
            return
        for i in range(self.n_layers):
            self.layer_into(i, x, x, stream)

    def status(self) -> int:
        st = self.decoder.status() | self.dense.status()
        if self.fused:
            v = ctypes.c_uint32(0)
            _lib.check(_lib.load().fleet_decode_step_status(_ptr(self.step_ws), ctypes.byref(v),
                                                            None), "fleet_decode_step_status")
            st |= int(v.value)
        return st


class AttnDecoder:
    """Absorbed-MLA attention half of a layer, the embedding and lm_head +
    argmax (fleet_attn_decode / fleet_embed / fleet_lm_head_argmax), sharing
    one persistent workspace. Calls must be ordered on one stream."""

    def __init__(self, dims: MoeDims = DSV2_LITE, device="cuda"):
        self.dims = dims
        self._dims = c_dims(dims)
        n = _lib.load().fleet_attn_workspace_bytes(ctypes.byref(self._dims))
        self.workspace = torch.zeros(n, dtype=torch.uint8, device=device)

    def attn_into(self, layer: "_lib.FleetAttnLayer", x: torch.Tensor, x_out: torch.Tensor,
                  cache: torch.Tensor, pos: int = 0, pos_dev: torch.Tensor | None = None,
                  cos: torch.Tensor = None, sin: torch.Tensor = None, stream=None) -> None:
        """x_out = bf16(x + attention(x)) at position `pos` (or *pos_dev);
        cache: int16 [max_pos][576] of this layer."""
        rc = _lib.load().fleet_attn_decode(
            ctypes.byref(layer), _ptr(x), _ptr(x_out), _ptr(cache), int(cache.shape[0]),
            int(pos), _ptr(pos_dev), _ptr(cos), _ptr(sin), _ptr(self.workspace),
            self.workspace.numel(), ctypes.byref(self._dims), _stream(stream))
        _lib.check(rc, "fleet_attn_decode")

    def embed_into(self, embed_ptr: int, token: torch.Tensor, x: torch.Tensor, stream=None):
        rc = _lib.load().fleet_embed(embed_ptr, _ptr(token), _ptr(x), _ptr(self.workspace),
                                     self.workspace.numel(), _stream(stream))
        _lib.check(rc, "fleet_embed")

    def lm_head_into(self, x: torch.Tensor, final_norm_ptr: int | None, lm_head_ptr: int,
                     logits: torch.Tensor | None = None, token_out: torch.Tensor | None = None,
                     token_next: torch.Tensor | None = None,
                     pos_advance: torch.Tensor | None = None, stream=None) -> None:
        rc = _lib.load().fleet_lm_head_argmax(
            _ptr(x), final_norm_ptr, lm_head_ptr, _ptr(logits), _ptr(token_out),
            _ptr(token_next), _ptr(pos_advance), _ptr(self.workspace), self.workspace.numel(),
            ctypes.byref(self._dims), _stream(stream))
        _lib.check(rc, "fleet_lm_head_argmax")

    def status(self, stream=None) -> int:
        v = ctypes.c_uint32(0)
        rc = _lib.load().fleet_moe_workspace_status(_ptr(self.workspace), ctypes.byref(v),
                                                    _stream(stream))
        _lib.check(rc, "fleet_moe_workspace_status")
        return int(v.value)


class Decoder:
    """Batch-1 greedy decode of the whole model on the GPU.

    `blob` is the packed uint8 device tensor of `layout`
    (fleet_moe.layout.model_layout). Per token (reference_decode.py:294-302
    per layer, the launcher's step order fleet_kernel.hip:966-1040):
    x = embed[token]; for each layer x = bf16(x + attn(x)), then
    x = bf16(x + ffn(rms_norm(x))) (dense below first_k_dense, MoE above);
    token = argmax(bf16(lm_head . rms_norm(x))). The KV cache is
    [layers][max_pos][576] bf16. The token and the position live in device
    memory (`token`, `pos`), so one step can be captured in a HIP graph and
    replayed: the argmax writes the next token and advances the position.
    With `fused` (the default) a step is ONE launch (fleet_decode_step) that
    runs all of it; otherwise one launch per stage (embed, per layer
    attention and FFN, lm_head, argmax). The results are the same bit for
    bit."""

    def __init__(self, blob: torch.Tensor, layout: Layout, dims: MoeDims = DSV2_LITE,
                 max_pos: int = 4096, fused: bool = True):
        from .rope import RopeParams, yarn_tables
        self.blob, self.layout, self.dims = blob, layout, dims
        dev = blob.device
        self.n_layers = int(layout.scalars["layers"])
        self.max_pos = int(max_pos)
        cos, sin = yarn_tables(self.max_pos, RopeParams.from_scalars(layout.scalars))
        self.cos = torch.from_numpy(cos).to(dev)
        self.sin = torch.from_numpy(sin).to(dev)
        self.cache = torch.zeros((self.n_layers, self.max_pos, 576), dtype=torch.int16,
                                 device=dev)
        self.ffn = FfnColumn(blob, layout, dims, fused=False)
        self.attn = AttnDecoder(dims, device=dev)
        self.attn_layers = [self._attn_layer(i) for i in range(self.n_layers)]
        self.x = torch.zeros(dims.hidden, dtype=torch.float32, device=dev)
        self.token = torch.zeros(1, dtype=torch.int32, device=dev)      # input of the next step
        self.token_out = torch.zeros(1, dtype=torch.int32, device=dev)  # last pick
        self.pos = torch.zeros(1, dtype=torch.int32, device=dev)        # position of the next step
        self.graph = None
        self.fused = bool(fused)
        if self.fused:
            self._init_step()

    def _addr(self, name: str) -> int:
        return self.blob.data_ptr() + self.layout.tensors[name].offset

    def _attn_layer(self, i: int) -> _lib.FleetAttnLayer:
        return _lib.FleetAttnLayer(self._addr(f"L{i}.norm_in"), self._addr(f"L{i}.qkv"),
                                   self._addr(f"L{i}.kv_a_norm"), self._addr(f"L{i}.kv_b"),
                                   self._addr(f"L{i}.o_proj"))

    def layer_into(self, i: int, x: torch.Tensor, pos: int = 0, use_pos_dev: bool = False,
                   stream=None) -> None:
        """Layer i in place on x (attention half, then FFN half)."""
        self.attn.attn_into(self.attn_layers[i], x, x, self.cache[i], pos,
                            self.pos if use_pos_dev else None, self.cos, self.sin, stream)
        self.ffn.layer_into(i, x, x, stream)

    def _init_step(self) -> None:
        """The device layer table and the workspace of fleet_decode_step."""
        lib = _lib.load()
        rows = (_lib.FleetStepLayer * self.n_layers)()
        for i in range(self.n_layers):
            r = rows[i]
            r.attn = self.attn_layers[i]
            r.cache = self.cache[i].data_ptr()
            if i < self.ffn.first_k_dense:
                r.moe = _lib.FleetMoeLayer(self._addr(f"L{i}.norm_post"), None, None, 0, None)
                r.dense = self._addr(f"L{i}.dense")
            else:
                r.moe = self.ffn.moe[i].c_layer()
                r.dense = None
        raw = bytes(memoryview(rows).cast("B"))
        self.step_layers = torch.frombuffer(bytearray(raw), dtype=torch.uint8).to(self.blob.device)
        self.step_model = _lib.FleetStepModel(
            self.step_layers.data_ptr(), self.n_layers, self.max_pos, self._addr("embed"),
            self._addr("final_norm") if "final_norm" in self.layout.tensors else None,
            self._addr("lm_head"), self.cos.data_ptr(), self.sin.data_ptr())
        n = lib.fleet_decode_step_workspace_bytes(ctypes.byref(self.attn._dims))
        if n == 0:
            raise ValueError("fleet_decode_step does not support these model dims")
        self.step_ws = torch.zeros(n, dtype=torch.uint8, device=self.blob.device)

    def enqueue_step(self, logits: torch.Tensor | None = None, feed_back: bool = True,
                     stream=None) -> None:
        """One token from device state: embed(*token), every layer at *pos,
        lm_head + argmax -> token_out (and -> token when feed_back), *pos += 1.
        No allocation, no synchronisation: capturable."""
        if self.fused:
            rc = _lib.load().fleet_decode_step(
                ctypes.byref(self.step_model), _ptr(self.token), _ptr(self.token_out),
                _ptr(self.token) if feed_back else None, _ptr(self.pos), _ptr(self.x),
                _ptr(logits), _ptr(self.step_ws), self.step_ws.numel(),
                ctypes.byref(self.attn._dims), _stream(stream))
            _lib.check(rc, "fleet_decode_step")
            return
        self.attn.embed_into(self._addr("embed"), self.token, self.x, stream)
        for i in range(self.n_layers):
            self.layer_into(i, self.x, use_pos_dev=True, stream=stream)
        self.attn.lm_head_into(self.x, self._addr("final_norm"), self._addr("lm_head"), logits,
                               self.token_out, self.token if feed_back else None, self.pos,
                               stream)

    def reset(self, pos: int = 0) -> None:
        self.pos.fill_(int(pos))

    def capture(self) -> None:
        """Capture enqueue_step() into a HIP graph (replayed by step())."""
        s = torch.cuda.Stream(device=self.blob.device)
        s.wait_stream(torch.cuda.current_stream())
        g = torch.cuda.CUDAGraph()
        with torch.cuda.stream(s):
            with torch.cuda.graph(g, stream=s):
                self.enqueue_step(stream=s)
        torch.cuda.current_stream().wait_stream(s)
        self.graph = g

    def step(self) -> None:
        if self.graph is not None:
            self.graph.replay()
        else:
            self.enqueue_step()

    def prefill(self, tokens: torch.Tensor) -> None:
        """Teacher-forced steps over tokens (device int32 [n]) from position 0:
        fills the cache rows 0..n-1; after it token_out holds the pick after
        the last prompt token and pos == n."""
        self.reset(0)
        for i in range(tokens.numel()):
            self.token.copy_(tokens[i:i + 1])
            self.step()

    def generate(self, n: int) -> torch.Tensor:
        """n greedy tokens continuing from the state prefill() left: the first
        input is token_out. Returns the device int32 [n] of picks."""
        out = torch.empty(n, dtype=torch.int32, device=self.blob.device)
        self.token.copy_(self.token_out)
        for j in range(n):
            self.step()
            out[j:j + 1].copy_(self.token_out)
        return out

    def status(self) -> int:
        st = self.attn.status() | self.ffn.status()
        if self.fused:
            v = ctypes.c_uint32(0)
            _lib.check(_lib.load().fleet_decode_step_status(_ptr(self.step_ws), ctypes.byref(v),
                                                            None), "fleet_decode_step_status")
            st |= int(v.value)
        return st
