"""The C-ABI library: it loads, exports every symbol include/fleet_moe.h
declares, and rejects bad arguments before touching a device (CPU-only)."""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from fleet_moe import _lib
from fleet_moe.layout import DSV2_LITE, MoeDims
from fleet_moe.ops import c_dims

HEADER = Path(__file__).resolve().parents[1] / "include" / "fleet_moe.h"


def declared_functions() -> set[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return set(re.findall(r"\b(fleet_\w+)\s*\(", text))


@pytest.fixture(scope="module")
def lib():
    return _lib.load()


def test_every_declared_symbol_is_exported_and_bound(lib):
    decl = declared_functions()
    assert decl, "no declarations parsed"
    bound = {name for name, _, _ in _lib.SYMBOLS}
    assert decl == bound, f"header vs binding: {sorted(decl ^ bound)}"
    for name in decl:
        assert getattr(lib, name) is not None


def test_struct_layouts_match_header():
    # fleet_moe_dims: 5 int32 + 2 float; fleet_moe_layer: 4 pointers + int64
    assert ctypes.sizeof(_lib.FleetMoeDims) == 28
    assert ctypes.sizeof(_lib.FleetMoeLayer) == 40
    assert _lib.FleetMoeLayer.expert_stride.offset == 24
    # fleet_attn_layer: 5 pointers
    assert ctypes.sizeof(_lib.FleetAttnLayer) == 40


def test_version_and_error_strings(lib):
    assert lib.fleet_moe_abi_version() == 101
    assert b"shape" in lib.fleet_moe_error_string(_lib.ERR_DIMS)
    assert b"workspace" in lib.fleet_moe_error_string(_lib.ERR_WORKSPACE)
    assert lib.fleet_moe_error_string(0) == b"success"


def test_workspace_sizes(lib):
    d = c_dims(DSV2_LITE)
    n = lib.fleet_moe_layer_workspace_bytes(ctypes.byref(d))
    assert n % 256 == 0 and 16_384 <= n <= 1 << 20
    g64 = lib.fleet_moe_grouped_workspace_bytes(ctypes.byref(d), 64)
    g16 = lib.fleet_moe_grouped_workspace_bytes(ctypes.byref(d), 16)
    assert g64 > g16 > 0
    assert lib.fleet_moe_grouped_workspace_bytes(ctypes.byref(d), 0) == 0
    assert lib.fleet_moe_grouped_workspace_bytes(ctypes.byref(d), 100_000) == 0


def test_bad_dims_rejected_without_device(lib):
    bad = c_dims(MoeDims(hidden=4096))
    layer = _lib.FleetMoeLayer(None, 16, 16, DSV2_LITE.expert_stride, 16)
    rc = lib.fleet_moe_layer_decode(ctypes.byref(layer), 16, 16, None, None, None, 256, 1 << 20,
                                    ctypes.byref(bad), None)
    assert rc == _lib.ERR_DIMS
    rc = lib.fleet_moe_router_topk(16, 16, 1, None, None, 16, 16, ctypes.byref(bad), None)
    assert rc == _lib.ERR_DIMS
    rc = lib.fleet_moe_grouped(ctypes.byref(layer), 4, 16, 16, 16, 16, 256, 1 << 24,
                               ctypes.byref(bad), None)
    assert rc == _lib.ERR_DIMS
    topk = c_dims(MoeDims(top_k=8))
    assert lib.fleet_moe_router_topk(16, 16, 1, None, None, 16, 16, ctypes.byref(topk), None) == _lib.ERR_DIMS


def test_bad_pointers_rejected_without_device(lib):
    d = c_dims(DSV2_LITE)
    layer = _lib.FleetMoeLayer(None, 256, 256, DSV2_LITE.expert_stride, 256)
    # null x
    assert lib.fleet_moe_layer_decode(ctypes.byref(layer), None, 256, None, None, None, 256,
                                      1 << 20, ctypes.byref(d), None) == _lib.ERR_ARG
    # misaligned experts base
    mis = _lib.FleetMoeLayer(None, 256, 258, DSV2_LITE.expert_stride, 256)
    assert lib.fleet_moe_layer_decode(ctypes.byref(mis), 256, 256, None, None, None, 256,
                                      1 << 20, ctypes.byref(d), None) == _lib.ERR_ARG
    # stride smaller than one expert
    short = _lib.FleetMoeLayer(None, 256, 256, DSV2_LITE.expert_stride - 8, 256)
    assert lib.fleet_moe_layer_decode(ctypes.byref(short), 256, 256, None, None, None, 256,
                                      1 << 20, ctypes.byref(d), None) == _lib.ERR_DIMS
    # workspace too small
    assert lib.fleet_moe_layer_decode(ctypes.byref(layer), 256, 256, None, None, None, 256,
                                      64, ctypes.byref(d), None) == _lib.ERR_WORKSPACE
    # token counts out of range
    assert lib.fleet_moe_router_topk(256, 256, 0, None, None, 256, 256, ctypes.byref(d), None) == _lib.ERR_ARG
    assert lib.fleet_moe_grouped(ctypes.byref(layer), 0, 256, 256, 256, 256, 256, 1 << 26,
                                 ctypes.byref(d), None) == _lib.ERR_ARG
    assert lib.fleet_moe_grouped(ctypes.byref(layer), 300, 256, 256, 256, 256, 256, 1 << 26,
                                 ctypes.byref(d), None) == _lib.ERR_ARG
    small = lib.fleet_moe_grouped_workspace_bytes(ctypes.byref(d), 4)
    assert lib.fleet_moe_grouped(ctypes.byref(layer), 8, 256, 256, 256, 256, 256, small,
                                 ctypes.byref(d), None) == _lib.ERR_WORKSPACE
    assert lib.fleet_moe_workspace_status(None, None, None) == _lib.ERR_ARG


def test_noalloc_grouped_rejects_bad_arguments_without_device(lib):
    d = c_dims(DSV2_LITE)
    layer = _lib.FleetMoeLayer(None, 256, 256, DSV2_LITE.expert_stride, 256)
    n = _lib.NOALLOC_MAX_TOKENS
    # the stated capacity and the scratch size match the workspace layout
    assert lib.fleet_moe_grouped_workspace_bytes(ctypes.byref(d), n) == _lib.NOALLOC_SCRATCH_BYTES
    call = lambda T, status=256: lib.fleet_moe_grouped_noalloc(  # noqa: E731
        ctypes.byref(layer), T, 256, 256, 256, 256, status, ctypes.byref(d), None)
    assert call(n + 1) == _lib.ERR_CAPACITY          # beyond the static scratch
    assert call(4, status=None) == _lib.ERR_ARG      # the status output is required
    assert call(4, status=258) == _lib.ERR_ARG       # misaligned status
    assert call(0) == _lib.ERR_ARG
    bad = c_dims(MoeDims(top_k=8))
    assert lib.fleet_moe_grouped_noalloc(ctypes.byref(layer), 4, 256, 256, 256, 256, 256,
                                         ctypes.byref(bad), None) == _lib.ERR_DIMS
    for code in (_lib.ERR_CAPACITY, _lib.ERR_CAPTURE):
        assert b"no-allocation" in lib.fleet_moe_error_string(code)


def test_attention_entry_points_reject_bad_arguments_without_device(lib):
    d = c_dims(DSV2_LITE)
    n = lib.fleet_attn_workspace_bytes(ctypes.byref(d))
    assert n % 256 == 0 and (1 << 20) < n < (8 << 20)
    assert lib.fleet_attn_workspace_bytes(ctypes.byref(c_dims(MoeDims(hidden=4096)))) == 0
    layer = _lib.FleetAttnLayer(256, 256, 256, 256, 256)
    args = dict(x=256, x_out=256, cache=256, max_pos=128, pos=0, pos_dev=None, cos=256, sin=256,
                ws=256, ws_bytes=n)

    def call(layer_=layer, dims=d, **kw):
        a = {**args, **kw}
        return lib.fleet_attn_decode(ctypes.byref(layer_), a["x"], a["x_out"], a["cache"],
                                     a["max_pos"], a["pos"], a["pos_dev"], a["cos"], a["sin"],
                                     a["ws"], a["ws_bytes"], ctypes.byref(dims), None)

    assert call(x=None) == _lib.ERR_ARG
    assert call(pos=128) == _lib.ERR_ARG                 # host position past max_pos
    assert call(pos=-1) == _lib.ERR_ARG
    assert call(max_pos=4097) == _lib.ERR_ARG            # beyond the cache the kernels index
    assert call(cache=258) == _lib.ERR_ARG               # misaligned
    assert call(layer_=_lib.FleetAttnLayer(256, None, 256, 256, 256)) == _lib.ERR_ARG
    assert call(ws_bytes=n - 256) == _lib.ERR_WORKSPACE
    assert call(dims=c_dims(MoeDims(moe_inter=1024))) == _lib.ERR_DIMS
    assert lib.fleet_embed(None, 256, 256, 256, n, None) == _lib.ERR_ARG
    assert lib.fleet_embed(256, 256, 256, 256, 64, None) == _lib.ERR_WORKSPACE
    assert lib.fleet_lm_head_argmax(256, None, None, None, None, None, None, 256, n,
                                    ctypes.byref(d), None) == _lib.ERR_ARG
    assert lib.fleet_lm_head_argmax(256, None, 256, None, 258, None, None, 256, n,
                                    ctypes.byref(d), None) == _lib.ERR_ARG


def test_trace_build_exports_the_library_and_its_trace_hooks():
    """The stage-trace build (a diagnostic variant of the same sources) binds
    like the library and adds only its three trace hooks; the library itself
    has none of them."""
    from fleet_moe import _build, stage_trace
    if not stage_trace.TRACE_LIB.exists():
        pytest.skip("trace build not made (python -m fleet_moe._build --trace)")
    prev = _lib._LIB
    try:
        tl = stage_trace.load()
        for name, _, _ in _lib.SYMBOLS:
            assert getattr(tl, name) is not None
    finally:
        _lib._LIB = prev
    lib = _lib.load()
    for hook in ("fleet_step_debug_set_trace", "fleet_moe_debug_set_trace",
                 "fleet_attn_debug_set_trace"):
        assert getattr(tl, hook) is not None
        assert not hasattr(lib, hook), hook
    assert _build.TRACE_OUT != _build.OUT
