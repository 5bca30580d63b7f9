"""ctypes binding of libfleet_moe.so (declarations in include/fleet_moe.h).

The library is built in-tree by `fleet_moe._build.build()`; this module only
loads it. A missing library is an error, never a silent fallback.
"""
from __future__ import annotations

import ctypes
from ctypes import POINTER, c_char_p, c_float, c_int, c_int32, c_int64, c_size_t, c_uint32, c_void_p
from pathlib import Path

LIB_NAME = "libfleet_moe.so"

ERR_DIMS = 10001
ERR_ARG = 10002
ERR_WORKSPACE = 10003
ERR_DEVICE = 10004
ERR_CAPACITY = 10005
ERR_CAPTURE = 10006

NOALLOC_MAX_TOKENS = 64
NOALLOC_SCRATCH_BYTES = 7574528

ABORT_ROUTER_WAIT = 0x1
ABORT_UNIT_WAIT = 0x2
ABORT_GROUP_WAIT = 0x4
ABORT_POSITION = 0x8
ABORT_TOKEN = 0x10
ABORT_ATTN_WAIT = 0x20
ABORT_BAD_ID = 0x40
ABORT_STEP_WAIT = 0x80


class FleetMoeDims(ctypes.Structure):
    """struct fleet_moe_dims."""
    _fields_ = [("hidden", c_int32), ("moe_inter", c_int32), ("n_routed", c_int32),
                ("n_shared", c_int32), ("top_k", c_int32), ("routed_scaling", c_float),
                ("rms_eps", c_float)]


class FleetMoeLayer(ctypes.Structure):
    """struct fleet_moe_layer (device pointers)."""
    _fields_ = [("norm", c_void_p), ("router", c_void_p), ("experts", c_void_p),
                ("expert_stride", c_int64), ("shared", c_void_p)]


class FleetAttnLayer(ctypes.Structure):
    """struct fleet_attn_layer (device pointers)."""
    _fields_ = [("norm_in", c_void_p), ("qkv", c_void_p), ("kv_a_norm", c_void_p),
                ("kv_b", c_void_p), ("o_proj", c_void_p)]


class FleetStepLayer(ctypes.Structure):
    """struct fleet_step_layer (device pointers)."""
    _fields_ = [("attn", FleetAttnLayer), ("moe", FleetMoeLayer), ("dense", c_void_p),
                ("cache", c_void_p)]


class FleetStepModel(ctypes.Structure):
    """struct fleet_step_model (layers: a device array of FleetStepLayer)."""
    _fields_ = [("layers", c_void_p), ("n_layers", c_int32), ("max_pos", c_int32),
                ("embed", c_void_p), ("final_norm", c_void_p), ("lm_head", c_void_p),
                ("rope_cos", c_void_p), ("rope_sin", c_void_p)]


# (name, restype, argtypes) of every symbol the header declares.
SYMBOLS = [
    ("fleet_moe_router_topk", c_int,
     [c_void_p, c_void_p, c_int32, c_void_p, c_void_p, c_void_p, c_void_p,
      POINTER(FleetMoeDims), c_void_p]),
    ("fleet_moe_residual_fold", c_int,
     [c_void_p, c_void_p, c_int32, c_void_p, POINTER(FleetMoeDims), c_void_p]),
    ("fleet_moe_layer_workspace_bytes", c_size_t, [POINTER(FleetMoeDims)]),
    ("fleet_moe_layer_decode", c_int,
     [POINTER(FleetMoeLayer), c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
      c_size_t, POINTER(FleetMoeDims), c_void_p]),
    ("fleet_moe_dense_workspace_bytes", c_size_t, [POINTER(FleetMoeDims), c_int32]),
    ("fleet_moe_dense_decode", c_int,
     [c_void_p, c_void_p, c_int32, c_void_p, c_void_p, c_void_p, c_void_p, c_size_t,
      POINTER(FleetMoeDims), c_void_p]),
    ("fleet_moe_grouped_workspace_bytes", c_size_t, [POINTER(FleetMoeDims), c_int32]),
    ("fleet_moe_grouped", c_int,
     [POINTER(FleetMoeLayer), c_int32, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
      c_size_t, POINTER(FleetMoeDims), c_void_p]),
    ("fleet_moe_grouped_noalloc", c_int,
     [POINTER(FleetMoeLayer), c_int32, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
      POINTER(FleetMoeDims), c_void_p]),
    ("fleet_attn_workspace_bytes", c_size_t, [POINTER(FleetMoeDims)]),
    ("fleet_attn_decode", c_int,
     [POINTER(FleetAttnLayer), c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_void_p,
      c_void_p, c_void_p, c_void_p, c_size_t, POINTER(FleetMoeDims), c_void_p]),
    ("fleet_decode_step_workspace_bytes", c_size_t, [POINTER(FleetMoeDims)]),
    ("fleet_decode_step", c_int,
     [POINTER(FleetStepModel), c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
      c_void_p, c_size_t, POINTER(FleetMoeDims), c_void_p]),
    ("fleet_decode_step_status", c_int, [c_void_p, POINTER(ctypes.c_uint32), c_void_p]),
    ("fleet_ffn_column", c_int,
     [c_void_p, c_int32, c_void_p, c_void_p, c_void_p, c_size_t, POINTER(FleetMoeDims),
      c_void_p]),
    ("fleet_embed", c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_size_t, c_void_p]),
    ("fleet_lm_head_argmax", c_int,
     [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
      c_size_t, POINTER(FleetMoeDims), c_void_p]),
    ("fleet_moe_stream_read", c_int, [c_void_p, c_size_t, c_void_p, c_void_p]),
    ("fleet_moe_workspace_status", c_int, [c_void_p, POINTER(c_uint32), c_void_p]),
    ("fleet_moe_error_string", c_char_p, [c_int]),
    ("fleet_moe_abi_version", c_int, []),
]

_LIB = None


def lib_path() -> Path:
    return Path(__file__).resolve().with_name(LIB_NAME)


def load() -> ctypes.CDLL:
    """Load the library once and attach the prototypes. Raises if absent."""
    global _LIB
    if _LIB is not None:
        return _LIB
    p = lib_path()
    if not p.exists():
        raise RuntimeError(f"{p} is not built: run `python -c 'import __graft_entry__ as g; "
                           "g.build()'` from the repository root")
    lib = ctypes.CDLL(str(p))
    for name, res, args in SYMBOLS:
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _LIB = lib
    return lib


class FleetMoeError(RuntimeError):
    def __init__(self, code: int, what: str):
        self.code = code
        msg = load().fleet_moe_error_string(code)
        super().__init__(f"{what}: {msg.decode() if msg else code} (code {code})")


def check(code: int, what: str) -> None:
    if code != 0:
        raise FleetMoeError(code, what)
