"""Stage traces of the library's one-launch kernels (a diagnostic build).

The trace build, libfleet_moe_trace.so (``python -m fleet_moe._build --trace``,
also made by ``__graft_entry__.build()``), is the library's own sources
compiled with FLEET_ATTN_TRACE, FLEET_MOE_TRACE and FLEET_STEP_TRACE: at
fixed points of a stage, lane 0 of every wave (or thread 0 of every
workgroup, for the whole-step kernel's stage ends) stores the 100 MHz
``s_memrealtime`` counter into a buffer that a ``*_debug_set_trace`` entry
point of that build hands to the next launch. This module runs one kernel of
that build on seeded synthetic weights and prints when the stamps land:

  python -m fleet_moe.stage_trace step     # decode step, one launch: stage timeline,
                                           # and one layer's attention and MoE stages
  python -m fleet_moe.stage_trace column   # FFN column, one launch
  python -m fleet_moe.stage_trace moe      # one MoE layer per launch
  python -m fleet_moe.stage_trace attn     # one attention layer per launch

The stamps cost a few percent; the traced times locate latency, bench.py's
figures are the library's. Nothing else loads this build.
"""
from __future__ import annotations

import argparse
import ctypes
from pathlib import Path

import numpy as np

from . import _lib

TRACE_LIB = Path(__file__).resolve().parent / "libfleet_moe_trace.so"

# the marks of each stage body (the k of ATTN_TRACE(k) / FLEET_TRACE(k))
ATTN_MARKS = [
    (0, "start"), (1, "x in"), (2, "x normed"), (3, "S1 published, S2/S3 loads out"),
    (4, "S2 q_nope polled"), (5, "S2 q_c published"), (6, "S3 inputs polled"),
    (7, "S3 row of pos ready"), (8, "S3 scores done"), (9, "S3 partials published"),
    (10, "S4 partials polled"), (11, "S4 o_c published"), (12, "S4 o_c polled"),
    (13, "S4 head outputs published"), (14, "S5 head outputs polled"), (15, "end"),
]
MOE_MARKS = [
    (0, "first loads issued"), (1, "x normed"), (10, "routed (control wave)"),
    (8, "exact router row published"), (2, "phase G starts"), (3, "phase G done"),
    (4, "down rows issued / shared rows in LDS"), (9, "exact weights (control wave)"),
    (5, "h ready"), (6, "down dots done"), (7, "end"),
]


def load() -> ctypes.CDLL:
    """The trace build, bound like the library (and made the one `_lib` uses)."""
    if not TRACE_LIB.exists():
        raise RuntimeError(f"{TRACE_LIB} is not built: python -m fleet_moe._build --trace")
    lib = ctypes.CDLL(str(TRACE_LIB))
    for name, res, args in _lib.SYMBOLS:
        f = getattr(lib, name)
        f.restype, f.argtypes = res, args
    lib.fleet_step_debug_set_trace.argtypes = [ctypes.c_void_p] * 3 + [ctypes.c_int]
    lib.fleet_moe_debug_set_trace.argtypes = [ctypes.c_void_p]
    lib.fleet_attn_debug_set_trace.argtypes = [ctypes.c_void_p]
    _lib._LIB = lib
    return lib


def wave_marks(buf, marks, t_ref, label):
    """Per mark: median / p90 / max over the waves that stamped it, in us
    after t_ref (a raw stamp)."""
    a = buf.view(256, 8, 16).cpu().numpy().astype(np.int64)
    print(f"  {label} (us after the reference point; median / p90 / max over waves)")
    for k, name in marks:
        v = a[:, :, k]
        v = v[v > 0]
        if v.size == 0:
            continue
        d = (v - t_ref) / 100.0
        print(f"    {k:2d} {name:38s} {np.median(d):7.2f} {np.percentile(d, 90):7.2f} "
              f"{d.max():7.2f}")


def _timed(torch, fn, n):
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for i in range(n):
        fn(i)
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) * 1e3 / n


def run_step(torch, lib, n_layers, pos, layer, reps):
    from . import ops, synth_gpu, layout as lay_mod
    from .layout import DSV2_LITE as dims
    lay = lay_mod.model_layout(dims, n_layers=n_layers)
    blob = torch.empty(lay.nbytes, dtype=torch.uint8, device="cuda")
    synth_gpu.fill_model(blob, lay, seed=7)
    dec = ops.Decoder(blob, lay, dims, max_pos=pos + 64, fused=True)
    g = torch.Generator(device="cuda").manual_seed(0)
    dec.cache[:, :pos] = torch.randn((n_layers, pos, lay_mod.KV_LORA + lay_mod.QK_ROPE),
                                     generator=g, device="cuda").to(torch.bfloat16).view(torch.int16)
    ns = 2 * n_layers + 2
    ts = torch.zeros(ns * 256, dtype=torch.int64, device="cuda")
    ta = torch.zeros(256 * 8 * 16, dtype=torch.int64, device="cuda")
    tm = torch.zeros(256 * 8 * 16, dtype=torch.int64, device="cuda")
    dec.reset(pos)
    dec.token.fill_(7)
    for _ in range(4):
        dec.enqueue_step()
    dec.reset(pos)
    us = _timed(torch, lambda i: dec.enqueue_step(), 16)
    print(f"decode step, {n_layers} layers, position {pos}: {us:.1f} us per step "
          f"(trace build, eager launches)")
    durs, tot, keep = [], [], None
    for r in range(reps):
        dec.reset(pos)
        for _ in range(3):
            dec.enqueue_step()
        ts.zero_(); ta.zero_(); tm.zero_()
        lib.fleet_step_debug_set_trace(ts.data_ptr(), ta.data_ptr(), tm.data_ptr(), layer)
        dec.enqueue_step()
        lib.fleet_step_debug_set_trace(None, None, None, -1)
        torch.cuda.synchronize()
        if dec.status() != 0:
            raise RuntimeError(f"status {dec.status():#x}")
        S = ts.view(ns, 256).cpu().numpy().astype(np.int64)
        t0 = S[0].min()
        T = (S - t0) / 100.0
        durs.append(np.diff(np.median(T, axis=1)))
        tot.append(T[-1].max())
        keep = (t0, T)
    D = np.median(np.array(durs), axis=0)
    attn = D[0:2 * n_layers:2]
    ffn = D[1:2 * n_layers:2]
    print(f"  stage durations, median over {reps} steps of (median workgroup end - previous "
          f"median end), us:")
    print(f"    attention {np.median(attn):.2f} (layers: min {attn.min():.2f}, max {attn.max():.2f})")
    print(f"    dense FFN (layer 0) {ffn[0]:.2f}")
    print(f"    MoE FFN {np.median(ffn[1:]):.2f} (min {ffn[1:].min():.2f}, max {ffn[1:].max():.2f})")
    print(f"    lm_head + argmax {D[-1]:.2f}")
    print(f"    whole step (last workgroup's end) {np.median(tot):.1f}")
    t0, T = keep
    start = t0 + int(round(np.median(T[2 * layer]) * 100))
    wave_marks(ta, ATTN_MARKS, start, f"layer {layer} attention stage, last step, after the "
                                      f"previous stage's median end")
    start = t0 + int(round(np.median(T[2 * layer + 1]) * 100))
    wave_marks(tm, MOE_MARKS, start, f"layer {layer} MoE stage, last step, after the attention "
                                     f"stage's median end")


def run_column(torch, lib, n_layers, layer, reps):
    from . import ops, synth_gpu, layout as lay_mod
    from .layout import DSV2_LITE as dims
    lay = lay_mod.model_layout(dims, n_layers=n_layers)
    blob = torch.empty(lay.nbytes, dtype=torch.uint8, device="cuda")
    synth_gpu.fill_model(blob, lay, seed=7)
    col = ops.FfnColumn(blob, lay, dims, fused=True)
    g = torch.Generator(device="cuda").manual_seed(0)
    xs = [torch.randn(dims.hidden, generator=g, device="cuda").to(torch.bfloat16).float()
          for _ in range(8)]
    for t in range(4):
        col.run_into(xs[t])
    us = _timed(torch, lambda i: col.run_into(xs[i % 8]), 16)
    print(f"FFN column, {n_layers} layers: {us:.1f} us per token (trace build)")
    ns = n_layers + 2
    ts = torch.zeros(ns * 256, dtype=torch.int64, device="cuda")
    tm = torch.zeros(256 * 8 * 16, dtype=torch.int64, device="cuda")
    durs, tot, keep = [], [], None
    for r in range(reps):
        ts.zero_(); tm.zero_()
        lib.fleet_step_debug_set_trace(ts.data_ptr(), None, tm.data_ptr(), layer)
        col.run_into(xs[r % 8])
        lib.fleet_step_debug_set_trace(None, None, None, -1)
        torch.cuda.synchronize()
        S = ts.view(ns, 256).cpu().numpy().astype(np.int64)[: n_layers + 1]
        t0 = S[0].min()
        T = (S - t0) / 100.0
        durs.append(np.diff(np.median(T, axis=1)))
        tot.append(T[-1].max())
        keep = (t0, T)
    D = np.median(np.array(durs), axis=0)
    print(f"  stage durations, median over {reps} tokens, us: dense {D[0]:.2f}, MoE "
          f"{np.median(D[1:]):.2f} (min {D[1:].min():.2f}, max {D[1:].max():.2f}); "
          f"whole column {np.median(tot):.1f}")
    t0, T = keep
    start = t0 + int(round(np.median(T[layer]) * 100))
    wave_marks(tm, MOE_MARKS, start, f"layer {layer} MoE stage, last token, after the previous "
                                     f"stage's median end")


def run_moe(torch, lib, reps):
    from . import ops, synth
    from .layout import DSV2_LITE as dims
    blob, lay = synth.moe_layer_blob(seed=0, layer=1, dims=dims)
    ml = ops.DeviceLayer.from_host(blob, lay, 1, dims, device="cuda")
    md = ops.LayerDecoder(dims, device="cuda")
    xs = torch.from_numpy(synth.hidden_inputs(0, 64, dims.hidden)).cuda()
    y = torch.empty_like(xs[0])
    for t in range(20):
        md.decode_into(ml, xs[t % 64], y)
    us = _timed(torch, lambda i: md.decode_into(ml, xs[i % 64], y), 200)
    print(f"MoE layer per launch: {us:.2f} us per launch (trace build, one layer back to back)")
    tr = torch.zeros(256 * 8 * 16, dtype=torch.int64, device="cuda")
    acc = []
    for r in range(reps):
        tr.zero_()
        lib.fleet_moe_debug_set_trace(tr.data_ptr())
        md.decode_into(ml, xs[r], y)
        torch.cuda.synchronize()
        lib.fleet_moe_debug_set_trace(None)
        acc.append(tr.clone())
    if md.status() != 0:
        raise RuntimeError(f"status {md.status():#x}")
    _marks_over_reps(acc, MOE_MARKS, f"{reps} launches, after each launch's first stamp")


def run_attn(torch, lib, pos, reps):
    from . import ops, rope
    from . import layout as L
    from .layout import DSV2_LITE as dims
    g = torch.Generator(device="cuda").manual_seed(0)

    def rnd(shape, s=0.02):
        return (torch.randn(shape, generator=g, device="cuda") * s).to(torch.bfloat16).view(
            torch.int16)
    h, lora, rope_d = dims.hidden, L.KV_LORA, L.QK_ROPE
    w = {"norm_in": rnd(h, 0.1), "qkv": rnd((L.QKV_ROWS, h)), "kv_a_norm": rnd(lora, 0.1),
         "kv_b": rnd((L.ATTN_HEADS * (L.QK_NOPE + L.V_HEAD), lora)),
         "o_proj": rnd((h, L.ATTN_HEADS * L.V_HEAD))}
    layer = _lib.FleetAttnLayer(*(w[k].data_ptr() for k in ("norm_in", "qkv", "kv_a_norm",
                                                          "kv_b", "o_proj")))
    cos, sin = rope.yarn_tables(pos + 64)
    cos_d, sin_d = torch.from_numpy(cos).cuda(), torch.from_numpy(sin).cuda()
    cache = rnd((pos + 64, lora + rope_d), 1.0)
    dec = ops.AttnDecoder(dims)
    x = torch.randn(h, generator=g, device="cuda").to(torch.bfloat16).float()
    y = torch.empty_like(x)
    for _ in range(5):
        dec.attn_into(layer, x, y, cache, pos, None, cos_d, sin_d)
    us = _timed(torch, lambda i: dec.attn_into(layer, x, y, cache, pos, None, cos_d, sin_d), 50)
    print(f"attention layer per launch, position {pos}: {us:.2f} us per launch (trace build, "
          f"one layer back to back)")
    tr = torch.zeros(256 * 8 * 16, dtype=torch.int64, device="cuda")
    acc = []
    for r in range(reps):
        tr.zero_()
        lib.fleet_attn_debug_set_trace(tr.data_ptr())
        dec.attn_into(layer, x, y, cache, pos, None, cos_d, sin_d)
        torch.cuda.synchronize()
        lib.fleet_attn_debug_set_trace(None)
        acc.append(tr.clone())
    if dec.status() != 0:
        raise RuntimeError(f"status {dec.status():#x}")
    _marks_over_reps(acc, ATTN_MARKS, f"{reps} launches, after each launch's first stamp")


def _marks_over_reps(acc, marks, label):
    vals = {}
    for tr in acc:
        a = tr.view(256, 8, 16).cpu().numpy().astype(np.int64)
        t0 = a[:, :, 0][a[:, :, 0] > 0].min()
        for k, _ in marks:
            v = a[:, :, k]
            v = v[v > 0]
            if v.size:
                vals.setdefault(k, []).append((v - t0) / 100.0)
    print(f"  {label} (us; median / p90 / max over waves)")
    for k, name in marks:
        if k in vals:
            d = np.concatenate(vals[k])
            print(f"    {k:2d} {name:38s} {np.median(d):7.2f} {np.percentile(d, 90):7.2f} "
                  f"{d.max():7.2f}")


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("what", choices=["step", "column", "moe", "attn"])
    ap.add_argument("--layers", type=int, default=27)
    ap.add_argument("--pos", type=int, default=1024)
    ap.add_argument("--layer", type=int, default=5, help="the layer whose stages are detailed")
    ap.add_argument("--reps", type=int, default=5)
    args = ap.parse_args(argv)
    import torch
    if not torch.cuda.is_available():
        raise RuntimeError("stage_trace needs a GPU")
    lib = load()
    if args.what == "step":
        run_step(torch, lib, args.layers, args.pos, args.layer, args.reps)
    elif args.what == "column":
        run_column(torch, lib, args.layers, args.layer, args.reps)
    elif args.what == "moe":
        run_moe(torch, lib, args.reps)
    else:
        run_attn(torch, lib, args.pos, args.reps)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
