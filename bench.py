#!/usr/bin/env python3
"""Benchmark of the batch-1 DeepSeek-V2-Lite MoE decode path on one MI355X.

A step is one token through one MoE layer (RMSNorm, router, top-6, six
routed SwiGLU experts, the shared expert, the weighted combine and the
residual add): seeded N(0,1) hidden vectors rounded to
bf16, processed one token at a time, weights N(0, 0.02^2) in bf16 in the
reference's packed layout, all resident in HBM before timing starts.

Prints ONE JSON line. `value` is the median us per MoE layer over batches of
back-to-back launches timed with HIP events on the launch stream;
`roofline.achieved` is the selected-expert bytes (138,412,032 B per token)
divided by the kernel's own average duration (an event pair around each of a
series of launches). `cpu_baseline` times the CPU oracle on a bounded sample
of the same tokens (rank 0, N=1). The grouped multi-token step (config 2) is
reported under `grouped`.

    python bench.py [--steps 1000] [--warmup 20] [--gpus 1]
"""
from __future__ import annotations

import argparse
import ctypes
import hashlib
import json
import os
import platform
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "fleet-mi300x_amd"))

HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0
METRIC = "batch-1 MoE layer µs + HBM GB/s (% of 8 TB/s); full decode ms/token"


def parse_args():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1000, help="tokens timed (one layer each)")
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--batch", type=int, default=50, help="tokens per event-timed batch")
    ap.add_argument("--cpu-seconds", type=float, default=15.0, help="CPU baseline budget")
    ap.add_argument("--cpu-tokens", type=int, default=1000,
                    help="tokens in the CPU baseline's sample (config 1's first N, whatever "
                         "--steps is), cut short by --cpu-seconds")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-grouped", action="store_true")
    ap.add_argument("--no-cold", action="store_true",
                    help="skip the cold-cache runs (config 1 and the grouped step cycling "
                         "over 4 distinct MoE layers, 4.7 GB of weights)")
    ap.add_argument("--no-column", action="store_true",
                    help="skip config 3 (27-layer FFN column, 29.8 GB of weights)")
    ap.add_argument("--no-decode", action="store_true",
                    help="skip config 4 (27-layer full decode, 31.4 GB of weights)")
    ap.add_argument("--no-attention", action="store_true",
                    help="skip the attention-layer and lm_head legs (config 4's kernels alone)")
    ap.add_argument("--calibrate", action="store_true",
                    help="also run the known-size kernels that scale rocprofv3 FETCH_SIZE / "
                         "WRITE_SIZE: fleet_moe_stream_read over 256 MiB and a 64 MiB fill, "
                         "3 launches each")
    return ap.parse_args()


COUNTERS = ROOT / "profiles" / "kernel_counters.json"


def csrc_digest() -> str:
    """First 16 hex digits of the SHA-256 over the device sources (every file
    of fleet-mi300x_amd/csrc and include/fleet_moe.h, by name and content):
    the counter file records the digest of the sources it was measured on."""
    h = hashlib.sha256()
    files = sorted((ROOT / "fleet-mi300x_amd" / "csrc").iterdir()) + [ROOT / "include" / "fleet_moe.h"]
    for f in files:
        if f.is_file():
            h.update(f.name.encode() + b"\0" + f.read_bytes() + b"\0")
    return h.hexdigest()[:16]


def load_counter_file() -> dict:
    try:
        return json.loads(COUNTERS.read_text())
    except (OSError, ValueError):
        return {}


def load_counters() -> dict:
    """Per-leg HBM bytes and MFMA busy cycles per launch or step, from the
    committed rocprofv3 counter passes (FETCH_SIZE / WRITE_SIZE calibrated
    against known-size kernels, SQ_VALU_MFMA_BUSY_CYCLES)."""
    return load_counter_file().get("kernels", {})


def counters_source() -> dict:
    """Which sources the committed counters were measured on, and whether
    they are the sources of this run."""
    meas = load_counter_file().get("csrc_sha16")
    cur = csrc_digest()
    return {"file": "profiles/kernel_counters.json", "measured_csrc_sha16": meas,
            "current_csrc_sha16": cur, "matches_current_sources": meas == cur}


def counter_view(result: dict, profiled: dict) -> dict:
    """The profiled bytes (and MFMA busy cycles) of each leg over this run's
    own time for it: counter-derived GB/s and MFMA busy fraction."""
    def get(*path):
        v = result
        for p in path:
            if not isinstance(v, dict) or p not in v:
                return None
            v = v[p]
        return v

    col = get("ffn_column", "us_per_token")
    dense = get("ffn_column", "dense_layer", "us")
    times = {
        "moe_layer": get("roofline", "kernel_us_mean"),
        "moe_layer_cold": get("cold", "us_per_layer"),
        "attention": get("attention", "us_cold"),
        "lm_head": get("attention", "lm_head", "us"),
        "dense": dense,
        "moe_layer_in_column": (col - dense) / 26 if col and dense else None,
        "column": col,
        "decode_step": (get("full_decode", "ms_per_token") or 0) * 1e3 or None,
    }
    for t in ("T4", "T16", "T64"):
        times[f"grouped_{t}"] = get("grouped", t, "us_per_step")
        times[f"grouped_{t}_cold"] = get("cold", "grouped", t, "us_per_step")
    out = {"source": "profiles/kernel_counters.json"}
    for name, us in times.items():
        p = profiled.get(name)
        if not p or not us:
            continue
        e = {"hbm_bytes": p["hbm_bytes"], "traffic_over_algorithmic": p["traffic_over_algorithmic"],
             "us": round(us, 3), "counter_gbs": round(p["hbm_bytes"] / (us * 1e-6) / 1e9, 1),
             "counter_frac": round(p["hbm_bytes"] / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
        if "mfma_busy_cycles" in p:
            e["mfma_busy_frac"] = round(p["mfma_busy_cycles"] / (1024 * us * 1e-6 * 2.4e9), 5)
        out[name] = e
    return out


def progress(msg: str) -> None:
    """One line per finished leg on stderr (stdout carries only the JSON line)."""
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def cpu_baseline(blob, lay, x_tok: np.ndarray, budget_s: float, gpu_ids: np.ndarray):
    """The reference's NumPy MoE layer per token on the host cores: the
    oracle's fp32 restatement of reference_decode.py's arithmetic
    (moe_layer_fp32; fp32 BLAS GEMVs, experts pre-widened to fp32 outside the
    timed region, as reference_decode's LayerWeights are)."""
    sys.path.insert(0, str(ROOT))
    from fleet_moe.layout import view_u16
    from oracle import moe_oracle as orc
    t = lay.tensors
    pl = orc.PackedLayer(router=view_u16(blob, t["L1.router"]), experts=view_u16(blob, t["L1.experts"]),
                         shared=view_u16(blob, t["L1.shared"]), expert_stride=orc.HIDDEN * orc.MOE_INTER * 3,
                         norm=view_u16(blob, t["L1.norm_post"]))
    pl.widen()
    for i in range(3):                               # warm-up calls (BLAS threads start)
        orc.moe_layer_fp32(pl, x_tok[i % x_tok.shape[0]])
    times, n_match = [], 0
    t_end = time.perf_counter() + budget_s
    for i in range(x_tok.shape[0]):
        t0 = time.perf_counter_ns()
        r = orc.moe_layer_fp32(pl, x_tok[i])
        times.append((time.perf_counter_ns() - t0) / 1e3)
        n_match += int(np.array_equal(r["ids"], gpu_ids[i]))
        if time.perf_counter() > t_end:
            break
    cores = len(os.sched_getaffinity(0))
    cpu_model = platform.processor() or "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu_model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {
        "value": float(np.median(times)), "unit": "us/layer", "cores": cores, "kind": "port",
        "tokens": len(times), "p10": round(float(np.percentile(times, 10)), 1),
        "p90": round(float(np.percentile(times, 90)), 1),
        "sample": f"{len(times)} of config 1's seeded tokens, one MoE layer each "
                  f"(oracle/moe_oracle.moe_layer_fp32: reference_decode.py's fp32 NumPy "
                  f"arithmetic, NumPy {np.__version__}, BLAS threads = "
                  f"{cores} visible cores, {cpu_model})",
        "ids_match_gpu": f"{n_match}/{len(times)}",
    }


def main() -> int:
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported "
              "(the MoE decode path runs on one GPU; across GPUs its experts would shard "
              "by id, with one all-to-all of the 4 KB hidden vector each way per layer)",
              file=sys.stderr)
        return 2
    import torch
    from fleet_moe import _lib, ops, synth
    from fleet_moe.layout import DSV2_LITE

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    dims = DSV2_LITE
    bytes_layer = 6 * 3 * dims.hidden * dims.moe_inter * 2 + 3 * dims.hidden * dims.shared_inter * 2

    blob, lay = synth.moe_layer_blob(seed=0, layer=1, dims=dims)
    layer = ops.DeviceLayer.from_host(blob, lay, 1, dims, device=dev)
    n_tok = max(args.steps, 1)
    n_cpu = 0 if args.no_cpu else max(args.cpu_tokens, 1)
    x_host = bf16_tokens(synth, max(n_tok, args.warmup, n_cpu))
    xd = torch.from_numpy(x_host).to(dev)
    outs = torch.empty_like(xd)
    ids = torch.empty((xd.shape[0], dims.top_k), dtype=torch.int32, device=dev)
    wts = torch.empty((xd.shape[0], dims.top_k), dtype=torch.float32, device=dev)
    dec = ops.LayerDecoder(dims, device=dev)

    lib = _lib.load()
    cl = layer.c_layer()
    cd = ops.c_dims(dims)
    stream = torch.cuda.current_stream(dev)
    sh = int(stream.cuda_stream)
    ws_ptr, ws_n = dec.workspace.data_ptr(), dec.workspace.numel()
    row = xd.shape[1] * 4
    xb, ob, ib, wb = xd.data_ptr(), outs.data_ptr(), ids.data_ptr(), wts.data_ptr()
    fn = lib.fleet_moe_layer_decode
    byref = ctypes.byref

    def launch(t: int) -> None:
        rc = fn(byref(cl), xb + t * row, ob + t * row, None, ib + t * 24, wb + t * 24,
                ws_ptr, ws_n, byref(cd), sh)
        if rc:
            _lib.check(rc, "fleet_moe_layer_decode")

    for t in range(args.warmup):
        launch(t % xd.shape[0])
    torch.cuda.synchronize()

    # Throughput: back-to-back launches, event pair per batch.
    K = args.steps
    B = max(1, min(args.batch, K))
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(K // B + 2)]
    torch.cuda.synchronize()
    evs[0].record(stream)
    nb = 0
    for t in range(K):
        launch(t)
        if (t + 1) % B == 0:
            nb += 1
            evs[nb].record(stream)
    end_all = torch.cuda.Event(enable_timing=True)
    end_all.record(stream)
    torch.cuda.synchronize()
    per_batch = [evs[i].elapsed_time(evs[i + 1]) * 1e3 / B for i in range(nb)]
    total_ms = evs[0].elapsed_time(end_all)
    us_layer = float(np.median(per_batch)) if per_batch else total_ms * 1e3 / K
    # the GPU's routing of the rest of the CPU baseline's sample (untimed), so
    # that every CPU token's ids are compared
    for t in range(K, n_cpu):
        launch(t)
    torch.cuda.synchronize()
    status = dec.status()

    # Kernel duration: the launches above run back to back on one stream, so
    # the event time of a batch divided by its launch count is the kernel's
    # average duration (plus the sub-microsecond dispatch gap).
    k_mean = total_ms * 1e3 / K
    achieved = bytes_layer / (k_mean * 1e-6) / 1e9

    profiled = load_counters()
    traffic = profiled.get("moe_layer", {}).get("hbm_bytes")

    gpu_ids = ids.cpu().numpy()
    progress(f"config 1: {us_layer:.3f} us/layer")
    result = {
        "metric": METRIC,
        "value": round(us_layer, 3),
        "unit": "us/layer",
        "n_gpus": 1,
        "steps": K,
        "warmup": args.warmup,
        "ms_per_step": round(us_layer / 1e3, 6),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) bf16 tokens; random-init N(0,0.02^2) bf16 weights)",
        "config": {
            "workload": "DeepSeek-V2-Lite MoE layer, batch-1 decode, one token per launch "
                        "(BASELINE config 1)",
            "hidden": dims.hidden, "moe_inter": dims.moe_inter, "n_routed": dims.n_routed,
            "top_k": dims.top_k, "shared_inter": dims.shared_inter,
            "selected_bytes_per_token": bytes_layer,
        },
        "hbm_gbs": round(bytes_layer / (us_layer * 1e-6) / 1e9, 1),
        "hbm_frac": round(bytes_layer / (us_layer * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
        "roofline": {
            "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
            "traffic_source": counters_source(),
            "kernel": "fleet_moe::decode::moe_decode_kernel",
            "kernel_us_mean": round(k_mean, 3),
            "kernel_us_batch_min": round(float(min(per_batch)), 3) if per_batch else None,
            "algorithmic_bytes": bytes_layer,
        },
        "workspace_status": status,
    }

    if not args.no_grouped:
        # the grouped step takes up to 64 tokens whatever --steps is
        gx = x_host if x_host.shape[0] >= 64 else bf16_tokens(synth, 64)
        result["grouped"] = bench_grouped(torch, dev, stream, layer, dims, gx)
        progress("grouped steps done")
    del layer
    torch.cuda.empty_cache()
    if not args.no_cold:
        gx = x_host if x_host.shape[0] >= 64 else bf16_tokens(synth, 64)
        result["cold"] = bench_cold(torch, dev, stream, dims, x_host[:K], gx, lib,
                                    bytes_layer, args.no_grouped)
        progress("cold legs done")
    if not args.no_attention:
        result["attention"] = bench_attention(torch, dev, stream, dims)
        progress("attention and lm_head legs done")
    if not args.no_column:
        result["ffn_column"] = bench_column(torch, dev, stream, dims)
        progress("FFN column done")
    if not args.no_decode:
        result["full_decode"] = bench_decode(torch, dev, stream, dims)
        progress("full decode done")
    result["stream_read"] = stream_ceiling(torch, dev, stream, lib)
    if args.calibrate:
        n = 256 << 20
        buf = torch.ones(n // 4, dtype=torch.int32, device=dev)
        sink = torch.zeros(1, dtype=torch.int32, device=dev)
        for _ in range(3):
            _lib.check(lib.fleet_moe_stream_read(buf.data_ptr(), n, sink.data_ptr(), sh),
                       "fleet_moe_stream_read")
        fill = torch.empty(64 << 20, dtype=torch.uint8, device=dev)
        for _ in range(3):
            fill.fill_(3)
        torch.cuda.synchronize()
        result["calibration"] = {"stream_read_bytes": n, "fill_bytes": 64 << 20, "launches": 3}

    result["counters"] = counter_view(result, profiled)
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(blob, lay, x_host[:n_cpu], args.cpu_seconds,
                                              gpu_ids)
    print(json.dumps(result), flush=True)
    return 0 if status == 0 else 1


def bench_cold(torch, dev, stream, dims, x_host, gx_host, lib, bytes_layer, no_grouped,
               n_layers: int = 4, warm: int = 8):
    """Config 1 and config 2 with no weight reuse through the 256 MB MALL:
    token t runs MoE layer 1 + t % 4 of a 4-layer stack drawn on the device,
    so 3 x 138 MB of other layers' weights stream between two uses of a layer
    (the column and the full decode see the same). The grouped step alternates
    over the same 4 layers (its T = 4 step reads 260 MB, about the MALL's
    size, so a single layer would stay partly cached)."""
    from fleet_moe import _lib, layout as lay_mod, ops, synth_gpu
    lay = lay_mod.column_layout(dims, n_layers=n_layers + 1)
    blob = torch.empty(lay.nbytes, dtype=torch.uint8, device=dev)
    synth_gpu.fill_column(blob, lay, seed=5)
    layers = [ops.DeviceLayer(blob, lay, i, dims) for i in range(1, n_layers + 1)]
    cls = [L.c_layer() for L in layers]
    dec = ops.LayerDecoder(dims, device=dev)
    xd = torch.from_numpy(x_host).to(dev)
    y = torch.empty_like(xd[0])
    cd = ops.c_dims(dims)
    sh = int(stream.cuda_stream)
    fn = lib.fleet_moe_layer_decode
    row = xd.shape[1] * 4

    def launch(t):
        rc = fn(ctypes.byref(cls[t % n_layers]), xd.data_ptr() + (t % xd.shape[0]) * row,
                y.data_ptr(), None, None, None, dec.workspace.data_ptr(), dec.workspace.numel(),
                ctypes.byref(cd), sh)
        if rc:
            _lib.check(rc, "fleet_moe_layer_decode")

    for t in range(warm):
        launch(t)
    K = xd.shape[0]
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    a.record(stream)
    for t in range(K):
        launch(t)
    b.record(stream)
    torch.cuda.synchronize()
    us = a.elapsed_time(b) * 1e3 / K
    out = {"workload": f"config 1 cycling over {n_layers} distinct MoE layers (token t on layer "
                       f"1 + t % {n_layers}), {K} tokens",
           "us_per_layer": round(us, 3),
           "hbm_gbs": round(bytes_layer / (us * 1e-6) / 1e9, 1),
           "frac": round(bytes_layer / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
           "status": dec.status()}
    if not no_grouped:
        out["grouped"] = bench_grouped(torch, dev, stream, layers, dims, gx_host)
    del layers, dec, blob, xd
    torch.cuda.empty_cache()
    return out


def bench_column(torch, dev, stream, dims, n_tok: int = 32, warm: int = 4):
    """Config 3: the FFN half of all 27 layers (dense layer 0 + 26 MoE layers)
    chained at batch 1 over 32 seeded tokens, weights drawn on the device, one
    launch per token (fleet_ffn_column); the same tokens also with one launch
    per layer. Also times the dense layer alone (its own roofline)."""
    from fleet_moe import layout as lay_mod, ops, synth, synth_gpu
    lay = lay_mod.column_layout(dims, n_layers=27)
    blob = torch.empty(lay.nbytes, dtype=torch.uint8, device=dev)
    synth_gpu.fill_column(blob, lay, seed=0)
    col = ops.FfnColumn(blob, lay, dims)
    xs = synth.hidden_inputs(3, n_tok + warm)
    xs = ((xs.view(np.uint32) + 0x7FFF + ((xs.view(np.uint32) >> 16) & 1))
          & 0xFFFF0000).astype(np.uint32).view(np.float32)
    xd = torch.from_numpy(xs).to(dev)
    for t in range(warm):
        col.run_into(xd[t], stream)
    torch.cuda.synchronize()
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    a.record(stream)
    for t in range(warm, warm + n_tok):
        col.run_into(xd[t], stream)
    b.record(stream)
    torch.cuda.synchronize()
    us_tok = a.elapsed_time(b) * 1e3 / n_tok
    # the same tokens with one launch per layer
    col.fused = False
    for t in range(warm):
        col.run_into(xd[t], stream)
    a2 = torch.cuda.Event(enable_timing=True)
    b2 = torch.cuda.Event(enable_timing=True)
    a2.record(stream)
    for t in range(warm, warm + n_tok):
        col.run_into(xd[t], stream)
    b2.record(stream)
    torch.cuda.synchronize()
    us_tok_sep = a2.elapsed_time(b2) * 1e3 / n_tok
    col.fused = True
    # dense layer 0 alone, back to back
    y = torch.empty_like(xd[0])
    nd = 50
    c = torch.cuda.Event(enable_timing=True)
    d = torch.cuda.Event(enable_timing=True)
    c.record(stream)
    for t in range(nd):
        col.layer_into(0, xd[t % (n_tok + warm)], y, stream)
    d.record(stream)
    torch.cuda.synchronize()
    us_dense = c.elapsed_time(d) * 1e3 / nd
    dense_bytes = 3 * lay_mod.DENSE_INTER * dims.hidden * 2
    moe_bytes = 6 * 3 * dims.hidden * dims.moe_inter * 2 + 3 * dims.hidden * dims.shared_inter * 2
    tok_bytes = dense_bytes + 26 * (moe_bytes + dims.n_routed * dims.hidden * 2)
    status = col.status()
    out = {
        "workload": "27-layer FFN column (dense layer 0 + 26 MoE layers), batch 1, "
                    f"{n_tok} chained tokens, weights N(0,0.02^2) bf16 drawn on the device, "
                    "one launch per token (BASELINE config 3)",
        "us_per_token": round(us_tok, 1), "tokens_per_s": round(1e6 / us_tok, 1),
        "us_per_token_separate_launches": round(us_tok_sep, 1),
        "bytes_per_token": tok_bytes,
        "hbm_gbs": round(tok_bytes / (us_tok * 1e-6) / 1e9, 1),
        "hbm_frac": round(tok_bytes / (us_tok * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
        "dense_layer": {"us": round(us_dense, 2), "bytes": dense_bytes,
                        "hbm_gbs": round(dense_bytes / (us_dense * 1e-6) / 1e9, 1),
                        "hbm_frac": round(dense_bytes / (us_dense * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)},
        "status": status,
    }
    del col, blob, xd
    torch.cuda.empty_cache()
    return out


def bench_decode(torch, dev, stream, dims, prompt_len: int = 1024, n_gen: int = 32):
    """Config 4: the full 27-layer model (absorbed-MLA attention, dense layer
    0, 26 MoE layers, lm_head + greedy argmax) at batch 1, weights drawn on the
    device. The KV cache is prefilled by teacher-forced steps over a seeded
    uniform prompt of 1024 tokens, then 32 greedy tokens are generated; each
    step is one replay of the captured HIP graph of the step (the token and
    the position live on the device, the argmax feeds both forward). The step
    is one launch (fleet_decode_step); the same 32 tokens are also timed with
    one launch per stage (embed, per layer attention and FFN, lm_head,
    argmax) for comparison."""
    from fleet_moe import layout as lay_mod, ops, synth_gpu
    lay = lay_mod.model_layout(dims, n_layers=27)
    blob = torch.empty(lay.nbytes, dtype=torch.uint8, device=dev)
    synth_gpu.fill_model(blob, lay, seed=0)
    max_pos = prompt_len + n_gen
    dec = ops.Decoder(blob, lay, dims, max_pos=max_pos)
    prompt = np.random.default_rng(0).integers(0, lay_mod.VOCAB, prompt_len).astype(np.int32)
    prompt_d = torch.from_numpy(prompt).to(dev)
    torch.cuda.synchronize()
    dec.capture()
    t0 = time.perf_counter()
    dec.prefill(prompt_d)
    torch.cuda.synchronize()
    prefill_s = time.perf_counter() - t0
    toks = torch.empty(n_gen, dtype=torch.int32, device=dev)
    dec.token.copy_(dec.token_out)
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    a.record(stream)
    for j in range(n_gen):
        dec.graph.replay()
        toks[j:j + 1].copy_(dec.token_out)
    b.record(stream)
    torch.cuda.synchronize()
    ms_tok = a.elapsed_time(b) / n_gen
    # the same steps launched eagerly (no graph), from the same state
    dec.graph = None
    dec.token.copy_(prompt_d[-1:])
    dec.pos.fill_(prompt_len - 1)
    dec.step()            # the last prompt step again: same cache row, same first pick
    c = torch.cuda.Event(enable_timing=True)
    d = torch.cuda.Event(enable_timing=True)
    toks_e = torch.empty_like(toks)
    c.record(stream)
    for j in range(n_gen):
        dec.step()
        toks_e[j:j + 1].copy_(dec.token_out)
    d.record(stream)
    torch.cuda.synchronize()
    ms_tok_eager = c.elapsed_time(d) / n_gen
    # the same steps as separate launches per stage (graph of ~56 launches)
    sep = ops.Decoder(blob, lay, dims, max_pos=max_pos, fused=False)
    sep.cache.copy_(dec.cache)
    sep.capture()
    sep.token.copy_(prompt_d[-1:])
    sep.pos.fill_(prompt_len - 1)
    sep.step()
    toks_s = torch.empty_like(toks)
    e = torch.cuda.Event(enable_timing=True)
    f = torch.cuda.Event(enable_timing=True)
    e.record(stream)
    for j in range(n_gen):
        sep.graph.replay()
        toks_s[j:j + 1].copy_(sep.token_out)
    f.record(stream)
    torch.cuda.synchronize()
    ms_tok_sep = e.elapsed_time(f) / n_gen
    sep_status = sep.status()
    del sep
    H = dims.hidden
    attn_bytes = (lay_mod.QKV_ROWS * H + lay_mod.ATTN_HEADS * (lay_mod.QK_NOPE + lay_mod.V_HEAD)
                  * lay_mod.KV_LORA + H * lay_mod.ATTN_HEADS * lay_mod.V_HEAD) * 2
    moe_bytes = (6 * 3 * H * dims.moe_inter + 3 * H * dims.shared_inter + dims.n_routed * H) * 2
    dense_bytes = 3 * lay_mod.DENSE_INTER * H * 2
    head_bytes = lay_mod.VOCAB * H * 2
    mean_rows = prompt_len + (n_gen + 1) / 2
    cache_bytes = int(27 * mean_rows * 576 * 2)
    tok_bytes = 27 * attn_bytes + 26 * moe_bytes + dense_bytes + head_bytes + cache_bytes
    out = {
        "workload": "27-layer DeepSeek-V2-Lite-shape decode, batch 1, absorbed MLA, "
                    f"KV cache prefilled with {prompt_len} seeded uniform tokens, {n_gen} greedy "
                    "tokens, weights N(0,0.02^2) bf16 drawn on the device, one launch per "
                    "token (BASELINE config 4)",
        "ms_per_token": round(ms_tok, 4), "tokens_per_s": round(1e3 / ms_tok, 1),
        "ms_per_token_eager": round(ms_tok_eager, 4),
        "ms_per_token_separate_launches": round(ms_tok_sep, 4),
        "bytes_per_token": tok_bytes,
        "hbm_gbs": round(tok_bytes / (ms_tok * 1e-3) / 1e9, 1),
        "hbm_frac": round(tok_bytes / (ms_tok * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "prefill_s": round(prefill_s, 3),
        "graph_equals_eager": bool(torch.equal(toks, toks_e)),
        "fused_equals_separate": bool(torch.equal(toks, toks_s)),
        "tokens_head": [int(t) for t in toks[:8].cpu()],
        "status": dec.status() | sep_status,
    }
    del dec, blob
    torch.cuda.empty_cache()
    return out


def bench_attention(torch, dev, stream, dims, pos: int = 1024, n_layers: int = 12,
                    rounds: int = 8, warm_launches: int = 50, head_launches: int = 20):
    """Config 4's per-layer attention kernel and its lm_head kernel alone.

    Attention: `n_layers` independent layers (qkv, kv_b, o_proj drawn
    N(0, 0.02^2), unit norms; 12 x 28.7 MB exceeds the 256 MB MALL), each with
    a KV cache whose rows 0..pos-1 are N(0,1) bf16, one call per layer in turn
    at position `pos` (the position the decode benchmark's tokens start at):
    the cold figure. The warm figure repeats layer 0 back to back.
    lm_head: final RMSNorm + the 102400 x 2048 GEMV + argmax (420 MB, always
    cold), back to back."""
    from fleet_moe import layout as lay_mod, ops
    from fleet_moe.rope import yarn_tables
    H = dims.hidden
    g = torch.Generator(device=dev)
    g.manual_seed(1234)

    def normal(n, std=0.02):
        return (torch.randn(n, generator=g, device=dev) * std).to(torch.bfloat16).view(torch.int16)

    one = torch.tensor(1.0, dtype=torch.bfloat16).view(torch.int16).item()
    kv_rows = lay_mod.ATTN_HEADS * (lay_mod.QK_NOPE + lay_mod.V_HEAD)
    w_bytes = (lay_mod.QKV_ROWS * H + kv_rows * lay_mod.KV_LORA
               + H * lay_mod.ATTN_HEADS * lay_mod.V_HEAD) * 2
    layers, keep = [], []
    max_pos = pos + 64
    for _ in range(n_layers):
        t = {"norm_in": torch.full((H,), one, dtype=torch.int16, device=dev),
             "qkv": normal(lay_mod.QKV_ROWS * H),
             "kv_a_norm": torch.full((lay_mod.KV_LORA,), one, dtype=torch.int16, device=dev),
             "kv_b": normal(kv_rows * lay_mod.KV_LORA),
             "o_proj": normal(H * lay_mod.ATTN_HEADS * lay_mod.V_HEAD),
             "cache": torch.zeros((max_pos, 576), dtype=torch.int16, device=dev)}
        t["cache"][:pos] = normal(pos * 576, 1.0).view(pos, 576)
        keep.append(t)
        layers.append(ops._lib.FleetAttnLayer(t["norm_in"].data_ptr(), t["qkv"].data_ptr(),
                                              t["kv_a_norm"].data_ptr(), t["kv_b"].data_ptr(),
                                              t["o_proj"].data_ptr()))
    cos, sin = yarn_tables(max_pos)
    cos, sin = torch.from_numpy(cos).to(dev), torch.from_numpy(sin).to(dev)
    ad = ops.AttnDecoder(dims, device=dev)
    x = torch.randn(H, generator=g, device=dev).to(torch.bfloat16).float()
    y = torch.empty_like(x)

    def timed(fn, n):
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for i in range(n):
            fn(i)
        b.record(stream)
        torch.cuda.synchronize()
        return a.elapsed_time(b) * 1e3 / n

    def call(i):
        k = i % n_layers
        ad.attn_into(layers[k], x, y, keep[k]["cache"], pos, None, cos, sin, stream)

    for i in range(2 * n_layers):
        call(i)
    torch.cuda.synchronize()
    us_cold = timed(call, rounds * n_layers)
    us_warm = timed(lambda i: call(0), warm_launches)
    # algorithmic bytes: the weights, the norms, the pos cached rows read and
    # the new row written
    a_bytes = w_bytes + (H + lay_mod.KV_LORA) * 2 + (pos + 1) * 576 * 2
    status = ad.status()
    del keep, layers
    # lm_head: 102400 x 2048 bf16
    head = normal(lay_mod.VOCAB * H)
    fnorm = torch.full((H,), one, dtype=torch.int16, device=dev)
    tok = torch.zeros(1, dtype=torch.int32, device=dev)
    for _ in range(3):
        ad.lm_head_into(x, fnorm.data_ptr(), head.data_ptr(), None, tok, None, None, stream)
    torch.cuda.synchronize()
    us_head = timed(lambda i: ad.lm_head_into(x, fnorm.data_ptr(), head.data_ptr(), None, tok,
                                              None, None, stream), head_launches)
    h_bytes = lay_mod.VOCAB * H * 2 + H * 2
    status |= ad.status()
    del head
    torch.cuda.empty_cache()
    return {
        "workload": f"config 4's attention half alone (absorbed MLA, 16 heads, KV cache of {pos} "
                    f"rows, one call at position {pos}); cold: {n_layers} layers in turn "
                    f"({n_layers * w_bytes / 1e6:.0f} MB of weights between reuses), warm: one "
                    "layer back to back",
        "us_cold": round(us_cold, 2), "us_warm": round(us_warm, 2), "bytes": a_bytes,
        "hbm_gbs": round(a_bytes / (us_cold * 1e-6) / 1e9, 1),
        "frac": round(a_bytes / (us_cold * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
        "kernel": "fleet_moe::attn::attn_layer_kernel",
        "lm_head": {"us": round(us_head, 2), "bytes": h_bytes,
                    "hbm_gbs": round(h_bytes / (us_head * 1e-6) / 1e9, 1),
                    "frac": round(h_bytes / (us_head * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                    "kernels": "fleet_moe::attn::lmhead_kernel + argmax_kernel"},
        "status": status,
    }


def stream_ceiling(torch, dev, stream, lib):
    """Achievable HBM read rate with the kernels' load pattern: the streaming
    probe over 2 GiB (far beyond the 256 MB of L2 + MALL), best of 10."""
    from fleet_moe import _lib
    n = 2 << 30
    buf = torch.ones(n // 4, dtype=torch.int32, device=dev)
    sink = torch.zeros(1, dtype=torch.int32, device=dev)
    sh = int(stream.cuda_stream)
    best = float("inf")
    for i in range(12):
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record(stream)
        _lib.check(lib.fleet_moe_stream_read(buf.data_ptr(), n, sink.data_ptr(), sh),
                   "fleet_moe_stream_read")
        b.record(stream)
        torch.cuda.synchronize()
        if i >= 2:
            best = min(best, a.elapsed_time(b) * 1e-3)
    del buf
    return {"bytes": n, "gbs": round(n / best / 1e9, 1), "frac_of_peak": round(n / best / 1e9 / HBM_PEAK_GBS, 4),
            "kernel": "fleet_moe::probe::stream_read_kernel"}


def bf16_tokens(synth, n):
    """The first n seeded N(0,1) hidden vectors (a prefix-stable stream),
    rounded to bf16 (RNE), as fp32."""
    x = synth.hidden_inputs(0, n)
    return ((x.view(np.uint32) + 0x7FFF + ((x.view(np.uint32) >> 16) & 1))
            & 0xFFFF0000).astype(np.uint32).view(np.float32)


def bench_grouped(torch, dev, stream, layers, dims, x_host):
    """Config 2: T in {4, 16, 64}, Zipf(1.1)-biased routing; times the grouped
    product alone (routing precomputed), per step. `layers`: one DeviceLayer,
    or a list the steps cycle over (one step per layer in turn)."""
    from fleet_moe import ops, synth
    out = {}
    layers = layers if isinstance(layers, list) else [layers]
    bias = torch.from_numpy(synth.zipf_logit_bias(0)).to(dev)
    runner = ops.GroupedRunner(64, dims, device=dev)
    for T in (4, 16, 64):
        if x_host.shape[0] < T:
            raise ValueError(f"grouped step T={T} needs {T} token rows, got {x_host.shape[0]}")
        x = torch.from_numpy(x_host[:T]).to(dev)
        # the router kernel takes normed input: the RMSNorm of config 2 (unit
        # gamma) is applied with torch here, outside the timed expert product
        xf = x.double()
        xn = x * torch.rsqrt((xf * xf).mean(-1, keepdim=True).float() + dims.rms_eps)
        xn = ops.bf16_bits_to_f32(ops.f32_to_bf16_bits(xn)).contiguous()
        routes = [ops.route(L, xn, bias)[1:] for L in layers]
        xb = ops.f32_to_bf16_bits(xn).contiguous()
        o = torch.empty((T, dims.hidden), dtype=torch.int16, device=dev)
        nl = len(layers)
        for i in range(5 * nl):
            runner.run_into(layers[i % nl], xb, *routes[i % nl], o)
        torch.cuda.synchronize()
        n = 48 if nl > 1 else 50
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for i in range(n):
            runner.run_into(layers[i % nl], xb, *routes[i % nl], o)
        b.record(stream)
        torch.cuda.synchronize()
        us = a.elapsed_time(b) * 1e3 / n
        dist = [int(torch.unique(r[0]).numel()) for r in routes]
        distinct = float(np.mean(dist)) if nl > 1 else dist[0]
        nbytes = distinct * 3 * dims.hidden * dims.moe_inter * 2 + 3 * dims.hidden * dims.shared_inter * 2
        flops = 2.0 * T * (6 * 3 * dims.hidden * dims.moe_inter + 3 * dims.hidden * dims.shared_inter)
        out[f"T{T}"] = {"us_per_step": round(us, 2), "distinct_experts": distinct,
                        "hbm_gbs": round(nbytes / (us * 1e-6) / 1e9, 1),
                        "hbm_frac": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                        "tflops": round(flops / (us * 1e-6) / 1e12, 2),
                        "mfma_frac": round(flops / (us * 1e-6) / 1e12 / MFMA_BF16_PEAK_TFLOPS, 5)}
    out["status"] = runner.status()
    return out


if __name__ == "__main__":
    sys.exit(main())
