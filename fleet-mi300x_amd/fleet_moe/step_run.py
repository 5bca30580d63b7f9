"""A short run of the one-launch decode step for counter passes.

The full-decode leg of bench.py prefills its KV cache with 1,024
graph-replayed steps (about 57,000 dispatches with the separate-launch
comparison); this run fills the cache rows 0..1023 with seeded bf16 values
instead and launches the step eagerly a few times from position 1024, so a
rocprofv3 counter pass sees a handful of step dispatches:

  cd fleet-mi300x_amd
  rocprofv3 --pmc FETCH_SIZE --kernel-include-regex 'step_kernel|stream_read|FillFunctor' \\
      --output-format csv -d ../gpurun_out/q_step_fetch -o step_fetch -- python3 -m fleet_moe.step_run

It also runs the known-size kernels that calibrate FETCH_SIZE and WRITE_SIZE
(fleet_moe_stream_read over 256 MiB, three times; a 64 MiB byte fill) and
prints one JSON line: the steps' event-timed mean and their algorithmic bytes.
"""
from __future__ import annotations

import argparse
import json
import time


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--steps", type=int, default=8, help="timed steps (eager, one launch each)")
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--pos", type=int, default=1024, help="position of the first step")
    args = ap.parse_args()

    import torch

    from . import _lib, layout as lay_mod, ops, synth_gpu
    from .layout import DSV2_LITE as dims

    dev = torch.device("cuda")
    lib = _lib.load()
    n_layers = 27
    lay = lay_mod.model_layout(dims, n_layers=n_layers)
    blob = torch.empty(lay.nbytes, dtype=torch.uint8, device=dev)
    synth_gpu.fill_model(blob, lay, seed=0)
    n_steps = args.warmup + args.steps
    dec = ops.Decoder(blob, lay, dims, max_pos=args.pos + n_steps)
    g = torch.Generator(device=dev).manual_seed(1)
    rows = dec.cache[:, : args.pos]
    rows.copy_((0.5 * torch.randn(rows.shape, generator=g, device=dev)).to(torch.bfloat16)
               .view(torch.int16))
    dec.reset(args.pos)
    dec.token.fill_(1)
    torch.cuda.synchronize()
    for _ in range(args.warmup):
        dec.step()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(args.steps):
        dec.step()
    b.record()
    torch.cuda.synchronize()
    ms = a.elapsed_time(b) / args.steps
    status = dec.status()

    # calibration: known-size reads and writes in the same process
    sh = int(torch.cuda.current_stream().cuda_stream)
    n = 256 << 20
    buf = torch.ones(n // 4, dtype=torch.int32, device=dev)
    sink = torch.zeros(1, dtype=torch.int32, device=dev)
    for _ in range(3):
        _lib.check(lib.fleet_moe_stream_read(buf.data_ptr(), n, sink.data_ptr(), sh),
                   "fleet_moe_stream_read")
    fill = torch.empty(64 << 20, dtype=torch.uint8, device=dev)
    fill.fill_(1)
    torch.cuda.synchronize()

    H = dims.hidden
    attn = (lay_mod.QKV_ROWS * H + lay_mod.ATTN_HEADS * (lay_mod.QK_NOPE + lay_mod.V_HEAD)
            * lay_mod.KV_LORA + H * lay_mod.ATTN_HEADS * lay_mod.V_HEAD) * 2
    moe = (6 * 3 * H * dims.moe_inter + 3 * H * dims.shared_inter + dims.n_routed * H) * 2
    dense = 3 * lay_mod.DENSE_INTER * H * 2
    head = lay_mod.VOCAB * H * 2
    first = args.pos + args.warmup
    mean_rows = first + (args.steps + 1) / 2           # rows read per step, averaged
    cache = int(n_layers * mean_rows * 576 * 2)
    print(json.dumps({
        "workload": f"one-launch decode step, {n_layers} layers, positions {first}.."
                    f"{first + args.steps - 1} (eager, cache rows seeded), batch 1",
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 4),
        "algorithmic_bytes_per_step": n_layers * attn + (n_layers - 1) * moe + dense + head + cache,
        "calibration": {"stream_read_bytes": n, "stream_read_launches": 3, "fill_bytes": 64 << 20},
        "status": status, "time": time.strftime("%Y-%m-%dT%H:%M:%S")}), flush=True)
    return 0 if status == 0 else 1


if __name__ == "__main__":
    raise SystemExit(main())
