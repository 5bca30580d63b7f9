"""Write the task-graph fixtures under tests/golden/taskgraph/.

Runs the reference's own graph emitter, src/host/taskgraph.py --emit
(/root/reference, only in the build container; it needs json, struct and
argparse only), on a 3-layer copy of reference/dsv2lite_config.json (layer 0
dense, layers 1 and 2 MoE) in five variants: the default graph and the
--topk-published, --split-workers 18, --oproj-row-split and --local-fold
graphs. Each variant's descriptor stream (64-byte descriptors,
taskgraph.py:172-184) and its `.events.txt` sidecar (taskgraph.py:832-839)
are stored gzipped as <variant>.bin.gz / <variant>.events.txt.gz, with the
command line and the emitter's exit status in index.json. These are the
graphs the descriptor adapter (fleet_moe.descriptors) must consume.

    python tests/golden/make_taskgraph_fixtures.py [--reference /root/reference]
"""
from __future__ import annotations

import argparse
import gzip
import json
import subprocess
import sys
import tempfile
from pathlib import Path

OUT = Path(__file__).resolve().parent / "taskgraph"
VARIANTS = {
    "default": [],
    "topk_published": ["--topk-published"],
    "split_workers_18": ["--split-workers", "18"],
    "oproj_row_split": ["--oproj-row-split"],
    "local_fold": ["--local-fold"],
}
LAYERS = 3


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--reference", type=Path, default=Path("/root/reference"))
    a = ap.parse_args()
    emitter = a.reference / "src" / "host" / "taskgraph.py"
    cfg = json.loads((a.reference / "reference" / "dsv2lite_config.json").read_text())
    cfg["num_hidden_layers"] = LAYERS
    OUT.mkdir(parents=True, exist_ok=True)
    index = {"layers": LAYERS, "first_k_dense": cfg["first_k_dense_replace"], "variants": {}}
    with tempfile.TemporaryDirectory() as td:
        td = Path(td)
        cfg_path = td / "dsv2lite_3layer.json"
        cfg_path.write_text(json.dumps(cfg))
        for name, flags in VARIANTS.items():
            bin_path = td / f"{name}.bin"
            cmd = [sys.executable, str(emitter), "--config", str(cfg_path), "--emit",
                   str(bin_path), *flags]
            r = subprocess.run(cmd, capture_output=True, text=True)
            if not bin_path.exists():
                raise SystemExit(f"{name}: emitter wrote nothing (rc {r.returncode}):\n"
                                 f"{r.stdout}\n{r.stderr}")
            events = Path(str(bin_path) + ".events.txt")
            raw = bin_path.read_bytes()
            (OUT / f"{name}.bin.gz").write_bytes(gzip.compress(raw, mtime=0))
            (OUT / f"{name}.events.txt.gz").write_bytes(
                gzip.compress(events.read_bytes(), mtime=0))
            index["variants"][name] = {
                "flags": flags, "emitter_rc": r.returncode,
                "descriptors": len(raw) // 64,
                "events": len(events.read_text().splitlines()),
            }
            print(f"{name}: {len(raw) // 64} descriptors, rc {r.returncode}")
    (OUT / "index.json").write_text(json.dumps(index, indent=1) + "\n")


if __name__ == "__main__":
    main()
