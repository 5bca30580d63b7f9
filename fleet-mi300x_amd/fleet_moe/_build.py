"""In-tree build of libfleet_moe.so for gfx950 with hipcc.

Every HIP source under ../csrc is compiled to an object (in parallel) and the
objects are linked into one shared library next to this file. Runs on a machine without a GPU (hipcc
cross-compiles gfx950).

`build(trace=True)` compiles the same sources with the stage-trace stamps on
(FLEET_ATTN_TRACE, FLEET_MOE_TRACE, FLEET_STEP_TRACE) into a second library,
libfleet_moe_trace.so, which only the diagnostic `fleet_moe.stage_trace`
loads.
"""
from __future__ import annotations

import os
import shutil
import subprocess
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG.parent / "csrc"
INCLUDE = PKG.parents[1] / "include"
OUT = PKG / "libfleet_moe.so"
TRACE_OUT = PKG / "libfleet_moe_trace.so"
TRACE_FLAGS = ["-DFLEET_ATTN_TRACE=1", "-DFLEET_MOE_TRACE=1", "-DFLEET_STEP_TRACE=1"]

HIPCC_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
    # keep the compiler from emitting packed fp32 arithmetic
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found")


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def _run(cmd: list[str], verbose: bool) -> subprocess.Popen:
    if verbose:
        print(" ".join(cmd), flush=True)
    return subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)


def _check(p: subprocess.Popen, what: str, verbose: bool) -> None:
    out, _ = p.communicate()
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in out.splitlines() if noise not in l)
    if p.returncode != 0:
        raise RuntimeError(f"hipcc failed on {what} ({p.returncode}):\n{err}")
    if verbose and err.strip():
        print(err)


def build(verbose: bool = False, trace: bool = False) -> Path:
    """Compile every source into OUT, or with trace into TRACE_OUT (always
    recompiles). Returns the path."""
    out = TRACE_OUT if trace else OUT
    objdir = PKG / ("_obj_trace" if trace else "_obj")
    objdir.mkdir(exist_ok=True)
    jobs, objs = [], []
    for src in sources():
        obj = objdir / (src.stem + ".o")
        cmd = [hipcc(), *HIPCC_FLAGS, *(TRACE_FLAGS if trace else []), f"-I{INCLUDE}",
               f"-I{CSRC}", "-c", "-o", str(obj), str(src)]
        jobs.append((_run(cmd, verbose), src.name))
        objs.append(obj)
    for p, name in jobs:
        _check(p, name, verbose)
    tmp = out.with_name(out.name + ".tmp")
    link = [hipcc(), "--offload-arch=gfx950", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    _check(_run(link, verbose), "the link", verbose)
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    import sys
    print(build(verbose=True, trace="--trace" in sys.argv[1:]))
