"""Write tests/golden/rope/yarn_tables.npz: the reference's YaRN rotary tables.

Imports the reference's NumPy decode module, src/host/reference_decode.py
(/root/reference, only in the build container; it needs numpy only), and
calls its yarn_find_correction_range and yarn_cos_sin
(reference_decode.py:85-117) for four parameter sets:

  config   DeepSeek-V2-Lite's rope scaling as the benchmark's config 4 runs
           it: dim 64, 1056 positions, base 1e4, factor 40, original 4096,
           beta 32 / 1, mscale 0.707 / 0.707 (reference_decode.py:294-302
           callers build it with these; dsv2lite_config.json);
  plain    factor 1 (no interpolation: the plain RoPE frequencies);
  other    base 1e6, factor 8, original 2048, beta 16 / 2, mscale 1 / 0.5
           (another correction range and an mscale ratio other than 1);
  guard    original 6, so the correction range is empty (low == high == 0)
           and the ramp takes its +0.001 guard.

For each set the file holds the correction range, the parameters and the cos
/ sin rows (fp32) at sampled positions (all 1056 are not needed: each row
depends on its position alone). Only the vectors are committed; the reference
itself never travels.

    python tests/golden/make_rope_fixtures.py [--reference /root/reference]
"""
from __future__ import annotations

import argparse
import importlib.util
import sys
from pathlib import Path

import numpy as np

OUT = Path(__file__).resolve().parent / "rope" / "yarn_tables.npz"
SETS = {
    # dim, seq_len, base, scale, original_max, beta_fast, beta_slow, mscale, mscale_all_dim
    "config": (64, 1056, 1e4, 40.0, 4096, 32.0, 1.0, 0.707, 0.707),
    "plain": (64, 1056, 1e4, 1.0, 4096, 32.0, 1.0, 1.0, 1.0),
    "other": (64, 1056, 1e6, 8.0, 2048, 16.0, 2.0, 1.0, 0.5),
    "guard": (64, 1056, 1e4, 40.0, 6, 32.0, 1.0, 0.707, 0.707),
}


def positions(seq_len: int) -> np.ndarray:
    rng = np.random.default_rng(0)
    fixed = [0, 1, 2, 3, 7, 8, 63, 64, 255, 256, 511, 512, 1000, 1022, 1023, 1024, seq_len - 1]
    return np.unique(np.concatenate([fixed, rng.integers(0, seq_len, 31)])).astype(np.int64)


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--reference", type=Path, default=Path("/root/reference"))
    a = ap.parse_args()
    src = a.reference / "src" / "host" / "reference_decode.py"
    spec = importlib.util.spec_from_file_location("reference_decode", src)
    ref = importlib.util.module_from_spec(spec)
    sys.modules[spec.name] = ref          # its dataclasses look the module up
    spec.loader.exec_module(ref)
    out = {}
    for name, (dim, seq_len, base, scale, orig, bf, bs, ms, msa) in SETS.items():
        low, high = ref.yarn_find_correction_range(bf, bs, dim, base, orig)
        cos, sin = ref.yarn_cos_sin(dim, seq_len, base, scale, orig, bf, bs, ms, msa)
        pos = positions(seq_len)
        out[f"{name}.params"] = np.array([dim, seq_len, base, scale, orig, bf, bs, ms, msa],
                                         np.float64)
        out[f"{name}.range"] = np.array([low, high], np.float64)
        out[f"{name}.positions"] = pos
        out[f"{name}.cos"] = np.asarray(cos, np.float32)[pos]
        out[f"{name}.sin"] = np.asarray(sin, np.float32)[pos]
        print(f"{name}: range ({low}, {high}), cos dtype {cos.dtype}, {len(pos)} positions")
    OUT.parent.mkdir(parents=True, exist_ok=True)
    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
