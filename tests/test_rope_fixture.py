"""The YaRN rotary tables against the reference's own: the product's
fleet_moe.rope.yarn_tables (uploaded to the GPU by every attention and decode
path) and the oracle's rope_tables must equal, bit for bit, the cos / sin rows
that reference_decode.yarn_cos_sin (reference_decode.py:85-117) wrote into
tests/golden/rope/yarn_tables.npz (tests/golden/make_rope_fixtures.py), for
DeepSeek-V2-Lite's scaling and three other parameter sets (factor 1, another
correction range and mscale ratio, and the empty range that takes the ramp's
+0.001 guard). All three evaluate the same fp32 NumPy operations, so equality
is exact. A correction range moved by one pair must fail."""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

from fleet_moe import rope
from oracle import moe_oracle as orc

FIXTURE = Path(__file__).resolve().parent / "golden" / "rope" / "yarn_tables.npz"
SETS = ("config", "plain", "other", "guard")


@pytest.fixture(scope="module")
def golden():
    with np.load(FIXTURE) as z:
        return {k: z[k] for k in z.files}


def params(g, name):
    dim, seq_len, base, scale, orig, bf, bs, ms, msa = g[f"{name}.params"].tolist()
    p = rope.RopeParams(dim=int(dim), base=base, factor=scale, original_max=int(orig),
                        beta_fast=bf, beta_slow=bs, mscale=ms, mscale_all_dim=msa)
    return p, int(seq_len)


def bits(a) -> np.ndarray:
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.mark.parametrize("name", SETS)
def test_correction_range_equals_the_reference(golden, name):
    p, _ = params(golden, name)
    low, high = golden[f"{name}.range"].tolist()
    got_low, got_high = rope._correction_range(p)
    assert got_low == low
    assert got_high == (high + 0.001 if low == high else high)


@pytest.mark.parametrize("name", SETS)
def test_product_tables_equal_the_reference(golden, name):
    p, seq_len = params(golden, name)
    pos = golden[f"{name}.positions"]
    cos, sin = rope.yarn_tables(seq_len, p)
    assert cos.dtype == np.float32 and cos.shape == (seq_len, p.dim)
    np.testing.assert_array_equal(bits(cos[pos]), bits(golden[f"{name}.cos"]))
    np.testing.assert_array_equal(bits(sin[pos]), bits(golden[f"{name}.sin"]))


@pytest.mark.parametrize("name", SETS)
def test_oracle_tables_equal_the_reference(golden, name):
    p, seq_len = params(golden, name)
    pos = golden[f"{name}.positions"]
    cos, sin = orc.rope_tables(seq_len, dim=p.dim, base=p.base, scale=p.factor,
                               original_max=p.original_max, beta_fast=p.beta_fast,
                               beta_slow=p.beta_slow, mscale=p.mscale,
                               mscale_all_dim=p.mscale_all_dim)
    np.testing.assert_array_equal(bits(cos[pos]), bits(golden[f"{name}.cos"]))
    np.testing.assert_array_equal(bits(sin[pos]), bits(golden[f"{name}.sin"]))


def test_the_benchmark_tables_are_the_config_set(golden):
    """The defaults every Decoder uses (RopeParams()) are the config set."""
    p, seq_len = params(golden, "config")
    assert p == rope.RopeParams()
    cos, _ = rope.yarn_tables(seq_len)
    np.testing.assert_array_equal(bits(cos[golden["config.positions"]]), bits(golden["config.cos"]))


@pytest.mark.parametrize("shift", [(1, 0), (-1, 0), (0, 1), (0, -1)])
def test_a_shifted_correction_range_is_caught(golden, monkeypatch, shift):
    p, seq_len = params(golden, "config")
    low, high = rope._correction_range(p)
    monkeypatch.setattr(rope, "_correction_range", lambda _p: (low + shift[0], high + shift[1]))
    cos, _ = rope.yarn_tables(seq_len, p)
    assert not np.array_equal(bits(cos[golden["config.positions"]]), bits(golden["config.cos"]))
