"""Shared test setup: import paths, the `gpu` marker, and fixtures."""
from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT, ROOT / "fleet-mi300x_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built HIP library")


@pytest.fixture(scope="session")
def full_layer():
    """One DeepSeek-V2-Lite MoE layer (seed 0, layer 1) in the packed layout:
    (uint8 blob, layout, oracle PackedLayer view)."""
    from fleet_moe import synth
    from fleet_moe.layout import DSV2_LITE, view_u16
    from oracle import moe_oracle as orc
    blob, lay = synth.moe_layer_blob(seed=0, layer=1, dims=DSV2_LITE)
    t = lay.tensors
    pl = orc.PackedLayer(router=view_u16(blob, t["L1.router"]),
                         experts=view_u16(blob, t["L1.experts"]),
                         shared=view_u16(blob, t["L1.shared"]),
                         expert_stride=DSV2_LITE.expert_stride,
                         norm=view_u16(blob, t["L1.norm_post"]))
    return blob, lay, pl
