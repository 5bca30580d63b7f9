"""fleet_moe: MI355X-native batch-1 MoE decode path for DeepSeek-V2-Lite.

Python host side over the C ABI of libfleet_moe.so (include/fleet_moe.h):
`layout` (packed-weight layout and manifest), `synth` (seeded synthetic
weights), `ops` (device buffers and calls), `taskgraph` (the reference's
64-byte task descriptors for the MoE task kinds).
"""
from .layout import DSV2_LITE, MoeDims  # noqa: F401

__all__ = ["DSV2_LITE", "MoeDims"]
