"""fleet_moe: MI355X-native batch-1 MoE decode path for DeepSeek-V2-Lite.

Python host side over the C ABI of libfleet_moe.so (include/fleet_moe.h):
`layout` (packed-weight layout and manifest), `hf_pack` (a local HF
checkpoint into that layout), `synth` / `synth_gpu` (seeded synthetic weights
on the host / device), `rope` (the YaRN rotary tables), `ops` (device buffers
and calls), `descriptors` (the reference's 64-byte task descriptors: the MoE
task kinds planned onto library calls). Diagnostics, run as modules:
`stage_trace` (stage timelines from the stamped build) and `step_run` (a short
run of the one-launch decode step for counter passes).
"""
from .layout import DSV2_LITE, MoeDims  # noqa: F401

__all__ = ["DSV2_LITE", "MoeDims"]
