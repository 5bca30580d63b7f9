"""YaRN rotary tables for DeepSeek-V2-Lite's decoupled RoPE (qk_rope = 64).

The tables depend only on the position, so they are built once on the host and
uploaded, as the reference launcher does (src/host/fleet_launch.hip:174-218).
The arithmetic is DeepseekV2YarnRotaryEmbedding's cache as
src/host/reference_decode.py:78-117 computes it, in fp32 throughout:
  inv_freq_i = inter_i * ramp_i + extra_i * (1 - ramp_i), extra_i = base^(-2i/d),
  inter_i = extra_i / factor, ramp_i = clip((i - low) / (high - low), 0, 1) over
  the correction range [low, high] of beta_fast / beta_slow rotations;
  angle[t][i] = angle[t][i + d/2] = t * inv_freq_i;
  cos, sin = cos(angle), sin(angle) times mscale(factor, mscale) /
  mscale(factor, mscale_all_dim), which is 1.0 for DeepSeek-V2-Lite.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np


@dataclass(frozen=True)
class RopeParams:
    """Manifest scalars rope_* / beta_* / mscale* (pack_weights.py:171-181)."""
    dim: int = 64
    base: float = 10000.0
    factor: float = 40.0
    original_max: int = 4096
    beta_fast: float = 32.0
    beta_slow: float = 1.0
    mscale: float = 0.707
    mscale_all_dim: float = 0.707

    @classmethod
    def from_scalars(cls, s: dict) -> "RopeParams":
        return cls(dim=int(s.get("qk_rope", 64)), base=float(s["rope_theta"]),
                   factor=float(s["rope_factor"]), original_max=int(s["rope_original_max"]),
                   beta_fast=float(s["beta_fast"]), beta_slow=float(s["beta_slow"]),
                   mscale=float(s["mscale"]), mscale_all_dim=float(s["mscale_all_dim"]))


def get_mscale(scale: float, m: float) -> float:
    """0.1 m ln(scale) + 1 above scale 1, else 1 (reference_decode.py:78-82)."""
    return 1.0 if scale <= 1 else 0.1 * m * math.log(scale) + 1.0


def softmax_scale(p: RopeParams = RopeParams(), q_head_dim: int = 192) -> float:
    """q_head_dim^-0.5 * mscale(factor, mscale_all_dim)^2 (reference_decode.py:197-203)."""
    m = get_mscale(p.factor, p.mscale_all_dim) if p.mscale_all_dim else 1.0
    return q_head_dim ** -0.5 * m * m


def _correction_range(p: RopeParams) -> tuple[float, float]:
    def dim_of(rotations: float) -> float:
        return (p.dim * math.log(p.original_max / (rotations * 2 * math.pi))) / (2 * math.log(p.base))
    low = max(math.floor(dim_of(p.beta_fast)), 0)
    high = min(math.ceil(dim_of(p.beta_slow)), p.dim - 1)
    return float(low), float(high) + (0.001 if low == high else 0.0)


def yarn_tables(max_pos: int, p: RopeParams = RopeParams()) -> tuple[np.ndarray, np.ndarray]:
    """(cos, sin), fp32 [max_pos][dim]."""
    exps = np.arange(0, p.dim, 2, dtype=np.float32) / p.dim
    extra = 1.0 / (p.base ** exps)
    inter = 1.0 / (p.factor * p.base ** exps)
    low, high = _correction_range(p)
    ramp = np.clip((np.arange(p.dim // 2, dtype=np.float32) - low) / (high - low), 0, 1)
    keep = 1.0 - ramp
    inv_freq = inter * (1 - keep) + extra * keep
    ang = np.outer(np.arange(max_pos, dtype=np.float32), inv_freq)
    ang = np.concatenate([ang, ang], axis=-1)
    m = get_mscale(p.factor, p.mscale) / get_mscale(p.factor, p.mscale_all_dim)
    return ((np.cos(ang) * m).astype(np.float32), (np.sin(ang) * m).astype(np.float32))
