"""The residual exchange of the one-launch kernels (fleet_decode_step,
fleet_ffn_column), replayed on the CPU: no stage may find a word left by an
earlier stage or step that already carries the tag it polls for.

The stage schedule is the one csrc/step_decode.hip runs: the decode step's
attention of layer i is stage 2i + 1 and its FFN stage 2i + 2, the lm_head
reads stage 2n; the column's FFN of layer i is stage i + 1. Stage s writes
exchange buffer s % 2 with tag ((epoch + 1) * stride + s) & 0xffff and polls
buffer (s - 1) % 2 for stage s - 1's tag; a one-layer column also stamps
buffer 0 with its stage-0 tag. A poll can pass early only if a word of the
buffer, before the producing stage overwrites it, already holds the expected
tag. The stride and the layer bound are read from the sources, so the test
follows the kernel; a stride of 64 (the earlier kernel) must be caught at 33
layers."""
from __future__ import annotations

import random
import re
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
SRC = ROOT / "fleet-mi300x_amd" / "csrc" / "step_decode.hip"
HEADER = ROOT / "include" / "fleet_moe.h"


def kernel_constants() -> tuple[int, int]:
    stride = re.search(r"constexpr uint32_t kTagStride = (\d+);", SRC.read_text())
    layers = re.search(r"#define FLEET_STEP_MAX_LAYERS (\d+)", HEADER.read_text())
    assert stride and layers, "constants not found in the sources"
    return int(stride.group(1)), int(layers.group(1))


def run_step(bufs: list, epoch: int, full: bool, n: int, stride: int,
             stamp: bool = True) -> list:
    """One launch; returns (s, tag) for every produced stage s whose poller
    (stage s + 1 or the lm_head) an old word could satisfy."""
    sbase = (epoch + 1) * stride

    def tag(s: int) -> int:
        return (sbase + s) & 0xFFFF

    stages = 2 * n if full else n
    polled = set(range(1, stages + 1)) if full else set(range(1, stages))
    aliases = []
    for s in range(1, stages + 1):
        before = bufs[s % 2]
        if s in polled and before == tag(s):
            aliases.append((s, tag(s)))
        bufs[s % 2] = tag(s)
    if stamp and not full and n == 1:
        bufs[0] = tag(0)
    return aliases


def run_sequence(calls, stride: int, stamp: bool = True) -> list:
    bufs = [0, 0]          # the workspace starts zero-filled
    found = []
    for epoch, (full, n) in enumerate(calls):
        found += [(epoch, full, n, s, t)
                  for s, t in run_step(bufs, epoch, full, n, stride, stamp)]
    return found


def test_constants_leave_room_for_every_stage():
    stride, max_layers = kernel_constants()
    assert stride >= 2 * max_layers + 2
    assert 65536 % stride == 0


def test_no_poll_sees_a_stale_tag_at_any_layer_count():
    stride, max_layers = kernel_constants()
    steps = 65536 // stride + 3       # past the 16-bit tag's wrap
    for n in range(1, max_layers + 1):
        for full in (True, False):
            assert run_sequence([(full, n)] * steps, stride) == [], (full, n)


def test_no_poll_sees_a_stale_tag_when_calls_mix():
    """One workspace shared by steps and columns of different depths,
    including runs of one-layer columns long enough for the tag to wrap."""
    stride, max_layers = kernel_constants()
    wrap = 65536 // stride
    for n in (2, 3, 33, max_layers):
        for full in (True, False):
            for gap in (wrap - 1, wrap, wrap + 1):
                calls = [(full, n)] + [(False, 1)] * gap + [(full, n)] * 2
                assert run_sequence(calls, stride) == [], (full, n, gap)
    rng = random.Random(7)
    calls = [(rng.random() < 0.5, rng.choice([1, 1, 1, 2, 27, 33, max_layers]))
             for _ in range(4000)]
    assert run_sequence(calls, stride) == []


def test_the_replay_catches_a_stride_of_64():
    # stages 1 and 2 (polled by 2 and 3) meet the previous step's 65 and 66
    found = run_sequence([(True, 33)] * 3, 64)
    assert found and {s for _, _, _, s, _ in found} == {1, 2}
    assert run_sequence([(False, 64)] * 3, 64) == []


def test_the_replay_catches_a_missing_stamp():
    """Without the one-layer column's stamp, buffer 0 keeps a one-layer
    step's stage-2 word through 65536 / stride - 1 one-layer columns, and its
    tag has come round when the next step polls stage 2."""
    stride, _ = kernel_constants()
    calls = [(True, 1)] + [(False, 1)] * (65536 // stride - 1) + [(True, 4)]
    assert run_sequence(calls, stride, stamp=False) != []
    assert run_sequence(calls, stride) == []
