"""The descriptor adapter on graphs the reference itself emitted.

The fixtures under tests/golden/taskgraph/ were written by the reference's
src/host/taskgraph.py --emit (tests/golden/make_taskgraph_fixtures.py) for a
3-layer DeepSeek-V2-Lite config (layer 0 dense, layers 1 and 2 MoE) in five
variants: default, --topk-published, --split-workers 18, --oproj-row-split
and --local-fold. Each graph has the reference's per-worker fan-out (37
descriptors per chiplet task), K-chunk local events and the variant's flags.

For every variant plan() must give [segment, MoE call 1, segment, MoE call 2,
segment] whose segments are self-contained (every wait they keep is signalled
earlier in the same segment), hold no task of the MoE layers, and keep no
fold of expert partials (FOLD_PARTIALS, LOCAL_FOLD readers, head-1 REDUCE
publishers); a call folds o_proj's partials unless o_proj splits rows."""
from __future__ import annotations

import gzip
import json
from dataclasses import replace
from pathlib import Path

import pytest

from fleet_moe import descriptors as D

FIX = Path(__file__).resolve().parent / "golden" / "taskgraph"
INDEX = json.loads((FIX / "index.json").read_text())
VARIANTS = sorted(INDEX["variants"])
K = D.TaskKind
F = D.Flags


def load(name):
    descs = D.unpack_all(gzip.decompress((FIX / f"{name}.bin.gz").read_bytes()))
    events = D.parse_events(gzip.decompress((FIX / f"{name}.events.txt.gz").read_bytes()).decode())
    return descs, events


def test_fixture_index_matches_the_streams():
    assert set(VARIANTS) == {"default", "topk_published", "split_workers_18", "oproj_row_split",
                             "local_fold"}
    for name, meta in INDEX["variants"].items():
        descs, events = load(name)
        assert len(descs) == meta["descriptors"] and len(events) == meta["events"]
        assert meta["emitter_rc"] == 0
        assert [d.index for d in descs] == list(range(len(descs)))


@pytest.mark.parametrize("name", VARIANTS)
def test_reference_graph_plans_into_two_moe_calls(name):
    descs, events = load(name)
    steps = D.plan(descs, events=events)
    assert [type(s).__name__ for s in steps] == ["Segment", "MoeCall", "Segment", "MoeCall",
                                                 "Segment"]
    calls = [s for s in steps if isinstance(s, D.MoeCall)]
    segs = [s.descriptors for s in steps if isinstance(s, D.Segment)]
    assert [c.layer for c in calls] == [1, 2]
    for c in calls:
        assert c.fold_oproj == (name != "oproj_row_split")
        # per-worker fan-out: 37 router tasks on each of the 8 XCDs
        assert len(c.source.routers) == 8 * 37
        assert sorted({d.expert_slot for d in c.source.down}) == [-2, -1, 0, 1, 2, 3, 4, 5]
    for seg in segs:
        signalled = set()
        for d in seg:
            assert not (d.layer in (1, 2) and d.kind in D.MOE_KINDS)
            assert not d.flags & F.FOLD_PARTIALS, f"{K(d.kind).name} keeps FOLD_PARTIALS"
            if d.kind in (K.QKV_FUSED, K.LM_HEAD):
                assert not d.flags & F.LOCAL_FOLD or d.layer == 0
            if d.kind == K.REDUCE:
                assert d.head == 0 and d.layer == 0, "only the dense layer's o_proj fold stays"
            # self-contained: what a segment still waits for, it produces itself
            if d.wait_event >= 0:
                assert d.wait_event in signalled, f"{K(d.kind).name} {d.index} waits outside"
            if d.signal_event >= 0:
                signalled.add(d.signal_event)
        assert [d.index for d in seg] == list(range(len(seg)))
    # every descriptor is accounted for: in a segment, a call's layer, or absorbed
    n_moe = sum(len(c.source.routers) + len(c.source.gate_up) + len(c.source.down) for c in calls)
    n_abs = sum(len(c.absorbed) for c in calls)
    assert sum(map(len, segs)) + n_moe + n_abs == len(descs)
    if name == "local_fold":
        for c in calls:
            heads = sorted(d.head for d in c.absorbed)
            assert heads == [0] * 8 + [1] * 8
            assert all(d.flags & F.LOCAL_FOLD for d in c.absorbed)
    else:
        assert n_abs == 0
    # the first tasks after each call read the residual the call left in x[1]
    for seg, layer in ((segs[1], 2), (segs[2], -1)):
        first = [d for d in seg if d.kind in (K.QKV_FUSED, K.LM_HEAD) and d.layer == layer]
        assert len(first) == 8 * 37
        assert all(d.wait_event == -1 for d in first)


def _local_fold():
    descs, events = load("local_fold")
    return descs, {e.label: e.id for e in events}


def test_plan_refuses_a_foreign_reader_of_an_absorbed_fold():
    descs, ev = _local_fold()
    qkv2 = next(d for d in descs if d.kind == K.QKV_FUSED and d.layer == 2)
    bad = [replace(d, wait_event=ev["L1.local_fold0.x0"]) if d is qkv2 else d for d in descs]
    with pytest.raises(D.PlanError, match="o_proj fold of MoE layer 1"):
        D.plan(bad)


def test_plan_refuses_tasks_that_wait_inside_a_moe_layer():
    descs, ev = _local_fold()
    o2 = next(d for d in descs if d.kind == K.O_PROJ and d.layer == 2)
    bad = [replace(d, wait_event=ev["L1.norm.x3"]) if d is o2 else d for d in descs]
    with pytest.raises(D.PlanError, match="internal event of MoE layer 1"):
        D.plan(bad)


def test_plan_refuses_an_unknown_fold_of_expert_partials():
    descs, ev = _local_fold()
    r = next(d for d in descs if d.kind == K.REDUCE and d.head == 1)
    bad = [replace(d, head=2) if d is r else d for d in descs]
    with pytest.raises(D.PlanError, match="cannot be mapped"):
        D.plan(bad)
