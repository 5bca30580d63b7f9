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


# ---------------------------------------------------------------- the emit side

EMIT_CFG = {
    "default": {},
    "topk_published": {"topk_published": True},
    "split_workers_18": {"split_workers": 18},
    "oproj_row_split": {"oproj_row_split": True},
    "local_fold": {"router_flags": int(F.LOCAL_FOLD)},
}


@pytest.mark.parametrize("name", VARIANTS)
@pytest.mark.parametrize("layer", [1, 2])
def test_emitted_moe_layer_equals_the_reference_emitters(name, layer):
    """emit_moe_layer writes, field for field, the MoE layer the reference's
    taskgraph.py wrote into the fixture: the same descriptors in the same
    order with the same indices, and the same events (id, scope, producer
    count, label) in the sidecar. Where the layer starts (first index, first
    event id) and what its routers wait on are read from the fixture."""
    descs, events = load(name)
    moe = [d for d in descs if d.layer == layer and d.kind in D.MOE_KINDS]
    lo, hi = moe[0].index, moe[-1].index
    assert [d.index for d in moe] == list(range(lo, hi + 1)), "contiguous in the stream"
    mine = [e for e in events if e.label.startswith(f"L{layer}.")
            and e.label.split(".")[1] in ("norm", "topk", "gate_up", "down")]
    routers = [d for d in moe if d.kind == K.NORM_ROUTER]
    waits = [next(d.wait_event for d in routers if d.xcd == x) for x in range(8)]
    if len(set(waits)) == 1:
        waits = waits[0]
    got = D.emit_moe_layer(layer, waits, mine[0].id, lo, wait_scope=routers[0].wait_scope,
                           wait_count=routers[0].wait_count, **EMIT_CFG[name])
    assert len(got.descriptors) == len(moe)
    for g, w in zip(got.descriptors, moe):
        assert g == w, f"{name} L{layer} index {w.index}:\n got  {g}\n want {w}"
    assert got.events == mine
    assert got.done_event == next(e.id for e in mine if e.label == f"L{layer}.down")
    assert D.events_text(got.events) == "".join(
        f"{e.id} {e.scope} {e.producers} {e.label}\n" for e in mine)


def test_emitted_layer_round_trips_through_the_planner():
    """A graph whose MoE layer is emitted here plans into one MoE call with
    the emitted done event, and its consumer loses FOLD_PARTIALS."""
    lay = D.emit_moe_layer(1, wait_event=0, first_event=1, first_index=1)
    head = D.Descriptor(int(K.O_PROJ), 1, 0, 0, signal_event=0, signal_scope=int(D.Scope.GLOBAL),
                        index=0)
    tail = D.Descriptor(int(K.LM_HEAD), -1, 0, 0, wait_event=lay.done_event,
                        wait_scope=int(D.Scope.GLOBAL), wait_count=8 * 37,
                        flags=int(F.FOLD_PARTIALS), index=1 + len(lay.descriptors))
    stream = D.unpack_all(D.pack_all([head] + lay.descriptors + [tail]))
    steps = D.plan(stream, events=[D.Event(0, 2, 1, "L1.oproj")] + lay.events)
    calls = [s for s in steps if isinstance(s, D.MoeCall)]
    assert len(calls) == 1 and calls[0].source.done_event == lay.done_event
    last = [s for s in steps if isinstance(s, D.Segment)][-1].descriptors
    assert last[0].kind == K.LM_HEAD and not last[0].flags & F.FOLD_PARTIALS
