"""Task-descriptor adapter (fleet_moe.descriptors), on the CPU.

The byte layout is pinned against the reference's device struct
(src/runtime/fleet_runtime.h:87-107, checked there by
tests/test_descriptor_layout.py): every field at its C offset with its C type,
64 bytes in all. The planner is checked on a graph in the reference's shape
(taskgraph.py:366-441): MoE layers become calls, cross-cut waits and
FOLD_PARTIALS are cleared, incomplete layers are refused."""
from __future__ import annotations

import struct

import pytest

from fleet_moe import descriptors as D

# (field, struct code, byte offset) of struct TaskDescriptor, fleet_runtime.h:88-106
C_LAYOUT = [("kind", "H", 0), ("layer", "h", 2), ("xcd", "h", 4), ("worker", "h", 6),
            ("wait_event", "h", 8), ("signal_event", "h", 10), ("signal_scope", "h", 12),
            ("n_split", "h", 14), ("head", "h", 16), ("kv_chunk", "h", 18),
            ("expert_slot", "h", 20), ("wait_scope", "h", 22), ("wait_count", "h", 24),
            ("local_event", "h", 26), ("flags", "h", 28), ("signal_xcd_count", "h", 30),
            ("index", "i", 32)]


def test_descriptor_bytes_match_the_device_struct():
    vals = {n: (i + 1) * (-1 if i % 3 == 1 else 1) for i, (n, _, _) in enumerate(C_LAYOUT)}
    vals["kind"] = 6
    vals["index"] = 123456          # > 32767: needs the int32
    b = D.Descriptor(**vals).pack()
    assert len(b) == 64 == D.DESCRIPTOR_BYTES
    for name, code, off in C_LAYOUT:
        assert struct.unpack_from("<" + code, b, off)[0] == vals[name], name
    assert b[36:] == bytes(28)
    assert D.Descriptor.unpack(b) == D.Descriptor(**vals)
    assert D.field_offsets() == {n: o for n, _, o in C_LAYOUT}


def test_unpack_rejects_partial_descriptors():
    with pytest.raises(ValueError):
        D.unpack_all(bytes(100))
    assert D.unpack_all(b"") == []


def test_parse_events_sidecar():
    ev = D.parse_events("0 2 1 embed\n1 1 37 L0.norm.x0\n\n2 2 296 L1.down with spaces\n")
    assert [e.id for e in ev] == [0, 1, 2]
    assert ev[1] == D.Event(1, 1, 37, "L0.norm.x0")
    assert ev[2].label == "L1.down with spaces"
    with pytest.raises(ValueError):
        D.parse_events("3 1\n")


def _graph():
    """embed -> dense layer 0 -> layer 1 (qkv, o_proj, MoE) -> layer 2 (qkv
    folding layer 1's partials, o_proj, MoE) -> lm_head folding layer 2's ->
    argmax; events numbered in emission order."""
    K = D.TaskKind
    g = [D.Descriptor(K.EMBED, -1, 0, signal_event=0, signal_scope=D.Scope.GLOBAL)]
    g += [D.Descriptor(K.NORM_ROUTER, 0, x, wait_event=0, signal_event=1,
                       signal_scope=D.Scope.XCD_LOCAL) for x in range(8)]
    g += [D.Descriptor(K.DENSE_GATE_UP, 0, x, wait_event=1, signal_event=2,
                       signal_scope=D.Scope.GLOBAL) for x in range(8)]
    g += [D.Descriptor(K.DENSE_DOWN, 0, -1, wait_event=2, signal_event=3,
                       signal_scope=D.Scope.GLOBAL)]
    g += [D.Descriptor(K.QKV_FUSED, 1, 0, wait_event=3, signal_event=4),
          D.Descriptor(K.O_PROJ, 1, 0, wait_event=4, signal_event=5)]
    moe1, done1 = D.moe_layer_descriptors(1, wait_event=5, first_event=6)
    g += moe1
    g += [D.Descriptor(K.QKV_FUSED, 2, 0, wait_event=done1, signal_event=done1 + 1,
                       flags=D.Flags.FOLD_PARTIALS),
          D.Descriptor(K.O_PROJ, 2, 0, wait_event=done1 + 1, signal_event=done1 + 2)]
    moe2, done2 = D.moe_layer_descriptors(2, wait_event=done1 + 2, first_event=done1 + 3)
    g += moe2
    g += [D.Descriptor(K.LM_HEAD, -1, 0, wait_event=done2, signal_event=done2 + 1,
                       flags=D.Flags.FOLD_PARTIALS | D.Flags.SIGNAL_LAST),
          D.Descriptor(K.ARGMAX, -1, 0, wait_event=done2 + 1)]
    return [D.replace(d, index=i) for i, d in enumerate(g)], done1, done2


def test_plan_cuts_moe_layers_out_of_the_graph():
    g, done1, done2 = _graph()
    # the byte stream round trip feeds the planner the same list
    g = D.unpack_all(D.pack_all(g))
    steps = D.plan(g)
    kinds = [type(s).__name__ for s in steps]
    assert kinds == ["Segment", "MoeCall", "Segment", "MoeCall", "Segment"]
    assert [s.layer for s in steps if isinstance(s, D.MoeCall)] == [1, 2]
    seg0, seg1, seg2 = (s.descriptors for s in steps if isinstance(s, D.Segment))
    # the dense layer's NORM_ROUTER tasks stay in the graph
    assert sum(d.kind == D.TaskKind.NORM_ROUTER for d in seg0) == 8
    assert [d.kind for d in seg0][-2:] == [D.TaskKind.QKV_FUSED, D.TaskKind.O_PROJ]
    # waits inside a segment are kept, waits on earlier steps are cleared
    assert seg0[-1].wait_event == 4
    qkv2, oproj2 = seg1
    assert qkv2.wait_event == -1 and qkv2.wait_count == 0
    assert not qkv2.flags & D.Flags.FOLD_PARTIALS
    assert oproj2.wait_event == done1 + 1
    lm, am = seg2
    assert lm.wait_event == -1 and lm.flags == int(D.Flags.SIGNAL_LAST)
    assert am.wait_event == done2 + 1
    # indices are renumbered per segment; the MoE tasks are gone
    for seg in (seg0, seg1, seg2):
        assert [d.index for d in seg] == list(range(len(seg)))
        assert not any(d.kind in (D.TaskKind.EXPERT_GATE_UP, D.TaskKind.EXPERT_DOWN)
                       for d in seg)
    moe = steps[1].source
    assert moe.done_event == done1 and len(moe.routers) == 8 * D.WORKERS_PER_XCD
    assert sorted({d.expert_slot for d in moe.down}) == [-2, -1, 0, 1, 2, 3, 4, 5]


def test_plan_refuses_incomplete_moe_layers():
    g, _, _ = _graph()
    no_slot3 = [d for d in g if not (d.kind == D.TaskKind.EXPERT_DOWN and d.layer == 1
                                     and d.expert_slot == 3)]
    with pytest.raises(ValueError, match="EXPERT_DOWN slots"):
        D.plan(no_slot3)
    no_router = [d for d in g if not (d.kind == D.TaskKind.NORM_ROUTER and d.layer == 2
                                      and d.xcd == 5)]
    with pytest.raises(ValueError, match="NORM_ROUTER"):
        D.plan(no_router)
    split_down = [D.replace(d, signal_event=999) if (d.kind == D.TaskKind.EXPERT_DOWN and
                                                     d.layer == 1 and d.xcd == 0) else d
                  for d in g]
    with pytest.raises(ValueError, match="signal"):
        D.plan(split_down)


def test_plan_checks_events_against_the_sidecar():
    g, _, done2 = _graph()
    ev = [D.Event(i, 2, 1, f"e{i}") for i in range(done2 + 2)]
    assert len(D.plan(g, events=ev)) == 5
    with pytest.raises(ValueError, match="not in the event table"):
        D.plan(g, events=ev[:-1])


def test_moe_steps_need_weights_and_a_segment_runner():
    g, _, _ = _graph()
    steps = D.plan(g)
    with pytest.raises(KeyError):
        D.MoeSteps(steps, {1: object()}, decoder=None)
    calls = []

    class Dec:
        def decode_into(self, layer, x, x_out, stream=None):
            calls.append((layer, x is x_out))

    Dec.dims = None
    folds = []
    ms = D.MoeSteps(steps, {1: "w1", 2: "w2"}, Dec(),
                    fold=lambda x, p, out, dims, stream: folds.append((x, p, out)))
    with pytest.raises(RuntimeError):
        ms.run("x0", "x1", "p")
    with pytest.raises(ValueError, match="oproj_partials"):
        ms.run("x0", "x1", None, segment_runner=lambda s: None)
    segs = []
    calls.clear()
    folds.clear()
    ms.run("x0", "x1", "p", segment_runner=segs.append)
    # each call: x[1] = fold(x[0], partials), then the layer in place on x[1]
    assert folds == [("x0", "p", "x1")] * 2
    assert calls == [("w1", True), ("w2", True)] and len(segs) == 3
    # o_proj row-split graphs write x[1] themselves: no fold
    g2 = [D.replace(d, flags=d.flags | D.Flags.OPROJ_ROW_SPLIT)
          if d.kind == D.TaskKind.NORM_ROUTER and d.layer > 0 else d for d in g]
    folds.clear()
    D.MoeSteps(D.plan(g2), {1: "w1", 2: "w2"}, Dec(),
               fold=lambda *a: folds.append(a)).run("x0", "x1", segment_runner=segs.append)
    assert folds == []
