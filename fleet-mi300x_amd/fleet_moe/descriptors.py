"""Task-descriptor adapter: route a task graph's MoE layers to this library.

The reference decode runs one persistent kernel over a list of 64-byte task
descriptors (src/host/taskgraph.py:64-68 packs them; src/runtime/
fleet_runtime.h:87-107 is the device struct). A MoE layer is three task kinds
in that list (taskgraph.py:366-441):

  NORM_ROUTER (4)      one per XCD: post-attention RMSNorm + router logits
  EXPERT_GATE_UP (5)   one per XCD, `expert_slot` 0..top_k-1 (routed slot) or
                       -1 / -2 (the two halves of the shared expert)
  EXPERT_DOWN (6)      the same slots; all of them signal one GLOBAL event

and the consumer of that event (the next layer's first tasks, or LM_HEAD)
carries FOLD_PARTIALS: its prologue adds the eight expert partials to the
residual stream.

The residual stream is two buffers (fleet_types.h Activations.x): x[0], the
layer input, and x[1], the residual after attention. The NORM_ROUTER prologue
forms x[1] = bf16(x[0] + bf16(sum of o_proj's eight fp32 partials))
(fleet_kernel.hip:405-425), unless o_proj splits rows (OPROJ_ROW_SPLIT) and
writes x[1] itself. With --local-fold (taskgraph.py:752-829) the folds move
into REDUCE tasks, one per XCD: head 0 forms x[1] for the NORM_ROUTER tasks,
head 1 adds an MoE layer's expert partials for the next QKV_FUSED / LM_HEAD
tasks, which then read the REDUCE's per-XCD copy (LOCAL_FOLD).

`plan()` reads such a list (and the `.events.txt` sidecar, when given) and cuts
it into graph segments around every MoE layer. Each MoE layer becomes one
`MoeCall`: `fleet_moe_residual_fold` (x[0] + o_proj partials -> x[1]) when
the layer's o_proj is K-split, then `fleet_moe_layer_decode` in place on
x[1], which does the norm, routing, experts, combine and residual add, so
x[1] leaves the call as the next layer's input and no expert partials exist.
Accordingly:
  * the layer's head-0 REDUCE tasks are absorbed into its call (the call
    folds o_proj's partials itself);
  * head-1 REDUCE tasks that fold its expert partials are dropped, and their
    consumers lose LOCAL_FOLD and FOLD_PARTIALS and read x[1];
  * waits on events produced before a cut are satisfied by stream order and
    cleared; FOLD_PARTIALS is cleared on the consumers of the layer's done
    event.
Every MoE layer must be complete (a router task on every XCD, gate_up and down
for every routed slot and both shared halves), and no task outside the layer
may wait on one of its internal events, or `plan()` raises `PlanError`.

`MoeSteps.run()` executes the MoE calls of a plan on this library; the graph
segments are left to the runtime that owns them.
"""
from __future__ import annotations

import struct
from dataclasses import dataclass, field, replace
from enum import IntEnum, IntFlag

DESCRIPTOR_BYTES = 64
# Field order and widths of struct TaskDescriptor (fleet_runtime.h:87-107):
# kind u16, fifteen i16, index i32, 28 bytes of padding, little-endian.
_FORMAT = "<H15hi28x"
assert struct.calcsize(_FORMAT) == DESCRIPTOR_BYTES
FIELD_NAMES = ("kind", "layer", "xcd", "worker", "wait_event", "signal_event",
               "signal_scope", "n_split", "head", "kv_chunk", "expert_slot",
               "wait_scope", "wait_count", "local_event", "flags",
               "signal_xcd_count", "index")
N_XCDS = 8


class TaskKind(IntEnum):
    """Task kinds (taskgraph.py:73-88); the MoE path is 4, 5 and 6."""
    QKV_FUSED = 0
    ATTENTION = 1
    MERGE_UV = 2
    O_PROJ = 3
    NORM_ROUTER = 4
    EXPERT_GATE_UP = 5
    EXPERT_DOWN = 6
    REDUCE = 7
    DENSE_GATE_UP = 8
    DENSE_DOWN = 9
    EMBED = 10
    LM_HEAD = 11
    ARGMAX = 12
    PREFETCH = 13
    Q_ABSORB = 14


class Flags(IntFlag):
    """Descriptor flag bits (taskgraph.py:91-126, fleet_runtime.h TaskFlags)."""
    NONE = 0
    FOLD_PARTIALS = 1
    SIGNAL_LAST = 2
    CHUNK_SIGNAL = 8
    CHUNK_WAIT = 16
    KVA_SHARED = 32
    WORKER_GROUP = 64
    ROUTING_CACHED = 128
    TOPK_PUBLISH = 256
    TOPK_READ = 512
    PUB_WAIT = 1024
    OPROJ_ROW_SPLIT = 2048
    LOCAL_FOLD = 4096
    LOCAL_KVA = 8192


class Scope(IntEnum):
    """Event scope (taskgraph.py:147-151)."""
    NONE = 0
    XCD_LOCAL = 1
    GLOBAL = 2


MOE_KINDS = (TaskKind.NORM_ROUTER, TaskKind.EXPERT_GATE_UP, TaskKind.EXPERT_DOWN)


@dataclass(frozen=True)
class Descriptor:
    """One 64-byte task descriptor; -1 means "none" for event fields."""
    kind: int
    layer: int = -1
    xcd: int = -1
    worker: int = -1
    wait_event: int = -1
    signal_event: int = -1
    signal_scope: int = 0
    n_split: int = 1
    head: int = -1
    kv_chunk: int = -1
    expert_slot: int = -1
    wait_scope: int = 0
    wait_count: int = 0
    local_event: int = -1
    flags: int = 0
    signal_xcd_count: int = 0
    index: int = -1

    def pack(self) -> bytes:
        return struct.pack(_FORMAT, *(getattr(self, n) for n in FIELD_NAMES))

    @classmethod
    def unpack(cls, b: bytes) -> "Descriptor":
        return cls(*struct.unpack(_FORMAT, b))


def pack_all(descs) -> bytes:
    return b"".join(d.pack() for d in descs)


def unpack_all(buf: bytes) -> list[Descriptor]:
    if len(buf) % DESCRIPTOR_BYTES:
        raise ValueError(f"descriptor stream of {len(buf)} bytes is not a multiple of "
                         f"{DESCRIPTOR_BYTES}")
    return [Descriptor.unpack(buf[o:o + DESCRIPTOR_BYTES])
            for o in range(0, len(buf), DESCRIPTOR_BYTES)]


@dataclass(frozen=True)
class Event:
    id: int
    scope: int
    producers: int
    label: str


def parse_events(text: str) -> list[Event]:
    """The `.events.txt` sidecar: one `id scope producers label` per line
    (taskgraph.py:835-837)."""
    out = []
    for ln, line in enumerate(text.splitlines(), 1):
        if not line.strip():
            continue
        parts = line.split(maxsplit=3)
        if len(parts) < 3:
            raise ValueError(f"events line {ln}: expected `id scope producers label`")
        out.append(Event(int(parts[0]), int(parts[1]), int(parts[2]),
                         parts[3] if len(parts) > 3 else ""))
    return out


@dataclass
class MoeLayer:
    """The MoE tasks of one layer, as found in the graph."""
    layer: int
    routers: list[Descriptor] = field(default_factory=list)
    gate_up: list[Descriptor] = field(default_factory=list)
    down: list[Descriptor] = field(default_factory=list)

    @property
    def done_event(self) -> int:
        ev = {d.signal_event for d in self.down}
        if len(ev) != 1:
            raise ValueError(f"layer {self.layer}: expert down tasks signal {sorted(ev)}, "
                             "expected one event")
        return ev.pop()

    def check(self, top_k: int, n_xcds: int = N_XCDS) -> None:
        want = set(range(top_k)) | {-1, -2}
        if {d.xcd for d in self.routers} != set(range(n_xcds)):
            raise ValueError(f"layer {self.layer}: NORM_ROUTER tasks on XCDs "
                             f"{sorted({d.xcd for d in self.routers})}, expected all {n_xcds}")
        for name, group in (("EXPERT_GATE_UP", self.gate_up), ("EXPERT_DOWN", self.down)):
            got = {d.expert_slot for d in group}
            if got != want:
                raise ValueError(f"layer {self.layer}: {name} slots {sorted(got)}, "
                                 f"expected {sorted(want)}")
        _ = self.done_event


class PlanError(ValueError):
    """A task graph that cannot be mapped onto the library's MoE calls."""


@dataclass
class Segment:
    """Graph descriptors to run as one launch of the owning runtime."""
    descriptors: list[Descriptor]


@dataclass
class MoeCall:
    """One MoE layer replaced by library calls: the o_proj fold into x[1]
    (when `fold_oproj`), then fleet_moe_layer_decode in place on x[1].
    `absorbed` lists the graph's REDUCE tasks the call replaces."""
    layer: int
    source: MoeLayer
    fold_oproj: bool = True
    absorbed: list[Descriptor] = field(default_factory=list)


def _moe_layers(descs: list[Descriptor]) -> dict[int, MoeLayer]:
    expert_layers = {d.layer for d in descs
                     if d.kind in (TaskKind.EXPERT_GATE_UP, TaskKind.EXPERT_DOWN)}
    out: dict[int, MoeLayer] = {}
    for d in descs:
        if d.layer not in expert_layers or d.kind not in MOE_KINDS:
            continue
        m = out.setdefault(d.layer, MoeLayer(d.layer))
        {TaskKind.NORM_ROUTER: m.routers, TaskKind.EXPERT_GATE_UP: m.gate_up,
         TaskKind.EXPERT_DOWN: m.down}[TaskKind(d.kind)].append(d)
    return out


def _internal_events(m: MoeLayer) -> set[int]:
    """Events a MoE layer's tasks signal or use locally, except its done event."""
    ev = set()
    for d in m.routers + m.gate_up + m.down:
        for e in (d.signal_event, d.local_event):
            if e >= 0:
                ev.add(e)
    ev.discard(m.done_event)
    return ev


def plan(descs: list[Descriptor], top_k: int = 6, events: list[Event] | None = None,
         n_xcds: int = N_XCDS) -> list[Segment | MoeCall]:
    """Cut a descriptor list into runtime segments and MoE calls, in order.

    A MoE layer is a layer with EXPERT_GATE_UP / EXPERT_DOWN tasks; its
    NORM_ROUTER tasks go with it (a dense layer's NORM_ROUTER tasks stay in the
    graph). The call takes the place of the layer's first MoE descriptor."""
    if events is not None:
        ids = {e.id for e in events}
        for d in descs:
            for ev in (d.wait_event, d.signal_event):
                if ev >= 0 and ev not in ids:
                    raise PlanError(f"descriptor {d.index}: event {ev} not in the event table")
    layers = _moe_layers(descs)
    for m in layers.values():
        m.check(top_k, n_xcds)
    done = {m.done_event: m.layer for m in layers.values()}
    internal = {e: m.layer for m in layers.values() for e in _internal_events(m)}
    waiters: dict[int, list[Descriptor]] = {}
    for d in descs:
        if d.wait_event >= 0:
            waiters.setdefault(d.wait_event, []).append(d)

    calls: dict[int, MoeCall] = {}
    for L, m in layers.items():
        split = {bool(d.flags & Flags.OPROJ_ROW_SPLIT) for d in m.routers}
        if len(split) != 1:
            raise PlanError(f"layer {L}: NORM_ROUTER tasks disagree on OPROJ_ROW_SPLIT")
        calls[L] = MoeCall(L, m, fold_oproj=not split.pop())

    # --local-fold publishers: head 0 before an MoE layer's routers (absorbed),
    # head 1 after it (dropped; its readers read x[1] instead)
    absorbed: set[int] = set()          # id() of REDUCE descriptors taken out
    retired: dict[int, int] = {}        # head-1 publication event -> MoE layer
    for d in descs:
        if d.kind != TaskKind.REDUCE or not d.flags & Flags.LOCAL_FOLD:
            continue
        readers = waiters.get(d.signal_event, [])
        if d.head == 0 and d.layer in layers:
            bad = [r for r in readers if not (r.kind == TaskKind.NORM_ROUTER and r.layer == d.layer)]
            if bad:
                raise PlanError(f"REDUCE {d.index} (o_proj fold of MoE layer {d.layer}) is read "
                                f"by tasks other than the layer's routers: {[r.index for r in bad]}")
            calls[d.layer].absorbed.append(d)
            absorbed.add(id(d))
        elif d.head == 1 and d.wait_event in done:
            L = done[d.wait_event]
            bad = [r for r in readers if r.kind not in (TaskKind.QKV_FUSED, TaskKind.LM_HEAD)]
            if bad:
                raise PlanError(f"REDUCE {d.index} (expert fold of MoE layer {L}) is read by "
                                f"unexpected tasks {[r.index for r in bad]}")
            calls[L].absorbed.append(d)
            absorbed.add(id(d))
            retired[d.signal_event] = L
        elif d.wait_event in done or d.wait_event in internal:
            raise PlanError(f"REDUCE {d.index} (head {d.head}) waits on MoE layer "
                            f"{done.get(d.wait_event, internal.get(d.wait_event))}, "
                            "which this library replaces; its fold cannot be mapped")

    steps: list[Segment | MoeCall] = []
    produced_before: set[int] = set()     # events signalled by earlier steps
    cur: list[Descriptor] = []
    seg_events: set[int] = set()
    emitted: set[int] = set()

    def close_segment():
        nonlocal cur, seg_events
        if cur:
            steps.append(Segment(cur))
            produced_before.update(seg_events)
        cur, seg_events = [], set()

    for d in descs:
        if d.layer in layers and d.kind in MOE_KINDS:
            if d.layer not in emitted:
                close_segment()
                steps.append(calls[d.layer])
                emitted.add(d.layer)
                m = layers[d.layer]
                produced_before.update({t.signal_event for t in m.routers + m.gate_up + m.down
                                        if t.signal_event >= 0})
                produced_before.update({t.signal_event for t in calls[d.layer].absorbed})
            continue
        if id(d) in absorbed:
            continue
        if d.wait_event in internal:
            raise PlanError(f"descriptor {d.index} ({TaskKind(d.kind).name}) waits on an "
                            f"internal event of MoE layer {internal[d.wait_event]}")
        nd = d
        if d.wait_event in retired:
            L = retired[d.wait_event]
            if L not in emitted:
                raise PlanError(f"descriptor {d.index} reads MoE layer {L}'s fold before the layer")
            nd = replace(nd, flags=int(Flags(nd.flags) & ~(Flags.LOCAL_FOLD | Flags.FOLD_PARTIALS)))
        if d.wait_event in done:
            nd = replace(nd, flags=int(Flags(nd.flags) & ~Flags.FOLD_PARTIALS))
        if nd.wait_event >= 0 and nd.wait_event in produced_before:
            # satisfied by stream order: the producer ran in an earlier step
            nd = replace(nd, wait_event=-1, wait_scope=0, wait_count=0)
        cur.append(replace(nd, index=len(cur)))
        if d.signal_event >= 0:
            seg_events.add(d.signal_event)
    close_segment()
    return steps


class MoeSteps:
    """Runs the MoE calls of a plan: fleet_moe_residual_fold (for a call with
    `fold_oproj`), then fleet_moe_layer_decode in place on x[1].

    `layers` maps a graph layer index to a `DeviceLayer`; one decoder (and its
    workspace) serves all of them, in order, on one stream. `fold` is
    `ops.residual_fold` unless given."""

    def __init__(self, steps: list[Segment | MoeCall], layers: dict, decoder, fold=None):
        self.steps = steps
        self.layers = layers
        self.decoder = decoder
        if fold is None:
            from .ops import residual_fold as fold
        self.fold = fold
        missing = [s.layer for s in steps if isinstance(s, MoeCall) and s.layer not in layers]
        if missing:
            raise KeyError(f"no weights for MoE layers {missing}")

    def run(self, x_in, x_mid, oproj_partials=None, segment_runner=None, stream=None) -> None:
        """The runtime's residual buffers, fp32 device tensors: x_in = x[0]
        (the layer input), x_mid = x[1] (the residual after attention; each
        MoE call leaves the next layer's input there), oproj_partials = o_proj's
        K-split partials [n][hidden] (read by calls with `fold_oproj`).
        `segment_runner(segment)` runs the non-MoE descriptors (the owning
        runtime, which fills those buffers); without one, only MoE calls may
        appear in the plan. Nothing is allocated."""
        for s in self.steps:
            if isinstance(s, MoeCall):
                if s.fold_oproj:
                    if oproj_partials is None:
                        raise ValueError(f"MoE layer {s.layer} folds o_proj's partials: "
                                         "pass oproj_partials")
                    self.fold(x_in, oproj_partials, x_mid, self.decoder.dims, stream)
                self.decoder.decode_into(self.layers[s.layer], x_mid, x_mid, stream=stream)
            elif segment_runner is not None:
                segment_runner(s)
            else:
                raise RuntimeError("plan has graph segments but no segment_runner")


WORKERS_PER_XCD = 37       # worker workgroups per XCD of the reference runtime
WAVES_PER_WORKER = 4       # its waves per workgroup (producers of a K-chunk event)
EXPERT_K_CHUNK = 2048      # rows of h per gate_up -> down event (>= moe_inter: one chunk)


@dataclass
class LayerEmit:
    """One emitted MoE layer: its descriptors (finalized), the events it
    created (in id order, for the `.events.txt` sidecar) and the id of the
    event the next layer waits on."""
    descriptors: list[Descriptor]
    events: list[Event]
    done_event: int


def emit_moe_layer(layer: int, wait_event, first_event: int, first_index: int = 0, *,
                   wait_scope: int = Scope.GLOBAL, wait_count: int = N_XCDS * WORKERS_PER_XCD,
                   top_k: int = 6, moe_inter: int = 1408, k_chunk: int = EXPERT_K_CHUNK,
                   n_xcds: int = N_XCDS, workers: int = WORKERS_PER_XCD,
                   waves: int = WAVES_PER_WORKER, topk_published: bool = False,
                   split_workers: int = 0, oproj_row_split: bool = False,
                   router_flags: int = 0) -> LayerEmit:
    """The descriptors of one MoE layer as the reference's emitter writes them
    (taskgraph.py:366-441, then finalize :500-523), for a caller that builds
    its own task list around this library's MoE calls or checks a graph.

    Events, from `first_event` on: per XCD the router event `L{l}.norm.x{x}`
    (XCD-local, one producer per worker) and, with `topk_published`, the
    top-k publication `L{l}.topk.x{x}`; per XCD the K-chunk events
    `L{l}.gate_up.x{x}.k{c}` (XCD-local, one producer per wave of the gate_up
    workers; ceil(moe_inter / k_chunk) of them, consecutive ids); then the
    layer's GLOBAL `L{l}.down` (one producer per down worker and XCD).
    Descriptors, from `first_index` on, one per worker of each XCD's chiplet
    task: NORM_ROUTER, then EXPERT_GATE_UP, then EXPERT_DOWN, the expert slot
    of XCD x being x for x < top_k and -(x - top_k + 1) (a shared half) after.
    `split_workers` G > 0 puts gate_up on workers [0, G) and down on [G,
    workers) of every XCD (WORKER_GROUP; head = the group's first worker,
    n_split = its size); otherwise down carries ROUTING_CACHED.
    `wait_event` is what the router tasks wait on: one id, or one per XCD
    (the --local-fold per-XCD folds, whose `router_flags` add LOCAL_FOLD),
    with that event's `wait_scope` and `wait_count`. finalize's fields are
    filled in: every waiter carries its event's scope and producer count,
    every signaller the count of its event's producers on its own XCD."""
    waits = list(wait_event) if isinstance(wait_event, (list, tuple)) else [wait_event] * n_xcds
    if len(waits) != n_xcds:
        raise ValueError(f"{len(waits)} wait events for {n_xcds} XCDs")
    if not 0 <= split_workers < workers:
        raise ValueError(f"split_workers {split_workers} outside [0, {workers})")
    events: list[Event] = []

    def new_event(scope, producers, label) -> int:
        events.append(Event(first_event + len(events), int(scope), int(producers), label))
        return events[-1].id

    n_chunks = -(-moe_inter // k_chunk)
    G = split_workers
    gu_group = list(range(G)) if G else list(range(workers))
    dn_group = list(range(G, workers)) if G else list(range(workers))
    e_router, e_pub = [], []
    for x in range(n_xcds):
        e_router.append(new_event(Scope.XCD_LOCAL, workers, f"L{layer}.norm.x{x}"))
        e_pub.append(new_event(Scope.XCD_LOCAL, workers, f"L{layer}.topk.x{x}")
                     if topk_published else -1)
    e_chunk0 = []
    for x in range(n_xcds):
        ids = [new_event(Scope.XCD_LOCAL, len(gu_group) * waves, f"L{layer}.gate_up.x{x}.k{c}")
               for c in range(n_chunks)]
        e_chunk0.append(ids[0])
    e_down = new_event(Scope.GLOBAL, n_xcds * len(dn_group), f"L{layer}.down")
    by_id = {e.id: e for e in events}

    def slot_of(x: int) -> int:
        return x if x < top_k else -(x - top_k + 1)

    read = Flags.TOPK_READ if topk_published else Flags.NONE
    out: list[Descriptor] = []

    def add(kind, x, group, split, **kw):
        extra = {}
        if split:
            extra = {"flags": kw.pop("flags") | Flags.WORKER_GROUP, "head": group[0],
                     "n_split": len(group)}
        for w in group:
            out.append(Descriptor(int(kind), layer, x, w, index=first_index + len(out),
                                  **{**kw, **extra}))

    def internal_wait(e: int) -> dict:
        ev = by_id[e]
        return {"wait_event": e, "wait_scope": ev.scope, "wait_count": ev.producers}

    nr = (Flags.TOPK_PUBLISH if topk_published else Flags.NONE) | \
         (Flags.OPROJ_ROW_SPLIT if oproj_row_split else Flags.NONE) | Flags(router_flags)
    for x in range(n_xcds):
        add(TaskKind.NORM_ROUTER, x, list(range(workers)), False, wait_event=waits[x],
            wait_scope=int(wait_scope), wait_count=int(wait_count),
            signal_event=e_router[x], signal_scope=int(Scope.XCD_LOCAL), n_split=workers,
            local_event=e_pub[x], flags=int(nr), signal_xcd_count=workers)
    for x in range(n_xcds):
        add(TaskKind.EXPERT_GATE_UP, x, gu_group, bool(G), **internal_wait(e_router[x]),
            expert_slot=slot_of(x), local_event=e_chunk0[x], kv_chunk=n_chunks,
            flags=int(Flags.CHUNK_SIGNAL | read))
    dn_flags = Flags.CHUNK_WAIT | read | (Flags.NONE if G else Flags.ROUTING_CACHED)
    for x in range(n_xcds):
        add(TaskKind.EXPERT_DOWN, x, dn_group, bool(G), **internal_wait(e_chunk0[x]),
            signal_event=e_down, signal_scope=int(Scope.GLOBAL), expert_slot=slot_of(x),
            local_event=e_chunk0[x], kv_chunk=n_chunks, flags=int(dn_flags),
            signal_xcd_count=len(dn_group))
    return LayerEmit(out, events, e_down)


def moe_layer_descriptors(layer: int, wait_event: int, first_event: int, top_k: int = 6,
                          n_xcds: int = N_XCDS, workers: int = WORKERS_PER_XCD,
                          oproj_row_split: bool = False) -> tuple[list[Descriptor], int]:
    """emit_moe_layer's descriptors and done event (indices from 0)."""
    e = emit_moe_layer(layer, wait_event, first_event, top_k=top_k, n_xcds=n_xcds,
                       workers=workers, oproj_row_split=oproj_row_split)
    return e.descriptors, e.done_event


def events_text(events) -> str:
    """The `.events.txt` sidecar of `events` (taskgraph.py:832-839 grammar)."""
    return "".join(f"{e.id} {e.scope} {e.producers} {e.label}\n" for e in events)


def field_offsets() -> dict[str, int]:
    """Byte offset of every named field in the packed descriptor."""
    offs, off = {}, 0
    for n in FIELD_NAMES:
        offs[n] = off
        off += 2 if n != "index" else 4
    return offs


__all__ = ["DESCRIPTOR_BYTES", "FIELD_NAMES", "TaskKind", "Flags", "Scope", "Descriptor",
           "Event", "MoeLayer", "PlanError", "Segment", "MoeCall", "MoeSteps", "pack_all", "unpack_all",
           "parse_events", "plan", "LayerEmit", "emit_moe_layer", "moe_layer_descriptors",
           "events_text", "field_offsets", "WORKERS_PER_XCD", "WAVES_PER_WORKER",
           "EXPERT_K_CHUNK"]
