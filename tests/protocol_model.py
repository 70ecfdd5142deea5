"""Host models of the two synchronisation protocols of the whole-step kernels,
explored over every interleaving of their workgroups.

Each workgroup is a list of operations (write an exchange slot, read one,
publish a counter or flag, wait for counters or flags) taken from the
kernels' own schedules:

* column kernel (lich_amd/csrc/ipc_narrow.hip, ``narrow_kernel`` /
  ``grid_barrier`` / ``barrier_exit``): phase A of every column block, a grid
  barrier on an arrival counter, phase B of every weight tile, a barrier
  between steps, and the exit counter whose last arrival clears both counters
  for the next launch;
* layer-resident kernel (lich_amd/csrc/ipc_resident.hip, ``run_hidden`` /
  ``run_top`` / ``publish`` / ``wait_peers`` / ``load_epoch``): hidden
  workgroup l writes eps[l] and W[l]^T eps[l] records (double-buffered,
  triple next to the top layer), the top chunks write partial products and
  chunk 0 of each row block the summed eps[L-1], every workgroup raises its
  step flag and waits for its peers (the top chunks for workgroup L-2 one
  step behind); the flags count steps across launches and are never
  cleared.

A slot remembers the step whose value it holds; every read names the step it
must see, so a read before its write (a missing wait) and an overwrite before
the last read (a missing wait in the other direction, or too few buffers)
both show up as a read of the wrong step.  A state in which no workgroup can
move and some have not finished is a deadlock.  Publishes and waits are
modelled as release / acquire operations (the kernels' agent-scope release
fence before a flag store, acquire fence after the poll): the model checks the
ordering logic of the schedules, not the hardware's memory ordering.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Callable


@dataclass(frozen=True)
class Op:
    kind: str                 # "write", "read", "publish", "wait", "add", "exit"
    key: tuple = ()           # slot or flag name
    value: int = 0            # step written / expected, or flag value
    conds: tuple = ()         # wait: ((flag, minimum), ...)


class Violation(AssertionError):
    pass


@dataclass
class Model:
    programs: dict                          # workgroup -> list[Op]
    init_flags: dict = field(default_factory=dict)
    init_slots: dict = field(default_factory=dict)
    final_check: Callable | None = None     # called with the flags once every workgroup has finished

    def explore(self, limit: int = 2_000_000) -> int:
        """Visits every reachable state; returns how many.  Raises Violation on
        a wrong read or a deadlock.  The shared state is a function of the
        program counters (every slot and flag has one writer per value), so
        visited program-counter tuples identify states."""
        names = list(self.programs)
        progs = [self.programs[n] for n in names]
        start = tuple(0 for _ in names)
        seen = {start}
        stack = [(start, dict(self.init_flags), dict(self.init_slots))]
        while stack:
            pcs, flags, slots = stack.pop()
            moved = False
            for i, prog in enumerate(progs):
                pc = pcs[i]
                if pc >= len(prog):
                    continue
                op = prog[pc]
                nflags, nslots = flags, slots
                if op.kind == "wait":
                    if not all(flags.get(f, 0) >= v for f, v in op.conds):
                        continue
                elif op.kind == "publish":
                    nflags = dict(flags)
                    nflags[op.key] = op.value
                elif op.kind == "add":
                    nflags = dict(flags)
                    nflags[op.key] = flags.get(op.key, 0) + 1
                elif op.kind == "exit":
                    # last arrival on the exit counter clears the counters it names
                    nflags = dict(flags)
                    prev = flags.get(op.key, 0)
                    nflags[op.key] = prev + 1
                    if prev + 1 == op.value:
                        for k in op.conds:
                            nflags[k] = 0
                elif op.kind == "write":
                    nslots = dict(slots)
                    nslots[op.key] = op.value
                elif op.kind == "read":
                    got = slots.get(op.key)
                    if got != op.value:
                        raise Violation(f"{names[i]} read {op.key} holding step {got}, expected step {op.value}")
                else:
                    raise ValueError(op.kind)
                moved = True
                npcs = pcs[:i] + (pc + 1,) + pcs[i + 1:]
                if npcs not in seen:
                    seen.add(npcs)
                    if len(seen) > limit:
                        raise RuntimeError("state limit reached")
                    stack.append((npcs, nflags, nslots))
            if not moved and any(pcs[i] < len(progs[i]) for i in range(len(progs))):
                blocked = [names[i] for i in range(len(progs)) if pcs[i] < len(progs[i])]
                raise Violation(f"deadlock: {blocked} cannot move")
            if not moved and self.final_check is not None:
                self.final_check(flags)
        return len(seen)


# --------------------------------------------------------------------------- column kernel
def column_kernel(nblocks: int, ntile: int, steps: int, launches: int = 2, *, drop_barrier: bool = False,
                  exit_clears: tuple = ("bar0", "bar1")) -> Model:
    """One or more multi-step launches of the column kernel with one column
    block (block 0 runs phase A) and ``ntile`` weight tiles dealt to the
    blocks round-robin.  Phase A reads every W tile and writes eps; phase B
    reads eps and writes its W tile.  Launch n+1 starts when every block of
    launch n has finished (stream order), so its operations follow the
    previous launch's in each block's program and the counters carry over.
    ``drop_barrier`` (no wait at the first barrier) and ``exit_clears`` (the
    counters the last exit clears) plant mistakes for the tests."""
    progs = {b: [] for b in range(nblocks)}
    version = 0  # W version at the start of the launch
    for _ in range(launches):
        nbar = 0
        for s in range(steps):
            wv = version + s
            # phase A (column block 0 on block 0)
            progs[0] += [Op("read", ("W", t), wv) for t in range(ntile)]
            progs[0].append(Op("write", ("e",), wv))
            for b in range(nblocks):
                progs[b].append(Op("add", ("bar0",)))
                if not drop_barrier:
                    progs[b].append(Op("wait", conds=((("bar0",), (nbar + 1) * nblocks),)))
            nbar += 1
            # phase B
            for t in range(ntile):
                b = t % nblocks
                progs[b] += [Op("read", ("e",), wv), Op("read", ("W", t), wv), Op("write", ("W", t), wv + 1)]
            if s + 1 < steps:
                for b in range(nblocks):
                    progs[b] += [Op("add", ("bar0",)), Op("wait", conds=((("bar0",), (nbar + 1) * nblocks),))]
                nbar += 1
        for b in range(nblocks):
            progs[b].append(Op("exit", ("bar1",), nblocks, tuple((c,) for c in exit_clears)))
        version += steps
    return _with_launch_order(progs, nblocks, ntile, launches)


def _with_launch_order(progs, nblocks, ntile, launches):
    """Stream order between launches: after its exit each block raises a
    "done" flag, and no block starts launch n + 1 before every block's flag of
    launch n is up.  Checks at the end that the counters are back at zero."""
    out = {}
    for b, prog in progs.items():
        new, n = [], 0
        for op in prog:
            new.append(op)
            if op.kind == "exit":
                n += 1
                new.append(Op("publish", ("done", b, n), 1))
                if n < launches:
                    new.append(Op("wait", conds=tuple((("done", c, n), 1) for c in range(nblocks))))
        out[b] = new

    def final(flags):
        if flags.get(("bar0",), 0) != 0 or flags.get(("bar1",), 0) != 0:
            raise Violation(f"counters not cleared at the end: bar0={flags.get(('bar0',))} "
                            f"bar1={flags.get(('bar1',))}")

    return Model(out, init_slots={("W", t): 0 for t in range(ntile)}, final_check=final)


# --------------------------------------------------------------------------- layer-resident kernel
def resident_kernel(hidden: int, chunks: int, halves: int, steps: int, *, launches: int = 1, g_buffers_top: int = 3,
                    top_waits_l2: bool = True, chunk0_waits_siblings: bool = True,
                    hidden_waits_up: bool = True, reset_base: bool = False, xn_wait: bool = True) -> Model:
    """``launches`` launches of the layer-resident kernel: hidden workgroups
    0..hidden-1 (hidden = L - 1; workgroup hidden-1 sits next to the top
    layer) and the top chunks (h, j), h < halves, j < chunks.  The flags are
    never cleared: every workgroup publishes once per step, so a launch starts
    with every flag at the steps of the launches before it (``load_epoch``
    reads the workgroup's own flag as that base) and publishes and waits for
    base + s + 1.  Slots remember the step counted across launches; the
    exchange buffers are chosen by the step within the launch, as in the
    kernel.  Launch n + 1 starts once every workgroup of launch n has finished
    (stream order).  Every launch after the first starts warm: its top chunks
    take their first step's partial products from xn, which each chunk writes
    at the end of the launch before (after its siblings' flags pass base + 1),
    so their first step neither computes, publishes nor waits before summing
    (it raises its flag afterwards only when it is the launch's only step).
    The keyword switches plant the mistakes the tests expect the model to catch
    (``reset_base``: a launch that counts from zero again while the flags hold
    the previous launch's steps; ``xn_wait=False``: xn rewritten without
    waiting for the siblings' first step)."""
    L2 = hidden - 1
    progs = {}
    names = [("hidden", l) for l in range(hidden)] + [("top", h, j) for h in range(halves) for j in range(chunks)]
    for name in names:
        progs[name] = []
    for n in range(launches):
        base = 0 if reset_base else n * steps
        for l in range(hidden):
            from_top = l == L2
            prog = progs[("hidden", l)]
            peers = []  # the workgroups it exchanges with
            if l >= 1:
                peers.append(("f", l - 1))
            if not from_top:
                if hidden_waits_up:
                    peers.append(("f", l + 1))
            else:
                peers += [("xsf", h) for h in range(halves)]
            for s in range(steps):
                g, buf = n * steps + s, s % 2
                if l >= 1:
                    prog.append(Op("write", ("xe", l, buf), g))
                gslot = s % g_buffers_top if from_top else buf
                prog.append(Op("write", ("xg", l, gslot), g))
                prog.append(Op("publish", ("f", l), base + s + 1))
                prog.append(Op("wait", conds=tuple((f, base + s + 1) for f in peers)))
                if l >= 1:
                    prog.append(Op("read", ("xg", l - 1, buf), g))
                if from_top:
                    prog += [Op("read", ("xs", h, buf), g) for h in range(halves)]
                else:
                    prog.append(Op("read", ("xe", l + 1, buf), g))
        for h in range(halves):
            for j in range(chunks):
                prog = progs[("top", h, j)]
                for s in range(steps):
                    g, buf = n * steps + s, s % 2
                    pre = n >= 1 and s == 0
                    if not pre:
                        prog.append(Op("write", ("xp", h, j, buf), g))
                        prog.append(Op("publish", ("f", ("top", h, j)), base + s + 1))
                        conds = [(("f", ("top", h, c)), base + s + 1) for c in range(chunks) if c != j]
                        if j == 0 and not chunk0_waits_siblings:
                            conds = []
                        if top_waits_l2:
                            conds.append((("f", L2), base + s))  # one step behind
                        prog.append(Op("wait", conds=tuple(conds)))
                    if s >= 1:
                        prog.append(Op("read", ("xg", L2, (s - 1) % g_buffers_top), g - 1))
                    if pre:
                        prog += [Op("read", ("xn", h, c), n) for c in range(chunks)]
                    else:
                        prog += [Op("read", ("xp", h, c, buf), g) for c in range(chunks)]
                    if j == 0:
                        prog.append(Op("write", ("xs", h, buf), g))
                        prog.append(Op("publish", ("xsf", h), base + s + 1))
                    if pre and steps == 1:  # else the next step's flag covers it
                        prog.append(Op("publish", ("f", ("top", h, j)), base + 1))
                # the next launch's first partials, after the siblings' first step
                if xn_wait:
                    prog.append(Op("wait", conds=tuple((("f", ("top", h, c)), base + 1)
                                                       for c in range(chunks) if c != j)))
                prog.append(Op("write", ("xn", h, j), n + 1))
        if n + 1 < launches:
            # stream order: every workgroup of launch n finishes before launch n + 1 starts
            for name in names:
                progs[name].append(Op("publish", ("done", name, n), 1))
            for name in names:
                progs[name].append(Op("wait", conds=tuple((("done", m, n), 1) for m in names)))
    return Model(progs)
