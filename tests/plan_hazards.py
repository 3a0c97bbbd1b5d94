"""Hazard check of the runtime's two-stream step schedule, independent of the runtime's own
dependency model.

A program image is decoded here from its byte layout, and every step's memory effects are
restated from the kernels the runtime launches for it (the launch wrappers in
synaptik_amd/csrc/*.hip), not from runtime.cpp's step_access:

- slots read and written (operands, outputs, optimizer tensors, the step counter);
- the reduction scratch of the stream the step runs on (GEMM split-K partials and column-sum
  partials, COLSUM, REDUCE_ALL, MSE and CE_INDEX partials): read and written;
- the device status word: OR-ed by atomics (commuting with each other), or read by steps that
  act only on a clear word (the optimizer's apply phase, the accumulator commit and clear, the
  step commit), and read and cleared by the run's publication kernel.

The schedule (`native.program_plan`) is then checked as the runtime enqueues it: a fork from
the context stream before the first step, every step on its stream in program order, one event
wait per step at most (recorded after the waited-for step), the join of both streams, and the
run's last launch (which performs the folded steps -- a classifier-loss MEAN, a small staged
optimizer pass -- in program order, then the trailing step commit and the status publication).
Every pair of steps whose effects conflict (read-after-write, write-after-read,
write-after-write, status read against status OR) must be ordered by a happens-before path.
"""
from __future__ import annotations

import struct
from dataclasses import dataclass, field

from synaptik_amd import program as P

_HDR = struct.Struct("<IIII")
_SLOT = struct.Struct("<QIIII")
_STEP = struct.Struct("<II8i16q8f")
_OPT = struct.Struct("<iiiiiiiiq")

@dataclass
class DecodedStep:
    index: int
    opcode: int
    slots: list
    iargs: list
    fargs: list
    payload: bytes


@dataclass
class Effects:
    reads: set = field(default_factory=set)
    writes: set = field(default_factory=set)
    status_or: bool = False
    status_read: bool = False


def decode(image: bytes) -> list[DecodedStep]:
    magic, version, n_slots, n_steps = _HDR.unpack_from(image, 0)
    assert magic == P.MAGIC and version == P.VERSION
    off = _HDR.size + n_slots * _SLOT.size
    steps = []
    for i in range(n_steps):
        rec = _STEP.unpack_from(image, off)
        off += _STEP.size
        opcode, nbytes = rec[0], rec[1]
        payload = image[off:off + nbytes]
        off += (nbytes + 7) & ~7
        steps.append(DecodedStep(i, opcode, list(rec[2:10]), list(rec[10:26]), list(rec[26:34]),
                                 payload))
    assert off == len(image)
    return steps


def _opt_rows(payload: bytes):
    return [_OPT.unpack_from(payload, o) for o in range(0, len(payload), _OPT.size)]


def effects(st: DecodedStep, stream: int | None, status_reads: bool = True) -> Effects:
    """Memory effects of one step run on `stream` (0 context stream, 1 side stream; None leaves
    the reduction scratch out). status_reads=False drops the optimizer's status-word reads (the
    runtime's dependency model before they were added; kept to show what the check catches)."""
    e = Effects()
    s, a = st.slots, st.iargs
    scratch = ("scratch", stream)

    def R(*xs):
        e.reads.update(("slot", x) for x in xs if x >= 0)

    def W(*xs):
        e.writes.update(("slot", x) for x in xs if x >= 0)

    op = st.opcode
    if op == P.OP_GEMM:
        # A, B, bias, aux (stored activation or upstream dY); C (read too when accumulating),
        # column sums, cotangent dz; split-K / column-sum partials in the stream's scratch
        R(s[0], s[1], s[3], s[4])
        W(s[2], s[5], s[7])
        if a[11]:
            R(s[2])
        _scratch(e, scratch)
        if st.payload:  # staged optimizer update in the epilogue
            p, _g, m, v, pn, mn, vn, _pad, _n = _opt_rows(st.payload)[0]
            R(p, m, v, s[6])
            W(pn, mn, vn)
            e.status_or = True
    elif op == P.OP_COLSUM:
        R(s[0])
        W(s[1])
        if a[3]:
            R(s[1])
        _scratch(e, scratch)
    elif op == P.OP_ROW_REDUCE:
        R(s[0])
        W(s[1])
    elif op == P.OP_REDUCE_ALL:
        R(s[0])
        W(s[1])
        _scratch(e, scratch)
    elif op == P.OP_POINTWISE:
        R(*s[0:6])
        W(s[6], s[7])
    elif op == P.OP_SOFTMAX:
        R(s[0])
        W(s[1], s[2])
    elif op == P.OP_SOFTMAX_BWD:
        R(s[0], s[1], s[3])
        W(s[2])
    elif op == P.OP_LSE_BWD:
        R(s[0], s[1], s[2])
        W(s[3])
    elif op == P.OP_MSE:
        R(s[0], s[1])
        W(s[2], s[3])
        _scratch(e, scratch)
    elif op == P.OP_CE_INDEX:
        R(s[0], s[1])
        W(s[2], s[3])
        _scratch(e, scratch)
        e.status_or = True
    elif op == P.OP_CE_HEAD:
        if a[4] == 1:  # loss MEAN of the per-row losses
            R(s[0])
            W(s[1])
        else:
            R(s[0], s[1], s[2], s[3])
            W(s[4], s[5], s[6], s[7])
            e.status_or = True
    elif op == P.OP_OPTIMIZER:
        kind, phase = a[0], a[1]
        for p, g, m, v, pn, mn, vn, _pad, _n in _opt_rows(st.payload):
            if kind == 3:      # p = m + g (checked)
                R(m, g)
                W(p)
                e.status_or = True
            elif kind == 4:    # m = g if the status word is clear
                R(g)
                W(m)
                e.status_read = status_reads
            elif kind == 5:    # m = 0 if the status word is clear
                W(m)
                e.status_read = status_reads
            else:
                R(p, g, m, v, s[0])
                if phase == 1:    # apply in place if the status word is clear
                    W(p, m, v)
                    e.status_read = status_reads
                elif phase == 2:  # stage into the other set, flag failures
                    W(pn, mn, vn)
                    e.status_or = True
                else:             # check only
                    e.status_or = True
    elif op == P.OP_STEP_COMMIT:
        R(s[0])
        W(s[0])
        e.status_read = True
    elif op == P.OP_FILL:
        W(s[0])
    elif op in (P.OP_COPY, P.OP_TRANSPOSE):
        R(s[0])
        W(s[1])
    else:
        raise ValueError(f"step {st.index}: opcode {op} has no effects model")
    return e


def _scratch(e: Effects, scratch) -> None:
    if scratch[1] is not None:
        e.reads.add(scratch)
        e.writes.add(scratch)


def conflict(x: Effects, y: Effects, read_read: bool = False) -> list[str]:
    """Why the two steps (x first in program order) must stay ordered; empty when they commute.
    read_read also orders two readers of the status word (the runtime's planner does, which
    costs nothing: they never both run beside the chain)."""
    why = []
    for r in sorted(x.writes & y.reads, key=str):
        why.append(f"RAW {r}")
    for r in sorted(x.reads & y.writes, key=str):
        why.append(f"WAR {r}")
    for r in sorted(x.writes & y.writes, key=str):
        why.append(f"WAW {r}")
    if x.status_read and y.status_or:
        why.append("status read before OR")
    if y.status_read and x.status_or:
        why.append("status OR before read")
    if read_read and x.status_read and y.status_read:
        why.append("status read twice")
    return why


@dataclass
class Hazard:
    first: int
    second: int
    reasons: list

    def __str__(self):
        return f"steps {self.first} -> {self.second} unordered: {', '.join(self.reasons)}"


def check_plan(steps: list[DecodedStep], stream_of, wait_for, folded=()) -> list[Hazard]:
    """Returns every conflicting pair of steps without a happens-before path under the plan
    (empty: the schedule is race-free), after checking the plan's own well-formedness. `folded`:
    the steps the run's last launch performs (-1 entries ignored)."""
    n = len(steps)
    assert len(stream_of) == n and len(wait_for) == n
    commit_last = n > 0 and steps[-1].opcode == P.OP_STEP_COMMIT
    launched = n - 1 if commit_last else n
    # the last launch performs the folded steps and the trailing commit after the join
    folded = {int(f) for f in folded if f >= 0}
    in_pub = set([n - 1] if commit_last else []) | folded
    for f in folded:
        st = steps[f]
        assert (st.opcode == P.OP_CE_HEAD and st.iargs[4] == 1) or \
            (st.opcode == P.OP_OPTIMIZER and st.iargs[1] == 2 and st.iargs[0] <= 2), f
    for j, w in enumerate(wait_for):
        if w < 0:
            continue
        assert w < j, f"step {j} waits for a later step {w}"
        assert stream_of[w] != stream_of[j], f"step {j} waits for step {w} on its own stream"
        assert w not in in_pub, f"step {j} waits for step {w}, which is never launched"
    # happens-before as reachability: node per launched step, plus the publication node n
    preds = {j: set() for j in range(n + 1)}
    last_on = {0: None, 1: None}
    for j in range(launched):
        if j in in_pub:
            continue
        sj = stream_of[j]
        if last_on[sj] is not None:
            preds[j].add(last_on[sj])
        if wait_for[j] >= 0:
            preds[j].add(wait_for[j])
        last_on[sj] = j
    for sj in (0, 1):  # join, then the publication
        if last_on[sj] is not None:
            preds[n].add(last_on[sj])
    anc = {}
    for j in list(range(launched)) + [n]:
        if j in in_pub:
            continue
        a = set()
        for p in preds[j]:
            a.add(p)
            a |= anc[p]
        anc[j] = a
    node = {j: (n if j in in_pub else j) for j in range(n)}
    eff = [effects(st, 0 if node[j] == n else stream_of[j]) for j, st in enumerate(steps)]
    hazards = []
    for j in range(n):
        for i in range(j):
            why = conflict(eff[i], eff[j])
            if not why:
                continue
            ni, nj = node[i], node[j]
            if ni == nj == n:
                continue  # inside the publication kernel, in program order
            if ni == n:
                hazards.append(Hazard(i, j, why + ["(first runs in the publication)"]))
            elif ni not in anc[nj]:
                hazards.append(Hazard(i, j, why))
    return hazards


def critical_path_plan(steps: list[DecodedStep]):
    """A critical-path two-stream assignment: the longest cost-weighted dependency chain stays on
    the context stream, every other step goes to the side stream; each step waits for its latest
    conflicting predecessor on the other stream. Cost: multiply-adds for GEMMs, element counts
    for the rest. Dependencies come from this module's effects, on one stream's scratch."""
    n = len(steps)
    eff = [effects(st, 0) for st in steps]

    def cost(st):
        a = st.iargs
        if st.opcode == P.OP_GEMM:
            return max(1, a[0] * a[1] * a[2])
        return max(1, a[0] * max(1, a[1]))

    deps = [[i for i in range(j) if conflict(eff[i], eff[j])] for j in range(n)]
    finish = [0] * n
    best = [-1] * n
    for j in range(n):
        f, b = 0, -1
        for i in deps[j]:
            if finish[i] > f:
                f, b = finish[i], i
        finish[j] = f + cost(steps[j])
        best[j] = b
    stream_of = [1] * n
    j = max(range(n), key=lambda k: finish[k]) if n else -1
    while j >= 0:
        stream_of[j] = 0
        j = best[j]
    if n and steps[-1].opcode == P.OP_STEP_COMMIT:
        stream_of[-1] = 0
    wait_for = [-1] * n
    for j in range(n):
        other = [i for i in deps[j] if stream_of[i] != stream_of[j]]
        if other:
            wait_for[j] = max(other)
    return stream_of, wait_for


def greedy_plan(steps: list[DecodedStep], status_reads: bool = True):
    """The runtime's list schedule restated over this module's effects: a step goes to the side
    stream when it does not depend on the step at the tail of the context stream and is not a
    GEMM of at least 2^28 multiply-adds; it waits for its latest dependency on the other stream."""
    n = len(steps)
    eff = [effects(st, None, status_reads) for st in steps]
    stream_of, wait_for = [0] * n, [-1] * n
    tail0 = -1
    for j in range(n):
        deps = [i for i in range(j) if conflict(eff[i], eff[j], read_read=True)]
        a = steps[j].iargs
        large = steps[j].opcode == P.OP_GEMM and min(a[0], a[1], a[2]) > 0 and \
            a[0] * a[1] * a[2] >= 1 << 28
        on_tail = tail0 < 0 or tail0 in deps
        stream_of[j] = 0 if (on_tail or large) else 1
        if stream_of[j] == 0:
            tail0 = j
        other = [i for i in deps if stream_of[i] != stream_of[j]]
        if other:
            wait_for[j] = max(other)
    return stream_of, wait_for
