"""CPU model of a withdrawn design: the decoupled weight stream of the
persistent decode step (stream waves that issue a workgroup's weight rows of
every GEMV phase of the step into a ring of LDS units, ahead of the phases'
inputs, and consume them in the phases).

The kernel was built, measured slower than the shipped step kernel and taken
out; two throttled variants then read wrong weights, and one of them ended its
GPU run with a memory fault.  This model restates the ring's accounting as the
kept source wrote it (per-wave 32-bit unsigned counters: slots issued I,
consumed C, known landed L, units issued IU / consumed CU; an issuing cursor
over (phase, row, chunk); blocking and non-blocking pumps; the in-flight bound
kInFlight; vector-memory waits that make all but the newest n slots land, in
issue order), plus the two throttle rules as they were described:

* T1: while the control waves wait for a phase's input, at most 4 slots in
  flight instead of kInFlight;
* T2: no issue while a phase's last job is consumed (neither the blocking pump
  before it nor the non-blocking pump after it).

and enumerates small programs exhaustively: 1-2 GEMV phases (an attention
phase between them, which drains the wave's loads) with 0-3 rows for the wave,
1-5 slots per row, one or two matrices (SwiGLU), rings of 1-3 units, bounds of
4 and 8 slots, inputs arriving after 0-2 pump rounds.  At every step it checks
that the ring unit consumed holds the job the consumer expects, that its slots
have landed by the wait history (not only by the kernel's own belief L), that
no counter difference wraps, and that every index the issuer forms (row, chunk,
ring unit) is in range: an out-of-range row or chunk would be a load from
outside the weight matrix.

Finding (asserted below; 87,120 runs per rule set): the kept rules keep every
invariant, and so does T1.  T2 lets the consumer pass the issuer (C > I) in
1,794 of them: when the ring is full, the next job can only be issued after a
unit is consumed, and if that happens at a phase's last job and the next
phase's input is already staged (no idle pumps), the pumps that would issue it
are the ones T2 silences, so the job is consumed before it exists (the
smallest case: two one-job phases and a one-unit ring); I - C then wraps to ~2^32,
the landed test skips its wait, IU - CU wraps so no pump issues again, and
every later job reads whatever the ring unit last held: wrong weights.  T1
keeps the invariants.  In no case, with or without the throttles, does the
issuer form a row, chunk or ring unit out of range, so the counters' wrap
explains the wrong weights but cannot by itself produce a memory fault; the
faulting run's source was not kept, and the design stays off the GPU.
"""
import itertools

import pytest

JOB_SLOTS = 4
MASK = 0xFFFFFFFF


def u32(x):
    return x & MASK


class Violation(Exception):
    pass


class Ring:
    def __init__(self, units, in_flight):
        self.units, self.K = units, in_flight
        self.I = self.C = self.L = self.IU = self.CU = 0
        self.ipos = self.cpos = 0
        self.content = [None] * units   # (job, first slot, slots) per ring unit
        self.truth = 0                  # slots below this index have landed (waits seen so far)
        self.wrapped = False

    def wait_vm(self, n):               # s_waitcnt vmcnt(n): all but the newest n slots landed
        self.truth = max(self.truth, self.I - n)


class Cursor:
    def __init__(self, prog):
        self.prog = prog
        self.seek(0)

    def seek(self, p):
        for q in range(p, len(self.prog)):
            ph = self.prog[q]
            if ph is not None and ph[0] > 0:
                self.p, (self.rows, self.spr, self.M) = q, ph
                self.per = JOB_SLOTS // self.M
                self.j = self.c = 0
                self.cnt = min(self.per, self.spr)
                return
        self.p = len(self.prog)


def issue(r, c):
    if not (0 <= c.j < c.rows and 0 <= c.c * c.per < c.spr and 1 <= c.cnt <= c.per and 0 <= r.ipos < r.units):
        raise Violation(f"issue out of range: phase {c.p} row {c.j} chunk {c.c} cnt {c.cnt} unit {r.ipos}")
    n = c.M * c.cnt
    r.content[r.ipos] = ((c.p, c.j, c.c), r.I, n)
    r.I += n
    r.IU += 1
    r.ipos = (r.ipos + 1) % r.units
    c.c += 1
    if c.c * c.per >= c.spr:
        c.c = 0
        c.j += 1
        if c.j == c.rows:
            c.seek(c.p + 1)
            return
    c.cnt = min(c.per, c.spr - c.c * c.per)


def pump(r, c, block, limit):
    if c.p >= len(c.prog) or u32(r.IU - r.CU) >= r.units:
        return False
    n = c.M * c.cnt
    if u32(r.I - r.L) + n > limit:
        if not block:
            return False
        r.wait_vm(limit - n)
        r.L = u32(r.I - (limit - n))
    issue(r, c)
    return True


def landed(r, n):
    if r.C + n > r.L:
        younger = u32(r.I - r.C - n)
        if younger < r.K:
            r.wait_vm(younger)
        r.L = u32(r.C + n)


def consume(r, job, n):
    content = r.content[r.cpos]
    if content is None or content[0] != job:
        raise Violation(f"consumed {job} from a unit holding {content and content[0]}")
    if content[1] + content[2] > r.truth:
        raise Violation(f"consumed {job} before its slots landed")
    r.C = u32(r.C + n)
    r.CU = u32(r.CU + 1)
    r.cpos = (r.cpos + 1) % r.units


def run(prog, units, in_flight, arrivals, t1=False, t2=False):
    """One step of one stream wave over `prog` (a GEMV phase: (rows, slots per
    row, matrices); None: an attention phase); the input of GEMV phase i
    arrives after arrivals[i] pump rounds.  Raises Violation."""
    r, c = Ring(units, in_flight), Cursor(prog)
    wait_limit = 4 if t1 else in_flight
    while pump(r, c, False, in_flight):
        pass
    gemv = 0
    for p, ph in enumerate(prog):
        if ph is None:          # attention: the wave's own loads and stores drain the counter
            r.wait_vm(0)
            r.L = r.I
            continue
        for _ in range(arrivals[gemv]):
            pump(r, c, True, wait_limit)
        gemv += 1
        rows, spr, M = ph
        per = JOB_SLOTS // M
        for j in range(rows):
            for cb in range(0, spr, per):
                cnt = min(per, spr - cb)
                last = j == rows - 1 and cb + per >= spr
                quiet = t2 and last
                while u32(r.I - r.C) < M * cnt and not quiet and pump(r, c, True, in_flight):
                    pass
                if u32(r.I - r.C) < M * cnt:
                    r.wrapped = True
                    raise Violation(f"job {(p, j, cb // per)} consumed before it was issued (I {r.I}, C {r.C})")
                landed(r, M * cnt)
                consume(r, (p, j, cb // per), M * cnt)
                if not quiet:
                    pump(r, c, False, in_flight)
    return r


def programs():
    shapes = [(rows, spr, M) for rows in range(0, 4) for spr in range(1, 6) for M in (1, 2)]
    for a in shapes:
        yield [a]
    for a in shapes:
        for b in shapes:
            yield [a, None, b]


def sweep(t1, t2):
    ok, failures = 0, []
    for prog in programs():
        ngemv = sum(ph is not None for ph in prog)
        for units, in_flight in itertools.product((1, 2, 3), (4, 8)):
            for arrivals in itertools.product(range(3), repeat=ngemv):
                try:
                    run(prog, units, in_flight, arrivals, t1=t1, t2=t2)
                    ok += 1
                except Violation as e:
                    failures.append((prog, units, in_flight, arrivals, str(e)))
    return ok, failures


def test_kept_ring_rules_hold_every_invariant():
    ok, failures = sweep(t1=False, t2=False)
    assert ok > 10000 and not failures, failures[:3]


def test_in_flight_limit_while_waiting_holds_every_invariant():
    ok, failures = sweep(t1=True, t2=False)
    assert ok > 10000 and not failures, failures[:3]


@pytest.mark.parametrize("t1", [False, True])
def test_no_issue_in_last_job_lets_the_consumer_pass_the_issuer(t1):
    ok, failures = sweep(t1=t1, t2=True)
    assert failures, "the last-job rule should let the consumer reach an unissued job"
    # every failure is the consumer overtaking the issuer; none is an index out of range
    assert all("before it was issued" in f[4] for f in failures), [f for f in failures if "issued" not in f[4]][:3]
    # the smallest case: two one-job phases and a one-unit ring, the second
    # phase's input already staged when the wave reaches it: the unit frees
    # only when the first phase's (last) job is consumed, and the only pumps
    # that could then issue the second phase's job are the ones the rule
    # silences (after the first phase's last job, before the second's)
    size = lambda f: (len(f[0]), sum(ph[0] * ph[1] * ph[2] for ph in f[0] if ph), f[1])
    prog, units, in_flight, arrivals, _ = min(failures, key=size)
    assert prog == [(1, 1, 1), None, (1, 1, 1)] and units == 1 and arrivals[1] == 0


def test_wrapped_counters_stop_the_issuer_but_stay_in_range():
    """What the kernel did after the consumer passed the issuer: the unsigned
    differences wrap, every later pump refuses (IU - CU >= units), and the
    consumer keeps reading ring units in range (wrong weights, no stray
    address)."""
    r, c = Ring(2, 8), Cursor([(3, 4, 1)])
    while pump(r, c, False, 8):
        pass
    issued = r.IU
    # consume one job more than was issued, as the throttled loop did
    for job in range(issued + 1):
        n = 4
        landed(r, n)
        r.C, r.CU, r.cpos = u32(r.C + n), u32(r.CU + 1), (r.cpos + 1) % r.units
    assert u32(r.I - r.C) > 2 ** 31 and u32(r.IU - r.CU) >= r.units
    assert not pump(r, c, True, 8) and not pump(r, c, False, 8)
    assert 0 <= r.cpos < r.units and 0 <= r.ipos < r.units
