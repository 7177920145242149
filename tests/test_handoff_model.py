"""CPU model of the fused kernels' LDS hand-offs under random interleavings.

Each wave of a fused workgroup is modelled as a generator that yields after
every shared-memory step and spins (yields 'blocked') at every bounded wait
of the kernel.  A scheduler runs the generators in a random order; a run in
which every live wave stays blocked is a deadlock.  The model also checks
that the MAC / verify wave reads every payload row in order with the right
contents, that no ring or staging slot is overwritten before it is consumed,
and that a code row reads its own unit's scales.

The ring, staging and look-ahead sizes are read from the kernel sources, so
the model follows the constants the kernels are built with.

  egress (vlx-tee_amd/csrc/ztcp_egress.hip): producers take code rows in
    order, stage scales per unit, write the ring at the row's payload
    position; a storer wave stores every code row from the ring in payload
    order and, after a unit's last code row, makes the unit's scale row: it
    keeps it in the unit's staging slot until kScaleGroup rows of the
    section are made (or the section's last unit is), then stores them and
    frees their slots, publishing that scale rows are stored before it next
    waits for a row or once four are outstanding; a feeder copies
    each stored scale row into the ring at its payload position; the MAC
    wave absorbs rows in payload order; a slot is rewritten only once both
    the MAC wave and the storer have passed it.
  ingress (vlx-tee_amd/csrc/ztcp_ingress.hip): decoders take tasks in order
    (a unit's scale row kLookahead units ahead of its code rows), write code rows
    into the ring, stage decrypted scales; a feeder copies every other
    payload row (scales, padding) into the ring; the verify wave absorbs
    rows in payload order.
"""
import random
import re
from pathlib import Path

import pytest

CSRC = Path(__file__).resolve().parents[1] / "vlx-tee_amd" / "csrc"


def _const(fname, name):
    m = re.search(rf"constexpr int {name} = (\d+);", (CSRC / fname).read_text())
    assert m, (fname, name)
    return int(m.group(1))


# code rows per unit of each section kind (code_rows_per_unit, ztcp_layout.h):
# the reference's int8 / int4 / raw, and the extension kinds e4m3 (16-element
# groups), int4 per 32 and int8 asymmetric per 64 (16 groups per unit, so 16
# code rows and one parameter row).  Every kind but raw has one parameter row
# per unit.
NBLK = {"i8": 8, "i4": 4, "raw": 16, "e4": 8, "i4g32": 8, "a8": 16}
LAZY_SCALE_ONLY_AT_END = False  # planted mistake: the storer publishes stored scale rows only when it is done
IGNORE_STORER = False       # planted mistake: reuse a ring slot once the MAC wave alone has passed it
GROUP_WITHOUT_SECTION_END = False  # planted mistake: the storer stores held scale rows only in full groups
FAM0_TASK_SPLIT = False     # planted mistake: ingress splits extension-kind tasks with the reference kinds' divisors
CONFIGS = {  # sections (kind, units) of the layouts the kernels meet
    "k8v4": [("i8", 16), ("i8", 16), ("i4", 32)],
    "int4": [("i8", 16), ("i4", 16), ("i4", 32)],
    "fp8only": [("i8", 32), ("i8", 32)],
    "mla": [("i8", 8), ("i4", 64)],
    "raw_rope": [("raw", 4), ("i4", 8), ("i4", 16)],
    "tiny": [("i8", 1), ("i4", 1)],
    "one_unit_sections": [("i8", 1), ("i8", 3), ("i4", 2)],
    # extension kinds (egress kind families 1 / 2, ingress family 1), the
    # 16-token x 8-head x 128 pages and 64-token MLA pages of the workloads
    "k8v4asym_e4rope": [("e4", 16), ("a8", 8), ("i4g32", 16)],
    "e4m3": [("e4", 32), ("e4", 32)],
    "mla_int4g32_e4rope": [("e4", 8), ("i4g32", 32)],
    "asym8_small": [("a8", 1), ("a8", 3), ("i4g32", 2)],
    "mixed_raw_ext": [("raw", 2), ("a8", 2), ("e4", 3)],
}


def payload_rows(secs, padding=0):
    """Payload rows in order: ('code', section, unit, j) / ('scale', g) /
    ('pad', i); code rows also get their code index."""
    rows, g = [], 0
    for si, (kind, nu) in enumerate(secs):
        for u in range(nu):
            for j in range(NBLK[kind]):
                rows.append(("code", si, u, j))
        if kind != "raw":
            rows += [("scale", g + u) for u in range(nu)]
            g += nu
    rows += [("pad", i) for i in range(padding)]
    return rows


class Sched:
    def __init__(self, seed):
        self.rng = random.Random(seed)

    def run(self, actors, max_steps=5_000_000):
        live = list(range(len(actors)))
        blocked = 0
        for _ in range(max_steps):
            if not live:
                return True
            i = self.rng.choice(live)
            try:
                s = next(actors[i])
            except StopIteration:
                live.remove(i)
                blocked = 0
                continue
            if s == "blocked":
                blocked += 1
                # with bounded waits every wait ends by itself
                if BOUND is None and blocked > 50 * len(live) + 1000:
                    return False
            else:
                blocked = 0
        raise RuntimeError("step limit")


class Bounded:
    """The kernels' bounded waits (wait_ge, vlx-tee_amd/csrc/ztcp_rows.h): a
    wait gives up after `limit` polls, records the expiry in the workgroup's
    LDS word and returns; with `short_circuit` (the kernels' rule) a wait that
    finds the word set returns at its next poll.  After an expiry rows are
    handed over out of turn, so the model's content checks no longer apply
    (the kernel fails such a workgroup closed)."""

    def __init__(self, limit, short_circuit=True):
        self.limit, self.short_circuit = limit, short_circuit
        self.expired = False
        self.expiries = 0   # waits that ran out their own bound
        self.polls = 0      # polls of all waits together

    def wait(self, cond):
        spins = 0
        while not cond():
            if self.short_circuit and self.expired:
                return
            if spins >= self.limit:
                self.expired = True
                self.expiries += 1
                return
            spins += 1
            self.polls += 1
            yield "blocked"


BOUND = None  # a Bounded while a test runs the model with bounded waits


def wait(cond):
    if BOUND is not None:
        yield from BOUND.wait(cond)
        return
    while not cond():
        yield "blocked"


def check(cond, *msg):
    """The model's content checks; void once a bounded wait has expired."""
    if BOUND is not None and BOUND.expired:
        return
    assert cond, msg


MAC_GROUP_OFF = False  # planted mistake: the MAC wave tests only the first row of each group


def mac_groups(prow, ring, ring_flag, st, KRING):
    """The MAC / verify wave (mac_rows, vlx-tee_amd/csrc/ztcp_rows.h): rows
    in groups of kMacGroup.  One test of the group's flags: a group whose rows
    are all in the ring is read at once and `used` is published once for it;
    otherwise the group is taken a row at a time, each row once its flag is
    set, and `used` is published after each.  The last total % kMacGroup
    rows are always taken a row at a time."""
    G = _const("ztcp_rows.h", "kMacGroup")
    assert KRING % G == 0, "ring lengths are multiples of the MAC group"
    for g0 in range(0, len(prow), G):
        rows = range(g0, min(g0 + G, len(prow)))
        tested = rows[:1] if MAC_GROUP_OFF else rows
        if len(rows) == G and all(ring_flag[m % KRING] >= m + 1 for m in tested):
            for m in rows:
                check(ring[m % KRING] == prow[m], (m, ring[m % KRING], prow[m]))
                yield "ok"
            st["used"] = rows[-1] + 1
            yield "ok"
            continue
        for m in rows:
            yield from wait(lambda: ring_flag[m % KRING] >= m + 1)
            check(ring[m % KRING] == prow[m], (m, ring[m % KRING], prow[m]))
            yield "ok"
            st["used"] = m + 1
            yield "ok"


def egress_model(secs, n_prod, seed):
    KRING, KSTAGE = _const("ztcp_egress.hip", "kRing"), _const("ztcp_egress.hip", "kStage")
    KGROUP = _const("ztcp_egress.hip", "kScaleGroup")
    prow = payload_rows(secs)
    # code rows in production order, with their payload row and unit
    code, g0 = [], 0
    for m, r in enumerate(prow):
        if r[0] == "code":
            si, u, _ = r[1:]
            kind = secs[si][0]
            code.append(dict(m=m, quant=kind != "raw", g=g0 + u if kind != "raw" else None, nblk=NBLK[kind]))
        elif r[0] == "scale":
            g0 = r[1] + 1
    per_unit = {}
    for c in code:
        if c["quant"]:
            per_unit[c["g"]] = per_unit.get(c["g"], 0) + 1
    st = dict(task=0, used=0, stored=0)
    ring, ring_flag = [None] * KRING, [0] * KRING

    def slot_free(m):
        return st["used"] >= m - KRING + 1 and (IGNORE_STORER or st["stored"] >= m - KRING + 1)
    stage_flag = [0] * KSTAGE
    stage_units = [None] * KSTAGE
    staged, stored = {}, set()

    def producer():
        t = st["task"]; st["task"] += 1
        yield "ok"
        while t < len(code):
            tn = st["task"]; st["task"] += 1
            yield "ok"
            c = code[t]
            if c["quant"]:
                g = c["g"]
                yield from wait(lambda: stage_flag[g % KSTAGE] >= g - KSTAGE + 1)
                if staged.get(g, 0) == 0:
                    stage_units[g % KSTAGE] = g
                check(stage_units[g % KSTAGE] == g, "staging slot still holds another unit")
                staged[g] = staged.get(g, 0) + 1
                yield "ok"
            m = c["m"]
            yield from wait(lambda: slot_free(m))
            check(ring_flag[m % KRING] <= max(0, m - KRING + 1), "ring slot overwritten before use")
            ring[m % KRING] = prow[m]
            yield "ok"
            ring_flag[m % KRING] = m + 1
            yield "ok"
            t = tn

    def storer():
        made, pub = [], 0
        held = []  # encrypted scale rows kept in their staging slots until their group is complete
        for m in range(len(prow)):
            if prow[m][0] == "code":
                if pub < len(made) and ring_flag[m % KRING] < m + 1 and not LAZY_SCALE_ONLY_AT_END:
                    stored.update(made[pub:]); pub = len(made)  # published before waiting
                    yield "ok"
                yield from wait(lambda: ring_flag[m % KRING] >= m + 1)
                yield "ok"  # the slot's quads are read ...
                check(ring[m % KRING] == prow[m], ("storer read an overwritten slot", m, ring[m % KRING]))
            st["stored"] = m + 1  # ... before the release that frees it
            yield "ok"
            if prow[m][0] == "code":
                _, si, u, j = prow[m]
                kind = secs[si][0]
                if kind != "raw" and j == NBLK[kind] - 1:
                    g = code[[c["m"] for c in code].index(m)]["g"]
                    check(staged.get(g, 0) == per_unit[g], "scale row made before its unit was staged")
                    check(stage_units[g % KSTAGE] == g)
                    last_of_section = u + 1 == secs[si][1] and not GROUP_WITHOUT_SECTION_END
                    if len(held) < KGROUP - 1 and not last_of_section:
                        held.append(g)
                        yield "ok"
                        continue
                    for h in held + [g]:  # stored in order, each slot freed after its stores
                        check(stage_units[h % KSTAGE] == h, "a held scale row's slot was reused")
                        stage_flag[h % KSTAGE] = h + 1
                        made.append(h)
                    held.clear()
                    yield "ok"
                    if len(made) - pub >= 4 and not LAZY_SCALE_ONLY_AT_END:
                        stored.update(made[pub:]); pub = len(made)
                        yield "ok"
        stored.update(made[pub:])
        yield "ok"

    def feeder():
        # scale rows in payload order; within a section the next row's load
        # (which waits until that row is stored) is issued before the
        # current row is put
        rows = [(m, r[1]) for m, r in enumerate(prow) if r[0] == "scale"]
        for i, (m, g) in enumerate(rows):
            first = i == 0 or rows[i - 1][0] != m - 1
            if first:
                yield from wait(lambda: g in stored)
            if i + 1 < len(rows) and rows[i + 1][0] == m + 1:
                gn = rows[i + 1][1]
                yield from wait(lambda: gn in stored)
            yield from wait(lambda: slot_free(m))
            check(ring_flag[m % KRING] <= max(0, m - KRING + 1))
            ring[m % KRING] = prow[m]
            yield "ok"
            ring_flag[m % KRING] = m + 1
            yield "ok"

    def mac():
        yield from mac_groups(prow, ring, ring_flag, st, KRING)

    return Sched(seed).run([producer() for _ in range(n_prod)] + [feeder(), mac(), storer()])


def ingress_tasks(secs, L):
    """Decode order of the ingress kernel: per section the scale rows of the
    first L units, then the units' code rows two units at a time, with the
    scale rows of the two units L further on between them (an odd last unit
    of that part: its code rows, then one scale row), then the code rows of
    the last L units."""
    tasks, g0, m = [], 0, 0
    for si, (kind, nu) in enumerate(secs):
        nblk = NBLK[kind]
        code_m = m  # payload row of the section's first code row
        scale_m = m + nu * nblk
        def code(u, j):
            return dict(kind="code", g=g0 + u if kind != "raw" else None, nblk=nblk, m=code_m + u * nblk + j,
                        quant=kind != "raw")
        def scale(u):
            return dict(kind="scale", g=g0 + u, m=scale_m + u)
        if kind == "raw":
            tasks += [code(u, j) for u in range(nu) for j in range(nblk)]
        else:
            pre, full = min(L, nu), max(nu - L, 0)
            tasks += [scale(u) for u in range(pre)]
            for u in range(0, full, 2):
                tasks += [code(u, j) for j in range(nblk)] + [scale(u + L)]
                if u + 1 < full:
                    tasks += [scale(u + 1 + L)] + [code(u + 1, j) for j in range(nblk)]
            for u in range(full, nu):
                tasks += [code(u, j) for j in range(nblk)]
            g0 += nu
        m = scale_m + (nu if kind != "raw" else 0)
    return tasks


def kernel_task(secs, t, L):
    """Task t as the ingress kernel computes it (task_info, div_nblk, div_rpu2
    in ztcp_ingress.hip): integer arithmetic per section, with the divisors
    of a two-unit block chosen by the kind's code rows per unit (family 1:
    8 -> /18, 4 -> /10, otherwise /34; family 0 knows only int8 -> /18 and
    int4 -> /10)."""
    fam1 = any(k not in ("i8", "i4", "raw") for k, _ in secs)
    def div_nblk(x, kind):
        return x // NBLK[kind]
    def div_rpu2(x, kind):
        nblk = NBLK[kind]
        if fam1 and not FAM0_TASK_SPLIT:
            return x // 18 if nblk == 8 else (x // 10 if nblk == 4 else x // 34)
        return x // 18 if kind == "i8" else x // 10
    tb = cb = qb = m = 0
    for kind, nu in secs:
        nblk, quant = NBLK[kind], kind != "raw"
        rpu = nblk + (1 if quant else 0)
        n = nu * nblk + (nu if quant else 0)
        if tb <= t < tb + n:
            x = t - tb
            scale, j = False, 0
            if not quant:
                u = div_nblk(x, kind)
                j = x - u * nblk
            else:
                pre, full = min(L, nu), max(nu - L, 0)
                if x < pre:
                    scale, u = True, x
                elif x - pre < full * rpu:
                    x -= pre
                    span, pairs = 2 * rpu, full // 2
                    if x < pairs * span:
                        p2 = div_rpu2(x, kind)
                        u0, off = 2 * p2, x - p2 * span
                    else:
                        u0, off = full - 1, x - pairs * span
                    if off < nblk:
                        u, j = u0, off
                    elif off <= nblk + 1:
                        scale, u = True, u0 + L + (off - nblk)
                    else:
                        u, j = u0 + 1, off - nblk - 2
                else:
                    x -= pre + full * rpu
                    u0 = div_nblk(x, kind)
                    u, j = full + u0, x - u0 * nblk
            if scale:
                return dict(kind="scale", g=qb + u, m=m + nu * nblk + u)
            return dict(kind="code", g=qb + u if quant else None, nblk=nblk, m=m + u * nblk + j, quant=quant)
        tb += n
        cb += nu * nblk
        m += nu * nblk + (nu if quant else 0)
        if quant:
            qb += nu
    return None


def ingress_model(secs, n_dec, seed, padding=0):
    KRING = _const("ztcp_ingress.hip", "kRing")
    KSTAGE = _const("ztcp_ingress.hip", "kStage")
    L = _const("ztcp_ingress.hip", "kLookahead")
    prow = payload_rows(secs, padding)
    # the decoders take tasks as the kernel computes them; the code rows they
    # put into the ring must be exactly the payload's
    tasks = [kernel_task(secs, t, L) for t in range(len(ingress_tasks(secs, L)))]
    code_m = {t["m"] for t in tasks if t["kind"] == "code"}
    check(len(code_m) == sum(1 for r in prow if r[0] == "code"))
    st = dict(task=0, used=0, stored=0)
    ring, ring_flag = [None] * KRING, [0] * KRING

    def slot_free(m):
        return st["used"] >= m - KRING + 1 and (IGNORE_STORER or st["stored"] >= m - KRING + 1)
    ready, free, count = [0] * KSTAGE, [0] * KSTAGE, [0] * KSTAGE
    stage = [None] * KSTAGE

    def decoder():
        t = st["task"]; st["task"] += 1
        yield "ok"
        while t < len(tasks):
            tn = st["task"]; st["task"] += 1
            yield "ok"
            k = tasks[t]
            if k["kind"] == "scale":
                g = k["g"]
                yield from wait(lambda: free[g % KSTAGE] >= g - KSTAGE + 1)
                stage[g % KSTAGE] = g
                yield "ok"
                ready[g % KSTAGE] = g + 1
                yield "ok"
            else:
                m = k["m"]
                yield from wait(lambda: st["used"] >= m - KRING + 1)
                check(ring_flag[m % KRING] <= max(0, m - KRING + 1), "ring slot overwritten before use")
                ring[m % KRING] = prow[m]
                yield "ok"
                ring_flag[m % KRING] = m + 1
                yield "ok"
                if k["quant"]:
                    g = k["g"]
                    yield from wait(lambda: ready[g % KSTAGE] >= g + 1)
                    check(stage[g % KSTAGE] == g, "code row read another unit's scales")
                    old = count[g % KSTAGE]; count[g % KSTAGE] += 1
                    yield "ok"
                    if old == k["nblk"] - 1:
                        count[g % KSTAGE] = 0
                        free[g % KSTAGE] = g + 1
                        yield "ok"
            t = tn

    def feeder():
        for m, r in enumerate(prow):
            if m in code_m:
                continue
            yield from wait(lambda: st["used"] >= m - KRING + 1)
            check(ring_flag[m % KRING] <= max(0, m - KRING + 1))
            ring[m % KRING] = r
            yield "ok"
            ring_flag[m % KRING] = m + 1
            yield "ok"

    def verify():
        yield from mac_groups(prow, ring, ring_flag, st, KRING)

    return Sched(seed).run([decoder() for _ in range(n_dec)] + [feeder(), verify()])


@pytest.mark.parametrize("cfg", sorted(CONFIGS))
@pytest.mark.parametrize("waves", [1, 3, 12, 48])
def test_egress_handoffs(cfg, waves):
    for seed in range(3):
        assert egress_model(CONFIGS[cfg], waves, seed), f"deadlock {cfg} waves={waves} seed={seed}"


@pytest.mark.parametrize("cfg", sorted(CONFIGS))
@pytest.mark.parametrize("waves", [1, 3, 12, 48])
def test_ingress_handoffs(cfg, waves):
    for seed in range(3):
        assert ingress_model(CONFIGS[cfg], waves, seed), f"deadlock {cfg} waves={waves} seed={seed}"
        assert ingress_model(CONFIGS[cfg], waves, seed + 100, padding=5)


def test_egress_model_catches_scale_rows_published_only_at_the_end():
    """A planted mistake: a storer that publishes its stored scale rows only
    when it is done holds up the feeder, through it the MAC wave, and through
    the ring the producers whose rows the storer waits for: a deadlock."""
    global LAZY_SCALE_ONLY_AT_END
    LAZY_SCALE_ONLY_AT_END = True
    try:
        assert not all(egress_model(CONFIGS["k8v4"], 12, seed) for seed in range(5))
    finally:
        LAZY_SCALE_ONLY_AT_END = False


def test_egress_model_catches_scale_rows_held_past_their_section():
    """A planted mistake: a storer that stores held scale rows only in full
    groups of kScaleGroup keeps a section's last rows (when its unit count is
    not a multiple of the group) until rows of later sections complete the
    group, or for good after the last section: the feeder, and through it the
    MAC wave, wait for rows that are never stored."""
    global GROUP_WITHOUT_SECTION_END
    GROUP_WITHOUT_SECTION_END = True
    try:
        for cfg in ("tiny", "one_unit_sections"):
            assert not all(egress_model(CONFIGS[cfg], 12, seed) for seed in range(5)), cfg
    finally:
        GROUP_WITHOUT_SECTION_END = False


def test_egress_model_catches_a_slot_reused_before_the_storer_read_it():
    """A planted mistake: producers that reuse a ring slot as soon as the MAC
    wave has passed it can overwrite a row the storer has not stored yet."""
    global IGNORE_STORER
    IGNORE_STORER = True
    try:
        with pytest.raises(AssertionError, match="storer read an overwritten slot"):
            for seed in range(20):
                egress_model(CONFIGS["fp8only"], 48, seed)
    finally:
        IGNORE_STORER = False


def test_model_catches_a_staging_ring_smaller_than_the_lookahead():
    """A planted mistake: with fewer staging slots than units of look-ahead,
    a scale row waits for a unit whose code rows come after it in task
    order, and the model reports the deadlock."""
    global _const
    real = _const
    try:
        _const = lambda f, n: 1 if n == "kStage" else real(f, n)  # noqa: E731
        assert not ingress_model(CONFIGS["k8v4"], 3, 0)
    finally:
        _const = real


@pytest.mark.parametrize("cfg", sorted(CONFIGS))
def test_kernel_task_split_equals_the_decode_order(cfg):
    """The kernel's integer task split (task_info) enumerates exactly the
    decode order built unit by unit, for every kind's code rows per unit."""
    L = _const("ztcp_ingress.hip", "kLookahead")
    want = ingress_tasks(CONFIGS[cfg], L)
    assert [kernel_task(CONFIGS[cfg], t, L) for t in range(len(want))] == want


def test_model_catches_the_reference_divisors_on_extension_kinds():
    """A planted mistake: splitting an asym8 section's tasks by 9 / 5 (the
    reference kinds' rows per unit + 1) instead of 17 hands out code rows of
    the wrong unit and scale rows at the wrong places; the model reports a
    deadlock or a row the verify wave reads out of order."""
    global FAM0_TASK_SPLIT
    FAM0_TASK_SPLIT = True
    try:
        L = _const("ztcp_ingress.hip", "kLookahead")
        secs = CONFIGS["k8v4asym_e4rope"]
        want = ingress_tasks(secs, L)
        assert [kernel_task(secs, t, L) for t in range(len(want))] != want
        caught = 0
        for seed in range(3):
            try:
                caught += not ingress_model(secs, 12, seed)
            except AssertionError:
                caught += 1
        assert caught == 3
    finally:
        FAM0_TASK_SPLIT = False


def _run_bounded(limit, short_circuit, model):
    global BOUND
    BOUND = Bounded(limit, short_circuit)
    try:
        done = model()
        return done, BOUND
    finally:
        BOUND = None


@pytest.mark.parametrize("cfg", ["k8v4", "k8v4asym_e4rope"])
def test_bounded_waits_never_expire_in_a_healthy_workgroup(cfg):
    for seed in range(2):
        done, b = _run_bounded(10**6, True, lambda: egress_model(CONFIGS[cfg], 12, seed))
        assert done and not b.expired
        done, b = _run_bounded(10**6, True, lambda: ingress_model(CONFIGS[cfg], 12, seed))
        assert done and not b.expired


def test_one_expired_wait_ends_every_later_wait_of_the_workgroup():
    """A planted deadlock (the storer holding back its stored scale rows) with
    the kernels' bounded waits: the first wait to run out its bound marks the
    workgroup, every other wait returns at its next poll, and the workgroup
    finishes after at most one expiry per wave.  Without that rule each later
    wait spins out its own bound again, so the time to failure grows with the
    number of waits left (hundreds of bounds per wave in the kernel)."""
    global LAZY_SCALE_ONLY_AT_END
    LAZY_SCALE_ONLY_AT_END = True
    n_prod, limit = 12, 400
    waves = n_prod + 3  # producers, feeder, MAC wave, storer
    try:
        for seed in range(3):
            done, b = _run_bounded(limit, True, lambda: egress_model(CONFIGS["k8v4"], n_prod, seed))
            assert done and b.expired
            assert 1 <= b.expiries <= waves
            assert b.polls <= waves * limit
            done, old = _run_bounded(limit, False, lambda: egress_model(CONFIGS["k8v4"], n_prod, seed))
            assert done and old.expiries > 4 * waves
            assert old.polls > 4 * waves * limit
    finally:
        LAZY_SCALE_ONLY_AT_END = False


def test_one_expired_wait_ends_a_broken_ingress_workgroup():
    """The same rule in the ingress hand-offs, on the planted staging ring
    smaller than the look-ahead (a deadlock without bounded waits)."""
    global _const
    real = _const
    try:
        _const = lambda f, n: 1 if n == "kStage" else real(f, n)  # noqa: E731
        for seed in range(3):
            done, b = _run_bounded(400, True, lambda: ingress_model(CONFIGS["k8v4"], 12, seed))
            assert done and b.expired and 1 <= b.expiries <= 14
    finally:
        _const = real


# ---------------------------------------------------------------------------
# The small-batch egress kernel (egress_small_kernel): three producer waves
# make task t = 192 k + 64 w + lane of pass k (code row t // ppw of page
# t % ppw) and publish pass counts; after every wave's last pass they make
# the scale rows and count themselves done.  The MAC wave reads payload rows
# in order, a code row once every wave has published the pass that holds its
# last page's task (need = (c ppw + ppw - 1) // 192 + 1 passes; rows below
# need * 192 // ppw are then complete), a scale row once all three waves are
# done.  The model runs the waves lane by lane in random order and checks
# that every row the MAC wave reads has been written for every page.
# ---------------------------------------------------------------------------
PASS_OFF_BY_ONE = False  # planted mistake: the MAC wave waits for one pass fewer than it needs


def small_egress_model(secs, ppw, seed):
    waves = _const("ztcp_egress.hip", "kSmallWaves") - 1
    tasks_per_pass = 64 * waves
    rows = payload_rows(secs)
    code_rows = [r for r in rows if r[0] == "code"]
    ncode, nq = len(code_rows), sum(1 for r in rows if r[0] == "scale")
    ntask = ncode * ppw
    npass = -(-ntask // tasks_per_pass)
    written = set()     # (page, payload row) written to the LDS copy
    passes = [0] * waves
    done = [0]

    def producer(w):
        for k in range(npass):
            lanes = list(range(64))
            random.Random(seed * 31 + w * 7 + k).shuffle(lanes)
            for lane in lanes:
                t = k * tasks_per_pass + w * 64 + lane
                if t < ntask:
                    c, i = divmod(t, ppw)
                    written.add((i, rows.index(code_rows[c])))
                    yield "step"
            passes[w] = k + 1
            yield "step"
        yield from wait(lambda: min(passes) >= npass)
        for t in range(w * 64, nq * ppw, tasks_per_pass):
            for lane_t in range(t, min(t + 64, nq * ppw)):
                g, i = divmod(lane_t, ppw)
                written.add((i, rows.index(("scale", g))))
                yield "step"
        done[0] += 1

    def mac():
        ready, scales, c = 0, False, 0
        for r, row in enumerate(rows):
            if row[0] == "code":
                if c >= ready:
                    need = (c * ppw + ppw - 1) // tasks_per_pass + 1 - (1 if PASS_OFF_BY_ONE else 0)
                    yield from wait(lambda: min(passes) >= need)
                    ready = min(ncode, need * tasks_per_pass // ppw)
                c += 1
            elif not scales:
                yield from wait(lambda: done[0] >= waves)
                scales = True
            for i in range(ppw):
                check((i, r) in written, "row read before it was written", r, i, row)
            yield "step"

    assert Sched(seed).run([mac()] + [producer(w) for w in range(waves)])


@pytest.mark.parametrize("cfg", ["k8v4", "int4", "raw_rope", "tiny", "one_unit_sections"])
@pytest.mark.parametrize("ppw", [1, 2, 3, 4])
def test_small_egress_passes(cfg, ppw):
    for seed in range(3):
        small_egress_model(CONFIGS[cfg], ppw, seed)


def test_small_egress_model_catches_a_missing_pass():
    global PASS_OFF_BY_ONE
    PASS_OFF_BY_ONE = True
    try:
        with pytest.raises(AssertionError, match="before it was written"):
            for seed in range(20):
                small_egress_model(CONFIGS["k8v4"], 3, seed)
    finally:
        PASS_OFF_BY_ONE = False


def test_model_catches_a_group_read_on_its_first_flag_only():
    global MAC_GROUP_OFF
    MAC_GROUP_OFF = True
    try:
        with pytest.raises(AssertionError):
            for seed in range(20):
                egress_model(CONFIGS["k8v4"], 11, seed)
    finally:
        MAC_GROUP_OFF = False
