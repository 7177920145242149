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
    order and, after a unit's last code row, makes the unit's scale row (its
    staging slot is then free), publishing that scale rows are stored before
    it next waits for a row or once four are outstanding; a feeder copies
    each stored scale row into the ring at its payload position; the MAC
    wave absorbs rows in payload order; a slot is rewritten only once both
    the MAC wave and the storer have passed it.
  ingress (vlx-tee_amd/csrc/ztcp_ingress.hip): decoders take tasks in order
    (a unit's scale row two units ahead of its code rows), write code rows
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


NBLK = {"i8": 8, "i4": 4, "raw": 16}
LAZY_SCALE_ONLY_AT_END = False  # planted mistake: the storer publishes stored scale rows only when it is done
IGNORE_STORER = False       # planted mistake: reuse a ring slot once the MAC wave alone has passed it
CONFIGS = {  # sections (kind, units) of the layouts the kernels meet
    "k8v4": [("i8", 16), ("i8", 16), ("i4", 32)],
    "int4": [("i8", 16), ("i4", 16), ("i4", 32)],
    "fp8only": [("i8", 32), ("i8", 32)],
    "mla": [("i8", 8), ("i4", 64)],
    "raw_rope": [("raw", 4), ("i4", 8), ("i4", 16)],
    "tiny": [("i8", 1), ("i4", 1)],
    "one_unit_sections": [("i8", 1), ("i8", 3), ("i4", 2)],
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
                if blocked > 50 * len(live) + 1000:
                    return False
            else:
                blocked = 0
        raise RuntimeError("step limit")


def wait(cond):
    while not cond():
        yield "blocked"


def egress_model(secs, n_prod, seed):
    KRING, KSTAGE = _const("ztcp_egress.hip", "kRing"), _const("ztcp_egress.hip", "kStage")
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
                assert stage_units[g % KSTAGE] == g, "staging slot still holds another unit"
                staged[g] = staged.get(g, 0) + 1
                yield "ok"
            m = c["m"]
            yield from wait(lambda: slot_free(m))
            assert ring_flag[m % KRING] <= max(0, m - KRING + 1), "ring slot overwritten before use"
            ring[m % KRING] = prow[m]
            yield "ok"
            ring_flag[m % KRING] = m + 1
            yield "ok"
            t = tn

    def storer():
        made, pub = [], 0
        for m in range(len(prow)):
            if prow[m][0] == "code":
                if pub < len(made) and ring_flag[m % KRING] < m + 1 and not LAZY_SCALE_ONLY_AT_END:
                    stored.update(made[pub:]); pub = len(made)  # published before waiting
                    yield "ok"
                yield from wait(lambda: ring_flag[m % KRING] >= m + 1)
                yield "ok"  # the slot's quads are read ...
                assert ring[m % KRING] == prow[m], ("storer read an overwritten slot", m, ring[m % KRING])
            st["stored"] = m + 1  # ... before the release that frees it
            yield "ok"
            if prow[m][0] == "code":
                _, si, u, j = prow[m]
                kind = secs[si][0]
                if kind != "raw" and j == NBLK[kind] - 1:
                    g = code[[c["m"] for c in code].index(m)]["g"]
                    assert staged.get(g, 0) == per_unit[g], "scale row made before its unit was staged"
                    assert stage_units[g % KSTAGE] == g
                    stage_flag[g % KSTAGE] = g + 1
                    made.append(g)
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
            assert ring_flag[m % KRING] <= max(0, m - KRING + 1)
            ring[m % KRING] = prow[m]
            yield "ok"
            ring_flag[m % KRING] = m + 1
            yield "ok"

    def mac():
        for m in range(len(prow)):
            yield from wait(lambda: ring_flag[m % KRING] >= m + 1)
            assert ring[m % KRING] == prow[m], (m, ring[m % KRING], prow[m])
            st["used"] = m + 1
            yield "ok"

    return Sched(seed).run([producer() for _ in range(n_prod)] + [feeder(), mac(), storer()])


def ingress_tasks(secs, L):
    """Decode order of the ingress kernel: per section the scale rows of the
    first L units, then each unit's code rows followed by the scale row of
    the unit L further on."""
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
            for u in range(full):
                tasks += [code(u, j) for j in range(nblk)] + [scale(u + L)]
            for u in range(full, nu):
                tasks += [code(u, j) for j in range(nblk)]
            g0 += nu
        m = scale_m + (nu if kind != "raw" else 0)
    return tasks


def ingress_model(secs, n_dec, seed, padding=0):
    KRING = _const("ztcp_ingress.hip", "kRing")
    KSTAGE = _const("ztcp_ingress.hip", "kStage")
    L = _const("ztcp_ingress.hip", "kLookahead")
    prow = payload_rows(secs, padding)
    tasks = ingress_tasks(secs, L)
    code_m = {t["m"] for t in tasks if t["kind"] == "code"}
    assert len(code_m) == sum(1 for r in prow if r[0] == "code")
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
                assert ring_flag[m % KRING] <= max(0, m - KRING + 1), "ring slot overwritten before use"
                ring[m % KRING] = prow[m]
                yield "ok"
                ring_flag[m % KRING] = m + 1
                yield "ok"
                if k["quant"]:
                    g = k["g"]
                    yield from wait(lambda: ready[g % KSTAGE] >= g + 1)
                    assert stage[g % KSTAGE] == g, "code row read another unit's scales"
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
            assert ring_flag[m % KRING] <= max(0, m - KRING + 1)
            ring[m % KRING] = r
            yield "ok"
            ring_flag[m % KRING] = m + 1
            yield "ok"

    def verify():
        for m in range(len(prow)):
            yield from wait(lambda: ring_flag[m % KRING] >= m + 1)
            assert ring[m % KRING] == prow[m], (m, ring[m % KRING], prow[m])
            st["used"] = m + 1
            yield "ok"

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
