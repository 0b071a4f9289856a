"""Wait counts of the prefill grouped GEMM's DMA pipeline (split_pipeline.h).

The kernel (gemm_item_split, grouped_gemm.hip) issues, per wavefront: a
prologue of the sub-steps q = -Q .. -1 of the steady pattern, then at each
sub-step j = H*s + half a wait `s_waitcnt vmcnt(split_after(...))`, a barrier,
A(j + DA) (NAD DMA instructions) and, on half 0, B(s + DB) (NBD), then the
multiply of A(j) against B(s).  The wide gate/up tiles (grouped_gemm_wide_kernel)
have a pipeline of their own, checked the same way (simulate_wide).  Indices outside the item load a clamped stage
into the slot of the unclamped index.  Vector memory loads complete in issue
order, so the wait is safe when no more than split_after instructions were
issued after both A(j) and B(s) -- counted here by brute force over whole
items of 1..9 K stages, for every configuration the library builds (the
parameters come from the header itself through tests/split_pipeline/driver).
The ring slots written at sub-step j must not be the ones read at j, and the
rings must fit the 160 KB of LDS.  Where the header allows it
(split_a_may_skip), a wavefront issues only the A instructions of the tile's
used rows (0 .. NAD per stage, fixed per item): the waits must stay safe for
every such count.
"""
import os
import subprocess

import pytest

DRIVER_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "split_pipeline")


def driver_lines():
    subprocess.run(["make", "-s", "-C", DRIVER_DIR], check=True)
    out = subprocess.run([os.path.join(DRIVER_DIR, "driver")], capture_output=True, text=True, check=True).stdout
    return out.strip().splitlines()


@pytest.fixture(scope="module")
def configs():
    rows = [list(map(int, line.split())) for line in driver_lines() if not line.startswith("wide")]
    keys = ["rows", "swiglu", "h", "cb", "da", "db", "nad", "nbd", "after0", "after1", "lds", "a_skip"]
    return [dict(zip(keys, r)) for r in rows]


@pytest.fixture(scope="module")
def wide():
    line = [ln for ln in driver_lines() if ln.startswith("wide")]
    assert len(line) == 1
    return dict(zip(["nad", "nwh", "after", "wper1", "wper2"], map(int, line[0].split()[1:])))


def simulate(c, nk, nad=None):
    """Issue sequence of one item with nad A instructions per stage (default
    NAD); checks every wait and slot reuse.  Loads of indices outside the
    item issue nothing; a sub-step whose preceding loads would reach past the
    item (A(j - 1 + DA) or B(floor((j - 1) / H) + DB) missing) waits for all."""
    H, DA, DB, NBD = c["h"], c["da"], c["db"], c["nbd"]
    NAD = c["nad"] if nad is None else nad
    RA, RB = DA + 1, DB + 1
    nj = nk * H
    seq = []  # (kind, index, ops)

    def issue_a(j):
        if 0 <= j < nj:
            seq.append(("A", j, NAD))

    def issue_b(s):
        if 0 <= s < nk:
            seq.append(("B", s, NBD))

    Q = max(DA, H * DB)
    for q in range(-Q, 0):
        issue_a(q + DA)
        if q % H == 0:
            issue_b(q // H + DB)
    for s in range(nk):
        for half in range(H):
            j = s * H + half
            ia = [i for i, (k, x, _) in enumerate(seq) if k == "A" and x == j]
            ib = [i for i, (k, x, _) in enumerate(seq) if k == "B" and x == s]
            assert len(ia) == 1 and len(ib) == 1
            later = max(ia[0], ib[0])
            after = sum(n for (_, _, n) in seq[later + 1:])
            steady = (j - 1) + DA < nj and (j - 1) // H + DB < nk
            allowed = (c["after0"] if half == 0 else c["after1"]) if steady else 0
            assert 0 <= allowed <= after, (c, nk, j, allowed, after)
            assert allowed < 64  # vmcnt field
            # the slots written after the barrier are not the ones multiplied now
            assert (j + DA) % RA != j % RA
            if half == 0:
                assert (s + DB) % RB != s % RB
            issue_a(j + DA)
            if half == 0:
                issue_b(s + DB)
    # every load of the item has landed once the last sub-step has waited
    last = max(i for i, (k, x, _) in enumerate(seq) if (k == "A" and x == nj - 1) or (k == "B" and x == nk - 1))
    assert last == len(seq) - 1, "no load may follow the last stage's"


def test_every_configuration_is_safe(configs):
    assert len(configs) == 8
    for c in configs:
        assert c["lds"] <= 160 * 1024
        for nk in range(1, 10):
            simulate(c, nk)
            if c["a_skip"]:
                for nad in range(c["nad"]):
                    simulate(c, nk, nad)


def test_prefill_tiles_may_skip_unused_rows(configs):
    # Every 192-row configuration skips; the skip flag is exactly "some A count
    # below NAD still passes every wait" (checked by brute force).
    for c in configs:
        safe = True
        try:
            for nk in range(1, 10):
                simulate(c, nk, 0)
        except AssertionError:
            safe = False
        assert bool(c["a_skip"]) == safe, c
        if c["rows"] == 192:
            assert c["a_skip"] == 1, c


def test_a_count_that_is_one_too_large_is_caught(configs):
    # The check has teeth: allowing one more outstanding instruction than the
    # header does breaks at least one configuration.
    broken = 0
    for c in configs:
        bad = dict(c, after0=c["after0"] + 1, after1=c["after1"] + 1 if c["h"] == 2 else -1)
        try:
            for nk in range(1, 10):
                simulate(bad, nk)
        except AssertionError:
            broken += 1
    assert broken == len(configs)


def simulate_wide(w, H, nk, nad):
    """The wide gate/up tiles' issue sequence for one item (split_pipeline.h,
    wide_after, wide_w_per_substep): a prologue of A(0) and weight
    half-stages 0, 1, 2, then per sub-step j = H*s + half a wait, A(j + 1)
    (nad instructions) and weight half-stages 2s + 3 + half, ... (both on a
    one-half stage, one per sub-step of a two-half stage).  The first sub-step
    of a stage reads half-stages 2s and 2s + 1 from the ring (a second one
    keeps their fragments).  Every wait must cover the loads the sub-step
    multiplies; a ring slot refilled at a sub-step must hold no half-stage
    that is still to be read (the sub-step's own reads come before its weight
    DMAs)."""
    NWH = w["nwh"]
    per = w["wper1"] if H == 1 else w["wper2"]
    assert per * H == 2
    nj = nk * H
    seq = []
    slot = {}  # ring slot -> half-stage it holds

    def issue(kind, i, n):
        if kind == "A" and i < nj or kind == "W" and i < 2 * nk:
            seq.append((kind, i, n))
            if kind == "W":
                held = slot.get(i % 3)
                # the half-stage the slot held was read at its stage's first sub-step
                assert held is None or 2 * (held // 2) <= 2 * s_now, (H, nk, i, held)
                slot[i % 3] = i

    s_now = -1
    issue("A", 0, nad)
    for q in range(3):
        issue("W", q, NWH)
    for j in range(nj):
        s, half = divmod(j, H)
        s_now = s
        need = [("A", j)] + ([("W", 2 * s), ("W", 2 * s + 1)] if half == 0 else [])
        if half == 0:
            assert slot[(2 * s) % 3] == 2 * s and slot[(2 * s + 1) % 3] == 2 * s + 1
        idx = [next(i for i, (k, x, _) in enumerate(seq) if (k, x) == nd) for nd in need]
        after = sum(n for (_, _, n) in seq[max(idx) + 1:])
        steady = s + 1 < nk
        allowed = w["after"] if steady else 0
        assert 0 <= allowed <= after, (H, nk, nad, j, allowed, after)
        issue("A", j + 1, nad)
        q0 = 2 * s + 3 + half + w.get("shift", 0)
        for q in range(q0, q0 + per):
            issue("W", q, NWH)
    assert all(x < (nj if k == "A" else 2 * nk) for k, x, _ in seq)


def test_wide_tiles_waits_are_safe(wide):
    for H in (1, 2):
        for nk in range(1, 12):
            for nad in range(wide["nad"] + 1):
                simulate_wide(wide, H, nk, nad)


def test_wide_tiles_one_more_outstanding_is_caught(wide):
    # A sub-step leaves exactly the last weight half-stage's DMAs outstanding:
    # one more, and the wait no longer covers half-stage 2s + 1 (a first
    # sub-step) or A(j) (a second one).
    for H in (1, 2):
        with pytest.raises(AssertionError):
            simulate_wide(dict(wide, after=wide["after"] + 1), H, 4, wide["nad"])
    with pytest.raises(AssertionError):
        simulate_wide(dict(wide, after=wide["after"] + 1), 2, 4, 0)


def test_wide_tiles_early_refill_is_caught(wide):
    # Each weight half-stage one sub-step earlier goes into the slot of
    # half-stage 2s + 2, not yet read.
    for H in (1, 2):
        with pytest.raises(AssertionError, match=r"^\(%d, 4, " % H):
            simulate_wide(dict(wide, shift=-1), H, 4, wide["nad"])
