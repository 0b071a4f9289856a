"""Streamed-expert cache and copy-ahead policy, on the CPU.

The oracle's restatement (oracle/stream_policy.py) is pinned first: its cache
against a brute-force LRU over last-use times, its predictor against routing
histories worked out by hand (gate timing at the floor, carry-over of the
current layer's selection, a disjoint alternation that never opens the gate,
the popularity boost changing a victim).  The library's own policy code
(hummingflight_amd/csrc/expert_stream_policy.h), built with g++ into
tests/stream_policy/driver, must then make the same decision at every step of
randomised correlated routing histories.
"""
import os
import random
import shutil
import subprocess

import numpy as np
import pytest

from oracle.stream_policy import COUNTERS, Options, StreamPolicy

HERE = os.path.dirname(os.path.abspath(__file__))
DRIVER_DIR = os.path.join(HERE, "stream_policy")
DRIVER = os.path.join(DRIVER_DIR, "driver")


def brute_lru(slots, calls):
    """Slots by last-use time: an empty slot (lowest index), else the oldest unheld."""
    key, last, clock, out = [None] * slots, [0] * slots, 0, []
    for layer, topk in calls:
        held, res = [], []
        for e in topk:
            k = (layer, e)
            if k in key:
                s, copy = key.index(k), False
            else:
                empty = [i for i in range(slots) if key[i] is None and i not in held]
                s = empty[0] if empty else min((i for i in range(slots) if i not in held), key=lambda i: last[i])
                key[s], copy = k, True
            clock += 1
            last[s] = clock
            held.append(s)
            res.append((s, copy))
        out.append(res)
    return out


def test_oracle_cache_is_lru():
    rng = random.Random(5)
    for case in range(200):
        k = rng.randint(1, 4)
        slots = rng.randint(k, 3 * k + 2)
        calls = [(rng.randrange(3), rng.sample(range(12), k)) for _ in range(40)]
        p = StreamPolicy(slots, Options(prefetch=False))
        got = [p.call(layer, topk, True)[0] for layer, topk in calls]
        assert got == brute_lru(slots, calls), case
        assert p.n["hits"] + p.n["misses"] == p.n["lookups"] == 40 * k
        assert p.n["copies"] == p.n["misses"]


def run_tokens(p, layers, tokens):
    """tokens: list of per-layer selections; layer l+1 is streamed for l < layers-1."""
    for sel in tokens:
        for layer in range(layers):
            p.call(layer, sel[layer], layer + 1 < layers)


def test_oracle_gate_opens_at_floor():
    # Same routing every token.  A layer's overlap EMA is 0 after its first
    # event and 0.5 after its second, so layer 1's guesses pass a 0.5 floor
    # from the third token on (already resident: no copy).
    sel = [[3, 4], [5, 6]]
    p = StreamPolicy(16)
    run_tokens(p, 2, [sel] * 4)
    assert (p.n["misses"], p.n["hits"], p.n["pred_resident"], p.n["pred_staged"]) == (4, 12, 4, 0)
    # A floor just above 0.5 waits for the third event (EMA 0.75).
    p = StreamPolicy(16, Options(overlap_floor=0.51))
    run_tokens(p, 2, [sel] * 4)
    assert p.n["pred_resident"] == 2


def test_oracle_disjoint_alternation_never_stages():
    a, b = [[0, 1], [2, 3]], [[4, 5], [6, 7]]
    p = StreamPolicy(4)  # too small to keep both: every token misses
    run_tokens(p, 2, [a, b] * 5)
    assert p.n["pred_staged"] == p.n["pred_resident"] == 0
    assert p.n["misses"] == 40  # 10 tokens x 4 keys, none kept from the token before


def test_oracle_carry_over_consumed_and_wasted():
    # Floor 0: on the first token layer 1 has no history, so layer 0's own
    # selection is copied ahead as layer 1's guess.  Expert 3 is then used
    # (consumed), expert 4 never is; evicting it later counts as wasted.
    p = StreamPolicy(4, Options(overlap_floor=0.0))
    looked, staged = p.call(0, [3, 4], True)
    assert looked == [(0, True), (1, True)] and staged == [(3, 2), (4, 3)]
    looked, staged = p.call(1, [3, 5], False)
    assert looked == [(2, False), (0, True)]
    assert (p.n["pred_staged"], p.n["pred_consumed"], p.n["pred_wasted"]) == (2, 1, 0)
    p.call(1, [6, 7], False)  # least recent unheld: slot 1 (expert 0:4), then slot 3 (1:4, unused)
    assert (p.n["pred_wasted"], p.find((1, 4)), p.find((0, 4))) == (1, -1, -1)


def test_oracle_popularity_boost_changes_victims():
    # Three slots.  Expert 0, routed at the first two calls, is the layer's
    # hottest at the second and resident by then (the routing is reported
    # before the lookups): its one-sweep protection makes the third call evict
    # experts 1 and 2 instead of 1 and 0.
    calls = [(0, [0, 1]), (0, [0, 2]), (0, [3, 4])]
    plain = StreamPolicy(3, Options(prefetch=False))
    boosted = StreamPolicy(3, Options(prefetch=False, ema_predictor=True))
    for layer, topk in calls:
        a = plain.call(layer, topk, False)[0]
        b = boosted.call(layer, topk, False)[0]
    assert a == [(1, True), (0, True)]
    assert b == [(1, True), (2, True)]
    assert boosted.find((0, 0)) == 0 and plain.find((0, 0)) == -1


def test_oracle_extra_depth_copies_the_most_probable_winners():
    # setRouterPrefetch(extra, ...): after the overlap gate (closed on the first
    # token), this token's winners by descending routing weight become layer
    # 1's guesses, up to extra_depth of them; ties keep rank order.
    p = StreamPolicy(16, Options(extra_depth=2))
    looked, staged = p.call(0, [3, 4, 5], 1, probs=[0.2, 0.5, 0.3])
    assert [s for s, _ in looked] == [0, 1, 2] and staged == [(4, 3), (5, 4)]
    assert p.n["pred_staged"] == 2
    p = StreamPolicy(16, Options(extra_depth=3))
    assert p.call(0, [3, 4, 5], 1, probs=[0.4, 0.4, 0.4])[1] == [(3, 3), (4, 4), (5, 5)]
    # No next layer: nothing (the reference stops before its guesses).
    p = StreamPolicy(16, Options(extra_depth=2))
    assert p.call(0, [3, 4, 5], 0, probs=[0.2, 0.5, 0.3])[1] == []
    # An open gate's guesses come first and are not repeated.
    p = StreamPolicy(16, Options(extra_depth=1, overlap_floor=0.0))
    assert p.call(0, [3, 4], 1, probs=[0.3, 0.6])[1] == [(3, 2), (4, 3)]


def test_oracle_probability_pins_survive_eviction():
    # probPriority: expert 0 (weight 0.95 >= 0.9 x the layer's running maximum
    # 1.0, looked up twice before) is pinned at its third call, so three later
    # cold experts evict experts 1 and 2 around it; without the rule, or with
    # no next layer (the reference returns before its pin rule), expert 0 goes.
    def run(opt, next_layer):
        p = StreamPolicy(3, opt)
        for e, w in [(0, 1.0), (0, 1.0), (0, 0.95), (1, 0.5), (2, 0.5)]:
            p.call(0, [e], next_layer, probs=[w])
        return p, p.call(0, [3], next_layer, probs=[0.5])[0]
    p, looked = run(Options(prefetch=False, prob_resident=True), 2)
    assert looked == [(1, True)] and p.n["pinned"] == 1 and p.find((0, 0)) == 0
    for opt, nl in [(Options(prefetch=False), 2), (Options(prefetch=False, prob_resident=True), 0)]:
        p, looked = run(opt, nl)
        assert looked == [(0, True)] and p.n["pinned"] == 0
    # Weight 0.85 < 0.9: no pin.
    p = StreamPolicy(3, Options(prefetch=False, prob_resident=True))
    for e, w in [(0, 1.0), (0, 1.0), (0, 0.85)]:
        p.call(0, [e], 2, probs=[w])
    assert p.n["pinned"] == 0


def test_oracle_demand_lookup_takes_a_pinned_slot_when_nothing_else_is_left():
    p = StreamPolicy(2, Options(prefetch=False, prob_resident=True))
    for _ in range(3):
        p.call(0, [0, 1], 2, probs=[1.0, 1.0])
    assert p.n["pinned"] == 2
    looked, _ = p.call(0, [5], 2, probs=[1.0])
    assert looked == [(0, True)] and p.find((0, 0)) == -1  # least recent of the pinned


def correlated_history(rng, layers, tokens, k, n_experts, p_change):
    cur = [rng.sample(range(n_experts), k) for _ in range(layers)]
    hist = []
    for _ in range(tokens):
        step = []
        for layer in range(layers):
            sel = list(cur[layer])
            for i in range(k):
                if rng.random() < p_change:
                    sel[i] = rng.choice([e for e in range(n_experts) if e not in sel])
            cur[layer] = sel
            step.append(sel)
        hist.append(step)
    return hist


@pytest.fixture(scope="module")
def driver():
    if not shutil.which("g++"):
        pytest.skip("g++ not available")
    subprocess.run(["make", "-s", "-C", DRIVER_DIR], check=True)
    return DRIVER


def test_library_policy_matches_oracle(driver):
    rng = random.Random(11)
    for case in range(60):
        k = rng.choice([1, 2, 4, 8])
        layers = rng.randint(1, 4)
        slots = rng.choice([2 * k, 3 * k, layers * k, 2 * layers * k + 1])
        opt = Options(prefetch=rng.random() < 0.8, ema_predictor=rng.random() < 0.5,
                      ema_alpha=rng.choice([0.1, 0.5, 1.0]), overlap_floor=rng.choice([0.0, 0.3, 0.5, 0.8]),
                      overlap_alpha=rng.choice([0.5, 0.3, 1.0]), extra_depth=rng.choice([0, 0, 1, 3, 8]),
                      prob_resident=rng.random() < 0.5)
        hist = correlated_history(rng, layers, 12, k, 24, rng.choice([0.0, 0.2, 0.5, 1.0]))
        lines = [f"opt {int(opt.prefetch)} {int(opt.ema_predictor)} {opt.ema_alpha} {opt.overlap_floor} "
                 f"{opt.overlap_alpha} {opt.extra_depth} {int(opt.prob_resident)}", f"reset {slots}"]
        p = StreamPolicy(slots, opt)
        want = []
        last_next = rng.choice([0, 2])  # the last layer: no next layer, or an HBM-resident one
        for step in hist:
            for layer in range(layers):
                sel = step[layer]
                nl = 1 if layer + 1 < layers else last_next
                # routing weights as float32 values, some tied
                probs = [float(np.float32(rng.choice([0.5, 1.0, rng.uniform(0.05, 2.5)]))) for _ in sel]
                lines.append(f"call {layer} {nl} {k} " + " ".join(map(str, sel)) + " " +
                             " ".join(repr(v) for v in probs))
                looked, staged = p.call(layer, sel, nl, probs=probs)
                want.append("L" + "".join(f" {s} {int(c)}" for s, c in looked))
                want.append("S" + "".join(f" {e} {s}" for e, s in staged))
        want.append("C " + " ".join(str(p.n[c]) for c in COUNTERS))
        r = subprocess.run([driver], input="\n".join(lines) + "\n", capture_output=True, text=True, check=True)
        got = r.stdout.strip().split("\n")
        assert len(got) == len(want), case
        for i, (g, w) in enumerate(zip(got, want)):
            assert g.strip() == w.strip(), f"case {case} line {i}: library {g!r} oracle {w!r}"


def test_library_forget_layer_drops_only_that_layer(driver):
    # Re-registering a layer's weights must not serve its old cached copies;
    # the other layers' entries and slots stay (no counterpart in the
    # reference, whose device cache is never re-keyed).
    lines = ["opt 0 0 0.1 0.5 0.5", "reset 8", "call 0 0 2 1 2", "call 1 0 2 1 2", "forget 0",
             "call 0 0 2 1 2", "call 1 0 2 1 2"]
    r = subprocess.run([driver], input="\n".join(lines) + "\n", capture_output=True, text=True, check=True)
    out = r.stdout.strip().split("\n")
    assert out[0] == "L 0 1 1 1" and out[2] == "L 2 1 3 1"
    assert out[4] == "L 0 1 1 1"  # layer 0 copied again into its freed slots
    assert out[6] == "L 2 0 3 0"  # layer 1 still resident
    assert out[-1].split()[1:4] == ["8", "2", "6"]  # lookups, hits, misses


def test_library_drop_slot_recopies(driver):
    # A copy that could not be queued leaves its slot empty: the next lookup of
    # that expert copies it again instead of serving a slot that never received
    # it (no counterpart in the reference, whose staging either succeeds or
    # falls back to the CPU).
    lines = ["opt 0 0 0.1 0.5 0.5", "reset 4", "call 0 0 2 5 6", "drop 1", "call 0 0 2 5 6", "drop 9", "drop -1"]
    r = subprocess.run([driver], input="\n".join(lines) + "\n", capture_output=True, text=True, check=True)
    out = r.stdout.strip().split("\n")
    assert out[0] == "L 0 1 1 1"
    assert out[2] == "L 0 0 1 1"  # expert 5 still resident, expert 6 copied again into the freed slot
    assert out[-1].split()[1:4] == ["4", "1", "3"]  # lookups, hits, misses
