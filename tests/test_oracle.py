"""Pins the CPU oracle (oracle/oracle.c) before the HIP path is tested against it.

Each function is checked against the reference's own outputs
(tests/golden/reference_vectors.json, written by gen_golden.py from the
reference's compiled sources), the reference's known-answer tests
(src/self_test.cpp:53-200), and what the mathematics fixes (closed forms,
brute force on tiny inputs, invariants).
"""
import ctypes as C
import itertools

import numpy as np
import pytest


def f32(bits):
    return np.array(bits, np.uint32).view(np.float32)


# ---------------------------------------------------------------- BF16 ----

def test_bf16_matches_reference_outputs(oracle_lib, golden):
    O = oracle_lib
    g = golden["bf16"]
    for vb, ob in zip(g["in"], g["out"]):
        v = f32([vb])[0]
        assert O.lib().orc_bf16_from_f32(float(v)) == ob


def test_bf16_known_answers(oracle_lib):
    # src/self_test.cpp:56-69: exact round trips and precision bound.
    O = oracle_lib
    L = O.lib()
    for v in [1.0, 2.0, -1.5, 0.5, 0.0]:
        assert L.orc_bf16_to_f32(L.orc_bf16_from_f32(v)) == v
    assert L.orc_bf16_to_f32(L.orc_bf16_from_f32(-0.0)) == 0.0
    for v in [0.1, 0.3, 1 / 3, 123.456, -987.654, 1e-3, 1e3]:
        r = L.orc_bf16_to_f32(L.orc_bf16_from_f32(v))
        assert abs(r - v) / abs(v) < 1e-2


def test_bf16_round_to_nearest_even_closed_form(oracle_lib):
    # Ties go to the even mantissa: 1 + 2^-8 (halfway) -> 1.0; 1 + 3*2^-8 -> 1 + 2^-6.
    O = oracle_lib
    L = O.lib()
    assert L.orc_bf16_to_f32(L.orc_bf16_from_f32(1.0 + 2 ** -8)) == 1.0
    assert L.orc_bf16_to_f32(L.orc_bf16_from_f32(1.0 + 3 * 2 ** -8)) == 1.0 + 2 ** -6
    assert L.orc_bf16_to_f32(L.orc_bf16_from_f32(1.0 + 2 ** -8 + 2 ** -20)) == 1.0 + 2 ** -7
    # Vectorised helper agrees with the C function on random bits.
    rng = np.random.default_rng(0)
    u = rng.integers(0, 2 ** 32, 20000, dtype=np.uint64).astype(np.uint32)
    u = u[(u & 0x7F800000) != 0x7F800000]  # finite only
    vals = u.view(np.float32)
    vec = O.f32_to_bf16(vals)
    ref = np.array([L.orc_bf16_from_f32(float(v)) for v in vals[:2000]], np.uint16)
    assert np.array_equal(vec[:2000], ref)


# ---------------------------------------------------------------- GEMV ----

def test_gemv_bit_exact_vs_reference(oracle_lib, golden):
    O = oracle_lib
    for case in golden["gemv"]:
        M, K = case["M"], case["K"]
        A = O.fill_bf16(M * K, case["seedA"], 1, 0.0, 0.5).reshape(M, K)
        x = O.fill_f32(K, case["seedx"], 2, 0.0, 1.0)
        y0 = O.fill_f32(M, case["seedy"], 3, 0.0, 1.0)
        y = O.gemv(A, x, case["alpha"], case["beta"], y=y0)
        assert np.array_equal(y.view(np.uint32), np.array(case["out"], np.uint32)), (M, K)


def test_gemv_serial_order_closed_form(oracle_lib):
    # Serial float32 order: y = (((a0*x0) + a1*x1) + a2*x2) ... with one
    # rounding per product and per sum (no FMA) -- built here in numpy float32.
    O = oracle_lib
    rng = np.random.default_rng(1)
    M, K = 5, 37
    A = O.f32_to_bf16(rng.uniform(-1, 1, (M, K)).astype(np.float32)).reshape(M, K)
    x = rng.uniform(-1.5, 1.5, K).astype(np.float32)
    Af = O.bf16_to_f32(A)
    exp = np.zeros(M, np.float32)
    for j in range(K):
        exp = (exp + (Af[:, j] * x[j]).astype(np.float32)).astype(np.float32)
    assert np.array_equal(O.gemv(A, x), exp)


def test_gemv_avx2_restatement_close_to_serial(oracle_lib):
    # cpu_kernels.cpp:47-81 reorders the sum: same value to FP32 rounding
    # (self_test.cpp:96-101 allows 1e-3 for this difference).
    O = oracle_lib
    rng = np.random.default_rng(2)
    for M, K in [(8, 33), (16, 2048), (4, 6144), (3, 16), (2, 7)]:
        A = O.f32_to_bf16(rng.uniform(-1, 1, (M, K)).astype(np.float32)).reshape(M, K)
        x = (1.5 * rng.uniform(-1, 1, K)).astype(np.float32)
        ys = O.gemv(A, x)
        ya = O.gemv(A, x, avx2=True)
        exact = O.bf16_to_f32(A).astype(np.float64) @ x.astype(np.float64)
        assert np.max(np.abs(ya - exact)) < 1e-3 * max(1.0, np.max(np.abs(exact)))
        assert np.max(np.abs(ys - exact)) < 1e-3 * max(1.0, np.max(np.abs(exact)))


# ------------------------------------------------------------- sigmoid ----

def test_sigmoid_matches_reference(oracle_lib, golden):
    O = oracle_lib
    g = golden["sigmoid"]
    xs = f32(g["in"])
    got = np.array([O.lib().orc_sigmoid(float(v)) for v in xs], np.float32)
    assert np.array_equal(got.view(np.uint32), np.array(g["out"], np.uint32))


def test_sigmoid_identities(oracle_lib):
    # src/self_test.cpp:170-177.
    s = oracle_lib.lib().orc_sigmoid
    assert abs(s(0.0) - 0.5) < 1e-6
    assert abs(s(100.0) - 1.0) < 1e-6
    assert abs(s(-100.0)) < 1e-6
    for v in [0.3, 2.0, 7.5]:
        assert abs(s(v) + s(-v) - 1.0) < 1e-6


# --------------------------------------------------------------- top-k ----

def test_topk_reference_kat(oracle_lib):
    # src/self_test.cpp:180-200.
    O = oracle_lib
    scores = np.array([0.1, 0.6, 0.9, 0.4, 0.7, 0.2, 0.8, 0.3], np.float32)
    idx, w = O.topk_flat(scores, None, 3, 1.0, False)
    assert idx.tolist() == [2, 6, 4]
    idx_n, w_n = O.topk_flat(scores, None, 3, 1.0, True)
    assert abs(float(w_n.sum()) - 1.0) < 1e-5
    _, w_s = O.topk_flat(scores, None, 3, 2.5, False)
    assert w_s[0] > w[0] + 1e-8
    bias = np.array([0, 0, -10, 0, 0, 0, 0, 0], np.float32)
    idx_b, _ = O.topk_flat(scores, bias, 3, 1.0, False)
    assert idx_b[0] == 6


def test_topk_matches_reference_outputs(oracle_lib, golden):
    O = oracle_lib
    for case in golden["topk"]:
        s = f32(case["scores"])
        bias = None if case["seed_bias"] is None else O.fill_f32(case["E"], case["seed_bias"], 5, 0.0, 0.01)
        idx, w = O.topk_flat(s, bias, case["k"], case["scale"], bool(case["norm"]))
        assert idx.tolist() == case["idx"]
        assert np.array_equal(w.view(np.uint32), np.array(case["w"], np.uint32))


def test_topk_brute_force_tiny(oracle_lib):
    # Selection = the k largest biased scores (lower index on ties), checked
    # against a full sort for every k on small random and tied inputs.
    O = oracle_lib
    rng = np.random.default_rng(3)
    for trial in range(200):
        E = int(rng.integers(1, 12))
        s = rng.choice(np.array([0.1, 0.2, 0.3, 0.5, 0.7], np.float32), E) if trial % 3 == 0 else \
            rng.uniform(0, 1, E).astype(np.float32)
        bias = rng.normal(0, 0.05, E).astype(np.float32) if trial % 2 else None
        key = s + (bias if bias is not None else 0)
        for k in range(1, min(E, 8) + 1):
            order = sorted(range(E), key=lambda i: (-float(np.float32(key[i])), i))[:k]
            idx, w = O.topk_flat(s, bias, k, 1.0, False)
            assert idx.tolist() == order
            assert np.array_equal(w, s[order])


def _grouped_by_sorting(s, bias, k, n_group, topk_group):
    """Group-limited selection written with sorts (an independent formulation)."""
    E = len(s)
    key = (s + (bias if bias is not None else np.float32(0))).astype(np.float32)
    gs = E // n_group
    gscore = []
    for gi in range(n_group):
        members = sorted(range(gi * gs, (gi + 1) * gs), key=lambda i: (-float(key[i]), i))
        top = [float(key[i]) for i in members[:2]]
        gscore.append(float(np.float32(top[0]) + np.float32(top[1])) if len(top) == 2 else top[0])
    kept = sorted(range(n_group), key=lambda gi: (-gscore[gi], gi))[:topk_group]
    cand = [i for i in range(E) if i // gs in kept]
    return sorted(cand, key=lambda i: (-float(key[i]), i))[:k]


def test_grouped_topk_reduces_to_flat(oracle_lib):
    O = oracle_lib
    rng = np.random.default_rng(4)
    for _ in range(100):
        E = int(rng.choice([8, 64, 256]))
        s = rng.uniform(0, 1, E).astype(np.float32)
        b = rng.normal(0, 0.01, E).astype(np.float32)
        a = O.topk_flat(s, b, 8, 2.5, True)
        g1 = O.topk_grouped(s, b, 8, 1, 1, 2.5, True)
        gall = O.topk_grouped(s, b, 8, 8, 8, 2.5, True)  # all groups kept
        assert a[0].tolist() == g1[0].tolist() == gall[0].tolist()
        assert np.array_equal(a[1], g1[1]) and np.array_equal(a[1], gall[1])


def test_grouped_topk_brute_force(oracle_lib):
    O = oracle_lib
    rng = np.random.default_rng(5)
    for trial in range(300):
        n_group = int(rng.choice([2, 4, 8]))
        gs = int(rng.choice([1, 2, 3, 4]))
        E = n_group * gs
        topk_group = int(rng.integers(1, n_group + 1))
        k = int(rng.integers(1, min(8, topk_group * gs) + 1))
        if trial % 4 == 0:
            s = rng.choice(np.array([0.25, 0.5, 0.75], np.float32), E)
            b = None
        else:
            s = rng.uniform(0, 1, E).astype(np.float32)
            b = rng.normal(0, 0.05, E).astype(np.float32)
        idx, w = O.topk_grouped(s, b, k, n_group, topk_group, 1.0, False)
        assert idx.tolist() == _grouped_by_sorting(s, b, k, n_group, topk_group)
        assert np.array_equal(w, s[idx])


def test_grouped_topk_invariants_full_shape(oracle_lib):
    # 256 experts in 8 groups of 32, keep 4: every winner lies in a kept group,
    # and no expert outside the winners but inside kept groups outranks one.
    O = oracle_lib
    rng = np.random.default_rng(6)
    for _ in range(50):
        s = rng.uniform(0, 1, 256).astype(np.float32)
        b = rng.normal(0, 0.01, 256).astype(np.float32)
        idx, w = O.topk_grouped(s, b, 8, 8, 4, 2.5, True)
        key = s + b
        groups = key.reshape(8, 32)
        top2 = np.sort(groups, axis=1)[:, -2:]
        gsc = (top2[:, 1] + top2[:, 0]).astype(np.float32)
        kept = set(np.argsort(-gsc, kind="stable")[:4].tolist())
        assert all(i // 32 in kept for i in idx)
        others = [i for i in range(256) if i // 32 in kept and i not in idx]
        assert min(key[idx]) >= max(key[others])
        assert abs(float(w.sum()) - 2.5) < 1e-5


# ------------------------------------------------------------ dispatch ----

def test_dispatch_is_stable_sort(oracle_lib):
    O = oracle_lib
    rng = np.random.default_rng(7)
    for T, k, E in [(1, 8, 256), (64, 8, 256), (5, 2, 8), (0, 8, 16), (4096, 8, 256)]:
        idx = rng.integers(0, E, (T, k)).astype(np.int32)
        counts, offsets, perm = O.dispatch(idx, E)
        flat = idx.reshape(-1)
        assert np.array_equal(counts, np.bincount(flat, minlength=E))
        assert offsets[0] == 0 and np.array_equal(np.diff(offsets), counts)
        assert np.array_equal(perm, np.argsort(flat, kind="stable"))


# ------------------------------------------------------------- RMSNorm ----

def test_rmsnorm_matches_reference(oracle_lib, golden):
    O = oracle_lib
    for case in golden["rmsnorm"]:
        n = case["n"]
        x = O.fill_f32(n, case["seedx"], 6, 0.0, 1.3)
        w = O.fill_bf16(n, case["seedw"], 7, 1.0, 0.05)
        y = O.rmsnorm(w, x, case["eps"])
        assert np.array_equal(y.view(np.uint32), np.array(case["out"], np.uint32))


# ----------------------------------------------------------- generator ----

def _sm64(z):
    z = (z + np.uint64(0x9E3779B97F4A7C15))
    z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
    z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    return z ^ (z >> np.uint64(31))


def test_generator_matches_its_specification(oracle_lib):
    # SplitMix64 (Steele, Lea, Flood 2014) -> twelve 16-bit uniforms ->
    # (sum - 393210) / 65536, then z*std + mean with two float32 roundings.
    O = oracle_lib
    with np.errstate(over="ignore"):
        seed, tensor, first, n = 77, (3 << 40) | (5 << 32) | 9, 1000, 4096
        key = _sm64(np.uint64(seed) ^ _sm64(np.uint64(tensor)))
        i = np.arange(first, first + n, dtype=np.uint64)
        c = key + np.uint64(3) * i
        tot = np.zeros(n, np.int64)
        for q in range(3):
            v = _sm64(c + np.uint64(q))
            for sh in (0, 16, 32, 48):
                tot += ((v >> np.uint64(sh)) & np.uint64(0xFFFF)).astype(np.int64)
    z = (tot - 393210).astype(np.float32) * np.float32(1 / 65536)
    val = (z * np.float32(0.02)).astype(np.float32) + np.float32(0.5)
    got = O.fill_f32(n, seed, tensor, 0.5, 0.02, first=first)
    assert np.array_equal(got, val.astype(np.float32))
    assert np.array_equal(O.fill_bf16(n, seed, tensor, 0.5, 0.02, first=first), O.f32_to_bf16(val))


def test_generator_statistics(oracle_lib):
    z = oracle_lib.fill_f32(1 << 20, 5, 6, 0.0, 1.0)
    assert abs(float(z.mean())) < 5e-3
    assert abs(float(z.std()) - 1.0) < 5e-3
    assert float(np.abs(z).max()) <= 6.0


# ------------------------------------------------------------ MoE layer ----

def test_config_mini_fixture(golden):
    # The MoE surface of the reference's own config fixture, as its
    # tests/test_fixtures.py reads it.
    m = golden["config_mini"]
    assert (m["hidden_size"], m["n_routed_experts"], m["num_experts_per_tok"], m["n_shared_experts"],
            m["moe_intermediate_size"]) == (16, 8, 2, 1, 16)
    assert m["mlp_layer_types"].count("dense") == m["first_k_dense_replace"] == 1
    assert m["routed_scaling_factor"] == 2.5 and m["norm_topk_prob"] and m["topk_group"] == 1


@pytest.mark.parametrize("which", ["small", "full", "config_mini"])
def test_moe_layer_bit_exact_vs_reference(oracle_lib, golden, which):
    O = oracle_lib
    cases = [c for c in golden["moe_layer"] if c["name"] == which]
    assert cases
    c0 = cases[0]
    spec = O.LayerSpec(hidden=c0["hidden"], inter=c0["inter"], n_experts=c0["n_experts"],
                       top_k=c0["top_k"], n_shared=c0["n_shared"], norm_topk_prob=c0["norm"],
                       routed_scaling_factor=c0["scale"], seed=c0["seed"])
    L = O.SyntheticLayer(spec)
    xs = O.make_x(max(c["token"] for c in cases) + 1, spec.hidden, spec.seed)
    for c in cases:
        out, lg, idx, w = L.forward(xs[c["token"]])
        assert idx.tolist() == c["idx"]
        assert np.array_equal(w.view(np.uint32), np.array(c["w"], np.uint32))
        assert np.array_equal(out.view(np.uint32), np.array(c["out"], np.uint32))


def test_moe_combine_linearity(oracle_lib):
    # Scaling every routing weight by 2 doubles the routed part; zero weights
    # leave the shared expert alone (glm_forward.cpp:639-660).
    O = oracle_lib
    spec = O.LayerSpec(hidden=256, inter=128, n_experts=16, top_k=4, seed=21)
    L = O.SyntheticLayer(spec)
    x = O.make_x(1, 256, 21)[0]
    out, lg, idx, w = L.forward(x)
    shared_only = L.combine(x, idx, np.zeros_like(w))
    doubled = L.combine(x, idx, 2 * w)
    routed = out.astype(np.float64) - shared_only
    assert np.allclose(doubled - shared_only, 2 * routed, rtol=1e-5, atol=1e-5)
    spec0 = O.LayerSpec(hidden=256, inter=128, n_experts=16, top_k=4, seed=21, n_shared=0)
    L0 = O.SyntheticLayer(spec0)
    assert np.array_equal(L0.combine(x, idx, np.zeros_like(w)), np.zeros(256, np.float32))


# ------------------------------------------------------- dense MLP, LM head ----

def dense_weights(O, c):
    H, I, seed, sd = c["hidden"], c["inter"], c["seed"], c["w_std"]
    return (O.fill_bf16(I * H, seed, 1, 0.0, sd), O.fill_bf16(I * H, seed, 2, 0.0, sd),
            O.fill_bf16(H * I, seed, 3, 0.0, sd), O.fill_f32(H, seed, 4, 0.0, 1.0))


@pytest.mark.parametrize("i", [0, 1], ids=["small", "glm_shape"])
def test_dense_mlp_bit_exact_vs_reference(oracle_lib, golden, i):
    O = oracle_lib
    c = golden["dense_mlp"][i]
    gw, uw, dw, x = dense_weights(O, c)
    y = O.dense_mlp(gw, uw, dw, x, c["hidden"], c["inter"])
    assert np.array_equal(y.view(np.uint32), np.array(c["out"], np.uint32))


def test_dense_mlp_closed_forms(oracle_lib):
    # Down is linear (doubling it doubles the output exactly); up = 0 gives 0;
    # a 1x1 MLP is silu(g*x)*(u*x)*d in FP32.
    O = oracle_lib
    H, I = 64, 96
    gw = O.fill_bf16(I * H, 3, 1, 0.0, 0.1)
    uw = O.fill_bf16(I * H, 3, 2, 0.0, 0.1)
    dw = O.fill_bf16(H * I, 3, 3, 0.0, 0.1)
    x = O.fill_f32(H, 3, 4, 0.0, 1.0)
    y = O.dense_mlp(gw, uw, dw, x, H, I)
    d2 = O.f32_to_bf16(2.0 * O.bf16_to_f32(dw))
    assert np.array_equal(O.dense_mlp(gw, uw, d2, x, H, I), 2.0 * y)
    assert not np.any(O.dense_mlp(gw, np.zeros_like(uw), dw, x, H, I))
    g1, u1, dn1 = (O.f32_to_bf16(np.array([v], np.float32)) for v in (0.75, -1.5, 2.0))
    x1 = np.array([1.25], np.float32)
    gv, uv = np.float32(0.75 * 1.25), np.float32(-1.5 * 1.25)
    want = np.float32(np.float32(gv / np.float32(1.0 + np.exp(np.float32(-gv)))) * uv) * np.float32(2.0)
    assert np.isclose(O.dense_mlp(g1, u1, dn1, x1, 1, 1)[0], want, rtol=1e-6)


@pytest.mark.parametrize("i", [0, 1], ids=["small", "glm_vocab"])
def test_lm_head_matches_reference(oracle_lib, golden, i):
    O = oracle_lib
    c = golden["lm_head"][i]
    H, V, seed = c["hidden"], c["vocab"], c["seed"]
    W = O.fill_bf16(V * H, seed, 1, 0.0, 0.02)
    nw = O.fill_bf16(H, seed, 2, 1.0, 0.05)
    h = O.fill_f32(H, seed, 3, 0.0, 1.0)
    logits, best = O.lm_head(W, nw, h, V, c["eps"])
    assert best == c["best"]
    assert np.array_equal(logits[c["top"]].view(np.uint32), np.array(c["top_bits"], np.uint32))
    assert np.array_equal(logits[c["sample"]].view(np.uint32), np.array(c["sample_bits"], np.uint32))


def test_lm_head_argmax_closed_form(oracle_lib):
    # Rows that are scaled copies of the normalised hidden state: the largest
    # scale wins; on an exact tie the first row wins.
    O = oracle_lib
    H = 32
    h = O.fill_f32(H, 5, 1, 0.0, 1.0)
    xn = O.rmsnorm(None, h, 1e-5)
    rows = np.stack([O.f32_to_bf16(s * xn) for s in (0.5, -1.0, 2.0, 1.0, 2.0)])
    logits, best = O.lm_head(rows, None, h, 5, 1e-5)
    assert best == 2 and logits[2] == logits[4]


# --------------------------------------------------------- plugin helpers ----

def test_helpers_match_reference(oracle_lib, golden):
    O = oracle_lib
    h = golden["helpers"]
    e = h["embedding"]
    emb = O.fill_bf16(e["vocab"] * e["hidden"], e["seed"], 1, 0.0, 1.0)
    for r in e["rows"]:
        got = O.embedding(emb, r["token"], e["hidden"])
        assert np.array_equal(got.view(np.uint32), np.array(r["out"], np.uint32))
    for c in h["matvec"]:
        W = O.fill_bf16(c["M"] * c["K"], c["seed"], 1, 0.0, 0.05).reshape(c["M"], c["K"])
        x = O.fill_f32(c["K"], c["seed"], 2, 0.0, 1.0)
        assert np.array_equal(O.gemv(W, x).view(np.uint32), np.array(c["out"], np.uint32))
    for c in h["softmax"]:
        y = O.softmax(O.fill_f32(c["n"], c["seed"], 1, 0.0, c["std"]))
        assert np.array_equal(y[c["sample"]].view(np.uint32), np.array(c["sample_bits"], np.uint32))
        assert float(np.sum(y, dtype=np.float64)) == c["sum64"]
    for c in h["argmax"]:
        x = O.fill_f32(c["n"], c["seed"], 1, 0.0, 1.0)
        x[c["n"] // 3] = x[2 * c["n"] // 3] = float(np.max(x)) + 1.0
        assert O.argmax(x) == c["best"] == c["n"] // 3


def test_softmax_closed_forms(oracle_lib):
    # Equal inputs give 1/n exactly (n a power of two); a shift by a constant
    # changes nothing once the maximum is subtracted; one dominant entry -> 1.
    O = oracle_lib
    assert np.all(O.softmax(np.full(64, 3.25, np.float32)) == np.float32(1 / 64))
    x = O.fill_f32(100, 4, 1, 0.0, 1.0)
    xs = (x + np.float32(16.0)).astype(np.float32)
    assert np.allclose(O.softmax(x), O.softmax(xs), rtol=1e-5, atol=1e-8)
    y = O.softmax(np.array([0.0, 200.0, 0.0], np.float32))
    assert y[1] == 1.0 and y[0] == y[2] == 0.0  # exp(-200) underflows in FP32


def test_cpu_baseline_bench_form(oracle_lib):
    # orc_moe_layer_bench (the bench's CPU baseline) computes what orc_moe_layer
    # computes: bit for bit with the Linux GEMV, with or without the scheduler's
    # per-expert copy; within the AVX2 GEMV's reordering with the MSVC form.
    O = oracle_lib
    spec = O.LayerSpec(hidden=256, inter=128, n_experts=32, top_k=4, n_group=4, topk_group=2, seed=9)
    L = O.SyntheticLayer(spec)
    x = O.make_x(1, spec.hidden, 9)[0].copy()
    ref, _, idx, _ = L.forward(x)
    W, keep = L.weights(range(spec.n_experts))
    cfg = spec.cfg()
    scratch = np.zeros(3 * spec.hidden * spec.inter, np.uint16)
    for avx2, copy in [(0, None), (0, scratch), (1, None), (1, scratch)]:
        out = np.zeros(spec.hidden, np.float32)
        sec = O.lib().orc_moe_layer_bench(C.byref(cfg), C.byref(W), x.ctypes.data, out.ctypes.data, avx2,
                                          None if copy is None else copy.ctypes.data, 3)
        assert sec > 0
        if avx2:
            assert np.max(np.abs(out - ref)) < 1e-3 * max(1.0, np.max(np.abs(ref)))
        else:
            assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))
    # The copy path really computes from the copy: the last selected expert's bytes are in it.
    e = int(idx[-1])
    g, u, d = L.expert(e)
    assert np.array_equal(scratch, np.concatenate([g, u, d]))
