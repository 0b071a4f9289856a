"""Full-shape prefill (T = 4096, d = 6144, 256 experts top-8 + 1 shared) checked
over every output.

The prefill chunk runs the MFMA grouped GEMMs on M tiles of 512 weight rows
(gate/up on 192 rows, or 160 with FP32 activations; down on 160), h entering
the down projection as BF16 hi + lo halves.  Each batch is
checked three ways:
  * dispatch offsets and permutation bit-exact with the oracle's stable
    counting sort, every token's selection and routing weights bit-exact with
    the oracle's given the GPU's router logits;
  * every one of the 25M outputs against a float32 reference of the whole
    layer (the oracle's weights and routing, FP32 FFNs, float64 combine), as
    a share of the 1e-2 relative + 2e-3 absolute tolerance, which must stay
    below 0.8 (it measures ~0.01-0.03; an FP16 h measured 0.61 here with
    near-uniform routing and 1.1-1.7 with skewed weights);
  * a token of every M tile of both tile lists of the dispatch (every routed
    expert's tiles, all of a hot expert's and all 22 / 26 of the shared
    expert's) against the oracle's own moeLayer restatement;
  * (uniform and Zipf) bit for bit against the narrower tiles (192 x 256
    gate/up, 192 x 384 down).

Routing: near-uniform (bias ~N(0, 0.001)), with BF16-valued and with FP32
activations; skewed routing weights (a trained router's spread: tokens with
one, two or three dominant experts whose normalised x 2.5 weights reach
~1.5-2, beside light pairs of ~0.02); Zipf(1.1)-skewed expert popularity.
"""
import json
import os

import numpy as np
import pytest

import oracle as O
from hummingflight_amd import capi
from moe_harness import (FULL, DeviceBackedLayer, Run, assert_close, layer_reference_f32, tile_cover_tokens,
                         tolerance_share, ulp_diff)

pytestmark = pytest.mark.gpu

T, D, E, K = 4096, FULL["hidden"], FULL["n_experts"], FULL["top_k"]
TILE, GU_TILE = 192, 160  # prefill M-tile rows at this size: the two tile lists


@pytest.fixture(scope="module")
def layer66(hf):
    bias = O.fill_f32(E, 66, O.tensor_id(0, O.ROLE_BIAS), 0.0, 0.001)
    r = Run(FULL, n_group=8, topk_group=4, seed=66, T=T, bias=bias)
    host = DeviceBackedLayer(r.spec, r.dev)
    yield r, host
    r.free()


def check_routing(r, res):
    counts, offsets, perm = O.dispatch(res["idx"], E)
    assert np.array_equal(res["offsets"], offsets), "expert offsets differ from the oracle"
    assert np.array_equal(res["perm"], perm), "dispatch permutation differs from the oracle"
    for t in range(T):
        ridx, rw = r.ref.route(res["logits"][t])
        assert res["idx"][t].tolist() == ridx.tolist(), f"token {t}: selection differs"
        assert ulp_diff(res["w"][t], rw).max() == 0, f"token {t}: routing weights differ"
    return counts


def check_every_output(host, xh, res, what):
    print(f"{what}: float32 reference of all {T} tokens", flush=True)
    ref = layer_reference_f32(host, xh, res["idx"], res["w"])
    share = tolerance_share(res["out"], ref)
    print(f"{what}: worst share of the tolerance over {ref.size} outputs: {share:.4f}", flush=True)
    assert share < 0.8, share
    return share


def check_tiles_against_oracle(host, xh, res, what):
    picks = sorted(set(tile_cover_tokens(res["offsets"], res["perm"], T, K, TILE, 1)) |
                   set(tile_cover_tokens(res["offsets"], res["perm"], T, K, GU_TILE, 1)))
    print(f"{what}: {len(picks)} tokens cover every M tile; oracle moeLayer on each", flush=True)
    for t in picks:
        ref = host.combine(xh[t], res["idx"][t], res["w"][t])
        assert_close(res["out"][t], ref, f"{what}: token {t}")


def narrow_tiles_agree(r, x, res, monkeypatch):
    # The wide tiles (512 weight rows per item) accumulate every output in
    # the same order as the narrower ones (192 x 256 gate/up, 192 x 384 down;
    # HFMOE_PREFILL_WIDE=0): K stage by stage, hi then lo, k half 0 then 1.
    monkeypatch.setenv("HFMOE_PREFILL_WIDE", "0")
    narrow = r.forward(x, T)
    monkeypatch.delenv("HFMOE_PREFILL_WIDE")
    assert np.array_equal(res["out"].view(np.uint32), narrow["out"].view(np.uint32)), "wide and narrow tiles differ"


@pytest.mark.parametrize("fp32_x", [False, True], ids=["bf16_valued_x", "fp32_x"])
def test_prefill_4096_uniform_every_output(layer66, fp32_x, monkeypatch):
    # Config 4: near-uniform routing, ~128 rows per expert, every routing
    # weight ~2.5 / 8.
    r, host = layer66
    xh = O.make_x(T, D, 66).astype(np.float32)
    if fp32_x:  # activations that are not BF16-valued: the x lo half enters the GEMMs too
        rng = np.random.default_rng(7)
        xh = (xh * (1.0 + np.float32(2.0 ** -10) * rng.standard_normal(xh.shape).astype(np.float32))).astype(
            np.float32)
    x = capi.DeviceBuffer.of(xh)
    res = r.forward(x, T)
    # Workgroups draw GEMM items from counters in whatever order they arrive;
    # every item is computed the same way wherever it runs: a second call is
    # bit-identical.
    again = r.forward(x, T)
    assert np.array_equal(res["out"].view(np.uint32), again["out"].view(np.uint32))
    narrow_tiles_agree(r, x, res, monkeypatch)
    x.free()
    counts = check_routing(r, res)
    assert counts.sum() == T * K
    what = "uniform, " + ("FP32 x" if fp32_x else "BF16-valued x")
    check_every_output(host, xh, res, what)
    if not fp32_x:
        check_tiles_against_oracle(host, xh, res, what)


def skewed_tokens(router_bits, seed, mu=6.0, delta=10.0):
    """Activations whose routing weights spread as a trained router's do.

    With the router rows W (E x d), x = z + m + sum of plants: z ~ N(0, 1);
    m solves W m = -mu (minimal norm), pulling every logit down by mu so that
    the top-8 sigmoid scores of unplanted experts fall to ~0.03-0.2; a plant
    adds delta * W_e / |W_e|^2, lifting expert e's logit by delta to a score
    of ~0.95-1.  Each token gets 0, 1, 2 or 3 plants (p = .2, .4, .3, .1) on
    uniformly drawn experts, so expert load stays near-uniform while the
    normalised x 2.5 weights range from ~1.5 (one dominant expert) down to
    ~0.05.  Rounded to BF16 values."""
    W = O.bf16_to_f32(router_bits).reshape(E, D).astype(np.float64)
    rng = np.random.default_rng(seed)
    m = -mu * (W.T @ np.linalg.solve(W @ W.T, np.ones(E)))
    plants = np.zeros((T, E))
    n = rng.choice(4, size=T, p=[0.2, 0.4, 0.3, 0.1])
    for t in range(T):
        plants[t, rng.choice(E, n[t], replace=False)] = delta
    x = rng.standard_normal((T, D)) + m + plants @ (W / np.einsum("ed,ed->e", W, W)[:, None])
    return O.bf16_to_f32(O.f32_to_bf16(x.astype(np.float32))).reshape(T, D)


def test_prefill_4096_skewed_routing_weights(layer66):
    r, host = layer66
    xh = skewed_tokens(r.ref.router, seed=67)
    x = capi.DeviceBuffer.of(xh)
    res = r.forward(x, T)
    x.free()
    counts = check_routing(r, res)
    top = res["w"].max(axis=1)
    sq = (res["w"].astype(np.float64) ** 2).sum(axis=1)
    print(f"skewed: top weight >= 1 for {np.mean(top >= 1):.2f} of tokens, max {top.max():.3f}, "
          f"smallest weight {res['w'].min():.4f}, sum of squared weights up to {sq.max():.2f}; "
          f"rows per expert {counts.min()}..{counts.max()}", flush=True)
    assert np.mean(top >= 1.0) > 0.3 and top.max() > 1.3 and res["w"].min() < 0.1
    check_every_output(host, xh, res, "skewed weights")
    heavy = np.argsort(-top)[:8].tolist()
    for t in heavy:  # the heaviest-weighted tokens against the oracle
        assert_close(res["out"][t], host.combine(xh[t], res["idx"][t], res["w"][t]), f"token {t}")


def test_prefill_4096_zipf_every_output(hf, monkeypatch):
    # Zipf(1.1)-skewed expert popularity: hot experts span several 192-row
    # tiles, cold ones leave their one tile mostly empty.  (Reconfigures the
    # library: runs after the tests on the shared layer.)
    with open(os.path.join(os.path.dirname(__file__), "golden", "zipf_bias_e256.json")) as fh:
        zb = json.load(fh)
    seed = zb["layer_seed"]
    r = Run(FULL, n_group=8, topk_group=4, seed=seed, T=T, bias=np.array(zb["bias"], np.float32))
    host = DeviceBackedLayer(r.spec, r.dev)
    xh = O.make_x(T, D, seed).astype(np.float32)
    x = capi.DeviceBuffer.of(xh)
    res = r.forward(x, T)
    narrow_tiles_agree(r, x, res, monkeypatch)
    x.free()
    counts = check_routing(r, res)
    assert counts.max() > 2 * TILE and counts.min() < 96
    check_every_output(host, xh, res, "Zipf popularity")
    check_tiles_against_oracle(host, xh, res, "Zipf popularity")
    r.free()
