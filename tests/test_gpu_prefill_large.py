"""Full-shape prefill chunks larger than 4096 tokens (d = 6144, 256 experts
top-8 + 1 shared, near-uniform routing):

  * T = 6000: ~187 rows per expert, so most experts span two M tiles of the
    160-row tile list (the down projection's, and gate/up's with FP32
    activations) and many two of the 192-row list (gate/up's with BF16-valued
    activations); the shared expert's 6000 rows take 38 and 32 tiles;
  * T = 8192, the largest batch a configuration accepts (max_tokens): ~256
    rows per expert, nearly every expert over two tiles of both lists, the
    shared expert's rows in 52 and 43 tiles, 73,728 rows of h and y (the
    largest workspace of this layer shape).

With BF16-valued and with FP32 activations:
  * dispatch and every token's selection and routing weights bit-exact with
    the oracle's given the GPU's router logits;
  * every output against a float32 reference of the whole layer (the
    oracle's weights and routing), as a share of the 1e-2 relative + 2e-3
    absolute tolerance (must stay below 0.8);
  * a token of every M tile of both tile lists against the oracle's moeLayer
    restatement;
  * bit for bit against the narrower split tiles (HFMOE_PREFILL_WIDE=0).
"""
import numpy as np
import pytest

import oracle as O
from hummingflight_amd import capi
from moe_harness import (FULL, DeviceBackedLayer, Run, assert_close, layer_reference_f32, tile_cover_tokens,
                         tolerance_share, ulp_diff)

pytestmark = pytest.mark.gpu

D, E, K = FULL["hidden"], FULL["n_experts"], FULL["top_k"]
SEEDS = {6000: 67, 8192: 68}  # batch size -> seed of the layer and its tokens


@pytest.fixture(scope="module", params=sorted(SEEDS), ids=lambda t: f"T{t}")
def big_layer(request, hf):
    T = request.param
    seed = SEEDS[T]
    print(f"T = {T}: building the full-shape layer (seed {seed})", flush=True)
    bias = O.fill_f32(E, seed, O.tensor_id(0, O.ROLE_BIAS), 0.0, 0.001)
    r = Run(FULL, n_group=8, topk_group=4, seed=seed, T=T, bias=bias)
    host = DeviceBackedLayer(r.spec, r.dev)
    yield T, seed, r, host
    r.free()


@pytest.mark.parametrize("fp32_x", [False, True], ids=["bf16_valued_x", "fp32_x"])
def test_prefill_large_multi_tile_experts(big_layer, fp32_x, monkeypatch):
    T, seed, r, host = big_layer
    xh = O.make_x(T, D, seed).astype(np.float32)
    if fp32_x:  # not BF16-valued: the x lo half enters the gate/up GEMM too
        rng = np.random.default_rng(seed)
        xh = (xh * (1.0 + np.float32(2.0 ** -10) * rng.standard_normal(xh.shape).astype(np.float32))).astype(
            np.float32)
    what = f"T = {T}, " + ("FP32 x" if fp32_x else "BF16-valued x")
    print(f"{what}: forward", flush=True)
    x = capi.DeviceBuffer.of(xh)
    res = r.forward(x, T)
    monkeypatch.setenv("HFMOE_PREFILL_WIDE", "0")
    narrow = r.forward(x, T)
    monkeypatch.delenv("HFMOE_PREFILL_WIDE")
    x.free()
    assert np.array_equal(res["out"].view(np.uint32), narrow["out"].view(np.uint32)), "wide and narrow tiles differ"

    counts, offsets, perm = O.dispatch(res["idx"], E)
    assert np.array_equal(res["offsets"], offsets) and np.array_equal(res["perm"], perm)
    for t in range(T):
        ridx, rw = r.ref.route(res["logits"][t])
        assert res["idx"][t].tolist() == ridx.tolist(), f"token {t}: selection differs"
        assert ulp_diff(res["w"][t], rw).max() == 0, f"token {t}: routing weights differ"
    two160, two192 = int((counts > 160).sum()), int((counts > 192).sum())
    print(f"{what}: experts over 160 rows {two160}, over 192 rows {two192}, max {int(counts.max())}", flush=True)
    assert two160 > 64 and two192 > 8

    print(f"{what}: float32 reference of all {T} tokens", flush=True)
    ref = layer_reference_f32(host, xh, res["idx"], res["w"])
    share = tolerance_share(res["out"], ref)
    print(f"{what}: worst share of the tolerance over {ref.size} outputs: {share:.4f}", flush=True)
    assert share < 0.8, share

    picks = sorted(set(tile_cover_tokens(res["offsets"], res["perm"], T, K, 192, 1)) |
                   set(tile_cover_tokens(res["offsets"], res["perm"], T, K, 160, 1)))
    print(f"{what}: {len(picks)} tokens cover every M tile of both lists; oracle moeLayer on each", flush=True)
    for t in picks:
        assert_close(res["out"][t], host.combine(xh[t], res["idx"][t], res["w"][t]), f"{what}: token {t}")
