"""Streamed experts with the HBM expert cache and next-layer copy-ahead.

Three layers with routed experts in pinned host RAM and a small slot pool (a
token's 12 experts do not all fit), over a run of correlated tokens.  Checks:
every token's layer-0 and layer-2 outputs against the oracle; the library's
cache and prediction counters equal to the oracle policy's replay of the same
routing; outputs bit-identical to a run with copy-ahead off (copy-ahead moves
weights earlier, never changes them).
"""
import ctypes as C

import numpy as np
import pytest

import oracle as O
from hummingflight_amd import capi, synth
from moe_harness import assert_close, ulp_diff
from oracle.stream_policy import COUNTERS, Options, StreamPolicy

pytestmark = pytest.mark.gpu

DIMS = dict(hidden=1024, inter=512, n_experts=32, top_k=4)
LAYERS, SLOTS, SEED = 3, 10, 81


def set_options(**kw):
    o = capi.StreamOptions()
    capi.call("hfmoe_stream_get_options", C.byref(o))
    for k, v in kw.items():
        setattr(o, k, v)
    capi.call("hfmoe_stream_set_options", C.byref(o))


def read_counters():
    c = capi.StreamCounters()
    capi.call("hfmoe_stream_read_counters", C.byref(c))
    return c.as_dict()


def tokens(n, d, rng):
    base = rng.standard_normal(d).astype(np.float32)
    return [(base + 0.35 * rng.standard_normal(d)).astype(np.float32) for _ in range(n)]


def run_chain(xs, d, k, E):
    """Each token through layers 0..2 (same input to each): outputs, logits, selections."""
    out, lg, idx = capi.DeviceBuffer(d * 4), capi.DeviceBuffer(E * 4), capi.DeviceBuffer(k * 4)
    w = capi.DeviceBuffer(k * 4)
    dbg = capi.RouteDebug(lg.ptr, idx.ptr, w.ptr, None, None)
    res = []
    for x in xs:
        xd = capi.DeviceBuffer.of(x)
        for layer in range(LAYERS):
            capi.call("hfmoe_moe_forward_debug", layer, xd.ptr, 1, out.ptr, None, C.byref(dbg))
            capi.call("hfmoe_synchronize")
            res.append(dict(layer=layer, out=out.download(np.float32, d), logits=lg.download(np.float32, E),
                            idx=idx.download(np.int32, k).tolist(), w=w.download(np.float32, k)))
        xd.free()
    for b in (out, lg, idx, w):
        b.free()
    return res


@pytest.mark.parametrize("opts", [dict(), dict(overlap_floor=0.0, ema_predictor=1),
                                  dict(extra_depth=2, prob_resident=1)],
                         ids=["reference_defaults", "always_copy_ahead_with_popularity", "router_probability_mode"])
def test_streamed_cache_and_copy_ahead(hf, opts):
    d, k, E = DIMS["hidden"], DIMS["top_k"], DIMS["n_experts"]
    shape = synth.LayerShape(n_group=4, topk_group=2, **DIMS)
    cfg = shape.config(max_tokens=1)
    cfg.vram_budget_bytes = SLOTS * 6 * d * DIMS["inter"]
    capi.call("hfmoe_configure", cfg)
    layers = [synth.DeviceLayer(shape, layer=l, seed=SEED, experts_on_host=True) for l in range(LAYERS)]
    refs = [O.SyntheticLayer(O.LayerSpec(n_group=4, topk_group=2, seed=SEED, layer=l, **DIMS))
            for l in range(LAYERS)]
    xs = tokens(8, d, np.random.default_rng(SEED))

    full = dict(prefetch_next_layer=1, ema_predictor=0, ema_alpha=0.1, overlap_floor=0.5, overlap_alpha=0.5,
                extra_depth=0, prob_resident=0)
    full.update(opts)
    set_options(**full)
    capi.call("hfmoe_stream_reset")
    got = run_chain(xs, d, k, E)
    n = read_counters()
    assert n["slots"] == SLOTS

    # The oracle policy fed the same selections makes the same decisions.
    pol = StreamPolicy(SLOTS, Options(prefetch=True, ema_predictor=bool(full["ema_predictor"]),
                                      ema_alpha=full["ema_alpha"], overlap_floor=full["overlap_floor"],
                                      overlap_alpha=full["overlap_alpha"], extra_depth=full["extra_depth"],
                                      prob_resident=bool(full["prob_resident"])))
    for r in got:  # the last layer has no next layer registered
        pol.call(r["layer"], r["idx"], 1 if r["layer"] + 1 < LAYERS else 0, probs=r["w"].tolist())
    assert {c: n[c] for c in COUNTERS} == pol.n
    assert n["misses"] > 0 and n["hits"] > 0
    if full["overlap_floor"] == 0.0 or full["extra_depth"]:
        assert n["pred_staged"] > 0 and n["pred_consumed"] > 0

    # Outputs: oracle per token (selection given the GPU's logits).
    for i, r in enumerate(got):
        if r["layer"] == 1:
            continue
        ref = refs[r["layer"]]
        x = xs[i // LAYERS]
        ridx, rw = ref.route(r["logits"])
        assert r["idx"] == ridx.tolist(), f"token {i // LAYERS} layer {r['layer']}: selection"
        assert ulp_diff(r["w"], rw).max() == 0
        assert_close(r["out"], ref.combine(x, ridx, rw), f"token {i // LAYERS} layer {r['layer']}")

    # Copy-ahead off, cache emptied: the same bits.
    set_options(**dict(full, prefetch_next_layer=0))
    capi.call("hfmoe_stream_reset")
    again = run_chain(xs, d, k, E)
    assert read_counters()["pred_staged"] == 0
    for a, b in zip(got, again):
        assert np.array_equal(a["out"].view(np.uint32), b["out"].view(np.uint32))
    set_options(prefetch_next_layer=1, ema_predictor=0, ema_alpha=0.1, overlap_floor=0.5, overlap_alpha=0.5,
                extra_depth=0, prob_resident=0)
    for L in layers:
        L.free()


def test_reregistered_streamed_layer_drops_cached_experts(hf):
    # The same token through layer 0 registered with one weight set, then
    # re-registered with another: the second output must be the second
    # layer's, not a mix with experts cached from the first.
    d, k = DIMS["hidden"], DIMS["top_k"]
    shape = synth.LayerShape(n_group=4, topk_group=2, **DIMS)
    cfg = shape.config(max_tokens=1)
    cfg.vram_budget_bytes = 64 * 6 * d * DIMS["inter"]  # room for every expert
    capi.call("hfmoe_configure", cfg)
    x = np.random.default_rng(5).standard_normal((1, d)).astype(np.float32)
    outs = []
    for seed in (91, 92):
        L = synth.DeviceLayer(shape, layer=0, seed=seed, experts_on_host=True)
        got = run_chain_one(x, d, k, DIMS["n_experts"])
        ref = O.SyntheticLayer(O.LayerSpec(n_group=4, topk_group=2, seed=seed, layer=0, **DIMS))
        ridx, rw = ref.route(got["logits"])
        assert got["idx"] == ridx.tolist()
        assert_close(got["out"], ref.combine(x[0], ridx, rw), f"weights of seed {seed}")
        outs.append((L, got))
    assert read_counters()["misses"] == 2 * k  # both registrations copied their experts
    for L, _ in outs:
        L.free()


def run_chain_one(x, d, k, E):
    out, lg, idx, w = capi.DeviceBuffer(d * 4), capi.DeviceBuffer(E * 4), capi.DeviceBuffer(k * 4), capi.DeviceBuffer(k * 4)
    dbg = capi.RouteDebug(lg.ptr, idx.ptr, w.ptr, None, None)
    xd = capi.DeviceBuffer.of(x)
    capi.call("hfmoe_moe_forward_debug", 0, xd.ptr, 1, out.ptr, None, C.byref(dbg))
    capi.call("hfmoe_synchronize")
    res = dict(out=out.download(np.float32, d), logits=lg.download(np.float32, E),
               idx=idx.download(np.int32, k).tolist())
    for b in (out, lg, idx, w, xd):
        b.free()
    return res
