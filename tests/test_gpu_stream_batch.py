"""Streamed experts for more than one token (prefill over host-resident experts).

A T > 1 call on a layer whose routed experts live in pinned host RAM routes the
batch on the device, reads the selections back, and multiplies the batch's
distinct experts a wave at a time: each wave's experts are copied into the HBM
slot pool (or found there) and the grouped GEMMs run with only that wave's
experts in the weight table.  The reference runs a batch token by token through
its streamed moeLayer (glm_forward.cpp:755, :562-602); the bar is the same
per token: selection bit-exact given the GPU's logits, output within 1e-2
relative + 2e-3 absolute of the oracle.  The same weights registered
HBM-resident under another layer id give the same bits (the waves change which
tiles a launch takes, not how a tile is computed).
"""
import ctypes as C

import numpy as np
import pytest

import oracle as O
from hummingflight_amd import capi, synth
from moe_harness import FULL, SMALL, assert_close, ulp_diff

pytestmark = pytest.mark.gpu

TWIN = 200


class AliasedLayer(O.SyntheticLayer):
    """The oracle layer with expert e carrying expert e % distinct's weights."""

    def __init__(self, spec, distinct):
        super().__init__(spec)
        self.distinct = distinct

    def expert(self, e: int):
        return super().expert(e % self.distinct)


def forward(layer, x, T, dims):
    d, E, k = dims["hidden"], dims["n_experts"], dims["top_k"]
    out, lg = capi.DeviceBuffer(T * d * 4), capi.DeviceBuffer(T * E * 4)
    idx, w = capi.DeviceBuffer(T * k * 4), capi.DeviceBuffer(T * k * 4)
    off, perm = capi.DeviceBuffer((E + 1) * 4), capi.DeviceBuffer(T * k * 4)
    dbg = capi.RouteDebug(lg.ptr, idx.ptr, w.ptr, off.ptr, perm.ptr)
    capi.call("hfmoe_moe_forward_debug", layer, x.ptr, T, out.ptr, None, C.byref(dbg))
    capi.call("hfmoe_synchronize")
    res = dict(out=out.download(np.float32, T * d).reshape(T, d), logits=lg.download(np.float32, T * E).reshape(T, E),
               idx=idx.download(np.int32, T * k).reshape(T, k), w=w.download(np.float32, T * k).reshape(T, k),
               offsets=off.download(np.int32, E + 1), perm=perm.download(np.int32, T * k))
    for b in (out, lg, idx, w, off, perm):
        b.free()
    return res


def counters():
    c = capi.StreamCounters()
    capi.call("hfmoe_stream_read_counters", C.byref(c))
    return c.as_dict()


@pytest.mark.parametrize("dims,T,distinct,check_every", [
    (SMALL, 24, None, 1),        # ~60 distinct experts over a 16-slot pool: waves of 8 (128-row tiles)
    (SMALL, 1024, None, 64),     # prefill tiles (192 rows) with per-XCD work counters, cleared per wave
    (FULL, 64, 32, 8),           # full shape, 75.5 MB slots, ~130 distinct experts in waves of 8
], ids=["small_t24", "small_t1024_prefill_tiles", "full_t64"])
def test_streamed_batch(hf, dims, T, distinct, check_every):
    seed = 300 + T
    shape = synth.LayerShape(n_group=8, topk_group=4, **dims)
    capi.call("hfmoe_configure", shape.config(max_tokens=T))
    streamed = synth.DeviceLayer(shape, layer=0, seed=seed, experts_on_host=True, distinct_experts=distinct)
    resident = synth.DeviceLayer(shape, layer=0, seed=seed, distinct_experts=distinct, register_as=TWIN)
    spec = O.LayerSpec(n_group=8, topk_group=4, seed=seed, layer=0, **dims)
    ref = AliasedLayer(spec, distinct) if distinct else O.SyntheticLayer(spec)
    capi.call("hfmoe_stream_reset")
    x = synth.make_x_dev(T, dims["hidden"], seed=seed)
    print(f"streamed T={T} hidden={dims['hidden']}", flush=True)
    got = forward(0, x, T, dims)
    n = counters()
    U = len(set(got["idx"].ravel().tolist()))
    assert n["lookups"] == U and n["misses"] == U and n["slots"] == 2 * dims["top_k"]
    assert U > n["slots"], "the batch must need several waves"
    # Dispatch and selection as the oracle's.
    counts, offsets, perm = O.dispatch(got["idx"], dims["n_experts"])
    assert np.array_equal(got["offsets"], offsets) and np.array_equal(got["perm"], perm)
    twin = forward(TWIN, x, T, dims)
    assert np.array_equal(got["out"].view(np.uint32), twin["out"].view(np.uint32)), "streamed vs HBM-resident"
    xh = x.download(np.float32, T * dims["hidden"]).reshape(T, -1)
    for t in range(0, T, check_every):
        ridx, rw = ref.route(got["logits"][t])
        assert got["idx"][t].tolist() == ridx.tolist(), f"token {t}: selection"
        assert ulp_diff(got["w"][t], rw).max() == 0
        assert_close(got["out"][t], ref.combine(xh[t], ridx, rw), f"token {t}")
    # A second call: experts still resident are hits, the output repeats.
    again = forward(0, x, T, dims)
    assert np.array_equal(again["out"].view(np.uint32), got["out"].view(np.uint32))
    assert counters()["hits"] > 0
    x.free()
    streamed.free()
    resident.free()
