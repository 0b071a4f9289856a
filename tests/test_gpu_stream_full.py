"""Streamed experts at full shape: the chains of the streamed-decode benchmark.

d = 6144, I = 2048, 256 experts in 8 groups keeping 4, top-8, one shared
expert; routed experts in pinned host RAM, 75.5 MB slots filled by three
hipMemcpyAsync each, and the default pool of 2k slots, so every token copies
most of its experts again.  To bound pinned host memory, expert e of a layer
carries the weights of expert e % 32 (every expert is still its own cache key
and crosses PCIe).  Three chained layers (h += MoE(h)) over four tokens, so the
next-layer copy-ahead runs at both layer boundaries.

Checks per token and layer: selection bit-exact given the GPU's logits, output
within 1e-2 relative + 2e-3 absolute of the oracle, and output bit-identical to
the same weights registered HBM-resident under another layer id.
"""
import ctypes as C

import numpy as np
import pytest

import oracle as O
from hummingflight_amd import capi, synth
from moe_harness import FULL, DeviceBackedLayer, assert_close, ulp_diff

pytestmark = pytest.mark.gpu

LAYERS, TOKENS, DISTINCT, SEED, TWIN = 3, 4, 32, 83, 100


class AliasedLayer(O.SyntheticLayer):
    """The oracle layer with expert e carrying expert e % DISTINCT's weights."""

    def expert(self, e: int):
        return super().expert(e % DISTINCT)


def test_streamed_chain_full_shape(hf):
    d, k, E = FULL["hidden"], FULL["top_k"], FULL["n_experts"]
    shape = synth.LayerShape(n_group=8, topk_group=4, **FULL)
    capi.call("hfmoe_configure", shape.config(max_tokens=1))
    capi.call("hfmoe_stream_reset")
    streamed = [synth.DeviceLayer(shape, layer=l, seed=SEED, experts_on_host=True, distinct_experts=DISTINCT)
                for l in range(LAYERS)]
    resident = [synth.DeviceLayer(shape, layer=l, seed=SEED, distinct_experts=DISTINCT, register_as=TWIN + l)
                for l in range(LAYERS)]
    refs = [AliasedLayer(O.LayerSpec(n_group=8, topk_group=4, seed=SEED, layer=l, **FULL)) for l in range(LAYERS)]
    out, twin = capi.DeviceBuffer(d * 4), capi.DeviceBuffer(d * 4)
    lg, idx, w = capi.DeviceBuffer(E * 4), capi.DeviceBuffer(k * 4), capi.DeviceBuffer(k * 4)
    dbg = capi.RouteDebug(lg.ptr, idx.ptr, w.ptr, None, None)
    rng = np.random.default_rng(SEED)
    for tok in range(TOKENS):
        h = rng.standard_normal(d).astype(np.float32)
        for l in range(LAYERS):
            print(f"token {tok} layer {l}", flush=True)
            xd = capi.DeviceBuffer.of(h)
            capi.call("hfmoe_moe_forward_debug", l, xd.ptr, 1, out.ptr, None, C.byref(dbg))
            capi.call("hfmoe_moe_forward", TWIN + l, xd.ptr, 1, twin.ptr, None)
            capi.call("hfmoe_synchronize")
            got = out.download(np.float32, d)
            ridx, rw = refs[l].route(lg.download(np.float32, E))
            assert idx.download(np.int32, k).tolist() == ridx.tolist(), f"token {tok} layer {l}: selection"
            assert ulp_diff(w.download(np.float32, k), rw).max() == 0
            assert_close(got, refs[l].combine(h, ridx, rw), f"token {tok} layer {l}")
            assert np.array_equal(got.view(np.uint32), twin.download(np.float32, d).view(np.uint32)), \
                f"token {tok} layer {l}: streamed and HBM-resident outputs differ"
            h = h + got
            xd.free()
    c = capi.StreamCounters()
    capi.call("hfmoe_stream_read_counters", C.byref(c))
    n = c.as_dict()
    assert n["slots"] == 2 * k and n["lookups"] == TOKENS * LAYERS * k and n["misses"] > 0
    for b in (out, twin, lg, idx, w):
        b.free()
    for L in streamed + resident:
        L.free()


def test_streamed_chain8_rmsnorm_residual_blocks(hf):
    """The benchmark's streamed chain as it is timed: eight full-shape layers,
    each RMSNorm -> MoE -> residual add through hfmoe_mlp_block
    (glm_forward.cpp:785-796), routed experts streamed from pinned host RAM,
    four tokens.  Per token and layer the streamed block's output must be
    bit-identical to the same weights registered HBM-resident (under other
    layer ids, through the same entry point), and its MoE part (output minus
    input) within 1e-2 / 2e-3 of the oracle: the oracle's RMSNorm of the
    layer's input, selection given the GPU's router logits of that input, the
    oracle's moeLayer restatement."""
    layers, tokens, seed = 8, 4, 84
    d, k, E = FULL["hidden"], FULL["top_k"], FULL["n_experts"]
    shape = synth.LayerShape(n_group=8, topk_group=4, **FULL)
    capi.call("hfmoe_configure", shape.config(max_tokens=1))
    capi.call("hfmoe_stream_reset")
    streamed = [synth.DeviceLayer(shape, layer=l, seed=seed, experts_on_host=True, distinct_experts=DISTINCT,
                                  with_norm=True) for l in range(layers)]
    resident = [synth.DeviceLayer(shape, layer=l, seed=seed, distinct_experts=DISTINCT, with_norm=True,
                                  register_as=TWIN + l) for l in range(layers)]
    hosts = [DeviceBackedLayer(O.LayerSpec(n_group=8, topk_group=4, seed=seed, layer=l, **FULL), streamed[l])
             for l in range(layers)]
    norms = [O.fill_bf16(d, seed, O.tensor_id(l, O.ROLE_NORM), 1.0, 0.05) for l in range(layers)]
    blk = capi.load().hfmoe_mlp_block
    hs, hr, xn_dev, moe = (capi.DeviceBuffer(d * 4) for _ in range(4))
    lg, idx, w = capi.DeviceBuffer(E * 4), capi.DeviceBuffer(k * 4), capi.DeviceBuffer(k * 4)
    dbg = capi.RouteDebug(lg.ptr, idx.ptr, w.ptr, None, None)
    rng = np.random.default_rng(seed)
    c0 = capi.StreamCounters()
    capi.call("hfmoe_stream_read_counters", C.byref(c0))
    for tok in range(tokens):
        h = rng.standard_normal(d).astype(np.float32)
        hs.upload(h)
        hr.upload(h)
        for l in range(layers):
            print(f"token {tok} layer {l}", flush=True)
            capi.check(blk(l, hs.ptr, 1, None))
            capi.check(blk(TWIN + l, hr.ptr, 1, None))
            capi.call("hfmoe_synchronize")
            got = hs.download(np.float32, d)
            assert np.array_equal(got.view(np.uint32), hr.download(np.float32, d).view(np.uint32)), \
                f"token {tok} layer {l}: streamed and HBM-resident blocks differ"
            xn = O.rmsnorm(norms[l], h, shape.rms_norm_eps)
            xn_dev.upload(xn)
            capi.call("hfmoe_moe_forward_debug", TWIN + l, xn_dev.ptr, 1, moe.ptr, None, C.byref(dbg))
            capi.call("hfmoe_synchronize")
            ridx, rw = hosts[l].route(lg.download(np.float32, E))
            assert idx.download(np.int32, k).tolist() == ridx.tolist(), f"token {tok} layer {l}: selection"
            assert ulp_diff(w.download(np.float32, k), rw).max() == 0
            ref = hosts[l].combine(xn, ridx, rw)
            assert_close(got.astype(np.float64) - h.astype(np.float64), ref, f"token {tok} layer {l}")
            h = got
    c1 = capi.StreamCounters()
    capi.call("hfmoe_stream_read_counters", C.byref(c1))
    assert c1.lookups - c0.lookups == tokens * layers * k and c1.copies > c0.copies
    for b in (hs, hr, xn_dev, moe, lg, idx, w):
        b.free()
    for L in streamed + resident:
        L.free()
