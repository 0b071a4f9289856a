"""The MoE forward and the dense MLP captured into a HIP graph and replayed.

A serving loop may capture a layer (or a chain of layers) once and replay it.
The forwards issue only kernel launches on the caller's stream -- no memsets,
no host synchronisation, no allocation -- so stream capture records them
whole.  Every replay is checked bit for bit against the same call made
eagerly, with other eager work on the stream between replays: the MoE layer
at T = 1 (decode kernels), T = 24 (128-row grouped GEMM) and T = 1024
(192-row tiles, multi-workgroup dispatch, per-XCD work counters that the
dispatch zeroes on every replay); the dense MLP at T = 1 (GEMVs), T = 64
(gate/up split over K, SwiGLU on the split sums, down in K splits) and
T = 300 (256-row tiles dealt per XCD); the LM head's logits and greedy
tokens at T = 1 (GEMV with the fused argmax and its merge launch), 5 and 150
(grouped GEMM, then the row argmax).
"""
import ctypes as C

import numpy as np
import pytest

import oracle as O
from hummingflight_amd import capi, synth
from moe_harness import SMALL, Run, assert_close

pytestmark = pytest.mark.gpu

CAPTURE_MODE_RELAXED = 2


def hip():
    lib = C.CDLL("libamdhip64.so")
    for name in ("hipStreamCreate", "hipStreamDestroy", "hipStreamSynchronize", "hipStreamBeginCapture",
                 "hipStreamEndCapture", "hipGraphInstantiate", "hipGraphLaunch", "hipGraphExecDestroy",
                 "hipGraphDestroy"):
        getattr(lib, name).restype = C.c_int
    return lib


def ok(rc, what):
    assert rc == 0, f"{what} failed with HIP error {rc}"


@pytest.mark.parametrize("T", [1, 24, 1024])
def test_forward_replays_from_hip_graph(hf, T):
    d = SMALL["hidden"]
    r = Run(SMALL, n_group=8, topk_group=4, seed=80 + T % 7, T=T)
    x = synth.make_x_dev(T, d, seed=80 + T % 7)
    x2 = synth.make_x_dev(T, d, seed=81 + T % 7)
    out_e = capi.DeviceBuffer(T * d * 4)
    out_g = capi.DeviceBuffer(T * d * 4)
    fwd = capi.load().hfmoe_moe_forward
    h = hip()
    s = C.c_void_p()
    ok(h.hipStreamCreate(C.byref(s)), "hipStreamCreate")
    graph, exe = C.c_void_p(), C.c_void_p()
    try:
        capi.check(fwd(0, x.ptr, T, out_e.ptr, s))
        ok(h.hipStreamSynchronize(s), "sync")
        ref = out_e.download(np.float32, T * d).copy()

        ok(h.hipStreamBeginCapture(s, CAPTURE_MODE_RELAXED), "hipStreamBeginCapture")
        rc = fwd(0, x.ptr, T, out_g.ptr, s)
        ok(h.hipStreamEndCapture(s, C.byref(graph)), "hipStreamEndCapture")
        capi.check(rc)
        ok(h.hipGraphInstantiate(C.byref(exe), graph, None, None, 0), "hipGraphInstantiate")

        for rep in range(4):
            capi.call("hfmoe_memset", out_g.ptr, 0, T * d * 4)
            ok(h.hipGraphLaunch(exe, s), "hipGraphLaunch")
            ok(h.hipStreamSynchronize(s), "sync")
            got = out_g.download(np.float32, T * d)
            assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), f"replay {rep} differs from eager"
            # Other work through the same workspace between replays.
            capi.check(fwd(0, x2.ptr, T, out_e.ptr, s))
            ok(h.hipStreamSynchronize(s), "sync")
        other = out_e.download(np.float32, T * d)
        assert not np.array_equal(other, ref)
        # The token's output is still the oracle's (selection and tolerance).
        res = r.forward(x, T)
        assert np.array_equal(res["out"].reshape(-1).view(np.uint32), ref.view(np.uint32))
        r.check_token(x.download(np.float32, d), res, 0)
    finally:
        if exe.value:
            h.hipGraphExecDestroy(exe)
        if graph.value:
            h.hipGraphDestroy(graph)
        h.hipStreamDestroy(s)
        for b in (x, x2, out_e, out_g):
            b.free()
        r.free()


def test_replays_follow_the_activation_type(hf):
    # One captured prefill-size forward (T = 1024: the wide gate/up tiles)
    # replayed on FP32 activations, then BF16-valued ones, then FP32 again,
    # written into the same input buffer between replays: the gate/up kernel
    # picks its M tiles on the device from the x lo-half flag (160-row tiles
    # with a lo half, 192-row without), so every replay must match the eager
    # call on the same values bit for bit.
    T, d = 1024, SMALL["hidden"]
    r = Run(SMALL, n_group=8, topk_group=4, seed=88, T=T)
    xb_dev = synth.make_x_dev(T, d, seed=88)
    xb = xb_dev.download(np.float32, T * d)
    xb_dev.free()
    xf = (xb * (1.0 + np.float32(2.0 ** -10) * np.random.default_rng(88).standard_normal(xb.shape))).astype(
        np.float32)
    assert not np.array_equal(xf, xb)
    xin = capi.DeviceBuffer.of(xf)
    out = capi.DeviceBuffer(T * d * 4)
    fwd = capi.load().hfmoe_moe_forward
    h = hip()
    s = C.c_void_p()
    ok(h.hipStreamCreate(C.byref(s)), "hipStreamCreate")
    graph, exe = C.c_void_p(), C.c_void_p()
    try:
        ref = {}
        for name, xv in (("fp32", xf), ("bf16", xb)):
            xin.upload(xv)
            capi.check(fwd(0, xin.ptr, T, out.ptr, s))
            ok(h.hipStreamSynchronize(s), "sync")
            ref[name] = out.download(np.float32, T * d).copy()
        assert not np.array_equal(ref["fp32"], ref["bf16"])

        ok(h.hipStreamBeginCapture(s, CAPTURE_MODE_RELAXED), "hipStreamBeginCapture")
        rc = fwd(0, xin.ptr, T, out.ptr, s)
        ok(h.hipStreamEndCapture(s, C.byref(graph)), "hipStreamEndCapture")
        capi.check(rc)
        ok(h.hipGraphInstantiate(C.byref(exe), graph, None, None, 0), "hipGraphInstantiate")

        for rep, (name, xv) in enumerate((("fp32", xf), ("bf16", xb), ("fp32", xf), ("bf16", xb))):
            xin.upload(xv)
            capi.call("hfmoe_memset", out.ptr, 0, T * d * 4)
            ok(h.hipGraphLaunch(exe, s), "hipGraphLaunch")
            ok(h.hipStreamSynchronize(s), "sync")
            got = out.download(np.float32, T * d)
            assert np.array_equal(got.view(np.uint32), ref[name].view(np.uint32)), \
                f"replay {rep} ({name} activations) differs from eager"
        # Both eager results are the oracle's for a token (selection and tolerance).
        for name, xv in (("fp32", xf), ("bf16", xb)):
            xin.upload(xv)
            res = r.forward(xin, T)
            assert np.array_equal(res["out"].reshape(-1).view(np.uint32), ref[name].view(np.uint32))
            r.check_token(xv.reshape(T, d)[0], res, 0)
    finally:
        if exe.value:
            h.hipGraphExecDestroy(exe)
        if graph.value:
            h.hipGraphDestroy(graph)
        h.hipStreamDestroy(s)
        for b in (xin, out):
            b.free()
        r.free()


@pytest.mark.parametrize("T", [1, 64, 300])
def test_dense_forward_replays_from_hip_graph(hf, T):
    H, I, seed = 1024, 3072, 90 + T % 7
    shape = synth.LayerShape(hidden=H, inter=512, n_experts=64, top_k=8, n_group=8, topk_group=4)
    capi.call("hfmoe_configure", shape.config(max_tokens=300))
    w = [capi.DeviceBuffer(2 * H * I) for _ in range(3)]
    for i, b in enumerate(w):
        synth.fill_bf16(b.ptr, H * I, seed, 100 + i, 0.0, 0.02)
    dw = capi.DenseWeights(w[0].ptr, w[1].ptr, w[2].ptr, None, I, 0)
    capi.call("hfmoe_register_dense_layer", 0, C.byref(dw))
    x = synth.make_x_dev(T, H, seed=seed)
    x2 = synth.make_x_dev(T, H, seed=seed + 1)
    out_e = capi.DeviceBuffer(T * H * 4)
    out_g = capi.DeviceBuffer(T * H * 4)
    fwd = capi.load().hfmoe_dense_mlp_forward
    h = hip()
    s = C.c_void_p()
    ok(h.hipStreamCreate(C.byref(s)), "hipStreamCreate")
    graph, exe = C.c_void_p(), C.c_void_p()
    try:
        capi.check(fwd(0, x.ptr, T, out_e.ptr, s))
        ok(h.hipStreamSynchronize(s), "sync")
        ref = out_e.download(np.float32, T * H).copy()

        ok(h.hipStreamBeginCapture(s, CAPTURE_MODE_RELAXED), "hipStreamBeginCapture")
        rc = fwd(0, x.ptr, T, out_g.ptr, s)
        ok(h.hipStreamEndCapture(s, C.byref(graph)), "hipStreamEndCapture")
        capi.check(rc)
        ok(h.hipGraphInstantiate(C.byref(exe), graph, None, None, 0), "hipGraphInstantiate")

        for rep in range(4):
            capi.call("hfmoe_memset", out_g.ptr, 0, T * H * 4)
            ok(h.hipGraphLaunch(exe, s), "hipGraphLaunch")
            ok(h.hipStreamSynchronize(s), "sync")
            got = out_g.download(np.float32, T * H)
            assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), f"replay {rep} differs from eager"
            # Other work through the same workspace between replays.
            capi.check(fwd(0, x2.ptr, T, out_e.ptr, s))
            ok(h.hipStreamSynchronize(s), "sync")
        assert not np.array_equal(out_e.download(np.float32, T * H), ref)
        # The last token against the oracle's denseMlp restatement.
        hw = [O.fill_bf16(H * I, seed, 100 + i, 0.0, 0.02) for i in range(3)]
        xt = x.download(np.float32, T * H).reshape(T, H)[T - 1]
        assert_close(ref.reshape(T, H)[T - 1], O.dense_mlp(hw[0], hw[1], hw[2], xt, H, I), f"T={T} last token")
    finally:
        if exe.value:
            h.hipGraphExecDestroy(exe)
        if graph.value:
            h.hipGraphDestroy(graph)
        h.hipStreamDestroy(s)
        for b in w + [x, x2, out_e, out_g]:
            b.free()


@pytest.mark.parametrize("T", [1, 5, 150])
def test_lm_head_replays_from_hip_graph(hf, T):
    H, V, seed = 1024, 5003, 95 + T % 7
    shape = synth.LayerShape(hidden=H, inter=512, n_experts=64, top_k=8, n_group=8, topk_group=4)
    capi.call("hfmoe_configure", shape.config(max_tokens=150))
    Wd = capi.DeviceBuffer(2 * V * H)
    synth.fill_bf16(Wd.ptr, V * H, seed, 300, 0.0, 0.02)
    nd = capi.DeviceBuffer(2 * H)
    synth.fill_bf16(nd.ptr, H, seed, 301, 1.0, 0.05)
    capi.call("hfmoe_register_lm_head", Wd.ptr, nd.ptr, V)
    x = synth.make_x_dev(T, H, seed=seed)
    x2 = synth.make_x_dev(T, H, seed=seed + 1)
    lg_e, lg_g = capi.DeviceBuffer(T * V * 4), capi.DeviceBuffer(T * V * 4)
    tk_e, tk_g = capi.DeviceBuffer(T * 4), capi.DeviceBuffer(T * 4)
    head = capi.load().hfmoe_lm_head
    h = hip()
    s = C.c_void_p()
    ok(h.hipStreamCreate(C.byref(s)), "hipStreamCreate")
    graph, exe = C.c_void_p(), C.c_void_p()
    try:
        capi.check(head(x.ptr, T, lg_e.ptr, tk_e.ptr, s))
        ok(h.hipStreamSynchronize(s), "sync")
        ref_lg = lg_e.download(np.float32, T * V).copy()
        ref_tk = tk_e.download(np.int32, T).copy()

        ok(h.hipStreamBeginCapture(s, CAPTURE_MODE_RELAXED), "hipStreamBeginCapture")
        rc = head(x.ptr, T, lg_g.ptr, tk_g.ptr, s)
        ok(h.hipStreamEndCapture(s, C.byref(graph)), "hipStreamEndCapture")
        capi.check(rc)
        ok(h.hipGraphInstantiate(C.byref(exe), graph, None, None, 0), "hipGraphInstantiate")

        for rep in range(4):
            capi.call("hfmoe_memset", lg_g.ptr, 0, T * V * 4)
            capi.call("hfmoe_memset", tk_g.ptr, 255, T * 4)
            ok(h.hipGraphLaunch(exe, s), "hipGraphLaunch")
            ok(h.hipStreamSynchronize(s), "sync")
            got = lg_g.download(np.float32, T * V)
            assert np.array_equal(got.view(np.uint32), ref_lg.view(np.uint32)), f"replay {rep}: logits differ"
            assert np.array_equal(tk_g.download(np.int32, T), ref_tk), f"replay {rep}: tokens differ"
            # Other work through the same workspace between replays.
            capi.check(head(x2.ptr, T, lg_e.ptr, tk_e.ptr, s))
            ok(h.hipStreamSynchronize(s), "sync")
        assert not np.array_equal(lg_e.download(np.float32, T * V), ref_lg)
        # The eager call's last token against the oracle's lmHeadAndSample restatement.
        W = O.fill_bf16(V * H, seed, 300, 0.0, 0.02)
        norm = O.fill_bf16(H, seed, 301, 1.0, 0.05)
        xt = x.download(np.float32, T * H).reshape(T, H)[T - 1]
        ref, _ = O.lm_head(W, norm, xt, V, 1e-5)
        assert_close(ref_lg.reshape(T, V)[T - 1], ref, f"T={T} last token logits")
        assert int(ref_tk[T - 1]) == int(np.argmax(ref_lg.reshape(T, V)[T - 1]))
    finally:
        if exe.value:
            h.hipGraphExecDestroy(exe)
        if graph.value:
            h.hipGraphDestroy(graph)
        h.hipStreamDestroy(s)
        for b in (Wd, nd, x, x2, lg_e, lg_g, tk_e, tk_g):
            b.free()
