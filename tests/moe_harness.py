"""Shared GPU-test harness: a configured layer on the device and its oracle twin.

Bar: expert indices and routing weights bit-exact given the same router
logits (the device sigmoid is glibc's expf algorithm, tests/test_expf.py);
outputs within 1e-2 relative + 2e-3 absolute of the oracle (BF16 weights,
FP32 accumulation).
"""
import ctypes as C

import numpy as np

import oracle as O
from hummingflight_amd import capi, synth

RTOL, ATOL = 1e-2, 2e-3


def assert_close(got, ref, what=""):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    err = np.abs(got - ref)
    tol = ATOL + RTOL * np.abs(ref)
    bad = np.flatnonzero(err > tol)
    assert bad.size == 0, (f"{what}: {bad.size} elements outside tolerance, first at {bad[0]}: "
                           f"got {got.flat[bad[0]]} ref {ref.flat[bad[0]]}")


def ulp_diff(a, b):
    ai = np.asarray(a, np.float32).view(np.int32).astype(np.int64)
    bi = np.asarray(b, np.float32).view(np.int32).astype(np.int64)
    return np.abs(ai - bi)


SMALL = dict(hidden=2048, inter=1024, n_experts=64, top_k=8)
FULL = dict(hidden=6144, inter=2048, n_experts=256, top_k=8)


class Run:
    """One configured layer on the device plus its oracle twin."""

    def __init__(self, dims, n_group=1, topk_group=1, seed=1, T=1, layer=0, n_shared=1,
                 on_host=False, with_norm=False, bias=None, max_tokens=None, w_std=0.02, **routing):
        # routing: norm_topk_prob / routed_scaling_factor, passed to both sides
        self.shape = synth.LayerShape(n_group=n_group, topk_group=topk_group, n_shared=n_shared,
                                      **dims, **routing)
        capi.call("hfmoe_configure", self.shape.config(max_tokens=max_tokens or T))
        self.dev = synth.DeviceLayer(self.shape, layer=layer, seed=seed, experts_on_host=on_host,
                                     with_norm=with_norm, bias=bias, w_std=w_std)
        self.spec = O.LayerSpec(n_group=n_group, topk_group=topk_group, n_shared=n_shared, seed=seed,
                                layer=layer, bias_override=bias, w_std=w_std, **dims, **routing)
        self.ref = O.SyntheticLayer(self.spec)
        self.T = T
        self.layer = layer

    def forward(self, x_dev, T=None):
        T = T or self.T
        s = self.shape
        out = capi.DeviceBuffer(T * s.hidden * 4)
        lg = capi.DeviceBuffer(T * s.n_experts * 4)
        idx = capi.DeviceBuffer(T * s.top_k * 4)
        w = capi.DeviceBuffer(T * s.top_k * 4)
        off = capi.DeviceBuffer((s.n_experts + 1) * 4)
        perm = capi.DeviceBuffer(T * s.top_k * 4)
        dbg = capi.RouteDebug(lg.ptr, idx.ptr, w.ptr, off.ptr, perm.ptr)
        capi.call("hfmoe_moe_forward_debug", self.layer, x_dev.ptr, T, out.ptr, None, C.byref(dbg))
        capi.call("hfmoe_synchronize")
        res = dict(out=out.download(np.float32, T * s.hidden).reshape(T, s.hidden),
                   logits=lg.download(np.float32, T * s.n_experts).reshape(T, s.n_experts),
                   idx=idx.download(np.int32, T * s.top_k).reshape(T, s.top_k),
                   w=w.download(np.float32, T * s.top_k).reshape(T, s.top_k),
                   offsets=off.download(np.int32, s.n_experts + 1),
                   perm=perm.download(np.int32, T * s.top_k))
        for b in (out, lg, idx, w, off, perm):
            b.free()
        return res

    def check_token(self, x, res, t):
        """Selection given the GPU's logits, then the output given that selection."""
        ridx, rw = self.ref.route(res["logits"][t])
        assert res["idx"][t].tolist() == ridx.tolist(), f"token {t}: selection differs"
        assert ulp_diff(res["w"][t], rw).max() == 0, f"token {t}: weights differ"
        ref = self.ref.combine(x, ridx, rw)
        assert_close(res["out"][t], ref, f"token {t} output")
        return ridx, ref

    def free(self):
        self.dev.free()


class DevView:
    """A pointer into an existing device buffer (no ownership)."""

    def __init__(self, buf, byte_offset: int):
        self.ptr = buf.ptr + byte_offset

