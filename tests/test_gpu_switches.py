"""The measurement switches documented as leaving results unchanged do so, bit
for bit: workgroup counts of the decode GEMVs (HFMOE_GU_BLOCKS,
HFMOE_DN_BLOCKS), routing as a kernel of its own (HFMOE_FUSE_SELECT=0), the
grouped GEMMs' workgroup count (HFMOE_GEMM_BLOCKS), the prefill down
projection on the split tiles (HFMOE_DOWN_WIDE=0) and the LM-head GEMV's
workgroup count (HFMOE_LM_BLOCKS).  Each output row is summed in one fixed
order whichever workgroup computes it, and every item of the grouped GEMMs
the same way wherever it runs.
"""
import numpy as np
import pytest

from hummingflight_amd import capi, synth
from moe_harness import FULL, SMALL, Run

pytestmark = pytest.mark.gpu


def same(a, b, what):
    for key in ("out", "idx", "w", "logits"):
        assert np.array_equal(a[key].view(np.uint32), b[key].view(np.uint32)), f"{what}: {key} differs"


def test_decode_switches_leave_results_unchanged(hf, monkeypatch):
    # Full shape, one token: 768 / 256 gate/up workgroups, 256 / 64 down
    # workgroups (64 rows each at most: 96 workgroups), routing fused or not.
    r = Run(FULL, n_group=8, topk_group=4, seed=21, T=1)
    x = synth.make_x_dev(1, FULL["hidden"], seed=21)
    base = r.forward(x, 1)
    for env, val in (("HFMOE_GU_BLOCKS", "256"), ("HFMOE_DN_BLOCKS", "64"), ("HFMOE_FUSE_SELECT", "0")):
        monkeypatch.setenv(env, val)
        same(base, r.forward(x, 1), f"{env}={val}")
        monkeypatch.delenv(env)
    r.check_token(x.download(np.float32, FULL["hidden"]), base, 0)
    x.free()
    r.free()


@pytest.mark.parametrize("fp32_x", [False, True], ids=["bf16_valued_x", "fp32_x"])
def test_prefill_switches_leave_results_unchanged(hf, monkeypatch, fp32_x):
    # 1024 tokens over 64 experts (~128 rows each): the wide gate/up and down
    # tiles with dynamic item counters, on 128 or 384 workgroups instead of
    # one per CU, and the down projection on the 192 x 384 split tiles.
    T, d = 1024, SMALL["hidden"]
    r = Run(SMALL, n_group=8, topk_group=4, seed=22, T=T)
    x = synth.make_x_dev(T, d, seed=22)
    if fp32_x:
        xv = x.download(np.float32, T * d)
        x.free()
        x = capi.DeviceBuffer.of((xv * (1.0 + np.float32(2.0 ** -10) *
                                        np.random.default_rng(22).standard_normal(xv.shape))).astype(np.float32))
    base = r.forward(x, T)
    for env, val in (("HFMOE_GEMM_BLOCKS", "128"), ("HFMOE_GEMM_BLOCKS", "384"), ("HFMOE_DOWN_WIDE", "0")):
        monkeypatch.setenv(env, val)
        same(base, r.forward(x, T), f"{env}={val}")
        monkeypatch.delenv(env)
    xh = x.download(np.float32, T * d).reshape(T, d)
    for t in (0, T // 2, T - 1):
        r.check_token(xh[t], base, t)
    x.free()
    r.free()


@pytest.mark.parametrize("T", [1, 5])
def test_lm_head_blocks_leave_results_unchanged(hf, monkeypatch, T):
    # The T = 1 GEMV with its fused argmax on another number of workgroups
    # than two per CU (the 128-row GEMM for T = 5 does not read the switch:
    # the same bits either way).
    H, V = 1024, 5003
    shape = synth.LayerShape(hidden=H, inter=512, n_experts=64, top_k=8, n_group=8, topk_group=4)
    capi.call("hfmoe_configure", shape.config(max_tokens=T))
    W = capi.DeviceBuffer(2 * V * H)
    synth.fill_bf16(W.ptr, V * H, 23, 300, 0.0, 0.02)
    capi.call("hfmoe_register_lm_head", W.ptr, None, V)
    x = synth.make_x_dev(T, H, seed=23)
    lg = capi.DeviceBuffer(T * V * 4)
    tok = capi.DeviceBuffer(T * 4)

    def run():
        capi.call("hfmoe_lm_head", x.ptr, T, lg.ptr, tok.ptr, None)
        capi.call("hfmoe_synchronize")
        return lg.download(np.float32, T * V).copy(), tok.download(np.int32, T).copy()

    l0, t0 = run()
    # 64 workgroups; then 4096, more than the per-workgroup winners
    # allocated at registration (two per CU): held to those.
    for val in ("64", "4096"):
        monkeypatch.setenv("HFMOE_LM_BLOCKS", val)
        l1, t1 = run()
        monkeypatch.delenv("HFMOE_LM_BLOCKS")
        assert np.array_equal(l0.view(np.uint32), l1.view(np.uint32)) and np.array_equal(t0, t1), val
    assert np.array_equal(t0, l0.reshape(T, V).argmax(axis=1))
    for b in (W, x, lg, tok):
        b.free()
