"""hfmoe_moe_forward_noalloc: the decode forward over the library's static
scratch array, against hfmoe_moe_forward (same kernels, so bit for bit) and
the oracle, on two calls in a row -- the full-shape layer, then a smaller one,
which finds the first call's contents still in the shared array.
"""
import numpy as np
import pytest

from hummingflight_amd import capi, synth
from moe_harness import FULL, SMALL, Run, assert_close

pytestmark = pytest.mark.gpu


def one_call(dims, seed):
    r = Run(dims, n_group=8, topk_group=4, seed=seed)
    d = dims["hidden"]
    x = synth.make_x_dev(1, d, seed=seed)
    out = capi.DeviceBuffer(d * 4)
    capi.call("hfmoe_moe_forward_noalloc", 0, x.ptr, 1, out.ptr, None)
    capi.call("hfmoe_synchronize")
    got = out.download(np.float32, d)
    res = r.forward(x)  # hfmoe_moe_forward_debug, the workspace path
    assert np.array_equal(got.view(np.uint32), res["out"][0].view(np.uint32)), f"{dims}: differs from hfmoe_moe_forward"
    _, ref = r.check_token(x.download(np.float32, d), res, 0)
    assert_close(got, ref, f"{dims}: oracle")
    L = capi.load()
    assert L.hfmoe_moe_forward_noalloc(0, x.ptr, 2, out.ptr, None) == capi.ERR_UNSUPPORTED
    assert L.hfmoe_moe_forward_noalloc(9, x.ptr, 1, out.ptr, None) == capi.ERR_NOT_REGISTERED
    assert L.hfmoe_moe_forward_noalloc(0, x.ptr, 0, out.ptr, None) == capi.OK
    x.free()
    out.free()
    r.free()


def test_noalloc_forward_two_calls_second_smaller(hf):
    one_call(FULL, seed=121)
    one_call(SMALL, seed=122)


def test_noalloc_forward_refuses_streamed_layers(hf):
    r = Run(SMALL, n_group=8, topk_group=4, seed=123, on_host=True)
    x = synth.make_x_dev(1, SMALL["hidden"], seed=123)
    out = capi.DeviceBuffer(SMALL["hidden"] * 4)
    assert capi.load().hfmoe_moe_forward_noalloc(0, x.ptr, 1, out.ptr, None) == capi.ERR_UNSUPPORTED
    x.free()
    out.free()
    r.free()


CHILD = r"""
import sys
sys.path[:0] = [{root!r}, {tests!r}]
import numpy as np
from hummingflight_amd import capi, synth
from moe_harness import SMALL, Run
L = capi.load()
assert L.hfmoe_init(0) == capi.OK, L.hfmoe_last_error()
r = Run(SMALL, n_group=8, topk_group=4, seed=124)
x = synth.make_x_dev(1, SMALL["hidden"], seed=124)
out = capi.DeviceBuffer(SMALL["hidden"] * 4)
rc = L.hfmoe_moe_forward_noalloc(0, x.ptr, 1, out.ptr, None)
assert rc == capi.ERR_NOT_INITIALIZED, rc
assert b"HFMOE_NOALLOC_DISABLE" in L.hfmoe_last_error(), L.hfmoe_last_error()
res = r.forward(x)
xh = x.download(np.float32, SMALL["hidden"])
r.check_token(xh, res, 0)
print("child ok", flush=True)
L.hfmoe_shutdown()
"""


def test_init_succeeds_without_the_noalloc_scratch(hf):
    # A library whose allocation-free scratch could not be set up still
    # initialises; only hfmoe_moe_forward_noalloc reports NOT_INITIALIZED.  The
    # setup is switched off by its environment switch in a child process (init
    # runs once per process), which then runs the regular forward.
    import os
    import subprocess
    import sys
    tests = os.path.dirname(os.path.abspath(__file__))
    code = CHILD.format(root=os.path.dirname(tests), tests=tests)
    env = dict(os.environ, HFMOE_NOALLOC_DISABLE="1")
    r = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True, timeout=300)
    assert r.returncode == 0 and "child ok" in r.stdout, r.stdout + r.stderr
