"""A MoE layer loaded from safetensors shards runs like the oracle's layer.

The oracle's seeded synthetic layer is written under the GLM tensor names into
two shards with an index (router, bias, shared expert and norm in one, the
routed experts in the other), loaded through hfmoe_checkpoint_load_moe_layer
with experts in HBM and, separately, in pinned host RAM, and checked token by
token against the oracle (selection given the GPU's logits, outputs within the
1e-2 / 2e-3 bar), including the multi-token path and the RMSNorm + residual
block that uses the loaded norm weight.
"""
import ctypes as C
import json

import numpy as np
import pytest

import oracle as O
from hummingflight_amd import capi, synth
from moe_harness import assert_close, ulp_diff
from safetensors_io import moe_layer_tensors, write_shard

pytestmark = pytest.mark.gpu

DIMS = dict(hidden=1024, inter=512, n_experts=32, top_k=4)
LAYER, SEED = 2, 91


@pytest.fixture(scope="module")
def ckpt_dir(tmp_path_factory):
    d = tmp_path_factory.mktemp("ckpt")
    ref = O.SyntheticLayer(O.LayerSpec(n_group=4, topk_group=2, seed=SEED, layer=LAYER, **DIMS))
    norm = O.fill_bf16(DIMS["hidden"], SEED, O.tensor_id(LAYER, O.ROLE_NORM), 1.0, 0.05)
    t = moe_layer_tensors(ref, LAYER, with_norm=norm)
    experts = {k: v for k, v in t.items() if ".experts." in k}
    rest = {k: v for k, v in t.items() if k not in experts}
    write_shard(d / "model-00001-of-00002.safetensors", rest)
    write_shard(d / "model-00002-of-00002.safetensors", experts)
    wm = {k: "model-00001-of-00002.safetensors" for k in rest}
    wm.update({k: "model-00002-of-00002.safetensors" for k in experts})
    (d / "model.safetensors.index.json").write_text(json.dumps({"metadata": {}, "weight_map": wm}))
    return d, ref, norm


def load(path, location):
    shape = synth.LayerShape(n_group=4, topk_group=2, **DIMS)
    capi.call("hfmoe_configure", shape.config(max_tokens=8))
    ck = C.c_void_p()
    capi.call("hfmoe_checkpoint_open", str(path).encode(), C.byref(ck))
    capi.call("hfmoe_checkpoint_load_moe_layer", ck, LAYER, location)
    return ck


def forward(T, x):
    d, E, k = DIMS["hidden"], DIMS["n_experts"], DIMS["top_k"]
    xd = capi.DeviceBuffer.of(x)
    out, lg = capi.DeviceBuffer(T * d * 4), capi.DeviceBuffer(T * E * 4)
    idx, w = capi.DeviceBuffer(T * k * 4), capi.DeviceBuffer(T * k * 4)
    dbg = capi.RouteDebug(lg.ptr, idx.ptr, w.ptr, None, None)
    capi.call("hfmoe_moe_forward_debug", LAYER, xd.ptr, T, out.ptr, None, C.byref(dbg))
    capi.call("hfmoe_synchronize")
    res = (out.download(np.float32, T * d).reshape(T, d), lg.download(np.float32, T * E).reshape(T, E),
           idx.download(np.int32, T * k).reshape(T, k), w.download(np.float32, T * k).reshape(T, k))
    for b in (xd, out, lg, idx, w):
        b.free()
    return res


def check(ref, x, res):
    out, lg, idx, w = res
    for t in range(x.shape[0]):
        ridx, rw = ref.route(lg[t])
        assert idx[t].tolist() == ridx.tolist(), f"token {t}: selection"
        assert ulp_diff(w[t], rw).max() == 0
        assert_close(out[t], ref.combine(x[t], ridx, rw), f"token {t}")


@pytest.mark.parametrize("location", [capi.EXPERTS_DEVICE, capi.EXPERTS_HOST_PINNED], ids=["hbm", "pinned_host"])
def test_checkpoint_layer_matches_oracle(hf, ckpt_dir, location):
    path, ref, norm = ckpt_dir
    ck = load(path, location)
    rng = np.random.default_rng(SEED + location)
    x1 = rng.standard_normal((1, DIMS["hidden"])).astype(np.float32)
    check(ref, x1, forward(1, x1))
    if location == capi.EXPERTS_DEVICE:
        x5 = rng.standard_normal((5, DIMS["hidden"])).astype(np.float32)
        check(ref, x5, forward(5, x5))
    # RMSNorm (loaded norm weight) + MoE + residual.
    h = capi.DeviceBuffer.of(x1[0])
    capi.call("hfmoe_mlp_block", LAYER, h.ptr, 1, None)
    capi.call("hfmoe_synchronize")
    xn = O.rmsnorm(norm, x1[0], 1e-5)
    want = x1[0] + ref.forward(xn)[0]
    assert_close(h.download(np.float32, DIMS["hidden"]), want, "mlp block")
    h.free()
    capi.load().hfmoe_checkpoint_close(ck)
    # Closing the checkpoint unregisters the layer it loaded.
    assert capi.load().hfmoe_moe_forward(LAYER, None, 1, None, None) == capi.ERR_NOT_REGISTERED


def test_checkpoint_missing_or_misshaped_tensor_is_named(hf, ckpt_dir, tmp_path):
    path, ref, norm = ckpt_dir
    t = moe_layer_tensors(ref, LAYER)
    del t[f"model.layers.{LAYER}.mlp.experts.7.up_proj.weight"]
    write_shard(tmp_path / "m.safetensors", t)
    shape = synth.LayerShape(n_group=4, topk_group=2, **DIMS)
    capi.call("hfmoe_configure", shape.config(max_tokens=1))
    L = capi.load()
    ck = C.c_void_p()
    capi.call("hfmoe_checkpoint_open", str(tmp_path / "m.safetensors").encode(), C.byref(ck))
    assert L.hfmoe_checkpoint_load_moe_layer(ck, LAYER, capi.EXPERTS_DEVICE) == capi.ERR_INVALID_ARGUMENT
    assert b"experts.7.up_proj.weight is missing" in L.hfmoe_last_error()
    assert L.hfmoe_checkpoint_load_moe_layer(ck, LAYER + 1, capi.EXPERTS_DEVICE) == capi.ERR_INVALID_ARGUMENT
    L.hfmoe_checkpoint_close(ck)
    # A checkpoint whose hidden size differs from the configured one.
    big = synth.LayerShape(n_group=4, topk_group=2, hidden=2048, inter=512, n_experts=32, top_k=4)
    capi.call("hfmoe_configure", big.config(max_tokens=1))
    capi.call("hfmoe_checkpoint_open", str(path).encode(), C.byref(ck))
    assert L.hfmoe_checkpoint_load_moe_layer(ck, LAYER, capi.EXPERTS_DEVICE) == capi.ERR_INVALID_ARGUMENT
    assert b"expected BF16 [32,2048]" in L.hfmoe_last_error()
    L.hfmoe_checkpoint_close(ck)


def test_close_leaves_a_later_registration_alone(hf, ckpt_dir):
    # Load layer 2 from the checkpoint, then register other weights under the
    # same id: closing the checkpoint must not unregister (or free) those.
    path, ref, norm = ckpt_dir
    ck = load(path, capi.EXPERTS_DEVICE)
    shape = synth.LayerShape(n_group=4, topk_group=2, **DIMS)
    other = synth.DeviceLayer(shape, layer=LAYER, seed=SEED + 1)
    capi.load().hfmoe_checkpoint_close(ck)
    x = np.random.default_rng(7).standard_normal((1, DIMS["hidden"])).astype(np.float32)
    ref2 = O.SyntheticLayer(O.LayerSpec(n_group=4, topk_group=2, seed=SEED + 1, layer=LAYER, **DIMS))
    check(ref2, x, forward(1, x))
    other.free()
