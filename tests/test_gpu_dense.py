"""Dense MLP layers (GLMForward::denseMlp) against the oracle.

The oracle's dense_mlp is pinned bit-exact to the reference's own denseMlp
(tests/test_oracle.py).  Here the library's decode path (T = 1: the expert
GEMVs over inter / slice slices) and multi-token path (one-group grouped GEMM,
128- and 256-row tiles, K splits) must agree with it within 1e-2 relative + 2e-3
absolute, at a small shape and at GLM-5.2's (hidden 6144, intermediate 12288);
the RMSNorm + residual block and a dense layer loaded from a checkpoint too.
"""
import ctypes as C
import json

import numpy as np
import pytest

import oracle as O
from hummingflight_amd import capi, synth
from moe_harness import assert_close
from safetensors_io import write_shard

pytestmark = pytest.mark.gpu


class Dense:
    """A seeded dense layer on the device and its host copy."""

    def __init__(self, hidden, inter, seed, layer=0, with_norm=True, std=0.02):
        self.hidden, self.inter, self.layer = hidden, inter, layer
        n = hidden * inter
        self.host = [O.fill_bf16(n, seed, 100 + i, 0.0, std) for i in range(3)]
        self.norm = O.fill_bf16(hidden, seed, 103, 1.0, 0.05) if with_norm else None
        self.dev = [capi.DeviceBuffer(2 * n) for _ in range(3)]
        for i, b in enumerate(self.dev):
            synth.fill_bf16(b.ptr, n, seed, 100 + i, 0.0, std)
        self.norm_dev = None
        if with_norm:
            self.norm_dev = capi.DeviceBuffer(2 * hidden)
            synth.fill_bf16(self.norm_dev.ptr, hidden, seed, 103, 1.0, 0.05)
        w = capi.DenseWeights(self.dev[0].ptr, self.dev[1].ptr, self.dev[2].ptr,
                              self.norm_dev.ptr if self.norm_dev else None, inter, 0)
        capi.call("hfmoe_register_dense_layer", layer, C.byref(w))

    def ref(self, x):
        return O.dense_mlp(self.host[0], self.host[1], self.host[2], x, self.hidden, self.inter)

    def forward(self, x):
        T = x.shape[0]
        xd = capi.DeviceBuffer.of(x)
        out = capi.DeviceBuffer(x.nbytes)
        capi.call("hfmoe_dense_mlp_forward", self.layer, xd.ptr, T, out.ptr, None)
        capi.call("hfmoe_synchronize")
        y = out.download(np.float32, x.size).reshape(x.shape)
        xd.free()
        out.free()
        return y

    def free(self):
        for b in self.dev + ([self.norm_dev] if self.norm_dev else []):
            b.free()


def configure(hidden, inter, n_experts, max_tokens):
    shape = synth.LayerShape(hidden=hidden, inter=inter, n_experts=n_experts, top_k=8, n_group=8, topk_group=4)
    capi.call("hfmoe_configure", shape.config(max_tokens=max_tokens))


def test_dense_small_decode_and_batches(hf):
    H, I_moe, I = 1024, 512, 3072
    configure(H, I_moe, 64, 300)
    L = Dense(H, I, seed=31)
    rng = np.random.default_rng(31)
    x1 = rng.standard_normal((1, H)).astype(np.float32)
    y1 = L.forward(x1)
    assert_close(y1[0], L.ref(x1[0]), "T=1")
    for T in (5, 300):  # 128-row and 192-row tiles (two M tiles)
        x = rng.standard_normal((T, H)).astype(np.float32)
        y = L.forward(x)
        for t in sorted({0, T // 2, T - 1}):
            assert_close(y[t], L.ref(x[t]), f"T={T} token {t}")
        # batch invariance against the decode path
        assert_close(y[T - 1], L.forward(x[T - 1:T])[0], f"T={T} vs decode")
    L.free()


def test_dense_glm_shape(hf):
    H, I = 6144, 12288
    configure(H, 2048, 256, 8)
    L = Dense(H, I, seed=32)
    x = np.random.default_rng(32).standard_normal((8, H)).astype(np.float32)
    y = L.forward(x)
    for t in (0, 7):
        assert_close(y[t], L.ref(x[t]), f"token {t}")
    assert_close(L.forward(x[:1])[0], L.ref(x[0]), "decode")
    L.free()


def ref_all(L, x):
    """The dense MLP of every token in float32 (the oracle's weights; FP32
    summation-order differences are ~1e-6 of the outputs, far inside the
    tolerance), for checks over every output of a batch."""
    H, I = L.hidden, L.inter
    Wg, Wu, Wd = (O.bf16_to_f32(m) for m in L.host)
    g = x @ Wg.reshape(I, H).T
    u = x @ Wu.reshape(I, H).T
    h = g / (1.0 + np.exp(-g)) * u
    return h @ Wd.reshape(H, I).T


def test_dense_glm_shape_prefill_tiles(hf):
    # T >= 192: prefill tiles (h as BF16 hi + lo, two K splits of the down
    # projection); every output against the float32 reference, three tokens
    # against the oracle.
    H, I, T = 6144, 12288, 256
    configure(H, 2048, 256, T)
    L = Dense(H, I, seed=35)
    x = np.random.default_rng(35).standard_normal((T, H)).astype(np.float32)
    y = L.forward(x)
    for t in (0, 129, T - 1):
        assert_close(y[t], L.ref(x[t]), f"token {t}")
    assert_close(y, ref_all(L, x), "every output")
    L.free()


@pytest.mark.parametrize("H,I,T", [(1024, 3072, 200), (6144, 12288, 256)])
def test_dense_down_k_splits(hf, H, I, T):
    # max_tokens well above T: the down projection's few items (one M tile)
    # are split 8 ways along K into partials summed in split order.
    configure(H, 2048 if H == 6144 else 512, 256 if H == 6144 else 64, 2048)
    L = Dense(H, I, seed=37)
    x = np.random.default_rng(37).standard_normal((T, H)).astype(np.float32)
    y = L.forward(x)
    for t in (0, T // 2, T - 1):
        assert_close(y[t], L.ref(x[t]), f"T={T} token {t}")
    assert_close(y, ref_all(L, x), f"T={T} every output")
    L.free()


@pytest.mark.parametrize("T", [64, 128, 191])
def test_dense_glm_shape_small_batch_k_splits(hf, T):
    # T <= 128: one 128-row tile, the down projection's 48 items; T = 191: one
    # 256-row tile, 24 items; split along K into partials summed in split
    # order.  Every output against the float32 reference, two tokens against
    # the oracle.
    H, I = 6144, 12288
    configure(H, 2048, 256, T)
    L = Dense(H, I, seed=41)
    x = np.random.default_rng(41).standard_normal((T, H)).astype(np.float32)
    y = L.forward(x)
    for t in (0, T - 1):
        assert_close(y[t], L.ref(x[t]), f"T={T} token {t}")
    assert_close(y, ref_all(L, x), f"T={T} every output")
    L.free()


@pytest.mark.parametrize("T,ks", [(64, None), (160, 3), (128, 4), (64, 8)])
def test_dense_gate_up_k_splits(hf, monkeypatch, T, ks):
    # One 256-row M tile gives the gate/up GEMM 96 items: from 64 to 256
    # tokens it splits K in two (None: the automatic choice), gate and up
    # partials in FP32 summed in split order before the SwiGLU.  The split
    # sums round differently from the unsplit GEMM's (so the outputs must
    # differ: the split path ran), and both hold every output to the float32
    # reference; a token of each against the oracle.
    H, I = 6144, 12288
    configure(H, 2048, 256, 512)  # partials for 2 splits x 256 tokens: room for 3 x 160, 4 x 128, 8 x 64
    L = Dense(H, I, seed=43)
    x = np.random.default_rng(43).standard_normal((T, H)).astype(np.float32)
    if ks:
        monkeypatch.setenv("HFMOE_DENSE_GU_KSPLIT", str(ks))
    y = L.forward(x)
    monkeypatch.setenv("HFMOE_DENSE_GU_KSPLIT", "1")
    y1 = L.forward(x)
    monkeypatch.delenv("HFMOE_DENSE_GU_KSPLIT")
    assert not np.array_equal(y.view(np.uint32), y1.view(np.uint32)), "the split path did not run"
    ref = ref_all(L, x)
    assert_close(y, ref, f"T={T} split every output")
    assert_close(y1, ref, f"T={T} unsplit every output")
    assert_close(y[T - 1], L.ref(x[T - 1]), f"T={T} split token {T - 1}")
    L.free()


@pytest.mark.parametrize("T", [512, 600])
def test_dense_item_orders_bit_identical(hf, monkeypatch, T):
    # Prefill tiles deal the items in blocks of N tiles x M tiles per XCD (M
    # tiles fastest) unless HFMOE_DENSE_BY_NTILE=0 (each XCD whole M tiles):
    # every item is computed the same way whichever workgroup takes it, so
    # the two orders agree bit for bit.  T = 512: two M tiles, 4 N groups x 2
    # M groups; T = 600: three M tiles (the last ragged), which do not split
    # in two, so 8 N groups x 1.
    H, I = 6144, 12288
    configure(H, 2048, 256, T)
    L = Dense(H, I, seed=39)
    x = np.random.default_rng(39).standard_normal((T, H)).astype(np.float32)
    y = L.forward(x)
    monkeypatch.setenv("HFMOE_DENSE_BY_NTILE", "0")
    y0 = L.forward(x)
    monkeypatch.delenv("HFMOE_DENSE_BY_NTILE")
    assert np.array_equal(y.view(np.uint32), y0.view(np.uint32))
    assert_close(y, ref_all(L, x), "every output")
    L.free()


def test_dense_large_weights(hf):
    # Weights ~N(0, 4): |h| passes 65504 (beyond FP16) on prefill tiles.  At
    # that weight scale an output is a small residual of terms near 1e6, so
    # FP32 summation order alone moves it by ~1e-5 of the token's largest
    # output: the absolute floor is 1e-4 of that instead of 2e-3 (as for the
    # MoE layer's prefill fallback test).
    H, I, T = 1024, 3072, 300
    configure(H, 512, 64, T)
    L = Dense(H, I, seed=36, std=4.0)
    x = np.random.default_rng(36).standard_normal((T, H)).astype(np.float32)
    y = L.forward(x)
    assert np.all(np.isfinite(y))
    for t in (0, 150, T - 1):
        ref = L.ref(x[t]).astype(np.float64)
        err = np.abs(y[t] - ref)
        assert np.all(err <= 1e-2 * np.abs(ref) + 1e-4 * np.abs(ref).max()), f"token {t}: {err.max()}"
    g = O.bf16_to_f32(L.host[0]).reshape(I, H) @ x[0].astype(np.float64)
    u = O.bf16_to_f32(L.host[1]).reshape(I, H) @ x[0].astype(np.float64)
    h_max = np.max(np.abs(g / (1.0 + np.exp(-g)) * u))
    assert h_max > 65504.0, h_max
    L.free()


def test_dense_block_and_moe_forward_rejected(hf):
    H = 1024
    configure(H, 512, 64, 4)
    L = Dense(H, 2048, seed=33, layer=3)
    x = np.random.default_rng(33).standard_normal(H).astype(np.float32)
    h = capi.DeviceBuffer.of(x)
    capi.call("hfmoe_mlp_block", 3, h.ptr, 1, None)
    capi.call("hfmoe_synchronize")
    want = x + L.ref(O.rmsnorm(L.norm, x, 1e-5))
    assert_close(h.download(np.float32, H), want, "dense block")
    assert capi.load().hfmoe_moe_forward(3, h.ptr, 1, h.ptr, None) == capi.ERR_INVALID_ARGUMENT
    h.free()
    L.free()


def test_dense_layer_from_checkpoint(hf, tmp_path):
    H, I = 1024, 2048
    configure(H, 512, 64, 4)
    gw, uw, dw = (O.fill_bf16(H * I, 34, 100 + i, 0.0, 0.02) for i in range(3))
    norm = O.fill_bf16(H, 34, 103, 1.0, 0.05)
    p = "model.layers.1."
    write_shard(tmp_path / "model-00001-of-00001.safetensors",
                {p + "mlp.gate_proj.weight": (gw, [I, H]), p + "mlp.up_proj.weight": (uw, [I, H]),
                 p + "mlp.down_proj.weight": (dw, [H, I]), p + "post_attention_layernorm.weight": (norm, [H])})
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps(
        {"weight_map": {k: "model-00001-of-00001.safetensors" for k in
                        (p + "mlp.gate_proj.weight", p + "mlp.up_proj.weight", p + "mlp.down_proj.weight",
                         p + "post_attention_layernorm.weight")}}))
    ck = C.c_void_p()
    capi.call("hfmoe_checkpoint_open", str(tmp_path).encode(), C.byref(ck))
    capi.call("hfmoe_checkpoint_load_dense_layer", ck, 1)
    x = np.random.default_rng(34).standard_normal(H).astype(np.float32)
    h = capi.DeviceBuffer.of(x)
    capi.call("hfmoe_mlp_block", 1, h.ptr, 1, None)
    capi.call("hfmoe_synchronize")
    want = x + O.dense_mlp(gw, uw, dw, O.rmsnorm(norm, x, 1e-5), H, I)
    assert_close(h.download(np.float32, H), want, "checkpoint dense block")
    h.free()
    capi.load().hfmoe_checkpoint_close(ck)
