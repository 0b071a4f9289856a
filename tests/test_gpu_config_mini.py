"""The reference's own test configuration (tests/fixtures/config_mini.json, MoE
fields in tests/golden/reference_vectors.json "config_mini") end to end.

Hidden 16, one dense layer (intermediate 48) then three MoE layers (8 routed
experts, top-2, one shared, expert intermediate 16, scale 2.5, normalised
weights, flat routing), vocabulary 64: embedding lookup, four RMSNorm + MLP +
residual blocks, final norm, LM head and greedy token, for single tokens and a
batch.  The oracle is pinned bit-exact to the reference's moeLayer at this
configuration (tests/test_oracle.py); the library agrees within 1e-2 relative
+ 2e-3 absolute at every layer, its selections are the oracle's given the
GPU's router logits, and its greedy token is the oracle's argmax (or a
candidate tied within the tolerance).  Hidden 16 is not a multiple of 64, so a
batch runs token by token on the decode kernels.
"""
import ctypes as C

import numpy as np
import pytest

import oracle as O
from hummingflight_amd import capi, synth
from moe_harness import ATOL, RTOL, Run, assert_close

pytestmark = pytest.mark.gpu

SEED = 17


@pytest.fixture
def mini(golden):
    return golden["config_mini"]


def moe_dims(m):
    return dict(hidden=m["hidden_size"], inter=m["moe_intermediate_size"], n_experts=m["n_routed_experts"],
                top_k=m["num_experts_per_tok"])


def routing(m):
    return dict(norm_topk_prob=m["norm_topk_prob"], routed_scaling_factor=m["routed_scaling_factor"])


@pytest.mark.parametrize("T", [1, 5])
def test_config_mini_moe_layer(hf, mini, T):
    r = Run(moe_dims(mini), seed=SEED, T=T, n_shared=mini["n_shared_experts"], **routing(mini))
    x = synth.make_x_dev(T, mini["hidden_size"], seed=SEED + T)
    res = r.forward(x, T)
    xh = x.download(np.float32, T * mini["hidden_size"]).reshape(T, -1)
    for t in range(T):
        r.check_token(xh[t], res, t)
    x.free()
    r.free()


class MiniModel:
    """Dense layer 0, MoE layers 1..n-1 (with post-attention norms), final norm
    and LM head, registered on the device, plus the host copies the oracle uses."""

    def __init__(self, m):
        d, Id, V = m["hidden_size"], m["intermediate_size"], m["vocab_size"]
        self.m, self.d, self.V = m, d, V
        self.nl = m["num_hidden_layers"]
        self.eps = m["rms_norm_eps"]
        assert m["mlp_layer_types"][:m["first_k_dense_replace"]] == ["dense"] * m["first_k_dense_replace"]
        self.shape = synth.LayerShape(n_group=1, topk_group=m["topk_group"], n_shared=m["n_shared_experts"],
                                      **moe_dims(m), **routing(m))
        capi.call("hfmoe_configure", self.shape.config(max_tokens=8))
        self.bufs = []
        # dense layers
        self.dense = {}
        for l in range(m["first_k_dense_replace"]):
            host = [O.fill_bf16(d * Id, SEED, 500 + 10 * l + i, 0.0, 0.02) for i in range(3)]
            norm = O.fill_bf16(d, SEED, 509 + 10 * l, 1.0, 0.05)
            dev = [capi.DeviceBuffer.of(a) for a in host + [norm]]
            self.bufs += dev
            w = capi.DenseWeights(dev[0].ptr, dev[1].ptr, dev[2].ptr, dev[3].ptr, Id, 0)
            capi.call("hfmoe_register_dense_layer", l, C.byref(w))
            self.dense[l] = (host, norm)
        # MoE layers
        self.moe = {}
        for l in range(m["first_k_dense_replace"], self.nl):
            dl = synth.DeviceLayer(self.shape, layer=l, seed=SEED, with_norm=True)
            spec = O.LayerSpec(n_group=1, topk_group=m["topk_group"], n_shared=m["n_shared_experts"], seed=SEED,
                               layer=l, **moe_dims(m), **routing(m))
            norm = O.fill_bf16(d, SEED, O.tensor_id(l, O.ROLE_NORM), 1.0, 0.05)
            self.moe[l] = (dl, O.SyntheticLayer(spec), norm)
        # embedding table, final norm, LM head
        self.emb = O.fill_bf16(V * d, SEED, 600, 0.0, 1.0)
        self.lm = O.fill_bf16(V * d, SEED, 601, 0.0, 0.02)
        self.fnorm = O.fill_bf16(d, SEED, 602, 1.0, 0.05)
        self.emb_d, self.lm_d, self.fnorm_d = (capi.DeviceBuffer.of(a) for a in (self.emb, self.lm, self.fnorm))
        self.bufs += [self.emb_d, self.lm_d, self.fnorm_d]
        capi.call("hfmoe_register_lm_head", self.lm_d.ptr, self.fnorm_d.ptr, V)

    def ref_block(self, l, h):
        if l in self.dense:
            (gw, uw, dw), norm = self.dense[l]
            return h + O.dense_mlp(gw, uw, dw, O.rmsnorm(norm, h, self.eps), self.d, self.m["intermediate_size"])
        _, ref, norm = self.moe[l]
        out, _, _, _ = ref.forward(O.rmsnorm(norm, h, self.eps))
        return h + out

    def free(self):
        for dl, _, _ in self.moe.values():
            dl.free()
        for b in self.bufs:
            b.free()


def test_config_mini_model(hf, mini):
    M = MiniModel(mini)
    d, V = M.d, M.V
    ids = np.array([3, 17, 42, 63, 0], np.int32)
    T = len(ids)
    idd = capi.DeviceBuffer.of(ids)
    h = capi.DeviceBuffer(T * d * 4)
    capi.call("hfmoe_embedding", M.emb_d.ptr, V, d, idd.ptr, T, h.ptr, None)
    capi.call("hfmoe_synchronize")
    hh = h.download(np.float32, T * d).reshape(T, d)
    for t in range(T):
        assert np.array_equal(hh[t].view(np.uint32), O.embedding(M.emb, int(ids[t]), d).view(np.uint32))
    # Layer by layer on the batch; each layer checked from the device's own input.
    for l in range(M.nl):
        capi.call("hfmoe_mlp_block", l, h.ptr, T, None)
        capi.call("hfmoe_synchronize")
        got = h.download(np.float32, T * d).reshape(T, d)
        for t in range(T):
            assert_close(got[t], M.ref_block(l, hh[t]), f"layer {l} token {t}")
        hh = got
    lg = capi.DeviceBuffer(T * V * 4)
    tok = capi.DeviceBuffer(T * 4)
    capi.call("hfmoe_lm_head", h.ptr, T, lg.ptr, tok.ptr, None)
    capi.call("hfmoe_synchronize")
    logits = lg.download(np.float32, T * V).reshape(T, V)
    tokens = tok.download(np.int32, T)
    for t in range(T):
        ref, best = O.lm_head(M.lm, M.fnorm, hh[t], V, M.eps)
        assert_close(logits[t], ref, f"logits token {t}")
        got = int(tokens[t])
        if got != best:
            assert abs(float(ref[got]) - float(ref[best])) <= ATOL + RTOL * abs(float(ref[best])), (t, got, best)
    for b in (idd, h, lg, tok):
        b.free()
    M.free()
