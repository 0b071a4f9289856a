"""LM head (GLMForward::lmHeadAndSample) against the oracle.

The oracle's lm_head is pinned bit-exact to the reference's own
lmHeadAndSample (tests/test_oracle.py, GLM-5.2's 154880-word vocabulary
included).  The library's logits must agree within 1e-2 relative + 2e-3
absolute, and its greedy token must be the oracle's argmax -- or, where two
logits are within the tolerance of each other, one of the tied candidates.
Paths: the T = 1 GEMV with fused argmax, and the grouped GEMM + row argmax for
batches (128- and 192-row tiles).
"""
import ctypes as C

import numpy as np
import pytest

import oracle as O
from hummingflight_amd import capi, synth
from moe_harness import ATOL, RTOL, assert_close
from safetensors_io import write_shard

pytestmark = pytest.mark.gpu


def configure(hidden, max_tokens):
    shape = synth.LayerShape(hidden=hidden, inter=512, n_experts=64, top_k=8, n_group=8, topk_group=4)
    capi.call("hfmoe_configure", shape.config(max_tokens=max_tokens))


class Head:
    def __init__(self, hidden, vocab, seed):
        self.hidden, self.vocab = hidden, vocab
        self.W = O.fill_bf16(vocab * hidden, seed, 300, 0.0, 0.02)
        self.norm = O.fill_bf16(hidden, seed, 301, 1.0, 0.05)
        self.Wd = capi.DeviceBuffer(2 * vocab * hidden)
        synth.fill_bf16(self.Wd.ptr, vocab * hidden, seed, 300, 0.0, 0.02)
        self.nd = capi.DeviceBuffer(2 * hidden)
        synth.fill_bf16(self.nd.ptr, hidden, seed, 301, 1.0, 0.05)
        capi.call("hfmoe_register_lm_head", self.Wd.ptr, self.nd.ptr, vocab)

    def run(self, h):
        T = h.shape[0]
        hd = capi.DeviceBuffer.of(h)
        lg = capi.DeviceBuffer(T * self.vocab * 4)
        tok = capi.DeviceBuffer(T * 4)
        capi.call("hfmoe_lm_head", hd.ptr, T, lg.ptr, tok.ptr, None)
        capi.call("hfmoe_synchronize")
        out = lg.download(np.float32, T * self.vocab).reshape(T, self.vocab), tok.download(np.int32, T)
        for b in (hd, lg, tok):
            b.free()
        return out

    def free(self):
        self.Wd.free()
        self.nd.free()


def check(head, h, logits, tokens, rows):
    for t in rows:
        ref, best = O.lm_head(head.W, head.norm, h[t], head.vocab, 1e-5)
        assert_close(logits[t], ref, f"token {t} logits")
        got = int(tokens[t])
        if got != best:  # only a near-tie may resolve differently
            assert abs(float(ref[got]) - float(ref[best])) <= ATOL + RTOL * abs(float(ref[best])), (t, got, best)
        assert got == int(np.argmax(logits[t]))


@pytest.mark.parametrize("T", [1, 5, 150, 300])
def test_lm_head_small(hf, T):
    H, V = 1024, 5003
    configure(H, 300)
    head = Head(H, V, seed=41)
    h = np.random.default_rng(41 + T).standard_normal((T, H)).astype(np.float32)
    logits, tokens = head.run(h)
    check(head, h, logits, tokens, sorted({0, T // 2, T - 1}))
    head.free()


def test_lm_head_glm_vocab(hf):
    H, V = 6144, 154880
    configure(H, 2)
    head = Head(H, V, seed=42)
    h = np.random.default_rng(42).standard_normal((2, H)).astype(np.float32)
    logits, tokens = head.run(h[:1])
    check(head, h, logits, tokens, [0])
    logits2, tokens2 = head.run(h)  # two tokens: the GEMM path
    check(head, h, logits2, tokens2, [0, 1])
    head.free()


def test_lm_head_from_checkpoint(hf, tmp_path):
    H, V = 512, 777
    configure(H, 1)
    W = O.fill_bf16(V * H, 43, 300, 0.0, 0.02)
    norm = O.fill_bf16(H, 43, 301, 1.0, 0.05)
    write_shard(tmp_path / "m.safetensors", {"lm_head.weight": (W, [V, H]), "model.norm.weight": (norm, [H])})
    ck = C.c_void_p()
    capi.call("hfmoe_checkpoint_open", str(tmp_path / "m.safetensors").encode(), C.byref(ck))
    capi.call("hfmoe_checkpoint_load_lm_head", ck)
    h = np.random.default_rng(43).standard_normal(H).astype(np.float32)
    hd = capi.DeviceBuffer.of(h)
    lg = capi.DeviceBuffer(V * 4)
    tok = capi.DeviceBuffer(4)
    capi.call("hfmoe_lm_head", hd.ptr, 1, lg.ptr, tok.ptr, None)
    capi.call("hfmoe_synchronize")
    ref, best = O.lm_head(W, norm, h, V, 1e-5)
    assert_close(lg.download(np.float32, V), ref, "logits")
    assert int(tok.download(np.int32, 1)[0]) == best
    for b in (hd, lg, tok):
        b.free()
    capi.load().hfmoe_checkpoint_close(ck)
    assert capi.load().hfmoe_lm_head(None, 1, None, None, None) == capi.ERR_NOT_REGISTERED
