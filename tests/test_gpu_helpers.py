"""Plugin helpers (cuda_backend.h:36-48) against the oracle.

The oracle's embedding, matvec, softmax and argmax are pinned bit-exact to the
reference's own CPU forms of these helpers (tests/test_oracle.py, golden
vectors).  The embedding widens BF16 exactly and argmax keeps the first
largest element, so both must match bit for bit; matvec and softmax agree
within 1e-2 relative + 2e-3 absolute.  Softmax outputs are probabilities far
below that absolute floor, so they are held to relative bounds: 1e-5 against
an FP64 softmax of the same inputs, and 1e-3 against the oracle, whose serial
FP32 sum over n terms (the reference's loop) drifts by up to about n * 2^-24
(2.2e-4 at n = 154880; 3e-7 at n = 1000).  Host-buffer entry points (the
reference's contract) and the device forms both.
"""
import ctypes as C

import numpy as np
import pytest

import oracle as O
from hummingflight_amd import capi, synth
from moe_harness import assert_close

pytestmark = pytest.mark.gpu


@pytest.fixture
def configured(hf):
    shape = synth.LayerShape(hidden=1024, inter=512, n_experts=64, top_k=8, n_group=8, topk_group=4)
    capi.call("hfmoe_configure", shape.config(max_tokens=4))


def ptr(a):
    return a.ctypes.data_as(C.c_void_p)


def check_softmax(y, x):
    e = np.exp(x.astype(np.float64) - np.max(x))
    np.testing.assert_allclose(y, e / e.sum(), rtol=1e-5, atol=1e-30)
    np.testing.assert_allclose(y, O.softmax(x), rtol=1e-3, atol=1e-30)


def test_embedding_lookup_host_and_device(configured):
    vocab, hidden = 1000, 6144
    emb = O.fill_bf16(vocab * hidden, 51, 1, 0.0, 1.0)
    for tok in (0, 517, vocab - 1):
        out = np.empty(hidden, np.float32)
        capi.call("hfmoe_embedding_lookup", ptr(emb), tok, ptr(out), hidden)
        assert np.array_equal(out.view(np.uint32), O.embedding(emb, tok, hidden).view(np.uint32)), tok
    ed = capi.DeviceBuffer.of(emb)
    ids = np.array([3, -1, vocab - 1, vocab, 0], np.int32)
    idd = capi.DeviceBuffer.of(ids)
    od = capi.DeviceBuffer(len(ids) * hidden * 4)
    capi.call("hfmoe_embedding", ed.ptr, vocab, hidden, idd.ptr, len(ids), od.ptr, None)
    capi.call("hfmoe_synchronize")
    got = od.download(np.float32, len(ids) * hidden).reshape(len(ids), hidden)
    for t, tok in enumerate(ids):
        want = O.embedding(emb, tok, hidden) if 0 <= tok < vocab else np.zeros(hidden, np.float32)
        assert np.array_equal(got[t].view(np.uint32), want.view(np.uint32)), (t, tok)
    one = capi.DeviceBuffer(hidden * 4)
    capi.call("hfmoe_embedding_gather", ed.ptr, 517, one.ptr, hidden, None)
    capi.call("hfmoe_synchronize")
    assert np.array_equal(one.download(np.uint32, hidden), O.embedding(emb, 517, hidden).view(np.uint32))
    for b in (ed, idd, od, one):
        b.free()


@pytest.mark.parametrize("M,K", [(300, 1024), (7, 6144), (129, 100), (5, 9000)],
                         ids=["fused_gemv", "glm_hidden", "ragged_k", "k_beyond_lds"])
def test_matvec(configured, M, K):
    W = O.fill_bf16(M * K, 52, 1, 0.0, 0.05).reshape(M, K)
    x = O.fill_f32(K, 52, 2, 0.0, 1.0)
    y = np.empty(M, np.float32)
    capi.call("hfmoe_matvec_bf16", ptr(W), ptr(x), ptr(y), M, K)
    ref = O.gemv(W, x)
    assert_close(y, ref, f"matvec {M}x{K}")
    # Device form, W aligned and W starting 2 bytes into its buffer.
    for shift in (0, 1):
        Wd = capi.DeviceBuffer.of(np.concatenate([np.zeros(shift, np.uint16), W.ravel()]))
        xd, yd = capi.DeviceBuffer.of(x), capi.DeviceBuffer(4 * M)
        capi.call("hfmoe_matvec_bf16_dev", Wd.ptr + 2 * shift, xd.ptr, yd.ptr, M, K, None)
        capi.call("hfmoe_synchronize")
        assert_close(yd.download(np.float32, M), ref, f"device matvec {M}x{K} shift {shift}")
        for b in (Wd, xd, yd):
            b.free()


@pytest.mark.parametrize("n", [1, 64, 1000, 154880])
def test_softmax_host(configured, n):
    x = O.fill_f32(n, 53, 1, 0.0, 4.0)
    y = x.copy()
    capi.call("hfmoe_softmax", ptr(y), n)
    check_softmax(y, x)
    assert int(np.argmax(y)) == O.argmax(O.softmax(x))


def test_softmax_rows_device(configured):
    T, n = 3, 5003
    x = np.stack([O.fill_f32(n, 54, 1 + t, 0.0, 3.0) for t in range(T)])
    x[2, :] = 7.5  # equal inputs: exactly 1/n
    xd = capi.DeviceBuffer.of(x)
    capi.call("hfmoe_softmax_rows", xd.ptr, T, n, None)
    capi.call("hfmoe_synchronize")
    y = xd.download(np.float32, T * n).reshape(T, n)
    for t in range(T):
        check_softmax(y[t], x[t])
    assert np.all(y[2] == np.float32(1.0) / np.float32(n))
    xd.free()


@pytest.mark.parametrize("n", [1, 77, 154880])
def test_argmax_first_of_ties(configured, n):
    x = O.fill_f32(n, 55, 1, 0.0, 1.0)
    x[n // 3] = x[2 * n // 3] = float(np.max(x)) + 1.0
    best = C.c_int32(-1)
    capi.call("hfmoe_argmax", ptr(x), n, C.byref(best))
    assert best.value == O.argmax(x) == n // 3
    rows = np.stack([x, x[::-1].copy()])
    xd, bd = capi.DeviceBuffer.of(rows), capi.DeviceBuffer(8)
    capi.call("hfmoe_argmax_rows", xd.ptr, 2, n, bd.ptr, None)
    capi.call("hfmoe_synchronize")
    assert bd.download(np.int32, 2).tolist() == [O.argmax(rows[0]), O.argmax(rows[1])]
    for b in (xd, bd):
        b.free()


def test_helpers_reject_bad_arguments(configured):
    lib = capi.load()
    x = np.zeros(4, np.float32)
    assert lib.hfmoe_softmax(ptr(x), 0) == capi.ERR_INVALID_ARGUMENT
    assert lib.hfmoe_argmax(None, 4, None) == capi.ERR_INVALID_ARGUMENT
    assert lib.hfmoe_embedding_lookup(None, 0, ptr(x), 4) == capi.ERR_INVALID_ARGUMENT
    assert lib.hfmoe_matvec_bf16(ptr(x), ptr(x), ptr(x), 0, 4) == capi.ERR_INVALID_ARGUMENT


def test_router_sigmoid_matches_the_c_library(hf):
    # The router's sigmoid on the device against 1/(1 + expf(-x)) with glibc's
    # expf (the oracle), bit for bit: every 256th float bit pattern (each
    # exponent, both signs, with the low byte varied), and every 97th float of
    # either sign below 16 in magnitude, where router logits live.
    i = np.arange(1 << 24, dtype=np.uint64)
    sweep = ((i << np.uint64(8)) | ((i * np.uint64(37)) & np.uint64(255))).astype(np.uint32)
    pos = np.arange(0, 0x41800000, 97, dtype=np.uint32)
    dense = np.concatenate([pos, pos | np.uint32(0x80000000)])
    for bits in (sweep, dense):
        x = bits.view(np.float32)
        x = x[~np.isnan(x)]
        xb = capi.DeviceBuffer.of(x)
        yb = capi.DeviceBuffer(x.size * 4)
        capi.call("hfmoe_router_sigmoid", xb.ptr, yb.ptr, x.size, None)
        capi.call("hfmoe_synchronize")
        got = yb.download(np.float32, x.size)
        ref = O.sigmoid(x)
        bad = np.flatnonzero(got.view(np.uint32) != ref.view(np.uint32))
        assert bad.size == 0, f"{bad.size} differ, first x={x[bad[0]]!r}: {got[bad[0]]!r} vs {ref[bad[0]]!r}"
        xb.free()
        yb.free()
