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



def tolerance_share(got, ref):
    """Largest |got - ref| / (ATOL + RTOL * |ref|) over all elements: 1.0 is the bar."""
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(np.asarray(got, np.float64) - ref) / (ATOL + RTOL * np.abs(ref))))


class DeviceBackedLayer(O.SyntheticLayer):
    """The oracle layer with its routed experts read back from the device
    layer's own block (HBM or pinned host RAM) rather than regenerated on the
    host: the device generator is bit-exact with the oracle's
    (tests/test_gpu_moe.py), and at full shape reading 19 GB back is far
    faster than generating it again."""

    def __init__(self, spec, dev_layer):
        super().__init__(spec)
        s = spec
        n = s.inter * s.hidden
        self.nd = min(dev_layer.distinct_experts or s.n_experts, s.n_experts)
        if dev_layer.experts_on_host:
            flat = dev_layer.experts.view(np.uint16, self.nd * 3 * n)
        else:
            flat = dev_layer.experts.download(np.uint16, self.nd * 3 * n)
        self.block = flat.reshape(self.nd, 3, n)

    def expert(self, e: int):
        b = self.block[e % self.nd]
        return b[0], b[1], b[2]


def _f32(bits):
    return (bits.astype(np.uint32) << 16).view(np.float32)


def _ffn_f32(x, g, u, d, I, H):
    gv = x @ g.reshape(I, H).T
    uv = x @ u.reshape(I, H).T
    h = gv / (np.float32(1.0) + np.exp(-gv)) * uv
    return h @ d.reshape(H, I).T


def layer_reference_f32(ref, x, idx, w, workers=6):
    """Every token's MoE output from the oracle layer's weights and the given
    routing: each expert's SwiGLU over all of its tokens in float32 (numpy),
    the routed outputs weighted and summed with the shared expert's in
    float64.  Only the FP32 summation order differs from the reference
    (~1e-6 of an output, far inside the 1e-2 / 2e-3 tolerance), so every
    output of a large batch can be checked, not a few tokens.  Weight
    conversions run a few experts ahead on a thread pool; the products use
    numpy's threaded BLAS."""
    from collections import deque
    from concurrent.futures import ThreadPoolExecutor

    s = ref.spec
    H, I = s.hidden, s.inter
    T, k = idx.shape
    x = np.ascontiguousarray(x, np.float32)
    out = np.zeros((T, H), np.float64)
    flat = idx.ravel()
    order = np.argsort(flat, kind="stable")
    experts, starts = np.unique(flat[order], return_index=True)
    ends = list(starts[1:]) + [flat.size]
    with ThreadPoolExecutor(workers) as ex:
        pend = deque()
        todo = iter(range(len(experts)))

        def submit():
            i = next(todo, None)
            if i is not None:
                pend.append((i, ex.submit(lambda e: [_f32(m) for m in ref.expert(int(e))], experts[i])))

        for _ in range(workers + 2):
            submit()
        while pend:
            i, fut = pend.popleft()
            g, u, dn = fut.result()
            submit()
            pairs = order[starts[i]:ends[i]]
            tok, rank = pairs // k, pairs % k
            y = _ffn_f32(x[tok], g, u, dn, I, H)
            out[tok] += w[tok, rank].astype(np.float64)[:, None] * y
    if s.n_shared:
        Is = s.n_shared * I
        out += _ffn_f32(x, _f32(ref.sg), _f32(ref.su), _f32(ref.sd), Is, H)
    return out


def tile_cover_tokens(offsets, perm, T, k, tile_rows, n_shared):
    """Tokens that between them touch every M tile of the canonical dispatch
    order (each expert's rows in tile_rows-row chunks, the shared expert's T
    rows likewise): a token per tile not covered by a token already taken."""
    E = offsets.size - 1
    tok_of_row = perm // k
    tile_of_pair = np.empty(T * k, np.int64)
    tiles = []
    for e in range(E):
        for r0 in range(offsets[e], offsets[e + 1], tile_rows):
            tiles.append(("e", e, r0))
            tile_of_pair[perm[r0:min(r0 + tile_rows, offsets[e + 1])]] = len(tiles) - 1
    covered = np.zeros(len(tiles) + (T + tile_rows - 1) // tile_rows * n_shared, bool)
    shared0 = len(tiles)
    picks = []
    for i in range(covered.size):
        if covered[i]:
            continue
        if i < shared0:
            t = int(tok_of_row[tiles[i][2]])
        else:
            t = (i - shared0) * tile_rows
        picks.append(t)
        covered[tile_of_pair[t * k:(t + 1) * k]] = True
        if n_shared:
            covered[shared0 + t // tile_rows] = True
    return picks
