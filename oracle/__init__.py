"""ctypes bindings for the CPU oracle (test infrastructure only).

`liboracle.so` is the C restatement of the reference MoE forward (oracle.c);
`_ref/libhfref.so` is the reference's own code behind a thin harness, built only
where the reference checkout exists.  Only tests/, the smoke() entry point and
bench.py's cpu_baseline leg import this package; the product never does.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from dataclasses import dataclass, field

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libhfref.so")

_u16p = C.POINTER(C.c_uint16)
_f32p = C.POINTER(C.c_float)
_i32p = C.POINTER(C.c_int)


class MoeCfg(C.Structure):
    _fields_ = [("hidden", C.c_int), ("inter", C.c_int), ("n_experts", C.c_int),
                ("top_k", C.c_int), ("n_group", C.c_int), ("topk_group", C.c_int),
                ("n_shared", C.c_int), ("norm_topk_prob", C.c_int),
                ("routed_scaling_factor", C.c_float)]


class MoeWeights(C.Structure):
    _fields_ = [("router", C.c_void_p), ("bias", C.c_void_p),
                ("shared_gate", C.c_void_p), ("shared_up", C.c_void_p),
                ("shared_down", C.c_void_p), ("expert_gate", C.c_void_p),
                ("expert_up", C.c_void_p), ("expert_down", C.c_void_p)]


def build(force: bool = False) -> None:
    """Compile liboracle.so (and the reference harness when its sources exist)."""
    if force or not os.path.exists(LIB_PATH):
        subprocess.run(["make", "-s", "-C", HERE, "liboracle.so"], check=True)


def build_ref() -> bool:
    """Compile _ref/libhfref.so from the reference checkout, if present."""
    if not os.path.isdir("/root/reference/src"):
        return os.path.exists(REF_PATH)
    subprocess.run(["make", "-s", "-C", HERE, "ref"], check=True)
    return True


_lib = None
_ref = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        L.orc_bf16_to_f32.restype = C.c_float
        L.orc_bf16_to_f32.argtypes = [C.c_uint16]
        L.orc_bf16_from_f32.restype = C.c_uint16
        L.orc_bf16_from_f32.argtypes = [C.c_float]
        L.orc_gemv_bf16_f32.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int,
                                        C.c_float, C.c_float]
        L.orc_gemv_bf16_f32_avx2.restype = C.c_int
        L.orc_gemv_bf16_f32_avx2.argtypes = L.orc_gemv_bf16_f32.argtypes
        L.orc_sigmoid.restype = C.c_float
        L.orc_sigmoid.argtypes = [C.c_float]
        L.orc_sigmoid_n.argtypes = [C.c_void_p, C.c_void_p, C.c_int64]
        L.orc_moe_layer_bench.restype = C.c_double
        L.orc_moe_layer_bench.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_void_p,
                                          C.c_int]
        L.orc_topk_flat.restype = C.c_int
        L.orc_topk_flat.argtypes = [C.c_void_p, C.c_int, C.c_void_p, C.c_int, C.c_float, C.c_int,
                                    C.c_void_p, C.c_void_p]
        L.orc_topk_grouped.restype = C.c_int
        L.orc_topk_grouped.argtypes = [C.c_void_p, C.c_int, C.c_void_p, C.c_int, C.c_int, C.c_int,
                                       C.c_float, C.c_int, C.c_void_p, C.c_void_p]
        L.orc_dispatch.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_void_p,
                                   C.c_void_p]
        L.orc_expert_ffn.argtypes = [C.c_void_p] * 5 + [C.c_int, C.c_int, C.c_void_p]
        L.orc_rmsnorm.argtypes = [C.c_void_p, C.c_void_p, C.c_int, C.c_float]
        L.orc_softmax.argtypes = [C.c_void_p, C.c_int]
        L.orc_argmax.restype = C.c_int
        L.orc_argmax.argtypes = [C.c_void_p, C.c_int]
        L.orc_moe_layer.restype = C.c_int
        L.orc_moe_layer.argtypes = [C.POINTER(MoeCfg), C.POINTER(MoeWeights), C.c_void_p,
                                    C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p]
        L.orc_route_from_logits.restype = C.c_int
        L.orc_route_from_logits.argtypes = [C.POINTER(MoeCfg), C.c_void_p, C.c_void_p,
                                            C.c_void_p, C.c_void_p]
        L.orc_moe_combine.restype = C.c_int
        L.orc_moe_combine.argtypes = [C.POINTER(MoeCfg), C.POINTER(MoeWeights), C.c_void_p,
                                      C.c_void_p, C.c_void_p, C.c_int, C.c_void_p]
        L.orc_rng_normal_f32.restype = C.c_float
        L.orc_rng_normal_f32.argtypes = [C.c_uint64, C.c_uint64, C.c_uint64, C.c_float, C.c_float]
        L.orc_fill_normal_bf16.argtypes = [C.c_void_p, C.c_uint64, C.c_uint64, C.c_uint64,
                                           C.c_uint64, C.c_float, C.c_float]
        L.orc_fill_normal_f32.argtypes = L.orc_fill_normal_bf16.argtypes
        _lib = L
    return _lib


def ref() -> C.CDLL | None:
    """The reference harness, or None where it was not built."""
    global _ref
    if _ref is None and os.path.exists(REF_PATH):
        R = C.CDLL(REF_PATH)
        R.ref_gemv_bf16_f32.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int,
                                        C.c_float, C.c_float]
        R.ref_sigmoid.restype = C.c_float
        R.ref_sigmoid.argtypes = [C.c_float]
        R.ref_bf16_from_f32.restype = C.c_uint16
        R.ref_bf16_from_f32.argtypes = [C.c_float]
        R.ref_bf16_to_f32.restype = C.c_float
        R.ref_bf16_to_f32.argtypes = [C.c_uint16]
        R.ref_topk_scores.restype = C.c_int
        R.ref_topk_scores.argtypes = [C.c_void_p, C.c_int, C.c_void_p, C.c_int, C.c_float, C.c_int,
                                      C.c_void_p, C.c_void_p]
        R.ref_moe_layer.restype = C.c_int
        R.ref_moe_layer.argtypes = [C.c_char_p, C.POINTER(MoeCfg), C.POINTER(MoeWeights),
                                    C.c_void_p, C.c_void_p]
        R.ref_moe_layer_timed.restype = C.c_int
        R.ref_moe_layer_timed.argtypes = [C.c_char_p, C.POINTER(MoeCfg), C.POINTER(MoeWeights),
                                          C.c_void_p, C.c_void_p, C.c_int, C.POINTER(C.c_double)]
        R.ref_rmsnorm.restype = C.c_int
        R.ref_rmsnorm.argtypes = [C.c_char_p, C.c_void_p, C.c_void_p, C.c_int, C.c_float]
        R.ref_dense_mlp.restype = C.c_int
        R.ref_dense_mlp.argtypes = [C.c_char_p] + [C.c_void_p] * 3 + [C.c_int, C.c_int, C.c_void_p, C.c_void_p]
        R.ref_embedding_lookup.argtypes = [C.c_void_p, C.c_int, C.c_void_p, C.c_int]
        R.ref_matvec_bf16.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int]
        R.ref_softmax.argtypes = [C.c_void_p, C.c_int]
        R.ref_argmax.restype = C.c_int
        R.ref_argmax.argtypes = [C.c_void_p, C.c_int]
        R.ref_lm_head.restype = C.c_int
        R.ref_lm_head.argtypes = [C.c_char_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_float,
                                  C.c_void_p, C.c_void_p, C.POINTER(C.c_int)]
        _ref = R
    return _ref


def _p(a: np.ndarray | None):
    return None if a is None else a.ctypes.data


# ---------------------------------------------------------------- helpers ----

def bf16_to_f32(a: np.ndarray) -> np.ndarray:
    return (a.astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(a: np.ndarray) -> np.ndarray:
    """dtype_bf16.h:27-33 round-to-nearest-even, vectorised."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def fill_bf16(n: int, seed: int, tensor: int, mean: float, std: float, first: int = 0) -> np.ndarray:
    out = np.empty(n, dtype=np.uint16)
    lib().orc_fill_normal_bf16(_p(out), n, seed, tensor, first, mean, std)
    return out


def fill_f32(n: int, seed: int, tensor: int, mean: float, std: float, first: int = 0) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    lib().orc_fill_normal_f32(_p(out), n, seed, tensor, first, mean, std)
    return out


def gemv(A: np.ndarray, x: np.ndarray, alpha=1.0, beta=0.0, y=None, avx2=False) -> np.ndarray:
    M, K = A.shape
    A = np.ascontiguousarray(A, dtype=np.uint16)
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.zeros(M, np.float32) if y is None else np.array(y, np.float32)
    fn = lib().orc_gemv_bf16_f32_avx2 if avx2 else lib().orc_gemv_bf16_f32
    rc = fn(_p(A), _p(x), _p(y), M, K, alpha, beta)
    if avx2 and rc != 0:
        raise RuntimeError("AVX2 restatement not built")
    return y


def sigmoid(x: np.ndarray) -> np.ndarray:
    """1/(1 + expf(-x)) per element in float (moe_router.h:19-21), glibc expf."""
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    lib().orc_sigmoid_n(_p(x), _p(y), x.size)
    return y


def topk_flat(scores, bias, k, scale, norm):
    s = np.ascontiguousarray(scores, np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, np.float32)
    idx = np.zeros(8, np.int32)
    w = np.zeros(8, np.float32)
    n = lib().orc_topk_flat(_p(s), len(s), _p(b), k, scale, int(norm), _p(idx), _p(w))
    return idx[:n].copy(), w[:n].copy()


def topk_grouped(scores, bias, k, n_group, topk_group, scale, norm):
    s = np.ascontiguousarray(scores, np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, np.float32)
    idx = np.zeros(8, np.int32)
    w = np.zeros(8, np.float32)
    n = lib().orc_topk_grouped(_p(s), len(s), _p(b), k, n_group, topk_group, scale, int(norm),
                               _p(idx), _p(w))
    if n < 0:
        raise ValueError("invalid group configuration")
    return idx[:n].copy(), w[:n].copy()


def dispatch(idx: np.ndarray, E: int):
    idx = np.ascontiguousarray(idx, np.int32)
    T, k = idx.shape
    counts = np.zeros(E, np.int32)
    offsets = np.zeros(E + 1, np.int32)
    perm = np.zeros(T * k, np.int32)
    lib().orc_dispatch(_p(idx), T, k, E, _p(counts), _p(offsets), _p(perm))
    return counts, offsets, perm


def rmsnorm(w: np.ndarray | None, x: np.ndarray, eps: float) -> np.ndarray:
    x = np.array(x, np.float32)
    wa = None if w is None else np.ascontiguousarray(w, np.uint16)
    lib().orc_rmsnorm(_p(wa), _p(x), len(x), eps)
    return x


def dense_mlp(gate: np.ndarray, up: np.ndarray, down: np.ndarray, x: np.ndarray, hidden: int,
              inter: int) -> np.ndarray:
    """GLMForward::denseMlp (glm_forward.cpp:410-432): the expert SwiGLU with the
    dense intermediate size (same serial GEMVs, same SiLU association)."""
    x = np.ascontiguousarray(x, np.float32)
    y = np.zeros(hidden, np.float32)
    scratch = np.zeros(3 * inter, np.float32)
    lib().orc_expert_ffn(_p(gate), _p(up), _p(down), _p(x), _p(y), hidden, inter, _p(scratch))
    return y


def lm_head(W: np.ndarray, norm: np.ndarray | None, h: np.ndarray, vocab: int, eps: float):
    """GLMForward::lmHeadAndSample (glm_forward.cpp:663-731): final RMSNorm (the
    rmsNorm formula with the norm weight widened to FP32), serial dot product per
    vocabulary row (dotBf16F32, :67-92), greedy argmax taking the first maximum.
    Returns (logits, best)."""
    xn = rmsnorm(norm, h, eps)
    logits = gemv(np.ascontiguousarray(W, np.uint16).reshape(vocab, -1), xn)
    return logits, int(np.argmax(logits))


def softmax(x: np.ndarray) -> np.ndarray:
    """The reference's softmax (cuda_backend.cpp:39-49): max, exp, one reciprocal."""
    y = np.array(x, np.float32)
    lib().orc_softmax(_p(y), len(y))
    return y


def argmax(x: np.ndarray) -> int:
    """The reference's argmax (cuda_backend.cpp:51-57): first largest element."""
    x = np.ascontiguousarray(x, np.float32)
    return int(lib().orc_argmax(_p(x), len(x)))


def embedding(emb: np.ndarray, token: int, hidden: int) -> np.ndarray:
    """Row `token` of a BF16 [vocab, hidden] table widened to FP32 (cuda_backend.cpp:27-29)."""
    return bf16_to_f32(np.ascontiguousarray(emb, np.uint16).reshape(-1, hidden)[token])


# ------------------------------------------------------------ MoE layer ----

@dataclass
class LayerSpec:
    """Shapes, routing rule and seeds of one synthetic MoE layer.

    Tensor ids (the generator's `tensor` argument) are fixed functions of
    (layer, role, expert) so any tensor can be regenerated independently.
    """
    hidden: int
    inter: int
    n_experts: int
    top_k: int = 8
    n_group: int = 1
    topk_group: int = 1
    n_shared: int = 1
    norm_topk_prob: bool = True
    routed_scaling_factor: float = 2.5
    seed: int = 1
    layer: int = 0
    w_std: float = 0.02
    bias_std: float = 0.01
    bias_override: np.ndarray | None = field(default=None, repr=False)

    def cfg(self) -> MoeCfg:
        return MoeCfg(self.hidden, self.inter, self.n_experts, self.top_k, self.n_group,
                      self.topk_group, self.n_shared, int(self.norm_topk_prob),
                      self.routed_scaling_factor)


ROLE_ROUTER, ROLE_BIAS, ROLE_SG, ROLE_SU, ROLE_SD, ROLE_EG, ROLE_EU, ROLE_ED, ROLE_X, ROLE_NORM = range(10)


def tensor_id(layer: int, role: int, expert: int = 0) -> int:
    return (layer << 40) | (role << 32) | expert


class SyntheticLayer:
    """Host copies of a synthetic layer's tensors, generated lazily per expert."""

    def __init__(self, spec: LayerSpec):
        self.spec = spec
        s = spec
        L = s.layer
        self.router = fill_bf16(s.n_experts * s.hidden, s.seed, tensor_id(L, ROLE_ROUTER), 0.0, s.w_std)
        if s.bias_override is not None:
            self.bias = np.ascontiguousarray(s.bias_override, np.float32)
        else:
            self.bias = fill_f32(s.n_experts, s.seed, tensor_id(L, ROLE_BIAS), 0.0, s.bias_std)
        Is = s.n_shared * s.inter
        if Is:
            self.sg = fill_bf16(Is * s.hidden, s.seed, tensor_id(L, ROLE_SG), 0.0, s.w_std)
            self.su = fill_bf16(Is * s.hidden, s.seed, tensor_id(L, ROLE_SU), 0.0, s.w_std)
            self.sd = fill_bf16(s.hidden * Is, s.seed, tensor_id(L, ROLE_SD), 0.0, s.w_std)
        else:
            self.sg = self.su = self.sd = None
        self.experts: dict[int, tuple[np.ndarray, np.ndarray, np.ndarray]] = {}

    def expert(self, e: int):
        if e not in self.experts:
            s = self.spec
            n = s.inter * s.hidden
            self.experts[e] = (fill_bf16(n, s.seed, tensor_id(s.layer, ROLE_EG, e), 0.0, s.w_std),
                               fill_bf16(n, s.seed, tensor_id(s.layer, ROLE_EU, e), 0.0, s.w_std),
                               fill_bf16(n, s.seed, tensor_id(s.layer, ROLE_ED, e), 0.0, s.w_std))
        return self.experts[e]

    def weights(self, experts) -> tuple[MoeWeights, list]:
        """A MoeWeights view with the listed experts materialised (others NULL)."""
        E = self.spec.n_experts
        g = (C.c_void_p * E)()
        u = (C.c_void_p * E)()
        d = (C.c_void_p * E)()
        for e in experts:
            eg, eu, ed = self.expert(int(e))
            g[e], u[e], d[e] = eg.ctypes.data, eu.ctypes.data, ed.ctypes.data
        W = MoeWeights(self.router.ctypes.data, self.bias.ctypes.data,
                       _p(self.sg), _p(self.su), _p(self.sd),
                       C.cast(g, C.c_void_p), C.cast(u, C.c_void_p), C.cast(d, C.c_void_p))
        return W, [g, u, d]

    def logits(self, x: np.ndarray) -> np.ndarray:
        s = self.spec
        return gemv(self.router.reshape(s.n_experts, s.hidden), x)

    def route(self, logits: np.ndarray):
        idx = np.zeros(8, np.int32)
        w = np.zeros(8, np.float32)
        lg = np.ascontiguousarray(logits, np.float32)
        k = lib().orc_route_from_logits(C.byref(self.spec.cfg()), _p(lg), _p(self.bias), _p(idx), _p(w))
        return idx[:k].copy(), w[:k].copy()

    def forward(self, x: np.ndarray):
        """Oracle moeLayer for one token: (out, logits, idx, w)."""
        s = self.spec
        x = np.ascontiguousarray(x, np.float32)
        lg = self.logits(x)
        idx, w = self.route(lg)
        W, keep = self.weights(idx)
        out = np.zeros(s.hidden, np.float32)
        rc = lib().orc_moe_combine(C.byref(s.cfg()), C.byref(W), _p(x), _p(idx), _p(w), len(idx), _p(out))
        if rc != 0:
            raise RuntimeError("oracle combine failed")
        return out, lg, idx, w

    def combine(self, x: np.ndarray, idx: np.ndarray, w: np.ndarray) -> np.ndarray:
        s = self.spec
        x = np.ascontiguousarray(x, np.float32)
        idx = np.ascontiguousarray(idx, np.int32)
        w = np.ascontiguousarray(w, np.float32)
        W, keep = self.weights(idx)
        out = np.zeros(s.hidden, np.float32)
        rc = lib().orc_moe_combine(C.byref(s.cfg()), C.byref(W), _p(x), _p(idx), _p(w), len(idx), _p(out))
        if rc != 0:
            raise RuntimeError("oracle combine failed")
        return out

    def ref_forward(self, x: np.ndarray, experts, path: str = "/tmp/hf_ref_layer.bin") -> np.ndarray:
        """The reference's own moeLayer on this layer (needs the harness)."""
        R = ref()
        if R is None:
            raise RuntimeError("reference harness not built")
        W, keep = self.weights(experts)
        x = np.ascontiguousarray(x, np.float32)
        out = np.zeros(self.spec.hidden, np.float32)
        rc = R.ref_moe_layer(path.encode(), C.byref(self.spec.cfg()), C.byref(W), _p(x), _p(out))
        if rc != 0:
            raise RuntimeError(f"ref_moe_layer failed rc={rc}")
        return out


def make_x(T: int, hidden: int, seed: int, layer: int = 0) -> np.ndarray:
    """Synthetic activations: BF16 ~N(0,1) values held as float32, [T, hidden]."""
    return bf16_to_f32(fill_bf16(T * hidden, seed, tensor_id(layer, ROLE_X), 0.0, 1.0)).reshape(T, hidden)
