"""ctypes binding of include/hfmoe.h (libhfmoe.so).

Plain pointers and sizes only; no torch.  Loading fails loudly when the library
has not been built: there is no other compute path.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libhfmoe.so")

OK = 0
ERR_NO_DEVICE = 1
ERR_NOT_INITIALIZED = 2
ERR_INVALID_ARGUMENT = 3
ERR_UNSUPPORTED = 4
ERR_OUT_OF_MEMORY = 5
ERR_NOT_REGISTERED = 6
ERR_HIP = 7

EXPERTS_DEVICE = 0
EXPERTS_HOST_PINNED = 1


class Config(C.Structure):
    _fields_ = [("hidden", C.c_int32), ("moe_intermediate", C.c_int32),
                ("n_routed_experts", C.c_int32), ("num_experts_per_tok", C.c_int32),
                ("n_group", C.c_int32), ("topk_group", C.c_int32),
                ("n_shared_experts", C.c_int32), ("norm_topk_prob", C.c_int32),
                ("routed_scaling_factor", C.c_float), ("rms_norm_eps", C.c_float),
                ("vram_budget_bytes", C.c_uint64), ("max_tokens", C.c_int32),
                ("reserved", C.c_int32)]


class LayerWeights(C.Structure):
    _fields_ = [("router_dev", C.c_void_p), ("score_bias_dev", C.c_void_p),
                ("shared_gate_dev", C.c_void_p), ("shared_up_dev", C.c_void_p),
                ("shared_down_dev", C.c_void_p), ("experts", C.c_void_p),
                ("post_attention_norm_dev", C.c_void_p), ("experts_location", C.c_int32),
                ("reserved", C.c_int32)]


class DenseWeights(C.Structure):
    _fields_ = [("gate_dev", C.c_void_p), ("up_dev", C.c_void_p), ("down_dev", C.c_void_p),
                ("post_attention_norm_dev", C.c_void_p), ("intermediate", C.c_int32), ("reserved", C.c_int32)]


class RouteDebug(C.Structure):
    _fields_ = [("logits_dev", C.c_void_p), ("idx_dev", C.c_void_p), ("weight_dev", C.c_void_p),
                ("offsets_dev", C.c_void_p), ("perm_dev", C.c_void_p)]


class KernelStat(C.Structure):
    _fields_ = [("name", C.c_char * 32), ("launches", C.c_int64), ("total_ms", C.c_double)]


class StreamOptions(C.Structure):
    _fields_ = [("prefetch_next_layer", C.c_int32), ("ema_predictor", C.c_int32),
                ("ema_alpha", C.c_float), ("overlap_floor", C.c_float), ("overlap_alpha", C.c_float),
                ("extra_depth", C.c_int32), ("prob_resident", C.c_int32), ("reserved", C.c_int32)]


class StreamCounters(C.Structure):
    _fields_ = [("lookups", C.c_uint64), ("hits", C.c_uint64), ("misses", C.c_uint64),
                ("pred_staged", C.c_uint64), ("pred_consumed", C.c_uint64), ("pred_wasted", C.c_uint64),
                ("pred_resident", C.c_uint64), ("copies", C.c_uint64),
                ("slots", C.c_int32), ("pinned", C.c_int32)]

    def as_dict(self) -> dict:
        return {name: getattr(self, name) for name, _ in self._fields_ if name != "reserved"}


class SafetensorsStats(C.Structure):
    _fields_ = [(n, C.c_uint64) for n in ("total", "accepted", "rejected", "duplicate_rejected", "dtype_rejected",
                                          "f32_allowed_accepted", "shape_rejected", "bounds_rejected",
                                          "byte_mismatch_rejected", "alignment_rejected")] + \
               [("shards", C.c_int32), ("reserved", C.c_int32)]

    def as_dict(self) -> dict:
        return {name: getattr(self, name) for name, _ in self._fields_ if name != "reserved"}


class TensorInfo(C.Structure):
    _fields_ = [("dtype", C.c_char * 8), ("ndim", C.c_int32), ("reserved", C.c_int32),
                ("shape", C.c_int64 * 8), ("nbytes", C.c_uint64), ("file_offset", C.c_uint64)]


# (name, restype, argtypes) for every entry point of include/hfmoe.h.
_SIGS = [
    ("hfmoe_init", C.c_int, [C.c_int]),
    ("hfmoe_shutdown", None, []),
    ("hfmoe_available", C.c_int, []),
    ("hfmoe_device_name", C.c_int, [C.c_char_p, C.c_size_t]),
    ("hfmoe_device_memory_mb", C.c_size_t, []),
    ("hfmoe_last_error", C.c_char_p, []),
    ("hfmoe_configure", C.c_int, [C.POINTER(Config)]),
    ("hfmoe_register_layer", C.c_int, [C.c_int, C.POINTER(LayerWeights)]),
    ("hfmoe_moe_forward", C.c_int, [C.c_int, C.c_void_p, C.c_int32, C.c_void_p, C.c_void_p]),
    ("hfmoe_moe_forward_debug", C.c_int,
     [C.c_int, C.c_void_p, C.c_int32, C.c_void_p, C.c_void_p, C.POINTER(RouteDebug)]),
    ("hfmoe_moe_forward_noalloc", C.c_int, [C.c_int, C.c_void_p, C.c_int32, C.c_void_p, C.c_void_p]),
    ("hfmoe_moe_forward_bf16", C.c_int, [C.c_int, C.c_void_p, C.c_int32, C.c_void_p, C.c_void_p]),
    ("hfmoe_moe_layer", C.c_int, [C.c_int, C.c_void_p, C.c_void_p]),
    ("hfmoe_mlp_block", C.c_int, [C.c_int, C.c_void_p, C.c_int32, C.c_void_p]),
    ("hfmoe_register_dense_layer", C.c_int, [C.c_int, C.POINTER(DenseWeights)]),
    ("hfmoe_register_lm_head", C.c_int, [C.c_void_p, C.c_void_p, C.c_int32]),
    ("hfmoe_embedding_lookup", C.c_int, [C.c_void_p, C.c_int, C.c_void_p, C.c_int]),
    ("hfmoe_matvec_bf16", C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int]),
    ("hfmoe_softmax", C.c_int, [C.c_void_p, C.c_int]),
    ("hfmoe_argmax", C.c_int, [C.c_void_p, C.c_int, C.POINTER(C.c_int32)]),
    ("hfmoe_embedding", C.c_int, [C.c_void_p, C.c_int32, C.c_int32, C.c_void_p, C.c_int32, C.c_void_p, C.c_void_p]),
    ("hfmoe_softmax_rows", C.c_int, [C.c_void_p, C.c_int32, C.c_int32, C.c_void_p]),
    ("hfmoe_embedding_gather", C.c_int, [C.c_void_p, C.c_int, C.c_void_p, C.c_int, C.c_void_p]),
    ("hfmoe_matvec_bf16_dev", C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_void_p]),
    ("hfmoe_argmax_rows", C.c_int, [C.c_void_p, C.c_int32, C.c_int32, C.c_void_p, C.c_void_p]),
    ("hfmoe_router_sigmoid", C.c_int, [C.c_void_p, C.c_void_p, C.c_int64, C.c_void_p]),
    ("hfmoe_lm_head", C.c_int, [C.c_void_p, C.c_int32, C.c_void_p, C.c_void_p, C.c_void_p]),
    ("hfmoe_dense_mlp_forward", C.c_int, [C.c_int, C.c_void_p, C.c_int32, C.c_void_p, C.c_void_p]),
    ("hfmoe_expert_cache_config", C.c_int, [C.c_int, C.c_int]),
    ("hfmoe_expert_cache_shutdown", None, []),
    ("hfmoe_experts_enabled", C.c_int, []),
    ("hfmoe_expert_stage", C.c_int, [C.c_int, C.c_int, C.c_void_p, C.c_int, C.c_int]),
    ("hfmoe_expert_ffn", C.c_int, [C.c_int, C.c_int, C.c_void_p, C.c_void_p, C.c_int, C.c_int]),
    ("hfmoe_self_test", C.c_int, []),
    ("hfmoe_malloc", C.c_int, [C.POINTER(C.c_void_p), C.c_size_t]),
    ("hfmoe_free", C.c_int, [C.c_void_p]),
    ("hfmoe_host_alloc", C.c_int, [C.POINTER(C.c_void_p), C.c_size_t]),
    ("hfmoe_host_free", C.c_int, [C.c_void_p]),
    ("hfmoe_memcpy_h2d", C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t]),
    ("hfmoe_memcpy_d2h", C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t]),
    ("hfmoe_memcpy_d2d", C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t]),
    ("hfmoe_memset", C.c_int, [C.c_void_p, C.c_int, C.c_size_t]),
    ("hfmoe_synchronize", C.c_int, []),
    ("hfmoe_fill_normal_bf16", C.c_int,
     [C.c_void_p, C.c_uint64, C.c_uint64, C.c_uint64, C.c_uint64, C.c_float, C.c_float]),
    ("hfmoe_fill_normal_f32", C.c_int,
     [C.c_void_p, C.c_uint64, C.c_uint64, C.c_uint64, C.c_uint64, C.c_float, C.c_float]),
    ("hfmoe_profile_enable", C.c_int, [C.c_int]),
    ("hfmoe_profile_read", C.c_int, [C.POINTER(KernelStat), C.c_int, C.POINTER(C.c_int)]),
    ("hfmoe_profile_reset", C.c_int, []),
    ("hfmoe_stream_set_options", C.c_int, [C.POINTER(StreamOptions)]),
    ("hfmoe_stream_get_options", C.c_int, [C.POINTER(StreamOptions)]),
    ("hfmoe_stream_read_counters", C.c_int, [C.POINTER(StreamCounters)]),
    ("hfmoe_stream_reset", C.c_int, []),
    ("hfmoe_checkpoint_open", C.c_int, [C.c_char_p, C.POINTER(C.c_void_p)]),
    ("hfmoe_checkpoint_stats", C.c_int, [C.c_void_p, C.POINTER(SafetensorsStats)]),
    ("hfmoe_checkpoint_tensor", C.c_int, [C.c_void_p, C.c_char_p, C.POINTER(TensorInfo)]),
    ("hfmoe_checkpoint_load_moe_layer", C.c_int, [C.c_void_p, C.c_int, C.c_int]),
    ("hfmoe_checkpoint_load_dense_layer", C.c_int, [C.c_void_p, C.c_int]),
    ("hfmoe_checkpoint_load_lm_head", C.c_int, [C.c_void_p]),
    ("hfmoe_checkpoint_close", None, [C.c_void_p]),
    ("hfmoe_stats", C.c_int, [C.POINTER(C.c_uint64), C.POINTER(C.c_uint64)]),
]

EXPORTS = [s[0] for s in _SIGS]

_lib: C.CDLL | None = None


class HfmoeError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"hfmoe error {code}: {msg}")
        self.code = code


def load() -> C.CDLL:
    """Load libhfmoe.so; raises if it was not built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: run __graft_entry__.build() first")
        L = C.CDLL(LIB_PATH)
        for name, res, args in _SIGS:
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(rc: int) -> None:
    if rc != OK:
        raise HfmoeError(rc, load().hfmoe_last_error().decode(errors="replace"))


def call(name: str, *args) -> None:
    check(getattr(load(), name)(*args))


class DeviceBuffer:
    """An HBM allocation owned by the library's allocator."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = C.c_void_p()
        call("hfmoe_malloc", C.byref(p), max(self.nbytes, 16))
        self.ptr = p.value

    def free(self) -> None:
        if self.ptr:
            call("hfmoe_free", self.ptr)
            self.ptr = None

    def upload(self, arr: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(arr)
        assert a.nbytes <= self.nbytes
        call("hfmoe_memcpy_h2d", self.ptr, a.ctypes.data, a.nbytes)
        return self

    def download(self, dtype, count: int) -> np.ndarray:
        out = np.empty(count, dtype=dtype)
        assert out.nbytes <= self.nbytes
        call("hfmoe_memcpy_d2h", out.ctypes.data, self.ptr, out.nbytes)
        return out

    @staticmethod
    def of(arr: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(arr)
        return DeviceBuffer(a.nbytes).upload(a)


class PinnedBuffer:
    """Pinned host memory from hipHostMalloc, viewable as a numpy array."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = C.c_void_p()
        call("hfmoe_host_alloc", C.byref(p), max(self.nbytes, 16))
        self.ptr = p.value

    def view(self, dtype, count: int, offset_bytes: int = 0) -> np.ndarray:
        buf = (C.c_char * (count * np.dtype(dtype).itemsize)).from_address(self.ptr + offset_bytes)
        return np.frombuffer(buf, dtype=dtype, count=count)

    def free(self) -> None:
        if self.ptr:
            call("hfmoe_host_free", self.ptr)
            self.ptr = None


def last_error() -> str:
    return load().hfmoe_last_error().decode(errors="replace")


def profile_read() -> dict[str, tuple[int, float]]:
    L = load()
    n = C.c_int()
    check(L.hfmoe_profile_read(None, 0, C.byref(n)))
    arr = (KernelStat * max(n.value, 1))()
    check(L.hfmoe_profile_read(arr, n.value, C.byref(n)))
    return {arr[i].name.decode(): (arr[i].launches, arr[i].total_ms) for i in range(n.value)}
