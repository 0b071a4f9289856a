"""Seeded synthetic MoE layers built directly in HBM (or pinned host RAM).

Weights come from the library's counter-based generator (hfmoe_fill_normal_*),
so the benchmark never moves 19 GB over PCIe and any tensor can be regenerated
elsewhere from (seed, tensor id, element index).  Tensor ids:
    (layer << 40) | (role << 32) | expert
with the roles below.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, field

import numpy as np

from . import capi

ROLE_ROUTER, ROLE_BIAS, ROLE_SG, ROLE_SU, ROLE_SD, ROLE_EG, ROLE_EU, ROLE_ED, ROLE_X, ROLE_NORM = range(10)


def tensor_id(layer: int, role: int, expert: int = 0) -> int:
    return (layer << 40) | (role << 32) | expert


@dataclass
class LayerShape:
    hidden: int
    inter: int
    n_experts: int
    top_k: int = 8
    n_group: int = 1
    topk_group: int = 1
    n_shared: int = 1
    norm_topk_prob: bool = True
    routed_scaling_factor: float = 2.5
    rms_norm_eps: float = 1e-5

    def config(self, max_tokens: int = 1, vram_budget: int = 0) -> capi.Config:
        return capi.Config(self.hidden, self.inter, self.n_experts, self.top_k, self.n_group,
                           self.topk_group, self.n_shared, int(self.norm_topk_prob),
                           self.routed_scaling_factor, self.rms_norm_eps, vram_budget,
                           max_tokens, 0)

    @property
    def expert_bytes(self) -> int:
        return 3 * self.hidden * self.inter * 2


def fill_bf16(buf_ptr: int, n: int, seed: int, tensor: int, mean: float, std: float, first: int = 0):
    capi.call("hfmoe_fill_normal_bf16", buf_ptr, n, seed, tensor, first, mean, std)


def fill_f32(buf_ptr: int, n: int, seed: int, tensor: int, mean: float, std: float, first: int = 0):
    capi.call("hfmoe_fill_normal_f32", buf_ptr, n, seed, tensor, first, mean, std)


@dataclass
class DeviceLayer:
    """One registered MoE layer with seeded weights.

    experts_on_host: routed experts live in pinned host RAM (streamed path).
    distinct_experts: when set, expert e uses the weights of expert
    e % distinct_experts (host-memory saving for full-shape streaming tests;
    every expert still has its own address range in the table only if
    distinct_experts >= n_experts).
    bias: optional explicit F32 [E] correction bias (else ~N(0, bias_std)).
    register_as: layer id to register under (default `layer`, which seeds the
    tensors), so one weight set can be registered twice, e.g. streamed and
    HBM-resident.
    """
    shape: LayerShape
    layer: int = 0
    seed: int = 1
    w_std: float = 0.02
    bias_std: float = 0.01
    bias: np.ndarray | None = None
    experts_on_host: bool = False
    distinct_experts: int | None = None
    with_norm: bool = False
    register_as: int | None = None
    buffers: list = field(default_factory=list, repr=False)

    def __post_init__(self):
        s = self.shape
        L = self.layer
        d, I, E = s.hidden, s.inter, s.n_experts
        Is = s.n_shared * I
        self.router = self._dev(E * d * 2)
        fill_bf16(self.router.ptr, E * d, self.seed, tensor_id(L, ROLE_ROUTER), 0.0, self.w_std)
        self.bias_buf = self._dev(E * 4)
        if self.bias is not None:
            self.bias_buf.upload(np.ascontiguousarray(self.bias, np.float32))
        else:
            fill_f32(self.bias_buf.ptr, E, self.seed, tensor_id(L, ROLE_BIAS), 0.0, self.bias_std)
        self.shared = [None, None, None]
        if Is:
            for q, role in enumerate((ROLE_SG, ROLE_SU, ROLE_SD)):
                b = self._dev(Is * d * 2)
                fill_bf16(b.ptr, Is * d, self.seed, tensor_id(L, role), 0.0, self.w_std)
                self.shared[q] = b
        self.norm = None
        if self.with_norm:
            self.norm = self._dev(d * 2)
            fill_bf16(self.norm.ptr, d, self.seed, tensor_id(L, ROLE_NORM), 1.0, 0.05)
        nd = self.distinct_experts or E
        nd = min(nd, E)
        proj = I * d
        eb = 3 * proj * 2
        ptrs = (C.c_void_p * (3 * E))()
        if not self.experts_on_host:
            self.experts = self._dev(nd * eb)
            for e in range(nd):
                base = self.experts.ptr + e * eb
                for q, role in enumerate((ROLE_EG, ROLE_EU, ROLE_ED)):
                    fill_bf16(base + q * proj * 2, proj, self.seed, tensor_id(L, role, e), 0.0, self.w_std)
        else:
            self.experts = capi.PinnedBuffer(nd * eb)
            self.buffers.append(self.experts)
            stage = self._dev(eb)
            for e in range(nd):
                for q, role in enumerate((ROLE_EG, ROLE_EU, ROLE_ED)):
                    fill_bf16(stage.ptr + q * proj * 2, proj, self.seed, tensor_id(L, role, e), 0.0, self.w_std)
                capi.call("hfmoe_memcpy_d2h", self.experts.ptr + e * eb, stage.ptr, eb)
        for e in range(E):
            base = self.experts.ptr + (e % nd) * eb
            for q in range(3):
                ptrs[3 * e + q] = base + q * proj * 2
        self._ptrs = ptrs
        self.weights = capi.LayerWeights(self.router.ptr, self.bias_buf.ptr,
                                         self.shared[0].ptr if Is else None,
                                         self.shared[1].ptr if Is else None,
                                         self.shared[2].ptr if Is else None,
                                         C.cast(ptrs, C.c_void_p),
                                         self.norm.ptr if self.norm else None,
                                         capi.EXPERTS_HOST_PINNED if self.experts_on_host else capi.EXPERTS_DEVICE, 0)
        self.layer_id = self.layer if self.register_as is None else self.register_as
        self.register()

    def register(self) -> None:
        """(Re-)register the layer, e.g. after its weights were changed in place."""
        capi.call("hfmoe_register_layer", self.layer_id, C.byref(self.weights))

    def _dev(self, nbytes: int) -> capi.DeviceBuffer:
        b = capi.DeviceBuffer(nbytes)
        self.buffers.append(b)
        return b

    def free(self) -> None:
        for b in self.buffers:
            b.free()
        self.buffers.clear()


def make_x_dev(T: int, hidden: int, seed: int, layer: int = 0) -> capi.DeviceBuffer:
    """Activations: BF16-valued ~N(0,1) held as FP32, [T, hidden], in HBM."""
    n = T * hidden
    tmp = capi.DeviceBuffer(n * 2)
    fill_bf16(tmp.ptr, n, seed, tensor_id(layer, ROLE_X), 0.0, 1.0)
    bits = tmp.download(np.uint16, n)
    tmp.free()
    x = (bits.astype(np.uint32) << 16).view(np.float32)
    return capi.DeviceBuffer.of(x)
