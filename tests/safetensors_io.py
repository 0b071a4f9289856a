"""Writes safetensors shards for the checkpoint tests (test helper).

Format: u64 little-endian header length, a JSON header padded with spaces to a
multiple of 8, then the data area; each tensor's data_offsets are relative to
the data area and 8-byte aligned.
"""
import json
import struct

import numpy as np

DTYPES = {np.dtype(np.uint16): "BF16", np.dtype(np.float32): "F32"}


def raw_shard(header: str, payload: int, align: bool = True) -> bytes:
    """Header text as given (padded to 8 unless align=False) + payload zero bytes."""
    h = header.encode()
    if align and len(h) % 8:
        h += b" " * (8 - len(h) % 8)
    return struct.pack("<Q", len(h)) + h + bytes(payload)


def tensor_entry(dtype, shape, begin, end):
    return {"dtype": dtype, "shape": list(shape), "data_offsets": [begin, end]}


def header_one(entry, name="w") -> str:
    return json.dumps({"__metadata__": {"format": "pt"}, name: entry})


def write_shard(path, tensors: dict) -> None:
    """tensors: name -> (numpy array, shape); uint16 arrays are BF16, float32 arrays F32."""
    entries, blobs, off = {}, [], 0
    for name, (arr, shape) in tensors.items():
        a = np.ascontiguousarray(arr)
        dt = DTYPES[a.dtype]
        b = a.tobytes()
        entries[name] = tensor_entry(dt, shape, off, off + len(b))
        pad = (-len(b)) % 8
        blobs.append(b + bytes(pad))
        off += len(b) + pad
    h = json.dumps({"__metadata__": {"format": "pt"}, **entries}).encode()
    h += b" " * ((-len(h)) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)))
        f.write(h)
        for b in blobs:
            f.write(b)


def moe_layer_tensors(ref, layer: int, with_norm=None) -> dict:
    """The GLM tensor names of one MoE layer, filled from an oracle SyntheticLayer."""
    s = ref.spec
    p = f"model.layers.{layer}.mlp."
    t = {p + "gate.weight": (ref.router, [s.n_experts, s.hidden]),
         p + "gate.e_score_correction_bias": (ref.bias, [s.n_experts])}
    if ref.sg is not None:
        Is = s.n_shared * s.inter
        t[p + "shared_experts.gate_proj.weight"] = (ref.sg, [Is, s.hidden])
        t[p + "shared_experts.up_proj.weight"] = (ref.su, [Is, s.hidden])
        t[p + "shared_experts.down_proj.weight"] = (ref.sd, [s.hidden, Is])
    for e in range(s.n_experts):
        g, u, d = ref.expert(e)
        t[p + f"experts.{e}.gate_proj.weight"] = (g, [s.inter, s.hidden])
        t[p + f"experts.{e}.up_proj.weight"] = (u, [s.inter, s.hidden])
        t[p + f"experts.{e}.down_proj.weight"] = (d, [s.hidden, s.inter])
    if with_norm is not None:
        t[f"model.layers.{layer}.post_attention_layernorm.weight"] = (with_norm, [s.hidden])
    return t
