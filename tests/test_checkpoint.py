"""Checkpoint parsing (safetensors shards + index), on the CPU.

The validation cases restate the reference's own strict-safetensors self-test
(src/self_test.cpp:536-690) through hfmoe_checkpoint_open, with the checkpoint
loader's options (strictStOpts, weight_index.cpp:20-27: BF16 only, F32 for the
router correction bias).  Loading a layer onto the GPU is tested in
test_gpu_checkpoint.py.
"""
import ctypes as C
import json

import numpy as np
import pytest

from hummingflight_amd import capi
from safetensors_io import header_one, raw_shard, tensor_entry, write_shard


def open_ck(path):
    ck = C.c_void_p()
    rc = capi.load().hfmoe_checkpoint_open(str(path).encode(), C.byref(ck))
    return rc, ck


def stats(ck):
    s = capi.SafetensorsStats()
    capi.call("hfmoe_checkpoint_stats", ck, C.byref(s))
    return s.as_dict()


def info(ck, name):
    t = capi.TensorInfo()
    rc = capi.load().hfmoe_checkpoint_tensor(ck, name.encode(), C.byref(t))
    return rc, t


def one(tmp_path, name, data: bytes):
    p = tmp_path / name
    p.write_bytes(data)
    rc, ck = open_ck(p)
    return rc, ck


def close(ck):
    capi.load().hfmoe_checkpoint_close(ck)


def test_valid_bf16_tensor(tmp_path):  # self_test.cpp case (1)
    rc, ck = one(tmp_path, "valid.safetensors", raw_shard(header_one(tensor_entry("BF16", [2, 3], 0, 12)), 12))
    assert rc == capi.OK
    s = stats(ck)
    assert (s["total"], s["accepted"], s["rejected"], s["shards"]) == (1, 1, 0, 1)
    rc, t = info(ck, "w")
    assert rc == capi.OK and t.dtype == b"BF16" and t.ndim == 2 and list(t.shape[:2]) == [2, 3]
    assert t.nbytes == 12 and t.file_offset % 8 == 0
    close(ck)


CASES = [
    # (what, header entry, name, payload, counter that must read 1)  -- self_test.cpp cases
    ("f32_off_list", tensor_entry("F32", [2], 0, 8), "w", 8, "dtype_rejected"),                       # (2)
    ("byte_mismatch", tensor_entry("BF16", [3], 0, 12), "w", 12, "byte_mismatch_rejected"),          # (3)
    ("out_of_bounds", tensor_entry("BF16", [2], 0, 100), "w", 12, "bounds_rejected"),                # (4)
    ("integer_dtype", tensor_entry("I8", [2], 0, 2), "w", 8, "dtype_rejected"),                      # (7)
    ("unaligned_data", tensor_entry("BF16", [2], 6, 10), "w", 10, "alignment_rejected"),             # (8)
    ("f32_other_name", tensor_entry("F32", [256], 0, 1024), "model.layers.4.mlp.gate.weight2", 1024,
     "dtype_rejected"),                                                                                # (10)
    ("unknown_dtype", tensor_entry("Q4", [2], 0, 8), "w", 8, "dtype_rejected"),
    ("negative_dim", tensor_entry("BF16", [-2], 0, 8), "w", 8, "shape_rejected"),
    ("fractional_dim", tensor_entry("BF16", [1.5], 0, 8), "w", 8, "shape_rejected"),
    ("scalar_shape", tensor_entry("BF16", [], 0, 2), "w", 8, "shape_rejected"),
    ("empty_span", tensor_entry("BF16", [0], 0, 0), "w", 8, "bounds_rejected"),
    # Not in the reference's list: inputs whose arithmetic would wrap 64 bits.
    # 20 * 5581 * 384773 * 429509837 = 2^64 + 4, so a wrapping element count
    # would match the 8-byte span.
    ("shape_product_wraps", tensor_entry("BF16", [20, 5581, 384773, 429509837], 0, 8), "w", 8, "shape_rejected"),
    ("offsets_past_the_file", tensor_entry("BF16", [4], 1e30, 1e30 + 8), "w", 8, "bounds_rejected"),
]


@pytest.mark.parametrize("what,entry,name,payload,counter", CASES, ids=[c[0] for c in CASES])
def test_rejected_tensor_counted(tmp_path, what, entry, name, payload, counter):
    rc, ck = one(tmp_path, what + ".safetensors", raw_shard(header_one(entry, name), payload))
    assert rc == capi.OK  # the shard opens; the tensor is counted and left out
    s = stats(ck)
    assert (s["total"], s["accepted"], s["rejected"], s[counter]) == (1, 0, 1, 1), s
    assert info(ck, name)[0] == capi.ERR_NOT_REGISTERED
    close(ck)


def test_router_bias_f32_allowed(tmp_path):  # self_test.cpp case (9), allow-list form
    name = "model.layers.4.mlp.gate.e_score_correction_bias"
    rc, ck = one(tmp_path, "bias.safetensors", raw_shard(header_one(tensor_entry("F32", [256], 0, 1024), name), 1024))
    assert rc == capi.OK
    s = stats(ck)
    assert (s["accepted"], s["f32_allowed_accepted"], s["dtype_rejected"]) == (1, 1, 0)
    close(ck)


def test_duplicate_name_second_rejected(tmp_path):
    # Two entries of one name in a header: the first is kept, the second counted.
    e = json.dumps(tensor_entry("BF16", [2], 0, 4))
    hdr = '{"w": ' + e + ', "w": ' + json.dumps(tensor_entry("BF16", [2], 8, 12)) + '}'
    rc, ck = one(tmp_path, "dup.safetensors", raw_shard(hdr, 16))
    s = stats(ck)
    assert (s["total"], s["accepted"], s["duplicate_rejected"]) == (2, 1, 1)
    rc, t = info(ck, "w")
    assert rc == capi.OK and t.file_offset == len(raw_shard(hdr, 0))  # the first entry's data (begin 0)
    close(ck)


def test_offsets_near_2_pow_64_rejected(tmp_path):
    # With a header of 4 KB or more, data start + end would wrap past 2^64 to a
    # place inside the file for these offsets (2048 bytes apart, both exact
    # doubles): the span must be rejected as out of bounds, not accepted.
    entry = tensor_entry("BF16", [1024], 2**64 - 4096, 2**64 - 2048)
    hdr = json.dumps({"__metadata__": {"pad": "x" * 4200}, "w": entry})
    rc, ck = one(tmp_path, "wrap.safetensors", raw_shard(hdr, 64))
    assert rc == capi.OK
    s = stats(ck)
    assert (s["total"], s["accepted"], s["bounds_rejected"]) == (1, 0, 1), s
    close(ck)


def test_header_length_near_2_pow_64_fails(tmp_path):
    rc, ck = one(tmp_path, "huge.safetensors", (2**64 - 8).to_bytes(8, "little") + b"{}" + b" " * 14)
    assert rc == capi.ERR_INVALID_ARGUMENT
    assert b"header" in capi.load().hfmoe_last_error()


def unaligned_header():
    h = header_one(tensor_entry("BF16", [2], 0, 4))
    return raw_shard(h + " " if len(h) % 8 == 0 else h, 4, align=False)


@pytest.mark.parametrize("what,data", [
    ("not_json", raw_shard("<not json at all", 16)),                    # (5)
    ("json_array", raw_shard("[1, 2, 3]", 16)),
    ("unaligned_header", unaligned_header()),                           # (6)
    ("header_past_end", (1 << 20).to_bytes(8, "little") + b" " * 16),
])
def test_unreadable_shard_fails(tmp_path, what, data):
    rc, ck = one(tmp_path, what + ".safetensors", data)
    assert rc == capi.ERR_INVALID_ARGUMENT
    assert b"header" in capi.load().hfmoe_last_error()


def test_index_picks_each_tensors_shard(tmp_path):
    a = np.arange(8, dtype=np.uint16)
    b = np.arange(16, dtype=np.uint16)
    # Both shards hold "x"; the index assigns it to shard 2, "y" to shard 1.
    write_shard(tmp_path / "model-00001-of-00002.safetensors", {"y": (a, [8]), "x": (a, [8])})
    write_shard(tmp_path / "model-00002-of-00002.safetensors", {"pad": (b, [16]), "x": (a, [8])})
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps(
        {"metadata": {}, "weight_map": {"x": "model-00002-of-00002.safetensors",
                                        "y": "model-00001-of-00002.safetensors"}}))
    rc, ck = open_ck(tmp_path)
    assert rc == capi.OK
    s = stats(ck)
    assert (s["shards"], s["total"], s["accepted"]) == (2, 4, 4)
    rc, tx = info(ck, "x")
    rc2, ty = info(ck, "y")
    assert rc == rc2 == capi.OK
    hdr2 = (tmp_path / "model-00002-of-00002.safetensors").read_bytes()
    n2 = int.from_bytes(hdr2[:8], "little")
    assert tx.file_offset == 8 + n2 + 32  # after shard 2's 32-byte "pad"
    assert info(ck, "pad")[0] == capi.ERR_NOT_REGISTERED  # not in the index
    close(ck)


def test_directory_without_index_takes_first_shard(tmp_path):
    a = np.arange(4, dtype=np.uint16)
    write_shard(tmp_path / "a.safetensors", {"x": (a, [4])})
    write_shard(tmp_path / "b.safetensors", {"pad": (a, [4]), "x": (a, [4])})
    rc, ck = open_ck(tmp_path)
    assert rc == capi.OK
    hdr = (tmp_path / "a.safetensors").read_bytes()
    rc, t = info(ck, "x")
    assert t.file_offset == 8 + int.from_bytes(hdr[:8], "little")
    assert stats(ck)["accepted"] == 3
    close(ck)


def test_missing_path_and_load_without_device_fail(tmp_path):
    rc, _ = open_ck(tmp_path / "nothing_here")
    assert rc == capi.ERR_INVALID_ARGUMENT
    a = np.zeros(4, np.uint16)
    write_shard(tmp_path / "m.safetensors", {"x": (a, [4])})
    rc, ck = open_ck(tmp_path / "m.safetensors")
    assert rc == capi.OK
    L = capi.load()
    if not L.hfmoe_available():
        assert L.hfmoe_checkpoint_load_moe_layer(ck, 0, capi.EXPERTS_DEVICE) == capi.ERR_NOT_INITIALIZED
    close(ck)
