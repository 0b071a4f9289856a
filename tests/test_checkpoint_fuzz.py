"""Checkpoint parser under mutated shards, on the CPU.

Seeded byte-level mutations of a valid shard's header (random bytes, JSON
tokens spliced in, header lengths near the limits, truncations, deletions) go
through hfmoe_checkpoint_open / _stats / _tensor / _close.  The parser must
neither crash nor accept a tensor whose data lies outside its file: every
tensor it reports has file_offset + nbytes within the shard, nbytes equal to
its shape times its dtype size, and an 8-byte-aligned start (the strict-mode
rules of safetensors.cpp:60-240 that checkpoint.cpp restates).  (Run against an
AddressSanitizer build of the library's host code, the same mutations report
no invalid access.)
"""
import ctypes as C
import os
import random
import struct

import numpy as np
import pytest

from hummingflight_amd import capi
from safetensors_io import write_shard

NAMES = (b"model.layers.0.mlp.gate.weight", b"model.layers.0.mlp.gate.e_score_correction_bias", b"x.y", b"")
TOKENS = (b'"', b"{", b"}", b"[", b"]", b":", b",", b"-1", b"1e309", b"18446744073709551615", b'"BF16"',
          b'"F32"', b"null", b"true", b'"shape"', b'"data_offsets"', b'"dtype"', b"\\u0000", b"\\", b"9" * 30,
          b" ", b"0")
SIZES = {b"BF16": 2, b"F32": 4}


def mutate(raw: bytearray, n: int, rng: random.Random) -> bytes:
    m = bytearray(raw)
    for _ in range(rng.randint(1, 6)):
        if len(m) <= 9:
            break
        hi = min(8 + n, len(m))
        r = rng.random()
        if r < 0.4:
            m[rng.randrange(8, hi)] = rng.randrange(256)
        elif r < 0.7:
            i = rng.randrange(8, hi)
            t = rng.choice(TOKENS)
            m[i:i + len(t)] = t
        elif r < 0.8:
            m[:8] = struct.pack("<Q", rng.choice([0, 7, 8, n - 8, n + 8, len(m), len(m) + 8, 2**63, 2**64 - 8]))
        elif r < 0.9:
            del m[rng.randrange(8, len(m)):]
        else:
            i = rng.randrange(8, hi)
            del m[i:i + rng.randint(1, 20)]
    return bytes(m)


@pytest.mark.parametrize("seed", [1, 2, 3])
def test_mutated_shards(tmp_path, seed):
    lib = capi.load()
    base = tmp_path / "base.safetensors"
    w = np.arange(64, dtype=np.uint16)
    write_shard(base, {NAMES[0].decode(): (w, [8, 8]),
                       NAMES[1].decode(): (np.zeros(8, np.float32).view(np.uint16), [8]),
                       NAMES[2].decode(): (w[:16], [4, 4])})
    raw = bytearray(base.read_bytes())
    n = struct.unpack("<Q", raw[:8])[0]
    rng = random.Random(seed)
    path = tmp_path / "m.safetensors"
    opened = accepted = 0
    for _ in range(3000):
        data = mutate(raw, n, rng)
        path.write_bytes(data)
        ck = C.c_void_p()
        if lib.hfmoe_checkpoint_open(str(path).encode(), C.byref(ck)) != 0:
            continue
        opened += 1
        s = capi.SafetensorsStats()
        assert lib.hfmoe_checkpoint_stats(ck, C.byref(s)) == 0
        for name in NAMES:
            t = capi.TensorInfo()
            if lib.hfmoe_checkpoint_tensor(ck, name, C.byref(t)) != 0:
                continue
            accepted += 1
            dt = t.dtype.split(b"\0")[0]
            assert dt in SIZES, dt
            assert 1 <= t.ndim <= 8
            elems = 1
            for d in t.shape[:t.ndim]:
                assert d >= 0
                elems *= d
            assert t.nbytes == elems * SIZES[dt] and t.nbytes > 0
            assert t.file_offset % 8 == 0
            assert t.file_offset + t.nbytes <= len(data), (name, t.file_offset, t.nbytes, len(data))
        lib.hfmoe_checkpoint_close(ck)
    # the mutations leave some shards valid, so acceptance is exercised too
    assert opened > 0 and accepted > 0
