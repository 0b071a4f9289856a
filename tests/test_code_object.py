"""The library's own gfx950 code: no kernel spills vector registers or uses
scratch memory.  A spill in a streaming kernel turns into memory traffic
inside its inner loop (one such build of the prefill gate/up GEMM ran 35 %
slower with 60 scratch instructions), so the check reads every kernel's
metadata (`.vgpr_spill_count`, `.private_segment_fixed_size`) from the code
objects bundled into libhfmoe.so, one bundle per source file."""
import os
import re
import struct
import subprocess

import pytest

from hummingflight_amd import capi

READELF = "/opt/rocm/llvm/bin/llvm-readelf"
MAGIC = b"__CLANG_OFFLOAD_BUNDLE__"


def gfx950_objects(tmp_path):
    fb = tmp_path / "fatbin.bin"
    subprocess.run(["objcopy", "-O", "binary", "--only-section=.hip_fatbin", capi.LIB_PATH, str(fb)], check=True)
    data = fb.read_bytes()
    objs, pos = [], 0
    while (i := data.find(MAGIC, pos)) >= 0:
        (count,) = struct.unpack_from("<Q", data, i + len(MAGIC))
        p = i + len(MAGIC) + 8
        for _ in range(count):
            off, size, tlen = struct.unpack_from("<QQQ", data, p)
            p += 24
            triple = data[p:p + tlen].decode()
            p += tlen
            if triple.endswith("gfx950"):
                objs.append(data[i + off:i + off + size])
        pos = i + len(MAGIC)
    return objs


def kernel_metadata(tmp_path):
    kernels = {}
    for n, co in enumerate(gfx950_objects(tmp_path)):
        f = tmp_path / f"co{n}.o"
        f.write_bytes(co)
        notes = subprocess.run([READELF, "--notes", str(f)], capture_output=True, text=True, check=True).stdout
        name = None
        for line in notes.splitlines():
            m = re.match(r"\s+\.(name|vgpr_spill_count|private_segment_fixed_size|vgpr_count):\s+(\S+)", line)
            if not m:
                continue
            if m.group(1) == "name":
                name = m.group(2)
                kernels[name] = {}
            elif name:
                kernels[name][m.group(1)] = int(m.group(2))
    return kernels


@pytest.mark.skipif(not os.path.exists(READELF), reason="llvm-readelf of the ROCm toolchain not installed")
def test_no_kernel_spills(tmp_path):
    kernels = kernel_metadata(tmp_path)
    # every source file's device code, the MoE GEMMs among them
    assert len(kernels) > 50
    assert any("grouped_gemm_wide_kernel" in k for k in kernels)
    assert any("gateup_t1_kernel" in k for k in kernels)
    bad = {k: v for k, v in kernels.items() if v.get("vgpr_spill_count", 0) or v.get("private_segment_fixed_size", 0)}
    assert not bad, bad
