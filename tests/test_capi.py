"""The C-ABI library loads and exports exactly what include/hfmoe.h declares.

CPU-only: no compute call is made without a GPU.
"""
import ctypes as C
import os
import re
import subprocess

import pytest

from hummingflight_amd import capi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_functions():
    txt = open(os.path.join(ROOT, "include", "hfmoe.h")).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b(hfmoe_[a-z0-9_]+)\s*\(", txt)))


def test_library_built_and_loads():
    assert os.path.exists(capi.LIB_PATH), "libhfmoe.so missing: run __graft_entry__.build()"
    capi.load()


def test_exports_match_header():
    declared = header_functions()
    assert declared, "no declarations parsed"
    assert sorted(capi.EXPORTS) == declared
    out = subprocess.run(["nm", "-D", "--defined-only", capi.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r"\bT (hfmoe_[a-z0-9_]+)$", out, flags=re.M))
    missing = [f for f in declared if f not in exported]
    assert not missing, missing
    L = capi.load()
    for f in declared:
        assert hasattr(L, f)


def test_gfx950_code_object_only(tmp_path):
    # The device code bundle of our own build targets gfx950 and nothing else.
    fb = tmp_path / "fatbin.bin"
    subprocess.run(["objcopy", "-O", "binary", "--only-section=.hip_fatbin", capi.LIB_PATH, str(fb)],
                   check=True)
    targets = set(re.findall(rb"hipv4-amdgcn-amd-amdhsa--(gfx[0-9a-z]+)", fb.read_bytes()))
    assert targets == {b"gfx950"}


def test_struct_layouts_match_header():
    # The ctypes mirrors must match the C structs byte for byte.
    assert C.sizeof(capi.Config) == 4 * 10 + 8 + 4 * 2
    assert C.sizeof(capi.LayerWeights) == 8 * 7 + 4 * 2
    assert C.sizeof(capi.RouteDebug) == 8 * 5
    assert C.sizeof(capi.KernelStat) == 32 + 8 + 8
    assert C.sizeof(capi.StreamOptions) == 4 * 8
    assert C.sizeof(capi.DenseWeights) == 8 * 4 + 4 * 2
    # The stream counters keep their first published layout: eight uint64
    # counters, then slots and pinned (the latter in the former reserved field).
    assert C.sizeof(capi.StreamCounters) == 8 * 8 + 4 * 2
    assert capi.StreamCounters.slots.offset == 64 and capi.StreamCounters.pinned.offset == 68


def test_calls_before_init_fail_loudly():
    L = capi.load()
    if L.hfmoe_available():
        pytest.skip("library already initialised in this process")
    cfg = capi.Config(2048, 1024, 64, 8, 1, 1, 1, 1, 2.5, 1e-5, 0, 1, 0)
    assert L.hfmoe_configure(C.byref(cfg)) == capi.ERR_NOT_INITIALIZED
    assert b"hfmoe_init" in L.hfmoe_last_error()
    assert L.hfmoe_moe_forward(0, None, 1, None, None) == capi.ERR_NOT_INITIALIZED
    assert L.hfmoe_expert_stage(0, 0, None, 64, 32) != capi.OK
    assert L.hfmoe_device_memory_mb() == 0


def test_engine_shim_builds_and_fails_cleanly_without_device():
    """The C++ caller compiles against include/hfmoe.h, links libhfmoe.so and,
    with no usable device, stops with the start-up error (exit code 2)."""
    shim_dir = os.path.join(ROOT, "tests", "engine_shim")
    subprocess.run(["make", "-s", "-C", shim_dir], check=True)
    r = subprocess.run([os.path.join(shim_dir, "engine_shim"), "1", "1"], capture_output=True, text=True,
                       timeout=120)
    if r.returncode == 2:
        assert "no usable device" in r.stderr
    else:  # a machine with a GPU: one line of hidden-size hex words
        assert r.returncode == 0, r.stderr
        assert len(r.stdout.split()) == 2048
