"""MoE-block benchmark on one MI355X.

Default workload: the full-shape MoE layer at decode, T=1 token (d=6144,
256 routed experts + 1 shared, SwiGLU I=2048, router 8 groups keep 4, top-8,
weights BF16 ~N(0,0.02) resident in HBM).  One step = one MoE-layer forward
over one token; inputs are already in HBM when the timed region starts.

Prints one JSON line: tokens/s as `value`, the dominant kernel's achieved HBM
bandwidth against the 8 TB/s peak as `roofline` (durations from hipEvents the
library records on its launch stream during the timed steps), and the
reference CPU path timed on this host as `cpu_baseline`.

    python bench.py [--steps K] [--warmup W] [--workload decode|batched|prefill|streamed]
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

from hummingflight_amd import capi, synth  # noqa: E402

METRIC = "MoE-layer decode tokens/s + achieved HBM GB/s (% peak) at d=6144, 256e top-8"
HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0

FULL = dict(hidden=6144, inter=2048, n_experts=256, top_k=8, n_group=8, topk_group=4, n_shared=1)


def algorithmic_bytes_t1(shape: synth.LayerShape) -> dict[str, int]:
    """Bytes each decode kernel must move at least once (T = 1)."""
    d, I, E = shape.hidden, shape.inter, shape.n_experts
    ns = shape.top_k + shape.n_shared
    router = E * d * 2 + d * 4 + E * 4
    select = E * 4 + E * 4 + shape.top_k * 8
    gateup = ns * 2 * I * d * 2 + d * 4 + ns * I * 4
    down = ns * d * I * 2 + ns * I * 4 + d * 4
    return {"router": router, "select": select, "expert_gateup": gateup, "expert_down": down,
            "layer": ns * 3 * I * d * 2 + E * d * 2 + E * 4 + d * 4 + d * 4}


def cpu_baseline_decode(shape: synth.LayerShape, seed: int, seconds: float) -> dict:
    """The reference's own moeLayer (oracle/_ref) on this host, else the C restatement."""
    import oracle as O
    spec = O.LayerSpec(hidden=shape.hidden, inter=shape.inter, n_experts=shape.n_experts,
                       top_k=shape.top_k, n_group=1, topk_group=1, n_shared=shape.n_shared, seed=seed)
    layer = O.SyntheticLayer(spec)
    x = O.make_x(1, shape.hidden, seed)[0].copy()
    idx, _ = layer.route(layer.logits(x))  # the reference routes flat (no groups)
    W, keep = layer.weights(idx)
    out = np.zeros(shape.hidden, np.float32)
    cores = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    R = O.ref()
    if R is not None:
        sec = C.c_double()
        # One call to size the sample, then a bounded timed sample.
        rc = R.ref_moe_layer_timed(b"/tmp/hfmoe_bench_ref_layer.bin", C.byref(spec.cfg()), C.byref(W),
                                   x.ctypes.data, out.ctypes.data, 1, C.byref(sec))
        if rc != 0:
            raise RuntimeError(f"reference harness failed rc={rc}")
        iters = max(3, min(500, int(seconds / max(sec.value, 1e-6))))
        rc = R.ref_moe_layer_timed(b"/tmp/hfmoe_bench_ref_layer.bin", C.byref(spec.cfg()), C.byref(W),
                                   x.ctypes.data, out.ctypes.data, iters, C.byref(sec))
        if rc != 0:
            raise RuntimeError(f"reference harness failed rc={rc}")
        kind, per_call = "reference", sec.value
    else:
        lib = O.lib()
        t0 = time.perf_counter()
        lib.orc_moe_layer(C.byref(spec.cfg()), C.byref(W), x.ctypes.data, out.ctypes.data, None, None, None)
        first = time.perf_counter() - t0
        iters = max(3, min(500, int(seconds / max(first, 1e-6))))
        t0 = time.perf_counter()
        for _ in range(iters):
            lib.orc_moe_layer(C.byref(spec.cfg()), C.byref(W), x.ctypes.data, out.ctypes.data, None, None, None)
        kind, per_call = "port", (time.perf_counter() - t0) / iters
    return {"value": 1.0 / per_call, "unit": "tokens/s", "cores": cores, "kind": kind,
            "sample": f"{iters} moeLayer calls, T=1, d={shape.hidden}, {shape.n_experts} experts top-{shape.top_k} "
                      f"+ {shape.n_shared} shared, flat routing, OpenMP threads={cores}; "
                      f"{per_call * 1e3:.2f} ms/call"}


def time_steps(step, steps: int, warmup: int) -> float:
    for _ in range(warmup):
        step()
    capi.call("hfmoe_synchronize")
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    capi.call("hfmoe_synchronize")
    return (time.perf_counter() - t0) / steps


def run_decode(args) -> dict:
    shape = synth.LayerShape(**FULL)
    capi.call("hfmoe_configure", shape.config(max_tokens=1))
    layer = synth.DeviceLayer(shape, layer=0, seed=args.seed, experts_on_host=False)
    x = synth.make_x_dev(1, shape.hidden, seed=args.seed)
    out = capi.DeviceBuffer(shape.hidden * 4)
    fwd = capi.load().hfmoe_moe_forward

    def step():
        rc = fwd(0, x.ptr, 1, out.ptr, None)
        if rc:
            capi.check(rc)

    sec = time_steps(step, args.steps, args.warmup)
    # Same steps again with per-kernel hipEvents on the launch stream.
    capi.call("hfmoe_profile_reset")
    capi.call("hfmoe_profile_enable", 1)
    sec_prof = time_steps(step, args.steps, 0)
    capi.call("hfmoe_profile_enable", 0)
    prof = capi.profile_read()
    algo = algorithmic_bytes_t1(shape)
    kernels = {}
    for name, (n, ms) in prof.items():
        avg_us = ms * 1e3 / max(n, 1)
        gbs = algo.get(name, 0) / (avg_us * 1e-6) / 1e9 if name in algo else None
        kernels[name] = {"launches": n, "avg_us": round(avg_us, 3),
                         "algorithmic_bytes": algo.get(name), "gbs": None if gbs is None else round(gbs, 1)}
    dom = kernels["expert_gateup"]
    layer_gbs = algo["layer"] / sec / 1e9
    res = {
        "value": 1.0 / sec,
        "ms_per_step": sec * 1e3,
        "config": {"workload": "moe_layer_decode", "tokens": 1, "hidden": shape.hidden,
                   "moe_intermediate": shape.inter, "routed_experts": shape.n_experts,
                   "shared_experts": shape.n_shared, "top_k": shape.top_k,
                   "n_group": shape.n_group, "topk_group": shape.topk_group,
                   "weights": "HBM-resident BF16 ~N(0,0.02)"},
        "roofline": {"bound": "hbm", "kernel": "expert_gateup", "achieved": round(dom["gbs"], 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(dom["gbs"] / HBM_PEAK_GBS, 4),
                     "traffic": traffic_from_profile("expert_gateup")},
        "layer_hbm": {"algorithmic_bytes": algo["layer"], "achieved_gbs": round(layer_gbs, 1),
                      "frac": round(layer_gbs / HBM_PEAK_GBS, 4)},
        "ms_per_step_with_kernel_events": sec_prof * 1e3,
        "kernels": kernels,
    }
    if not args.no_cpu_baseline:
        res["cpu_baseline"] = cpu_baseline_decode(shape, args.seed, args.cpu_seconds)
    layer.free()
    x.free()
    out.free()
    return res


def run_copy(args) -> None:
    """Counter calibration: 4 GiB device-to-device copies (HIP's own copy kernel)."""
    n = 4 << 30
    a = capi.DeviceBuffer(n)
    b = capi.DeviceBuffer(n)
    capi.call("hfmoe_memset", a.ptr, 1, n)
    t0 = time.perf_counter()
    for _ in range(max(args.steps, 1)):
        capi.call("hfmoe_memcpy_d2d", b.ptr, a.ptr, n)
    dt = (time.perf_counter() - t0) / max(args.steps, 1)
    print(json.dumps({"workload": "copy_calibration", "bytes_read_per_copy": n, "bytes_written_per_copy": n,
                      "copies": args.steps, "gbs_read_plus_write": round(2 * n / dt / 1e9, 1)}), flush=True)
    a.free()
    b.free()


def traffic_from_profile(kernel: str) -> int | None:
    """HBM bytes per launch of `kernel` from the committed counter summary."""
    path = os.path.join(ROOT, "profiles", "decode_t1_hbm_traffic.md")
    if not os.path.exists(path):
        return None
    for line in open(path):
        if line.startswith("traffic_bytes_per_launch:"):
            for item in line.split(":", 1)[1].split():
                name, _, val = item.partition("=")
                if name == kernel:
                    return int(val)
    return None


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="decode", choices=["decode", "copy"])
    ap.add_argument("--seed", type=int, default=2026)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: --gpus {args.gpus} is not supported "
              f"(the MoE block runs on a single MI355X; sharding is design-only)", file=sys.stderr)
        return 2
    capi.call("hfmoe_init", 0)
    if args.workload == "copy":
        run_copy(args)
        capi.load().hfmoe_shutdown()
        return 0
    res = run_decode(args)
    line = {"metric": METRIC, "value": round(res.pop("value"), 2), "unit": "tokens/s", "n_gpus": 1,
            "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(res.pop("ms_per_step"), 5),
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
            "data": "synthetic", **res}
    print(json.dumps(line), flush=True)
    capi.load().hfmoe_shutdown()
    return 0


if __name__ == "__main__":
    sys.exit(main())
