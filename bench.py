"""MoE-block benchmark on one MI355X.

Default workload (`decode`): the full-shape MoE layer at decode, T=1 token
(d=6144, 256 routed experts + 1 shared, SwiGLU I=2048, router 8 groups keep 4,
top-8, weights BF16 ~N(0,0.02) resident in HBM).  One step = one MoE-layer
forward over one token; inputs are already in HBM when the timed region starts.

Other workloads of the same layer:
  batched   T=64 tokens, correction bias calibrated for Zipf(1.1) expert
            popularity (tests/golden/zipf_bias_e256.json); HBM-bound
  prefill   T=4096 tokens, near-uniform routing (bias ~N(0,0.001)); HBM
            roofline, MFMA fraction beside it
  streamed  8 chained layers (RMSNorm + MoE + residual), T=1, routed experts in
            pinned host RAM, the selected ones copied to HBM on a side stream
  streamed_cached  the same with an HBM expert cache and next-layer copy-ahead
  streamed_prefill one layer, T=4096, routed experts in pinned host RAM: the
            batch's distinct experts cross PCIe a wave at a time
  dense     a dense-MLP layer (intermediate 12288), T=1 or --dense-tokens
  lm_head   final norm + LM head (vocab 154880) + greedy argmax, T=1
  load      a MoE layer from a safetensors shard into HBM (GB/s)
  plugin    the per-expert plugin calls: stage an expert, expert FFN with
            host buffers (calls/s)
  copy      counter calibration (4 GiB device-to-device copies)

Prints one JSON line: tokens/s as `value`, the dominant kernel's achieved rate
against its roofline as `roofline` (durations from the kernels' own dispatch
timestamps, recorded on the launch stream during a second pass of the timed
steps), and the reference CPU path timed on this host as `cpu_baseline`.  The
default (decode) line also carries `configs`: the batched, prefill (BF16-valued
and FP32 activations) and streamed-chain workloads, each timed in the same run
with steps of its own (--no-configs leaves them out).

    python bench.py [--steps K] [--warmup W]
                    [--workload decode|batched|prefill|streamed|streamed_cached|streamed_prefill|dense|lm_head|load|plugin|copy]
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import subprocess
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


def host_cpu() -> dict:
    """CPU model, sockets and cores of this host (lscpu), and the CPU share the bench uses."""
    info = {"model": None, "sockets": None, "cores_per_socket": None, "threads_per_core": None}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            key, _, val = line.partition(":")
            key, val = key.strip(), val.strip()
            if key == "Model name":
                info["model"] = val
            elif key == "Socket(s)":
                info["sockets"] = int(val)
            elif key == "Core(s) per socket":
                info["cores_per_socket"] = int(val)
            elif key == "Thread(s) per core":
                info["threads_per_core"] = int(val)
    except (OSError, ValueError, subprocess.SubprocessError):
        pass
    if info["sockets"] and info["cores_per_socket"]:
        info["physical_cores"] = info["sockets"] * info["cores_per_socket"]
    info["logical_cpus"] = os.cpu_count()
    try:
        info["cpus_allowed"] = len(os.sched_getaffinity(0))
    except OSError:
        info["cpus_allowed"] = None
    return info


def set_omp_threads(n: int) -> None:
    """Thread count of the OpenMP parallel regions started from this thread (both CPU libraries)."""
    C.CDLL("libgomp.so.1").omp_set_num_threads(int(n))


def cpu_baseline_decode(shape: synth.LayerShape, seed: int, seconds: float) -> dict:
    """The reference CPU MoE layer on this host, T = 1, full shape, weights in host RAM.

    `value`: the reference's own moeLayer (oracle/_ref, compiled from its
    sources with its Linux flags: the scalar serial GEMV) on the host's CPU
    share; beside it, `variants`: the same on one core, the restated MSVC
    AVX2+FMA GEMV build (the one behind the reference's published numbers) on
    the CPU share and on one core, and both builds with the scheduler's 72 MB
    copy of every used expert (scheduler.cpp:646-660).  The restatement routes
    with the GPU's 8-group rule; the reference routes flat (it has no group
    rule): the same 8 + 1 experts of work either way.
    """
    import oracle as O
    share = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or min(16, os.cpu_count() or 1)
    spec_flat = O.LayerSpec(hidden=shape.hidden, inter=shape.inter, n_experts=shape.n_experts,
                            top_k=shape.top_k, n_group=1, topk_group=1, n_shared=shape.n_shared, seed=seed)
    spec_grp = O.LayerSpec(hidden=shape.hidden, inter=shape.inter, n_experts=shape.n_experts,
                           top_k=shape.top_k, n_group=shape.n_group, topk_group=shape.topk_group,
                           n_shared=shape.n_shared, seed=seed)
    x = O.make_x(1, shape.hidden, seed)[0].copy()
    out = np.zeros(shape.hidden, np.float32)
    flat, grp = O.SyntheticLayer(spec_flat), O.SyntheticLayer(spec_grp)
    Wf, keep_f = flat.weights(flat.route(flat.logits(x))[0])
    Wg, keep_g = grp.weights(grp.route(grp.logits(x))[0])
    scratch = np.empty(3 * shape.hidden * shape.inter, np.uint16)

    def sample(call) -> tuple[float, int]:
        """(seconds per call, calls) of a bounded sample; `call(n)` runs n calls, returns seconds in all."""
        first = call(1)  # warm: pages in the weights, sizes the sample
        iters = max(2, min(500, int(seconds / max(first, 1e-6))))
        return call(iters) / iters, iters

    R = O.ref()

    def ref_call(n: int) -> float:
        sec = C.c_double()
        rc = R.ref_moe_layer_timed(b"/tmp/hfmoe_bench_ref_layer.bin", C.byref(spec_flat.cfg()), C.byref(Wf),
                                   x.ctypes.data, out.ctypes.data, n, C.byref(sec))
        if rc != 0:
            raise RuntimeError(f"reference harness failed rc={rc}")
        return sec.value * n  # the harness reports seconds per call

    def port_call(avx2: int, copy: bool):
        def call(n: int) -> float:
            sec = O.lib().orc_moe_layer_bench(C.byref(spec_grp.cfg()), C.byref(Wg), x.ctypes.data,
                                              out.ctypes.data, avx2, scratch.ctypes.data if copy else None, n)
            if sec < 0:
                raise RuntimeError("oracle bench failed")
            return sec
        return call

    runs = []
    for build, threads, copy in [("linux-scalar", share, False), ("linux-scalar", 1, False),
                                 ("msvc-avx2-fma", share, False), ("msvc-avx2-fma", 1, False),
                                 ("linux-scalar", share, True), ("msvc-avx2-fma", share, True)]:
        use_ref = build == "linux-scalar" and not copy and R is not None
        set_omp_threads(threads)
        per_call, iters = sample(ref_call if use_ref else port_call(int(build != "linux-scalar"), copy))
        runs.append({"kind": "reference" if use_ref else "port", "gemv": build, "threads": threads,
                     "scheduler_copy": copy, "tokens_per_s": round(1.0 / per_call, 2),
                     "ms_per_call": round(per_call * 1e3, 3), "calls": iters})
    set_omp_threads(share)
    head = runs[0]
    return {"value": head["tokens_per_s"], "unit": "tokens/s", "cores": share, "kind": head["kind"],
            "sample": f"{head['calls']} moeLayer calls, T=1, d={shape.hidden}, {shape.n_experts} experts "
                      f"top-{shape.top_k} + {shape.n_shared} shared, weights in host RAM, "
                      f"{head['gemv']} GEMV, {share} OpenMP threads (the host's CPU share); "
                      f"{head['ms_per_call']} ms/call",
            "host": host_cpu(), "variants": runs}


def time_steps(step, steps: int, warmup: int) -> float:
    for _ in range(warmup):
        step()
    capi.call("hfmoe_synchronize")
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    capi.call("hfmoe_synchronize")
    return (time.perf_counter() - t0) / steps


def decode_routing(x_all, ntok: int, shape: synth.LayerShape) -> dict:
    """Selections of the benchmark's tokens (one debug call each, untimed)."""
    d, k, E = shape.hidden, shape.top_k, shape.n_experts
    out, idx = capi.DeviceBuffer(d * 4), capi.DeviceBuffer(k * 4)
    dbg = capi.RouteDebug(None, idx.ptr, None, None, None)
    sel = []
    for t in range(ntok):
        capi.call("hfmoe_moe_forward_debug", 0, x_all.ptr + t * d * 4, 1, out.ptr, None, C.byref(dbg))
        sel.append(set(idx.download(np.int32, k).tolist()))
    out.free()
    idx.free()
    shared_prev = [len(sel[t] & sel[t - 1]) for t in range(ntok)]
    return {"tokens_cycled": ntok, "distinct_selections": len({frozenset(s) for s in sel}),
            "experts_hit": len(set().union(*sel)),
            "routed_experts_shared_with_previous_step": round(float(np.mean(shared_prev)), 3)}


def run_decode(args) -> dict:
    """T = 1 decode, one MoE layer; each step takes the next of 64 distinct tokens
    (different routing every step, as real decode), cycling."""
    shape = synth.LayerShape(**FULL)
    capi.call("hfmoe_configure", shape.config(max_tokens=1))
    layer = synth.DeviceLayer(shape, layer=0, seed=args.seed, experts_on_host=False)
    ntok = 64
    x_all = synth.make_x_dev(ntok, shape.hidden, seed=args.seed)
    x = capi.DeviceBuffer.of(x_all.download(np.float32, shape.hidden))  # token 0 alone
    out = capi.DeviceBuffer(shape.hidden * 4)
    fwd = capi.load().hfmoe_moe_forward
    routing = decode_routing(x_all, ntok, shape)
    tok = [0]

    def step():
        rc = fwd(0, x_all.ptr + (tok[0] % ntok) * shape.hidden * 4, 1, out.ptr, None)
        tok[0] += 1
        if rc:
            capi.check(rc)

    def same_step():
        rc = fwd(0, x.ptr, 1, out.ptr, None)
        if rc:
            capi.check(rc)

    sec_same = None if args.decode_only else time_steps(same_step, args.steps, args.warmup)
    sec = time_steps(step, args.steps, args.warmup)
    # Same steps again, each kernel recording its own dispatch timestamps.
    prof, sec_prof = profiled_pass(step, args.steps)
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
        "config": {"workload": "moe_layer_decode", "tokens": 1, "distinct_tokens_cycled": ntok,
                   "hidden": shape.hidden,
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
        "routing": routing,
    }
    if sec_same is not None:
        res["same_token_every_step"] = {"tokens_per_s": round(1.0 / sec_same, 1),
                                        "us_per_step": round(sec_same * 1e6, 2),
                                        "note": "one token replayed: its 9 experts re-read each step"}
    if args.decode_only:
        layer.free()
        for b in (x, x_all, out):
            b.free()
        return res
    # The reference's host contract (moeLayer: host float[hidden] in and out,
    # synchronous), PCIe copies included; a note beside `value`, not `value`.
    xh = x.download(np.float32, shape.hidden).copy()
    oh = np.zeros(shape.hidden, np.float32)
    host = capi.load().hfmoe_moe_layer

    def host_step():
        rc = host(0, xh.ctypes.data, oh.ctypes.data)
        if rc:
            capi.check(rc)

    sec_host = time_steps(host_step, args.steps, args.warmup)
    res["host_contract"] = {"us_per_call": round(sec_host * 1e6, 2), "tokens_per_s": round(1.0 / sec_host, 1),
                            "note": "hfmoe_moe_layer: x host -> HBM, layer, out -> host, synchronised per call"}
    if not args.no_cpu_baseline:
        res["cpu_baseline"] = cpu_baseline_decode(shape, args.seed, args.cpu_seconds)
    layer.free()
    for b in (x, x_all, out):
        b.free()
    return res


def run_dense(args) -> dict:
    """A dense MLP layer (GLM-5.2: hidden 6144, intermediate 12288; the first
    three decoder layers) on --dense-tokens tokens."""
    H, I, T = 6144, 12288, args.dense_tokens
    shape = synth.LayerShape(**FULL)
    capi.call("hfmoe_configure", shape.config(max_tokens=T))
    w = [capi.DeviceBuffer(2 * H * I) for _ in range(3)]
    for i, b in enumerate(w):
        synth.fill_bf16(b.ptr, H * I, args.seed, 200 + i, 0.0, 0.02)
    dw = capi.DenseWeights(w[0].ptr, w[1].ptr, w[2].ptr, None, I, 0)
    capi.call("hfmoe_register_dense_layer", 0, C.byref(dw))
    x = synth.make_x_dev(T, H, seed=args.seed)
    out = capi.DeviceBuffer(T * H * 4)
    fwd = capi.load().hfmoe_dense_mlp_forward

    def step():
        rc = fwd(0, x.ptr, T, out.ptr, None)
        if rc:
            capi.check(rc)

    sec = time_steps(step, args.steps, args.warmup)
    prof, sec_prof = profiled_pass(step, args.steps)
    wbytes = 3 * H * I * 2
    if T == 1:
        algo = {"dense_gateup": (2 * H * I * 2 + H * 4 + I * 4, 2 * 2 * H * I),
                "dense_down": (H * I * 2 + I * 4 + H * 4, 2 * H * I)}
        dom_name = "dense_gateup"
    else:
        algo = {"dense_gateup_gemm": (2 * H * I * 2 + T * H * 2 + T * I * 4, 2 * 2 * T * H * I),
                "dense_down_gemm": (H * I * 2 + T * I * 4 + T * H * 4, 2 * T * H * I),
                "split_x": (T * H * 4 + T * H * 4, 0)}
        dom_name = "dense_gateup_gemm"
    kernels = kernel_table(prof, algo)
    dom = kernels[dom_name]
    nbytes, flops = algo[dom_name]
    if flops / nbytes < MFMA_BF16_PEAK_TFLOPS * 1e12 / (HBM_PEAK_GBS * 1e9):
        roof = {"bound": "hbm", "kernel": dom_name, "achieved": dom["gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(dom["gbs"] / HBM_PEAK_GBS, 4), "traffic": None}
    else:
        roof = {"bound": "mfma", "kernel": dom_name, "achieved": dom["tflops"], "peak": MFMA_BF16_PEAK_TFLOPS,
                "unit": "TFLOP/s", "frac": round(dom["tflops"] / MFMA_BF16_PEAK_TFLOPS, 4), "traffic": None}
    res = {
        "value": T / sec,
        "ms_per_step": sec * 1e3,
        "config": {"workload": "dense_mlp", "tokens": T, "hidden": H, "intermediate": I,
                   "weights": "HBM-resident BF16 ~N(0,0.02)"},
        "roofline": roof,
        "layer": {"weight_bytes": wbytes, "gbs": round(wbytes / sec / 1e9, 1),
                  "tflops": round(2 * 3 * T * H * I / sec / 1e12, 2)},
        "ms_per_step_with_kernel_events": sec_prof * 1e3,
        "kernels": kernels,
    }
    for b in w + [x, out]:
        b.free()
    return res


def run_lm_head(args) -> dict:
    """Final norm + LM head + greedy argmax at GLM-5.2's size (vocab 154880,
    hidden 6144), one token."""
    H, V = 6144, 154880
    shape = synth.LayerShape(**FULL)
    capi.call("hfmoe_configure", shape.config(max_tokens=1))
    W = capi.DeviceBuffer(2 * V * H)
    synth.fill_bf16(W.ptr, V * H, args.seed, 300, 0.0, 0.02)
    norm = capi.DeviceBuffer(2 * H)
    synth.fill_bf16(norm.ptr, H, args.seed, 301, 1.0, 0.05)
    capi.call("hfmoe_register_lm_head", W.ptr, norm.ptr, V)
    x = synth.make_x_dev(1, H, seed=args.seed)
    lg = capi.DeviceBuffer(V * 4)
    tok = capi.DeviceBuffer(4)
    fwd = capi.load().hfmoe_lm_head

    def step():
        rc = fwd(x.ptr, 1, lg.ptr, tok.ptr, None)
        if rc:
            capi.check(rc)

    sec = time_steps(step, args.steps, args.warmup)
    prof, sec_prof = profiled_pass(step, args.steps)
    algo = {"lm_head_gemv": (V * H * 2 + H * 4 + V * 4, 2 * V * H)}
    kernels = kernel_table(prof, algo)
    dom = kernels["lm_head_gemv"]
    res = {
        "value": 1.0 / sec,
        "ms_per_step": sec * 1e3,
        "config": {"workload": "lm_head_greedy", "tokens": 1, "hidden": H, "vocab": V,
                   "weights": "HBM-resident BF16 ~N(0,0.02)"},
        "roofline": {"bound": "hbm", "kernel": "lm_head_gemv", "achieved": dom["gbs"], "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(dom["gbs"] / HBM_PEAK_GBS, 4), "traffic": None},
        "ms_per_step_with_kernel_events": sec_prof * 1e3,
        "kernels": kernels,
    }
    for b in (W, norm, x, lg, tok):
        b.free()
    return res


def grouped_algorithmic(shape: synth.LayerShape, T: int, U: int) -> dict[str, tuple[int, int]]:
    """(bytes, flops) each multi-token kernel must move / compute at least once.

    U = distinct routed experts hit by the batch; the shared expert is one more
    group in the same GEMM launches.  Weights are read once per launch,
    activations once per token (x as BF16 [T, d]), the SwiGLU intermediate
    counted at 4 bytes per element, expert outputs as FP32.
    """
    d, I, E, k, S = shape.hidden, shape.inter, shape.n_experts, shape.top_k, shape.n_shared
    R = T * k + S * T  # GEMM rows: routed (token, rank) pairs + shared-expert rows
    return {
        "router_gemm": (E * d * 2 + T * d * 2 + T * E * 4, 2 * T * E * d),
        "expert_gateup_gemm": ((U + S) * 2 * I * d * 2 + T * d * 2 + R * I * 4, 2 * R * 2 * I * d),
        "expert_down_gemm": ((U + S) * d * I * 2 + R * I * 4 + R * d * 4, 2 * R * d * I),
        "combine": (R * d * 4 + T * k * 4 + T * d * 4, 2 * T * k * d),
    }


def kernel_table(prof: dict, algo: dict) -> dict:
    kernels = {}
    for name, (n, ms) in prof.items():
        avg_us = ms * 1e3 / max(n, 1)
        row = {"launches": n, "avg_us": round(avg_us, 3)}
        if name in algo:
            nbytes, flops = algo[name]
            row.update(algorithmic_bytes=nbytes, gbs=round(nbytes / (avg_us * 1e-6) / 1e9, 1),
                       algorithmic_flops=flops, tflops=round(flops / (avg_us * 1e-6) / 1e12, 2))
        kernels[name] = row
    return kernels


def profiled_pass(step, steps: int) -> tuple[dict, float]:
    capi.call("hfmoe_profile_reset")
    capi.call("hfmoe_profile_enable", 1)
    sec = time_steps(step, steps, 0)
    capi.call("hfmoe_profile_enable", 0)
    return capi.profile_read(), sec


def run_grouped(args, workload: str, fp32_x: bool = False) -> dict:
    """Batched decode (T=64, Zipf routing) or a prefill chunk (T=4096, or
    --tokens, near-uniform routing).

    fp32_x: activations that are not BF16-valued (BF16 values scaled by
    1 + 2^-10 N(0, 1), FP32 like the reference's RMSNorm output), which the
    GEMMs take as BF16 hi + lo halves."""
    shape = synth.LayerShape(**FULL)
    if workload == "batched":
        T = 64
        with open(os.path.join(ROOT, "tests", "golden", "zipf_bias_e256.json")) as fh:
            zb = json.load(fh)
        seed = zb["layer_seed"]  # the bias is calibrated for this layer's router
        layer_kw = dict(bias=np.array(zb["bias"], np.float32))
        routing = "correction bias calibrated for Zipf(1.1) expert popularity"
    else:
        T = args.tokens
        seed = args.seed
        layer_kw = dict(bias_std=0.001)
        routing = "near-uniform, correction bias ~N(0,0.001)"
    capi.call("hfmoe_configure", shape.config(max_tokens=T))
    layer = synth.DeviceLayer(shape, layer=0, seed=seed, **layer_kw)
    x = synth.make_x_dev(T, shape.hidden, seed=seed)
    if fp32_x:
        xh = x.download(np.float32, T * shape.hidden)
        xh *= 1.0 + np.float32(2.0 ** -10) * np.random.default_rng(seed).standard_normal(xh.size).astype(np.float32)
        x.upload(xh)
        routing += "; FP32 activations (BF16 values x (1 + 2^-10 N(0,1)))"
    out = capi.DeviceBuffer(T * shape.hidden * 4)
    idx = capi.DeviceBuffer(T * shape.top_k * 4)
    dbg = capi.RouteDebug(None, idx.ptr, None, None, None)
    capi.call("hfmoe_moe_forward_debug", 0, x.ptr, T, out.ptr, None, C.byref(dbg))
    capi.call("hfmoe_synchronize")
    counts = np.bincount(idx.download(np.int32, T * shape.top_k), minlength=shape.n_experts)
    U = int((counts > 0).sum())
    fwd = capi.load().hfmoe_moe_forward

    def step():
        rc = fwd(0, x.ptr, T, out.ptr, None)
        if rc:
            capi.check(rc)

    sec = time_steps(step, args.steps, args.warmup)
    prof, sec_prof = profiled_pass(step, args.steps)
    algo = grouped_algorithmic(shape, T, U)
    kernels = kernel_table(prof, algo)
    d, I, E, S = shape.hidden, shape.inter, shape.n_experts, shape.n_shared
    layer_bytes = (U + S) * 3 * I * d * 2 + E * d * 2 + E * 4 + 2 * T * d * 4
    layer_flops = sum(f for _, f in algo.values())
    # Dominant kernel: the longest one.  Its roofline is HBM when its
    # arithmetic intensity (algorithmic FLOP per algorithmic byte) is below the
    # MI355X ridge point (2.5 PFLOP/s / 8 TB/s ~ 312), else MFMA.
    dom_name = max((n for n in algo if n in kernels), key=lambda n: kernels[n]["avg_us"])
    dom = kernels[dom_name]
    ai = dom["algorithmic_flops"] / dom["algorithmic_bytes"]
    # counter summaries exist for T = 64 (batched) and T = 4096 (prefill) only
    summary = "batched_t64_hbm_traffic.md" if workload == "batched" else \
        "prefill_t4096_hbm_traffic.md" if T == 4096 else ""
    tkey = "traffic_bytes_per_launch" + ("_fp32_x" if fp32_x else "")
    extra = {"arithmetic_intensity": round(ai, 1), "mfma_tflops": dom["tflops"],
             "mfma_frac": round(dom["tflops"] / MFMA_BF16_PEAK_TFLOPS, 4)}
    if ai < MFMA_BF16_PEAK_TFLOPS * 1e12 / (HBM_PEAK_GBS * 1e9):
        roof = {"bound": "hbm", "kernel": dom_name, "achieved": dom["gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(dom["gbs"] / HBM_PEAK_GBS, 4), "traffic": traffic_from_profile(dom_name, summary, tkey), **extra}
    else:
        roof = {"bound": "mfma", "kernel": dom_name, "achieved": dom["tflops"], "peak": MFMA_BF16_PEAK_TFLOPS,
                "unit": "TFLOP/s", "frac": round(dom["tflops"] / MFMA_BF16_PEAK_TFLOPS, 4),
                "traffic": traffic_from_profile(dom_name, summary, tkey), **extra}
    res = {
        "value": T / sec,
        "ms_per_step": sec * 1e3,
        "config": {"workload": f"moe_layer_{workload}", "tokens": T, "hidden": d, "moe_intermediate": I,
                   "routed_experts": E, "shared_experts": S, "top_k": shape.top_k,
                   "n_group": shape.n_group, "topk_group": shape.topk_group, "routing": routing,
                   "distinct_experts_hit": U, "max_rows_per_expert": int(counts.max()),
                   "weights": "HBM-resident BF16 ~N(0,0.02)"},
        "roofline": roof,
        "layer": {"algorithmic_bytes": layer_bytes, "achieved_gbs": round(layer_bytes / sec / 1e9, 1),
                  "hbm_frac": round(layer_bytes / sec / 1e9 / HBM_PEAK_GBS, 4),
                  "algorithmic_flops": layer_flops, "achieved_tflops": round(layer_flops / sec / 1e12, 2),
                  "mfma_frac": round(layer_flops / sec / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4)},
        "ms_per_step_with_kernel_events": sec_prof * 1e3,
        "kernels": kernels,
    }
    if not args.no_cpu_baseline:
        cb = cpu_baseline_decode(shape, seed, args.cpu_seconds)
        cb["sample"] += "; the reference runs a batch token by token (glm_forward.cpp:755), so its rate is per token"
        res["cpu_baseline"] = cb
    for b in (x, out, idx):
        b.free()
    layer.free()
    return res


def stream_counters() -> dict:
    c = capi.StreamCounters()
    capi.call("hfmoe_stream_read_counters", C.byref(c))
    return c.as_dict()


def run_streamed(args, cached: bool = False) -> dict:
    """8 chained layers, routed experts in pinned host RAM, T=1 per step.

    cached: an HBM expert cache of --cache-gb and a run of correlated tokens
    (each token's input = a shared base + --token-noise x N(0, 1)), so that
    consecutive tokens reuse experts and the next-layer copy-ahead has history
    to predict from.  Otherwise the pool holds two layers' selections and the
    tokens are independent: every selected expert crosses PCIe."""
    shape = synth.LayerShape(**FULL)
    n_layers = 8
    cfg = shape.config(max_tokens=1)
    if cached:
        cfg.vram_budget_bytes = int(args.cache_gb * 2**30)
    capi.call("hfmoe_configure", cfg)
    opt = capi.StreamOptions()
    capi.call("hfmoe_stream_get_options", C.byref(opt))
    opt.overlap_floor = args.overlap_floor
    opt.extra_depth = args.extra_depth
    opt.prob_resident = int(args.prob_resident)
    capi.call("hfmoe_stream_set_options", C.byref(opt))
    layers = [synth.DeviceLayer(shape, layer=l, seed=args.seed, experts_on_host=True, with_norm=True,
                                distinct_experts=args.distinct_experts) for l in range(n_layers)]
    d = shape.hidden
    ntok = args.warmup + 2 * args.steps
    if cached:
        rng = np.random.default_rng(args.seed)
        base = rng.standard_normal(d).astype(np.float32)
        xs = base + args.token_noise * rng.standard_normal((ntok, d)).astype(np.float32)
        h = capi.DeviceBuffer.of(xs.astype(np.float32))
    else:
        h = synth.make_x_dev(ntok, d, seed=args.seed)
    blk = capi.load().hfmoe_mlp_block
    cursor = [0]

    def step():
        ptr = h.ptr + cursor[0] * d * 4
        cursor[0] += 1
        for l in range(n_layers):
            rc = blk(l, ptr, 1, None)
            if rc:
                capi.check(rc)

    for _ in range(args.warmup):
        step()
    capi.call("hfmoe_synchronize")
    p0, a0 = C.c_uint64(), C.c_uint64()
    capi.call("hfmoe_stats", C.byref(p0), C.byref(a0))
    n0 = stream_counters()
    sec = time_steps(step, args.steps, 0)
    p1, a1 = C.c_uint64(), C.c_uint64()
    capi.call("hfmoe_stats", C.byref(p1), C.byref(a1))
    n1 = stream_counters()
    cache = {c: n1[c] - n0[c] for c in n1 if c != "slots"}
    cache["slots"] = n1["slots"]
    cache["hit_rate"] = round(cache["hits"] / max(cache["lookups"], 1), 4)
    prof, sec_prof = profiled_pass(step, args.steps)
    pcie = (p1.value - p0.value) / args.steps
    # Pinned host -> HBM copy rate of one layer's 8 selected experts, for the bound.
    nbytes = shape.top_k * shape.expert_bytes
    src = capi.PinnedBuffer(nbytes)
    dst = capi.DeviceBuffer(nbytes)
    capi.call("hfmoe_memcpy_h2d", dst.ptr, src.ptr, nbytes)
    t0 = time.perf_counter()
    for _ in range(5):
        capi.call("hfmoe_memcpy_h2d", dst.ptr, src.ptr, nbytes)
    h2d_gbs = 5 * nbytes / (time.perf_counter() - t0) / 1e9
    achieved = pcie / sec / 1e9
    res = {
        "value": 1.0 / sec,
        "ms_per_step": sec * 1e3,
        "config": {"workload": "moe_streamed_chain_cached" if cached else "moe_streamed_chain", "tokens": 1,
                   "layers": n_layers, "hidden": d,
                   "moe_intermediate": shape.inter, "routed_experts": shape.n_experts,
                   "shared_experts": shape.n_shared, "top_k": shape.top_k, "n_group": shape.n_group,
                   "topk_group": shape.topk_group,
                   "weights": f"routed experts in pinned host RAM ({args.distinct_experts} distinct weight "
                              f"sets per layer, every expert its own cache key); routers, shared experts "
                              f"and norms in HBM",
                   "hbm_expert_cache_gb": args.cache_gb if cached else None,
                   "copy_ahead_overlap_floor": args.overlap_floor,
                   "extra_depth": args.extra_depth, "prob_resident": bool(args.prob_resident),
                   "tokens_input": (f"correlated: base + {args.token_noise} x N(0,1) per token" if cached
                                    else "independent N(0,1) tokens")},
        "roofline": {"bound": "pcie", "kernel": "hipMemcpyAsync host->device", "achieved": round(achieved, 1),
                     "peak": round(h2d_gbs, 1), "unit": "GB/s", "frac": round(achieved / h2d_gbs, 4),
                     "traffic": int(pcie), "peak_source": "measured pinned copy of 8 experts"},
        "pcie_bytes_per_token": int(pcie),
        "expert_cache": cache,
        "ms_per_step_with_kernel_events": sec_prof * 1e3,
        "kernels": kernel_table(prof, {}),
    }
    if not args.no_cpu_baseline:
        cb = cpu_baseline_decode(shape, args.seed, args.cpu_seconds)
        cb["value"] /= n_layers
        cb["unit"] = "tokens/s"
        cb["sample"] += f"; one layer timed, a token crosses {n_layers} layers (variants: per layer)"
        res["cpu_baseline"] = cb
    src.free()
    dst.free()
    h.free()
    for L in layers:
        L.free()
    return res


def run_streamed_prefill(args) -> dict:
    """One full-shape layer, a prefill chunk of --prefill-tokens tokens, routed
    experts in pinned host RAM and the default slot pool (two layers' worth of
    selections): the batch's distinct experts cross PCIe a wave at a time."""
    shape = synth.LayerShape(**FULL)
    T = args.prefill_tokens
    capi.call("hfmoe_configure", shape.config(max_tokens=T))
    layer = synth.DeviceLayer(shape, layer=0, seed=args.seed, experts_on_host=True,
                              distinct_experts=args.distinct_experts)
    x = synth.make_x_dev(T, shape.hidden, seed=args.seed)
    out = capi.DeviceBuffer(T * shape.hidden * 4)
    fwd = capi.load().hfmoe_moe_forward

    def step():
        rc = fwd(0, x.ptr, T, out.ptr, None)
        if rc:
            capi.check(rc)

    for _ in range(args.warmup):
        step()
    capi.call("hfmoe_synchronize")
    p0, a0 = C.c_uint64(), C.c_uint64()
    capi.call("hfmoe_stats", C.byref(p0), C.byref(a0))
    n0 = stream_counters()
    sec = time_steps(step, args.steps, 0)
    p1, a1 = C.c_uint64(), C.c_uint64()
    capi.call("hfmoe_stats", C.byref(p1), C.byref(a1))
    n1 = stream_counters()
    cache = {c: (n1[c] - n0[c]) // args.steps for c in n1 if c != "slots"}
    cache["slots"] = n1["slots"]
    prof, sec_prof = profiled_pass(step, args.steps)
    pcie = (p1.value - p0.value) / args.steps
    nbytes = shape.top_k * shape.expert_bytes
    src = capi.PinnedBuffer(nbytes)
    dst = capi.DeviceBuffer(nbytes)
    capi.call("hfmoe_memcpy_h2d", dst.ptr, src.ptr, nbytes)
    t0 = time.perf_counter()
    for _ in range(5):
        capi.call("hfmoe_memcpy_h2d", dst.ptr, src.ptr, nbytes)
    h2d_gbs = 5 * nbytes / (time.perf_counter() - t0) / 1e9
    achieved = pcie / sec / 1e9
    res = {
        "value": T / sec,
        "ms_per_step": sec * 1e3,
        "config": {"workload": "moe_streamed_prefill", "tokens": T, "layers": 1, "hidden": shape.hidden,
                   "moe_intermediate": shape.inter, "routed_experts": shape.n_experts,
                   "shared_experts": shape.n_shared, "top_k": shape.top_k, "n_group": shape.n_group,
                   "topk_group": shape.topk_group,
                   "weights": f"routed experts in pinned host RAM ({args.distinct_experts} distinct weight sets, "
                              f"every expert its own cache key); router and shared expert in HBM",
                   "slot_pool": "default: 2 x top_k slots, waves of top_k experts"},
        "roofline": {"bound": "pcie", "kernel": "hipMemcpyAsync host->device", "achieved": round(achieved, 1),
                     "peak": round(h2d_gbs, 1), "unit": "GB/s", "frac": round(achieved / h2d_gbs, 4),
                     "traffic": int(pcie), "peak_source": "measured pinned copy of 8 experts"},
        "pcie_bytes_per_call": int(pcie),
        "expert_cache_per_call": cache,
        "ms_per_step_with_kernel_events": sec_prof * 1e3,
        "kernels": kernel_table(prof, {}),
    }
    src.free()
    dst.free()
    x.free()
    out.free()
    layer.free()
    return res


def run_load(args) -> None:
    """Checkpoint loading: one MoE layer (full d=6144 / I=2048 shapes, --load-experts
    routed experts) written as a safetensors shard, then timed through
    hfmoe_checkpoint_open + hfmoe_checkpoint_load_moe_layer into HBM.  The shard
    was just written, so it is read from the page cache: the bound is the
    host-memory read and the host->device copy, not the disk."""
    import shutil
    import tempfile
    shape = synth.LayerShape(**dict(FULL, n_experts=args.load_experts))
    capi.call("hfmoe_configure", shape.config(max_tokens=1))
    d, I, E = shape.hidden, shape.inter, shape.n_experts
    p = "model.layers.0.mlp."
    tensors = [(p + "gate.weight", "BF16", [E, d]), (p + "gate.e_score_correction_bias", "F32", [E]),
               (p + "shared_experts.gate_proj.weight", "BF16", [I, d]),
               (p + "shared_experts.up_proj.weight", "BF16", [I, d]),
               (p + "shared_experts.down_proj.weight", "BF16", [d, I])]
    for e in range(E):
        tensors += [(p + f"experts.{e}.gate_proj.weight", "BF16", [I, d]),
                    (p + f"experts.{e}.up_proj.weight", "BF16", [I, d]),
                    (p + f"experts.{e}.down_proj.weight", "BF16", [d, I])]
    header, off = {}, 0
    for name, dt, shp in tensors:
        nb = int(np.prod(shp)) * (2 if dt == "BF16" else 4)
        header[name] = {"dtype": dt, "shape": shp, "data_offsets": [off, off + nb]}
        off += nb + (-nb) % 8
    h = json.dumps(header).encode()
    h += b" " * ((-len(h)) % 8)
    tmp = tempfile.mkdtemp(prefix="hfmoe_ckpt_")
    path = os.path.join(tmp, "model-00001-of-00001.safetensors")
    buf = capi.DeviceBuffer(2 * I * d)
    t0 = time.perf_counter()
    with open(path, "wb") as f:
        f.write(len(h).to_bytes(8, "little"))
        f.write(h)
        for i, (name, dt, shp) in enumerate(tensors):
            n = int(np.prod(shp))
            if dt == "BF16":
                synth.fill_bf16(buf.ptr, n, args.seed, i, 0.0, 0.02)
                a = buf.download(np.uint16, n)
            else:
                a = np.zeros(n, np.float32)
            f.write(a.tobytes())
            f.write(bytes((-a.nbytes) % 8))
    t_write = time.perf_counter() - t0
    buf.free()
    total = sum(int(np.prod(shp)) * (2 if dt == "BF16" else 4) for _, dt, shp in tensors)
    L = capi.load()
    ck = C.c_void_p()
    t0 = time.perf_counter()
    capi.call("hfmoe_checkpoint_open", path.encode(), C.byref(ck))
    t_open = time.perf_counter() - t0
    capi.call("hfmoe_checkpoint_load_moe_layer", ck, 0, capi.EXPERTS_DEVICE)
    capi.call("hfmoe_synchronize")
    t_load = time.perf_counter() - t0
    L.hfmoe_checkpoint_close(ck)
    shutil.rmtree(tmp, ignore_errors=True)
    # The bound: a pinned host -> HBM copy of the same size class.
    nbytes = 1 << 30
    src = capi.PinnedBuffer(nbytes)
    dst = capi.DeviceBuffer(nbytes)
    capi.call("hfmoe_memcpy_h2d", dst.ptr, src.ptr, nbytes)
    t0 = time.perf_counter()
    for _ in range(3):
        capi.call("hfmoe_memcpy_h2d", dst.ptr, src.ptr, nbytes)
    h2d = 3 * nbytes / (time.perf_counter() - t0) / 1e9
    src.free()
    dst.free()
    print(json.dumps({"metric": "MoE layer checkpoint load GB/s (safetensors shard in page cache -> HBM)",
                      "value": round(total / t_load / 1e9, 2), "unit": "GB/s", "n_gpus": 1,
                      "higher_is_better": True, "bytes": total, "seconds": round(t_load, 3),
                      "open_seconds": round(t_open, 4), "write_seconds": round(t_write, 2),
                      "pinned_h2d_gbs": round(h2d, 1), "frac_of_pinned_h2d": round(total / t_load / 1e9 / h2d, 3),
                      "config": {"workload": "checkpoint_load", "hidden": d, "moe_intermediate": I,
                                 "routed_experts": E, "shared_experts": 1}}), flush=True)


def run_plugin(args) -> None:
    """Per-expert plugin surface (gpuExpertStage / gpuExpertFFN, cuda_backend.h:64-85)
    at the full expert shape: staging distinct experts from pageable host
    memory into the HBM expert cache, then synchronous expert FFN calls on a
    resident expert with host x and out (the reference's blocking contract:
    x up, FFN, out back, per call)."""
    d, I = FULL["hidden"], FULL["inter"]
    n_stage = 12
    ebytes = 3 * d * I * 2
    rng = np.random.default_rng(args.seed)
    w = (rng.standard_normal(3 * d * I, dtype=np.float32) * 0.02).view(np.uint32)
    w = ((w + 0x7FFF + ((w >> 16) & 1)) >> 16).astype(np.uint16)  # BF16, round to nearest even
    x = rng.standard_normal(d, dtype=np.float32)
    out = np.zeros(d, np.float32)
    L = capi.load()
    capi.call("hfmoe_expert_cache_config", n_stage + 4, 2)
    capi.call("hfmoe_expert_stage", 0, 0, w.ctypes.data, d, I)  # first call: slot pool set-up
    capi.call("hfmoe_synchronize")
    t0 = time.perf_counter()
    for e in range(1, n_stage + 1):
        capi.call("hfmoe_expert_stage", 0, e, w.ctypes.data, d, I)
    capi.call("hfmoe_synchronize")
    t_stage = (time.perf_counter() - t0) / n_stage
    ffn = L.hfmoe_expert_ffn
    for _ in range(args.warmup):
        capi.check(ffn(0, 1, x.ctypes.data, out.ctypes.data, d, I))
    t0 = time.perf_counter()
    for _ in range(args.steps):
        capi.check(ffn(0, 1, x.ctypes.data, out.ctypes.data, d, I))
    t_ffn = (time.perf_counter() - t0) / args.steps
    L.hfmoe_expert_cache_shutdown()
    gbs = ebytes / t_ffn / 1e9
    print(json.dumps({"metric": "per-expert plugin: expert FFN calls/s (host x/out, blocking) + stage GB/s, "
                                "d=6144, I=2048",
                      "value": round(1.0 / t_ffn, 1), "unit": "calls/s", "n_gpus": 1, "steps": args.steps,
                      "warmup": args.warmup, "us_per_call": round(t_ffn * 1e6, 2), "higher_is_better": True,
                      "dtype": "bf16", "data": "synthetic",
                      "roofline": {"bound": "hbm", "kernel": "expert_ffn (gate/up + down GEMV, one expert)",
                                   "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                   "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None,
                                   "note": "whole call: x H2D, two kernels, out D2H and the synchronisation"},
                      "stage": {"experts": n_stage, "bytes_each": ebytes, "ms_each": round(t_stage * 1e3, 3),
                                "gbs": round(ebytes / t_stage / 1e9, 2),
                                "source": "pageable numpy buffer, copied through pinned staging slots"},
                      "config": {"workload": "expert_plugin", "hidden": d, "moe_intermediate": I}}), flush=True)


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


def traffic_from_profile(kernel: str, summary: str = "decode_t1_hbm_traffic.md",
                         key: str = "traffic_bytes_per_launch") -> int | None:
    """HBM bytes per launch of `kernel` from a committed counter summary (the
    line that starts with `key:`)."""
    path = os.path.join(ROOT, "profiles", summary)
    if not summary or not os.path.isfile(path):
        return None
    for line in open(path):
        if line.startswith(key + ":"):
            for item in line.split(":", 1)[1].split():
                name, _, val = item.partition("=")
                if name == kernel:
                    return int(val)
    return None


METRICS = {
    "decode": METRIC,
    "batched": "MoE-layer batched-decode tokens/s + HBM GB/s at d=6144, 256e top-8, T=64 Zipf(1.1)",
    "prefill": "MoE-layer prefill tokens/s + BF16 MFMA TFLOP/s at d=6144, 256e top-8, T=4096",
    "streamed": "8-layer streamed-expert decode tokens/s + PCIe GB/s at d=6144, 256e top-8",
    "streamed_prefill": "streamed-expert prefill tokens/s + PCIe GB/s at d=6144, 256e top-8, T=4096",
    "dense": "dense-MLP layer tokens/s + HBM GB/s at d=6144, intermediate 12288",
    "lm_head": "LM head + greedy argmax tokens/s + HBM GB/s at d=6144, vocab 154880",
    "streamed_cached": "8-layer streamed-expert decode tokens/s with an HBM expert cache and next-layer "
                       "copy-ahead, correlated tokens, at d=6144, 256e top-8",
}


def run_configs(args, cpu_tokens_per_s: float | None = None) -> dict:
    """The other benchmark workloads of the same full-shape layer, timed in
    the default run beside the decode line: batched decode (T=64,
    Zipf popularity), prefill (T=4096, BF16-valued and FP32 activations) and
    the 8-layer streamed chain (T=1, experts from pinned host RAM).  Each
    with steps of its own; no CPU legs (the reference runs every batch token
    by token, so its rate per token is the decode line's cpu_baseline, per
    layer for the chain)."""
    import copy
    runs = [("batched_t64_zipf", lambda a: run_grouped(a, "batched"), 40, 5),
            ("prefill_t4096", lambda a: run_grouped(a, "prefill"), 10, 2),
            ("prefill_t4096_fp32_x", lambda a: run_grouped(a, "prefill", fp32_x=True), 10, 2),
            ("streamed_chain8", lambda a: run_streamed(a), 4, 1)]
    out = {}
    for name, fn, steps, warm in runs:
        a = copy.copy(args)
        a.steps, a.warmup, a.no_cpu_baseline, a.tokens = steps, warm, True, 4096
        t0 = time.perf_counter()
        r = fn(a)
        keep = {"tokens_per_s": round(r["value"], 1), "ms_per_step": round(r["ms_per_step"], 4), "steps": steps,
                "warmup": warm, "wall_s": round(time.perf_counter() - t0, 1)}
        for key in ("config", "roofline", "layer", "kernels", "pcie_bytes_per_token", "expert_cache"):
            if key in r:
                keep[key] = r[key]
        if cpu_tokens_per_s:
            # The reference runs a batch token by token (glm_forward.cpp:755), each token
            # reading its 8 routed + 1 shared experts of equal size, so its rate per token
            # is the decode line's; a token crosses all 8 layers of the chain.
            layers = r.get("config", {}).get("layers", 1)
            keep["cpu_baseline"] = {"value": round(cpu_tokens_per_s / layers, 2), "unit": "tokens/s",
                                    "kind": "reference",
                                    "sample": "the decode line's cpu_baseline per token"
                                              + (f", over {layers} layers" if layers > 1 else "")
                                              + ": the reference has no batched MoE; it calls moeLayer once per "
                                                "token of a batch, each call reading 8 routed + 1 shared experts "
                                                "of equal size, so its tokens/s at any batch size is its T = 1 "
                                                "call rate"}
        out[name] = keep
        print(f"{name}: {keep['tokens_per_s']} tokens/s", file=sys.stderr, flush=True)
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None, help="timed steps (default per workload)")
    ap.add_argument("--warmup", type=int, default=None)
    ap.add_argument("--workload", default="decode",
                    choices=["decode", "batched", "prefill", "streamed", "streamed_cached", "streamed_prefill",
                             "dense", "lm_head", "load", "plugin", "copy"])
    ap.add_argument("--seed", type=int, default=2026)
    ap.add_argument("--distinct-experts", type=int, default=32,
                    help="streamed: distinct expert weight sets per layer (bounds pinned host memory)")
    ap.add_argument("--cache-gb", type=float, default=40.0,
                    help="streamed_cached: HBM expert cache size (a quarter of the 8 layers' routed experts)")
    ap.add_argument("--token-noise", type=float, default=0.35,
                    help="streamed_cached: per-token deviation from the shared base input")
    ap.add_argument("--overlap-floor", type=float, default=0.5,
                    help="streamed: winner-overlap EMA below which next-layer copy-ahead is skipped")
    ap.add_argument("--extra-depth", type=int, default=0,
                    help="streamed: router-probability extra copy-ahead depth (setRouterPrefetch)")
    ap.add_argument("--prob-resident", action="store_true",
                    help="streamed: pin experts within 10%% of the layer's top routing weight (setRouterPrefetch)")
    ap.add_argument("--dense-tokens", type=int, default=1, help="dense: tokens per call")
    ap.add_argument("--prefill-tokens", type=int, default=4096, help="streamed_prefill: tokens per call")
    ap.add_argument("--tokens", type=int, default=4096,
                    help="prefill: tokens per call (near-uniform routing at any batch size, 2 or more)")
    ap.add_argument("--load-experts", type=int, default=64,
                    help="load: routed experts in the written checkpoint layer (75.5 MB each)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-configs", action="store_true",
                    help="decode: leave out the batched, prefill and streamed-chain extras")
    ap.add_argument("--fp32-x", action="store_true",
                    help="batched / prefill: FP32 activations (not BF16-valued)")
    ap.add_argument("--decode-only", action="store_true",
                    help="decode: only the distinct-token steps (no same-token, host-contract or CPU legs), "
                         "for kernel traces")
    ap.add_argument("--cpu-seconds", type=float, default=3.0, help="CPU baseline: seconds per variant")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: --gpus {args.gpus} is not supported "
              f"(the MoE block runs on a single MI355X; sharding is design-only)", file=sys.stderr)
        return 2
    defaults = {"decode": (200, 20), "batched": (100, 10), "prefill": (20, 3), "streamed": (20, 3),
                "streamed_cached": (30, 10), "streamed_prefill": (3, 1), "dense": (100, 10), "lm_head": (100, 10), "load": (1, 0),
                "plugin": (200, 20), "copy": (5, 0)}
    d_steps, d_warm = defaults[args.workload]
    args.steps = d_steps if args.steps is None else args.steps
    args.warmup = d_warm if args.warmup is None else args.warmup
    capi.call("hfmoe_init", 0)
    if args.workload in ("copy", "load", "plugin"):
        {"copy": run_copy, "load": run_load, "plugin": run_plugin}[args.workload](args)
        capi.load().hfmoe_shutdown()
        return 0
    if args.workload == "decode":
        res = run_decode(args)
        if not (args.no_configs or args.decode_only):
            res["configs"] = run_configs(args, res.get("cpu_baseline", {}).get("value"))
    elif args.workload == "dense":
        res = run_dense(args)
    elif args.workload == "lm_head":
        res = run_lm_head(args)
    elif args.workload in ("streamed", "streamed_cached"):
        res = run_streamed(args, cached=args.workload == "streamed_cached")
    elif args.workload == "streamed_prefill":
        res = run_streamed_prefill(args)
    else:
        res = run_grouped(args, args.workload, fp32_x=args.fp32_x)
    metric = METRICS[args.workload]
    if args.workload == "prefill" and args.tokens != 4096:
        metric = metric.replace("T=4096", f"T={args.tokens}")
    line = {"metric": metric, "value": round(res.pop("value"), 2), "unit": "tokens/s",
            "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "ms_per_step": round(res.pop("ms_per_step"), 5), "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "bf16", "data": "synthetic", **res}
    print(json.dumps(line), flush=True)
    capi.load().hfmoe_shutdown()
    return 0


if __name__ == "__main__":
    sys.exit(main())
