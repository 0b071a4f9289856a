"""Write golden input/output vectors from the reference's own compiled code.

Runs only where the reference checkout exists (oracle/_ref/libhfref.so is
built from its sources by `make -C oracle ref`).  Every vector below is an
output of the reference's functions -- gemv_bf16_f32 (cpu_kernels.cpp:43-94),
sigmoid_f32 (moe_router.h:19-21), topKScores (moe_router.h:29-57),
BFloat16::fromF32 (dtype_bf16.h:27-33), GLMForward::rmsNorm
(glm_forward.cpp:185-197), GLMForward::moeLayer (glm_forward.cpp:509-661),
GLMForward::denseMlp (:410-432), GLMForward::lmHeadAndSample (:663-731) and
the plugin helpers gpuEmbeddingLookup / gpuMatvecBf16 / gpuSoftmax / gpuArgmax
as built without CUDA (cuda_backend.cpp:564-594) --
on inputs from the seeded generator, so the fixtures hold seeds, a few inputs
and the reference's outputs, never reference source.

    python tests/golden/gen_golden.py
"""
from __future__ import annotations

import json
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
import oracle as O  # noqa: E402

OUT = os.path.dirname(os.path.abspath(__file__))


def bits(a: np.ndarray) -> list[int]:
    return np.ascontiguousarray(a, np.float32).view(np.uint32).tolist()


def main() -> None:
    O.build(force=True)
    if not O.build_ref():
        raise SystemExit("reference harness unavailable")
    R = O.ref()
    g: dict = {"about": "outputs of the reference's compiled functions; float32 values as uint32 bits"}

    # BF16 round trip of selected values (dtype_bf16.h:27-33).
    vals = np.array([1.0, 2.0, -1.5, 0.5, 0.0, -0.0, 0.1, 0.3, 1 / 3, 123.456, -987.654, 1e-3, 1e3,
                     1.00390625, 1.01171875, 3.4e38, 1e-40, -2.5e-39], np.float32)
    g["bf16"] = {"in": bits(vals), "out": [int(R.ref_bf16_from_f32(float(v))) for v in vals]}

    # Sigmoid on a sweep (moe_router.h:19-21).
    xs = np.concatenate([np.linspace(-20, 20, 97, dtype=np.float32),
                         np.array([0.0, 100.0, -100.0, 1e-8, -1e-8], np.float32)])
    g["sigmoid"] = {"in": bits(xs), "out": bits(np.array([R.ref_sigmoid(float(v)) for v in xs], np.float32))}

    # GEMV (cpu_kernels.cpp:43-94): shapes of the reference test (8x33) and the
    # MoE path, inputs from the seeded generator.
    gemv = []
    for i, (M, K, a, b) in enumerate([(8, 33, 1.0, 0.0), (8, 33, 2.0, 0.5), (16, 2048, 1.0, 0.0),
                                      (4, 6144, 1.0, 0.0), (3, 7, 1.0, 0.0)]):
        A = O.fill_bf16(M * K, 1000 + i, 1, 0.0, 0.5)
        x = O.fill_f32(K, 2000 + i, 2, 0.0, 1.0)
        y0 = O.fill_f32(M, 3000 + i, 3, 0.0, 1.0)
        y = y0.copy()
        R.ref_gemv_bf16_f32(A.ctypes.data, x.ctypes.data, y.ctypes.data, M, K, a, b)
        gemv.append({"M": M, "K": K, "alpha": a, "beta": b, "seedA": 1000 + i, "seedx": 2000 + i,
                     "seedy": 3000 + i, "out": bits(y)})
    g["gemv"] = gemv

    # topKScores (moe_router.h:29-57) on seeded scores/bias, with and without
    # normalisation; E and k as in the configs.
    topk = []
    for i, (E, k, norm, scale, with_bias) in enumerate([(8, 3, 0, 1.0, 0), (8, 3, 1, 1.0, 0), (64, 8, 1, 2.5, 1),
                                                        (256, 8, 1, 2.5, 1), (256, 8, 0, 1.0, 1), (16, 2, 1, 2.5, 1)]):
        logits = O.fill_f32(E, 4000 + i, 4, 0.0, 1.5)
        s = np.array([R.ref_sigmoid(float(v)) for v in logits], np.float32)
        bias = O.fill_f32(E, 5000 + i, 5, 0.0, 0.01) if with_bias else None
        idx = np.zeros(8, np.int32)
        w = np.zeros(8, np.float32)
        n = R.ref_topk_scores(s.ctypes.data, E, None if bias is None else bias.ctypes.data, k, scale, norm,
                              idx.ctypes.data, w.ctypes.data)
        topk.append({"E": E, "k": k, "norm": norm, "scale": scale, "seed_logits": 4000 + i,
                     "seed_bias": (5000 + i) if with_bias else None, "scores": bits(s),
                     "idx": idx[:n].tolist(), "w": bits(w[:n])})
    g["topk"] = topk

    # RMSNorm (glm_forward.cpp:185-197).
    rms = []
    for i, n in enumerate([128, 2048, 6144]):
        x = O.fill_f32(n, 6000 + i, 6, 0.0, 1.3)
        w = O.fill_bf16(n, 7000 + i, 7, 1.0, 0.05)
        y = x.copy()
        R.ref_rmsnorm(b"/tmp/hf_golden_rms.bin", w.ctypes.data, y.ctypes.data, n, 1e-5)
        rms.append({"n": n, "seedx": 6000 + i, "seedw": 7000 + i, "eps": 1e-5, "out": bits(y)})
    g["rmsnorm"] = rms

    # The MoE fields of the reference's own test fixture
    # (tests/fixtures/config_mini.json, read by config.cpp:107-117): hidden 16,
    # 8 routed experts, top-2, one shared expert, expert intermediate 16, dense
    # intermediate 48, scale 2.5, normalised weights, topk_group 1.
    mini_src = "/root/reference/tests/fixtures/config_mini.json"
    with open(mini_src, encoding="utf-8") as f:
        fx = json.load(f)
    keys = ["hidden_size", "intermediate_size", "vocab_size", "num_hidden_layers", "n_routed_experts",
            "num_experts_per_tok", "n_shared_experts", "moe_intermediate_size", "first_k_dense_replace",
            "routed_scaling_factor", "norm_topk_prob", "topk_group", "rms_norm_eps", "mlp_layer_types"]
    g["config_mini"] = {k: fx[k] for k in keys}
    mini = g["config_mini"]

    # Whole moeLayer, flat routing (the reference's rule): the small CPU config
    # (d=2048, I=1024, 64 experts) for three tokens, the full shape (d=6144,
    # I=2048, 256 experts) for one token, and the fixture's mini config for four.
    layers = []
    for name, spec, tokens in [
        ("small", O.LayerSpec(hidden=2048, inter=1024, n_experts=64, seed=11), 3),
        ("full", O.LayerSpec(hidden=6144, inter=2048, n_experts=256, seed=12), 1),
        ("config_mini", O.LayerSpec(hidden=mini["hidden_size"], inter=mini["moe_intermediate_size"],
                                    n_experts=mini["n_routed_experts"], top_k=mini["num_experts_per_tok"],
                                    n_shared=mini["n_shared_experts"], norm_topk_prob=mini["norm_topk_prob"],
                                    routed_scaling_factor=mini["routed_scaling_factor"], seed=13), 4),
    ]:
        L = O.SyntheticLayer(spec)
        xs = O.make_x(tokens, spec.hidden, spec.seed)
        for t in range(tokens):
            out, lg, idx, w = L.forward(xs[t])
            ro = L.ref_forward(xs[t], idx)
            if not np.array_equal(out.view(np.uint32), ro.view(np.uint32)):
                raise SystemExit(f"oracle and reference differ on {name} token {t}")
            layers.append({"name": name, "hidden": spec.hidden, "inter": spec.inter,
                           "n_experts": spec.n_experts, "top_k": spec.top_k, "n_shared": spec.n_shared,
                           "scale": spec.routed_scaling_factor, "norm": spec.norm_topk_prob,
                           "seed": spec.seed, "token": t, "idx": idx.tolist(), "w": bits(w), "out": bits(ro)})
        L.experts.clear()
    g["moe_layer"] = layers

    # Dense MLP (GLMForward::denseMlp, glm_forward.cpp:410-432): a small shape
    # and GLM-5.2's (hidden 6144, intermediate 12288), one seeded token each.
    dense = []
    for i, (H, I) in enumerate([(512, 1536), (6144, 12288)]):
        seed = 8000 + i
        gw = O.fill_bf16(I * H, seed, 1, 0.0, 0.02)
        uw = O.fill_bf16(I * H, seed, 2, 0.0, 0.02)
        dw = O.fill_bf16(H * I, seed, 3, 0.0, 0.02)
        x = O.fill_f32(H, seed, 4, 0.0, 1.0)
        out = np.zeros(H, np.float32)
        if R.ref_dense_mlp(b"/tmp/hf_golden_dense.bin", gw.ctypes.data, uw.ctypes.data, dw.ctypes.data, H, I,
                           x.ctypes.data, out.ctypes.data):
            raise SystemExit("ref_dense_mlp failed")
        dense.append({"hidden": H, "inter": I, "seed": seed, "w_std": 0.02, "out": bits(out)})
    g["dense_mlp"] = dense

    # LM head (GLMForward::lmHeadAndSample, glm_forward.cpp:663-731): final norm,
    # logits, greedy argmax; GLM-5.2's vocabulary (154880) at hidden 6144 and a
    # small one.  The fixture keeps the argmax, the ten largest logits and 64
    # seeded samples.
    import ctypes as C
    lm = []
    for i, (H, V) in enumerate([(512, 1000), (6144, 154880)]):
        seed = 9000 + i
        W = O.fill_bf16(V * H, seed, 1, 0.0, 0.02)
        nw = O.fill_bf16(H, seed, 2, 1.0, 0.05)
        h = O.fill_f32(H, seed, 3, 0.0, 1.0)
        lg = np.zeros(V, np.float32)
        best = C.c_int()
        if R.ref_lm_head(b"/tmp/hf_golden_lm.bin", W.ctypes.data, nw.ctypes.data, H, V, 1e-5, h.ctypes.data,
                         lg.ctypes.data, C.byref(best)):
            raise SystemExit("ref_lm_head failed")
        top = np.argsort(-lg, kind="stable")[:10]
        sample = np.random.default_rng(seed).choice(V, 64, replace=False)
        lm.append({"hidden": H, "vocab": V, "seed": seed, "eps": 1e-5, "best": best.value,
                   "top": top.tolist(), "top_bits": bits(lg[top]), "sample": sample.tolist(),
                   "sample_bits": bits(lg[sample])})
    g["lm_head"] = lm

    # Plugin helpers (cuda_backend.h:36-48, the reference's CPU forms
    # cuda_backend.cpp:564-594): embedding row, BF16 matvec, softmax, argmax.
    helpers = {}
    emb = O.fill_bf16(64 * 48, 9500, 1, 0.0, 1.0)
    rows = []
    for tok in (0, 5, 63):
        out = np.zeros(48, np.float32)
        R.ref_embedding_lookup(emb.ctypes.data, tok, out.ctypes.data, 48)
        rows.append({"token": tok, "out": bits(out)})
    helpers["embedding"] = {"vocab": 64, "hidden": 48, "seed": 9500, "rows": rows}
    mv = []
    for i, (M, K) in enumerate([(37, 300), (5, 6144)]):
        W = O.fill_bf16(M * K, 9600 + i, 1, 0.0, 0.05)
        x = O.fill_f32(K, 9600 + i, 2, 0.0, 1.0)
        y = np.zeros(M, np.float32)
        R.ref_matvec_bf16(W.ctypes.data, x.ctypes.data, y.ctypes.data, M, K)
        mv.append({"M": M, "K": K, "seed": 9600 + i, "out": bits(y)})
    helpers["matvec"] = mv
    sm = []
    for i, (n, sd) in enumerate([(1000, 3.0), (154880, 2.0), (7, 30.0)]):
        x = O.fill_f32(n, 9700 + i, 1, 0.0, sd)
        y = x.copy()
        R.ref_softmax(y.ctypes.data, n)
        sample = np.random.default_rng(9700 + i).choice(n, min(n, 64), replace=False)
        sm.append({"n": n, "std": sd, "seed": 9700 + i, "sample": sample.tolist(), "sample_bits": bits(y[sample]),
                   "sum64": float(np.sum(y, dtype=np.float64))})
    helpers["softmax"] = sm
    am = []
    for i, n in enumerate([1000, 154880]):
        x = O.fill_f32(n, 9800 + i, 1, 0.0, 1.0)
        x[n // 3] = x[2 * n // 3] = float(np.max(x)) + 1.0  # an exact tie: the first wins
        am.append({"n": n, "seed": 9800 + i, "best": int(R.ref_argmax(x.ctypes.data, n))})
    helpers["argmax"] = am
    g["helpers"] = helpers

    path = os.path.join(OUT, "reference_vectors.json")
    with open(path, "w") as f:
        json.dump(g, f, separators=(",", ":"))
    print(f"wrote {path} ({os.path.getsize(path)} bytes)")


if __name__ == "__main__":
    main()
