"""Calibrate the skewed-routing correction bias of the batched-decode workload.

The batched-decode workload (T=64 tokens, full-shape layer: d=6144, 256
experts, 8 groups keep 4, top-8) routes with a score-correction bias drawn so
that expert selection frequency follows Zipf(s=1.1) over a seeded permutation
of the experts.  Each token selects an expert at most once, so the target
per-token selection probability of the expert at Zipf rank r is
q_r = min(1, c * r^-1.1), with c fixed by sum(q) = top_k.

The bias is fitted by fixed-point iteration b += eta * (q - f) on a calibration
sample of tokens that is disjoint from the benchmark's own tokens, where f is
the realised selection frequency under the routing rule of
glm_forward.cpp:543-556 (sigmoid scores plus bias, group top-2 sums, keep
topk_group groups, top-k experts).  The router weights are those of the
seeded synthetic layer the benchmark builds (seed 2026, layer 0).

    python tests/golden/zipf_bias.py   # rewrites zipf_bias_e256.json
"""
from __future__ import annotations

import json
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
import oracle as O  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "zipf_bias_e256.json")

D, E, K, N_GROUP, TOPK_GROUP = 6144, 256, 8, 8, 4
LAYER_SEED = 2026          # seed of the synthetic layer (router weights)
PERM_SEED = 11             # permutation of experts onto Zipf ranks
SAMPLE_SEED = 7777         # calibration tokens (the benchmark uses LAYER_SEED's tokens)
ZIPF_S = 1.1


def zipf_targets() -> tuple[np.ndarray, np.ndarray]:
    perm = np.random.default_rng(PERM_SEED).permutation(E)
    rank = np.empty(E, np.int64)
    rank[perm] = np.arange(1, E + 1)
    base = rank.astype(np.float64) ** -ZIPF_S
    lo, hi = 0.0, 1e6
    for _ in range(200):
        c = 0.5 * (lo + hi)
        if np.minimum(1.0, c * base).sum() > K:
            hi = c
        else:
            lo = c
    return np.minimum(1.0, lo * base), rank


def scores_of(x: np.ndarray) -> np.ndarray:
    router = O.bf16_to_f32(O.fill_bf16(E * D, LAYER_SEED, O.tensor_id(0, O.ROLE_ROUTER), 0.0, 0.02))
    logits = x @ router.reshape(E, D).T
    return (1.0 / (1.0 + np.exp(-logits.astype(np.float64)))).astype(np.float32)


def route_counts(s: np.ndarray, b: np.ndarray) -> np.ndarray:
    """Per-expert selection counts under group-limited top-k (vectorised)."""
    n = s.shape[0]
    sb = s + b.astype(np.float32)
    gs = E // N_GROUP
    gscore = np.sort(sb.reshape(n, N_GROUP, gs), axis=2)[:, :, -2:].sum(axis=2)
    keep = np.argsort(-gscore, axis=1, kind="stable")[:, :TOPK_GROUP]
    mask = np.zeros((n, N_GROUP), bool)
    np.put_along_axis(mask, keep, True, axis=1)
    masked = np.where(np.repeat(mask, gs, axis=1), sb, -np.inf)
    sel = np.argsort(-masked, axis=1, kind="stable")[:, :K]
    return np.bincount(sel.reshape(-1), minlength=E)


def main() -> None:
    q, rank = zipf_targets()
    x = O.make_x(4096, D, SAMPLE_SEED)
    s = scores_of(x)
    b = np.zeros(E, np.float64)
    eta = 1.0
    for it in range(600):
        f = route_counts(s, b.astype(np.float32)) / s.shape[0]
        b += eta * (q - f)
        if it % 100 == 99:
            eta *= 0.6
    bias = b.astype(np.float32)
    f = route_counts(s, bias) / s.shape[0]
    doc = {
        "about": "score-correction bias giving Zipf(1.1) expert selection frequencies; "
                 "written by tests/golden/zipf_bias.py",
        "hidden": D, "n_experts": E, "top_k": K, "n_group": N_GROUP, "topk_group": TOPK_GROUP,
        "layer_seed": LAYER_SEED, "perm_seed": PERM_SEED, "sample_seed": SAMPLE_SEED,
        "sample_tokens": int(s.shape[0]), "zipf_s": ZIPF_S,
        "zipf_rank": rank.tolist(),
        "target_freq": [round(float(v), 6) for v in q],
        "sample_freq": [round(float(v), 6) for v in f],
        "max_abs_freq_error": round(float(np.abs(f - q).max()), 6),
        "bias": [float(v) for v in bias],
    }
    with open(OUT, "w") as fh:
        json.dump(doc, fh, indent=0)
    print(f"wrote {OUT}: max |f - q| = {doc['max_abs_freq_error']}")


if __name__ == "__main__":
    main()
