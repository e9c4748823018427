"""Writes wave64_conditioning.json: how far each leaf-net arithmetic model moves
the solve of every subgame of the 64-subgame wave (seed 3, 64 DCFR iterations,
512 -> 3x384 -> 567 net) from the float32 CPU solver.

Per subgame and model: the largest root-value difference divided by the largest
|root value| of the float32 solve, and the mean absolute strategy difference.
Models (oracle/oracle.c): F16 (f16 operands, wide sum), F16A (f16 operands,
float32 sum in ascending k order), F16X (compensated f16 pairs), BF16, F32W
(float32 operands, wide sum). Run from the repository root:
    python tests/golden/make_conditioning.py
"""
from __future__ import annotations

import json
import os
import sys
from concurrent.futures import ThreadPoolExecutor

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path[:0] = [os.path.join(ROOT, "war-chest-bot-9000-_amd"), os.path.join(ROOT, "oracle")]

import oracle as O  # noqa: E402
import workloads as W  # noqa: E402

MODELS = {"F16": O.NET_F16, "F16A": O.NET_F16A, "F16X": O.NET_F16X, "BF16": O.NET_BF16, "F32W": O.NET_F32W}
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "wave64_conditioning.json")


def errors(job, net, models=MODELS):
    """{model: (root error / max |root|, mean |strategy error|)} against the float32 solve,
    and under "F16~F16A" the two f16 realizations' root difference / max |root|."""
    ref = O.solve(job, net, O.NET_F32)
    scale = float(np.abs(ref["roots"]).max())
    out, roots = {}, {}
    for name, mode in models.items():
        o = O.solve(job, net, mode)
        roots[name] = o["roots"]
        out[name] = (float(np.abs(o["roots"] - ref["roots"]).max()) / scale,
                     float(np.abs(o["strategy"] - ref["strategy"]).mean()))
    if "F16" in roots and "F16A" in roots:
        out["F16~F16A"] = (float(np.abs(roots["F16"] - roots["F16A"]).max()) / scale, 0.0)
    return out


def main():
    jobs = W.jobs("wave64")
    net = W.net_for("wave64")
    with ThreadPoolExecutor(min(16, os.cpu_count() or 1)) as pool:
        rows = list(pool.map(lambda j: errors(j, net), jobs))
    doc = {
        "workload": "wave64: 64 depth-1 subgames, seed 3, 64 DCFR iterations, 512->3x384->567 net (seed 1)",
        "measure": "root: max |roots - roots_f32| / max |roots_f32|; strategy: mean |strategy - strategy_f32|",
        "models": {name: {"root": [r[name][0] for r in rows], "strategy": [r[name][1] for r in rows]}
                   for name in MODELS},
        "f16_realizations_root_difference": [r["F16~F16A"][0] for r in rows],
    }
    with open(OUT, "w") as f:
        json.dump(doc, f, indent=1)
    for name in MODELS:
        e = np.array(doc["models"][name]["root"])
        print(f"{name}: max {e.max():.2e}, median {np.median(e):.2e}, over 2e-3: {int((e > 2e-3).sum())}")
    e = np.array(doc["f16_realizations_root_difference"])
    print(f"F16 vs F16A: max {e.max():.2e}, median {np.median(e):.2e}")


if __name__ == "__main__":
    main()
