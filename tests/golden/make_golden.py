"""Writes tests/golden/reference_grid.json: expected tokens of the reference's
ranked-sampler test grids, computed with the restatement of the reference's
full-sort baseline reference_ranked_sample (crates/hi-cuda/src/gpu.rs:
29505-29580; oracle/sampler_oracle.c hro_ranked_sample_brute).

Grids (same parameters as the reference tests):
  * host grid, gpu.rs:29582-29633: LCG logits, seeds 0x1234+vi, spread 4,
    vocabs {64, 200, 1500, 4096} x T {0.7, 1.0, 1.3} x top_p {inf, 0.5, 0.9,
    0.95, 0.999} x top_k {None, 1, 10, 40, 2000} x u {0, 0.13, 0.5, 0.77, 0.999};
  * device grid, gpu.rs:29635-29760: LCG logits, seeds 0x8f21+vi, and the tie
    surface [1.5, 0.25, -2.0][i % 3], vocabs {200, 1500, 4096} x T {0.7, 1.0}
    x top_p {inf, 0.5, 0.9, 0.999} x top_k {None, 1, 10, 40, 2000}, skipping the
    temperature-only configs as the reference does.

Run: python tests/golden/make_golden.py
"""
import json
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from hi_amd.workloads import lcg_logits  # noqa: E402
from oracle import oracle as O  # noqa: E402

SAMPLES = [0.0, 0.13, 0.5, 0.77, 0.999]


def main():
    cases = []
    for vi, n in enumerate([64, 200, 1500, 4096]):
        x = lcg_logits(0x1234 + vi, n, 4.0)
        for t in [0.7, 1.0, 1.3]:
            for tp in [None, 0.5, 0.9, 0.95, 0.999]:
                for tk in [None, 1, 10, 40, 2000]:
                    for u in SAMPLES:
                        tok = O.ranked_sample_brute(x, t, float("inf") if tp is None else tp, tk, u)
                        cases.append(dict(grid="host", kind="lcg", seed=0x1234 + vi, n=n,
                                          temperature=t, top_p=tp, top_k=tk, sample=u, token=tok))
    for vi, n in enumerate([200, 1500, 4096]):
        for kind in ("lcg", "ties"):
            if kind == "lcg":
                x = lcg_logits(0x8F21 + vi, n, 4.0)
            else:
                x = np.array([[1.5, 0.25, -2.0][i % 3] for i in range(n)], np.float32)
            for t in [0.7, 1.0]:
                for tp in [None, 0.5, 0.9, 0.999]:
                    for tk in [None, 1, 10, 40, 2000]:
                        if tk is None and tp is None:
                            continue
                        for u in SAMPLES:
                            tok = O.ranked_sample_brute(x, t, float("inf") if tp is None else tp, tk, u)
                            cases.append(dict(grid="device", kind=kind,
                                              seed=0x8F21 + vi if kind == "lcg" else 0, n=n,
                                              temperature=t, top_p=tp, top_k=tk, sample=u,
                                              token=tok))
    out = os.path.join(os.path.dirname(os.path.abspath(__file__)), "reference_grid.json")
    with open(out, "w") as f:
        json.dump({"source": "gpu.rs:29505-29760 grids, expected by reference_ranked_sample",
                   "cases": cases}, f, separators=(",", ":"))
    print(f"wrote {len(cases)} cases to {out}")


if __name__ == "__main__":
    main()
