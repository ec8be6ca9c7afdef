"""Writes tests/golden/reference_tokens.json from the reference sampler.

Run in the build container only (the reference tree is not present on GPU
hosts):  python tests/golden/make_golden.py

For each case the reference's own `sample()` (mini_engine/sampling.py:30-69)
is called with a freshly seeded CPU torch.Generator, for several generator
seeds, and the returned token ids are recorded.  The inputs are not stored:
each case names a seeded workload row (mi355x_sampler.workloads) or a small
hand-written row given inline, so the fixture is a few KB.

What the vectors pin: tests/test_golden_reference.py replays every case
through oracle/torch_chain.cpu_ref (stable=False, multinomial draw) and
requires the same tokens, which fixes the restatement's op order, dedup,
greedy exit, top-k tie rule, top-p cut and draw against the reference itself.
"""

from __future__ import annotations

import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.abspath(os.path.join(HERE, "..", ".."))
sys.path.insert(0, os.path.join(ROOT, "llm-inference-scheduler_amd"))
sys.path.insert(0, "/root/reference")

from mini_engine.sampling import SamplingParams, sample  # noqa: E402  (reference)
from mi355x_sampler.workloads import make_workload  # noqa: E402

GEN_SEEDS = list(range(12))


def _params(T, k, p, pen):
    return SamplingParams(temperature=float(T), top_k=int(k), top_p=float(p),
                          repetition_penalty=float(pen))


def _tokens(row: np.ndarray, params, hist):
    out = []
    for s in GEN_SEEDS:
        g = torch.Generator().manual_seed(s)
        x = torch.from_numpy(row.copy())
        out.append(int(sample(x, params, list(hist), g)))
    return out


def workload_cases():
    cases = []
    picks = {"single": (1, [0]), "greedy": (4, [0, 1, 2, 3]),
             "peaked": (4, [0, 1, 2, 3]), "zipf": (12, list(range(12))),
             "flat16": (2, [0, 1])}
    for name, (B, rows) in picks.items():
        w = make_workload(name, B=B)
        for r in rows:
            hist = w.hist_ids[w.hist_offsets[r]:w.hist_offsets[r + 1]].tolist()
            params = _params(w.temperature[r], w.top_k[r], w.top_p[r], w.penalty[r])
            cases.append({"kind": "workload", "name": name, "B": B, "row": r,
                          "gen_seeds": GEN_SEEDS,
                          "tokens": _tokens(w.logits[r], params, hist)})
    return cases


def small_cases():
    """Hand-written rows that exercise edge rules on a tiny vocabulary."""
    specs = [
        # ties at the top-k threshold are all kept
        ([1.0, 3.0, 2.0, 3.0, 2.0, 2.0, 0.5, -1.0], 1.0, 3, 1.0, 1.0, []),
        # duplicate history ids penalize once
        ([2.0, -1.0, 0.5, 4.0, 4.0, -3.0], 0.9, 0, 1.0, 2.0, [3, 3, 3, 1, 1]),
        # greedy with penalty flips the winner; lowest index wins ties
        ([5.0, 4.0, 5.0, 1.0], 0.0, 0, 1.0, 1.5, [0]),
        # top_p small keeps only the first token of the sorted order
        ([0.1, 0.2, 3.0, 0.3, 2.9], 1.0, 0, 1e-6, 1.0, []),
        # top-k and top-p together
        ([0.0, 1.0, 2.0, 3.0, 4.0, 5.0, 6.0, 7.0], 2.0, 5, 0.6, 1.0, []),
        # negative temperature mirrors the reference's division
        ([0.5, -2.0, 1.5, -0.5], -1.0, 2, 1.0, 1.0, []),
        # penalty below one rewards history tokens
        ([1.0, 2.0, -1.0, 0.0], 1.0, 0, 0.95, 0.5, [0, 2, 3]),
    ]
    cases = []
    for (x, T, k, p, pen, hist) in specs:
        row = np.asarray(x, dtype=np.float32)
        cases.append({"kind": "inline", "logits": [float(v) for v in row],
                      "temperature": T, "top_k": k, "top_p": p, "penalty": pen,
                      "history": hist, "gen_seeds": GEN_SEEDS,
                      "tokens": _tokens(row, _params(T, k, p, pen), hist)})
    return cases


def main():
    doc = {
        "source": "mini_engine/sampling.py:30-69 (reference sample())",
        "torch": torch.__version__,
        "numpy": np.__version__,
        "cases": workload_cases() + small_cases(),
    }
    path = os.path.join(HERE, "reference_tokens.json")
    with open(path, "w") as f:
        json.dump(doc, f, indent=1)
    print(f"wrote {len(doc['cases'])} cases to {path}")


if __name__ == "__main__":
    main()
