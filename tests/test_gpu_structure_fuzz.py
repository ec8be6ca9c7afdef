"""Seeded structure fuzz: GPU sampler vs the oracle on pathological rows.

Each row is drawn from a palette of shapes that stress different paths of
the kernels: dense normal rows, rows masked with -inf almost everywhere
(the few finite values anywhere in the row, including its end), walls of
signed zeros, rows over a small alphabet of values (huge ties), Zipf rows,
and sprinkled NaN and infinities.  Parameters are drawn with their edge
values (greedy, negative and infinite temperatures, top_k 1, <= 1024,
> 1024 and >= V, top_p 1 and tiny, penalties below, at and above 1, long
histories with repeats and ids at the row's ends).  Batches of 72 rows take
the one-workgroup-per-row launch; batches of 16 the small-batch split.
Token ids and row statuses must equal the oracle's, probabilities within
1e-6.
"""

import numpy as np
import pytest

from mi355x_sampler.workloads import VOCAB

from test_gpu_parity import check, custom, run_gpu, run_oracle, say

pytestmark = pytest.mark.gpu

V = VOCAB


def _row(rng, kind, dtype):
    if kind == "normal":
        r = rng.standard_normal(V) * rng.choice([0.5, 3.0, 20.0])
    elif kind == "masked":
        r = rng.standard_normal(V) * 2.0
        r[rng.random(V) < rng.choice([0.5, 0.99, 0.9999])] = -np.inf
    elif kind == "few":
        r = np.full(V, -np.inf)
        n = int(rng.integers(1, 200))
        idx = rng.choice(V, n, replace=False)
        if rng.random() < 0.5:
            idx[0] = V - 1 - int(rng.integers(0, 8))      # one near the row's end
        r[idx] = rng.standard_normal(n)
    elif kind == "zeros":
        r = np.where(rng.random(V) < 0.5, 0.0, -0.0)
        n = int(rng.integers(0, 50))
        r[rng.choice(V, n, replace=False)] = rng.standard_normal(n)
    elif kind == "alphabet":
        r = rng.choice(rng.standard_normal(int(rng.integers(2, 12))), V)
    else:  # zipf
        rank = rng.permutation(V) + 1
        r = -1.1 * np.log(rank) + 0.1 * rng.standard_normal(V)
    r = r.astype(dtype)
    if rng.random() < 0.08:
        r[rng.integers(V)] = rng.choice([np.nan, np.inf, -np.inf]).astype(dtype)
    return r


def _params(rng):
    T = float(rng.choice([0.0, 0.7, 1.3, -0.8, 0.05, 5.0, np.inf], p=[.15, .3, .15, .1, .1, .1, .1]))
    k = int(rng.choice([0, 1, int(rng.integers(2, 64)), int(rng.integers(64, 1025)),
                        int(rng.integers(1025, 5000)), V]))
    p = float(rng.choice([1.0, 0.9, 0.5, 1e-6, float(rng.uniform(0.05, 1.0))]))
    pen = float(rng.choice([1.0, 1.0, 1.1, 1.3, 0.8, 2.0]))
    n = int(rng.choice([0, 1, 64, 1024, 2048]))
    hist = rng.integers(0, V, n)
    if n > 4:
        hist[:4] = [0, V - 1, hist[4], hist[4]]                    # ends of the row, a repeat
    return T, k, p, pen, hist.tolist(), float(rng.random())


def _batch(seed, B, dtype):
    rng = np.random.default_rng(seed)
    kinds = ["normal", "masked", "few", "zeros", "alphabet", "zipf"]
    rows, params = [], []
    for i in range(B):
        rows.append(_row(rng, kinds[i % len(kinds)] if i < len(kinds) else rng.choice(kinds), dtype))
        params.append(_params(rng))
    T, k, p, pen, hists, u = zip(*params)
    return custom(f"fuzz-{seed}-{B}-{np.dtype(dtype).name}", np.stack(rows), list(T), list(k), list(p),
                  list(pen), list(hists), list(u))


@pytest.mark.parametrize("seed,B,dtype", [
    (7001, 72, np.float32), (7002, 72, np.float32), (7003, 16, np.float32),
    (7004, 72, np.float16), (7005, 16, np.float16), (7006, 72, np.float32),
])
def test_structure_fuzz(oracle, cuda, seed, B, dtype):
    w = _batch(seed, B, dtype)
    say(f"[fuzz] seed {seed} B={B} {np.dtype(dtype).name}")
    tok, st, probs = run_gpu(w, cuda)
    check(w, run_oracle(oracle, w), tok, st, probs)
