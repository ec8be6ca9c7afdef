"""Seeded random batches that mix every row mode in one launch: greedy,
top-k below and above the candidate cap, top-k off, negative and extreme
temperatures, top-p off / tiny / ordinary, penalties above and below 1 with
long, repeating histories, and logits that are Gaussian at several widths,
Zipf-shaped, quantized into heavy ties or partly masked.  fp32 and fp16,
vocabularies from 17 to 151,936.  Tokens and statuses must equal the
oracle's, probabilities within 1e-6.
"""

import sys

import numpy as np
import pytest
import torch

from mi355x_sampler import sample_batch
from mi355x_sampler.workloads import VOCAB, Workload

pytestmark = pytest.mark.gpu

PROB_TOL = 1e-6


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def random_batch(seed, V, B, dtype):
    rng = np.random.default_rng(seed)
    x = np.empty((B, V), np.float32)
    for r in range(B):
        kind = rng.integers(0, 6)
        if kind == 0:
            x[r] = rng.standard_normal(V) * rng.choice([0.1, 1.0, 3.0])
        elif kind == 1:    # Zipf-shaped under a permutation
            x[r] = -1.1 * np.log(rng.permutation(V) + 1.0) + 0.1 * rng.standard_normal(V)
        elif kind == 2:    # heavy ties
            x[r] = rng.integers(0, int(rng.integers(2, 9)), V) * 0.5
        elif kind == 3:    # a few peaks over a flat floor
            x[r] = rng.standard_normal(V)
            x[r, rng.choice(V, min(V, 5), replace=False)] += 12.0
        elif kind == 4:    # partly masked
            x[r] = 2.0 * rng.standard_normal(V)
            x[r, rng.random(V) < rng.uniform(0.1, 0.9)] = -np.inf
        else:
            x[r] = rng.standard_normal(V)
            if rng.random() < 0.5:
                x[r, int(rng.integers(0, V))] = np.nan
    T = np.where(rng.random(B) < 0.15, 0.0, rng.uniform(0.2, 1.6, B)).astype(np.float32)
    T[rng.random(B) < 0.08] *= -1.0
    T[rng.random(B) < 0.04] = 1e-3
    k = np.where(rng.random(B) < 0.35, 0, rng.integers(1, 1100, B)).astype(np.int32)
    k[rng.random(B) < 0.08] = 2000
    k[rng.random(B) < 0.05] = V
    p = np.where(rng.random(B) < 0.3, 1.0, rng.uniform(0.05, 1.0, B)).astype(np.float32)
    p[rng.random(B) < 0.05] = 1e-6
    pen = np.where(rng.random(B) < 0.3, 1.0, rng.uniform(0.6, 1.4, B)).astype(np.float32)
    hists = []
    for r in range(B):
        n = int(rng.choice([0, 1, 64, 700, 2500]))
        h = rng.integers(0, V, n)
        if n and rng.random() < 0.5:   # repeats, and the row's maxima in the history
            h[: n // 4] = h[0]
            order = np.argsort(-np.nan_to_num(x[r], nan=-np.inf), kind="stable")
            h[n // 4: n // 4 + min(3, n - n // 4)] = order[: min(3, n - n // 4)]
        hists.append(h.astype(np.int32))
    off = np.zeros(B + 1, np.int32)
    off[1:] = np.cumsum([len(h) for h in hists])
    ids = np.concatenate(hists) if off[-1] else np.zeros(0, np.int32)
    u = rng.random(B).astype(np.float32)
    logits = x.astype(np.float16) if dtype == "f16" else x
    return Workload(f"mix{seed}", logits, T, k, p, pen, off, ids.astype(np.int32), u)


SIZES = [(VOCAB, 24), (40000, 32), (65537, 16), (4099, 40), (17, 40), (1000, 40), (32768, 24),
         (VOCAB, 12)]
CASES = [(seed, *SIZES[(seed - 1) % len(SIZES)], "f32" if seed % 2 else "f16") for seed in range(1, 25)]


@pytest.mark.parametrize("seed,V,B,dtype", CASES)
def test_random_mixed_batches(oracle, cuda, seed, V, B, dtype):
    w = random_batch(seed, V, B, dtype)
    probs = seed % 2 == 1
    say(f"[mix] seed={seed} V={V} B={B} {dtype} probs={probs}")
    ref = oracle.sample_rows(w.logits, w.temperature, w.top_k, w.top_p, w.penalty,
                             w.hist_offsets, w.hist_ids, w.uniforms, want_probs=probs)
    d = w.to_device(cuda)
    out = torch.zeros((w.B, w.V), dtype=torch.float32, device=cuda) if probs else None
    tok, st = sample_batch(**d, out_probs=out, return_status=True)
    torch.cuda.synchronize()
    st = st.cpu().numpy()
    tok = tok.cpu().numpy()
    assert np.array_equal(st, ref.status), f"status gpu {st} oracle {ref.status}"
    bad = np.nonzero(tok != ref.tokens)[0]
    assert bad.size == 0, f"rows {bad}: gpu {tok[bad]} oracle {ref.tokens[bad]}"
    if probs:
        err = np.abs(out.cpu().numpy() - ref.probs).max()
        assert err <= PROB_TOL, err
