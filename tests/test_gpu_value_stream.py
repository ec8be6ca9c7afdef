"""GPU parity for the top-k stream that tests hits on the values themselves.

The stream of the one-workgroup-per-row kernel (batches above 64 rows)
compares each logit with the value of the sampled bound (x >= tf, or
x <= tf for T < 0) instead of forming its selection key, keeps NaN-
propagating value extremes, and appends raw bits that the count pass turns
into keys.  These cases aim at what that changes: signed zeros on both
sides of the k-th value (a value test cannot tell -0 from +0, keys can),
both temperature signs, deferred and inline penalties, NaN and infinite
logits, masked rows, large ties at the k-th value, rows whose bound admits
most of the row, and rows that do not start on a 16-byte boundary (they
take the element-by-element loop, which visits every slot).  Token ids and
row statuses must equal the oracle's; probabilities within 1e-6.
"""

import numpy as np
import pytest
import torch

from mi355x_sampler import sample_batch
from mi355x_sampler.workloads import VOCAB

from test_gpu_parity import check, custom, run_oracle, say

pytestmark = pytest.mark.gpu

V = VOCAB
B_ROWS = 72          # above the small-batch split: one workgroup per row


def _rows(seed):
    rng = np.random.default_rng(seed)
    rows, params = [], []

    def add(r, T, k, p, pen, hist, u):
        rows.append(np.asarray(r, np.float32)); params.append((T, k, p, pen, list(hist), u))

    # signed zeros straddling the k-th value: 3000 zeros (half -0.0), all else below
    for T in (0.8, -0.8):
        base = (rng.standard_normal(V) * 0.1 - 3.0).astype(np.float32)
        if T < 0:
            base = -base                       # reversed order: the zeros lead again
        zi = rng.choice(V, 3000, replace=False)
        base[zi] = np.where(rng.random(3000) < 0.5, 0.0, -0.0).astype(np.float32)
        for k in (100, 1500, 2999, 3000, 3001):
            add(base.copy(), T, k, 0.9, 1.0, [], rng.random())
        hist = rng.choice(zi, 64, replace=False).tolist() + rng.choice(V, 64).tolist()
        add(base.copy(), T, 1000, 1.0, 1.15, hist, rng.random())     # penalty on zeros (no-op) and others
        add(base.copy(), T, 1000, 0.95, 0.85, hist, rng.random())    # penalty < 1: applied inline
    # a few positive values above a wall of signed zeros: the k-th is a zero
    w = np.full(V, -0.0, np.float32); w[rng.choice(V, V // 2, replace=False)] = 0.0
    w[rng.choice(V, 7, replace=False)] = rng.random(7).astype(np.float32) + 0.5
    for k in (5, 7, 8, 50):
        add(w.copy(), 0.6, k, 0.8, 1.0, [], rng.random())
    # negative temperatures with deferred-looking penalties (applied inline for T < 0)
    n = (rng.standard_normal(V) * 3).astype(np.float32)
    for pen in (1.0, 1.2, 0.7):
        add(n.copy(), -0.9, 40, 0.9, pen, rng.choice(V, 512).tolist(), rng.random())
    # NaN (both signs) and infinities in the streamed row
    for bits in (0x7FC00000, 0xFFC00000):
        r = n.copy(); r[rng.integers(V)] = np.frombuffer(np.uint32(bits).tobytes(), np.float32)[0]
        add(r, 0.8, 50, 0.9, 1.1, rng.choice(V, 64).tolist(), 0.5)
    r = n.copy(); r[rng.integers(V)] = np.inf
    add(r, 0.8, 50, 0.9, 1.0, [], 0.5)                                   # +inf maximum
    r = n.copy(); r[rng.choice(V, 5, replace=False)] = -np.inf
    add(r, 0.8, 50, 0.9, 1.1, [], 0.5)                                   # -inf entries below the bound
    r = n.copy(); r[rng.integers(V)] = -np.inf
    add(r, -0.8, 50, 0.9, 1.0, [], 0.5)                                  # -inf / T < 0 is +inf
    # masks: most of the row -inf; the k-th finite, and the k-th masked
    m = n.copy(); m[rng.choice(V, V - 4000, replace=False)] = -np.inf
    add(m.copy(), 1.0, 1000, 0.95, 1.1, rng.choice(V, 256).tolist(), rng.random())
    m2 = np.full(V, -np.inf, np.float32); m2[rng.choice(V, 30, replace=False)] = rng.standard_normal(30)
    add(m2, 1.0, 100, 0.9, 1.0, [], rng.random())
    # a tie of 5000 equal values at the k-th
    t = (rng.standard_normal(V) - 4.0).astype(np.float32); t[rng.choice(V, 5000, replace=False)] = 1.0
    t[rng.choice(V, 20, replace=False)] = 2.0
    for k in (10, 20, 21, 1000):
        add(t.copy(), 0.7, k, 0.97, 1.05, rng.choice(V, 300).tolist(), rng.random())
    # flat rows: the sampled bound admits a large share of the row
    f = np.zeros(V, np.float32); f[rng.choice(V, 2, replace=False)] = 1e-3
    add(f, 1.0, 1024, 0.5, 1.0, [], rng.random())
    # fill up with plain Zipf-like rows of mixed parameters
    while len(rows) < B_ROWS:
        rank = rng.permutation(V) + 1
        z = (-1.1 * np.log(rank) + 0.1 * rng.standard_normal(V)).astype(np.float32)
        add(z, float(rng.uniform(0.3, 1.5)) * (1 if rng.random() < 0.8 else -1), int(rng.integers(1, 1001)),
            float(rng.uniform(0.5, 1.0)), float(rng.uniform(0.8, 1.3)), rng.choice(V, 1024).tolist(), rng.random())
    return rows, params


def _workload(seed):
    rows, params = _rows(seed)
    assert len(rows) == B_ROWS
    T, k, p, pen, hists, u = zip(*params)
    return custom(f"value-stream-{seed}", np.stack(rows), list(T), list(k), list(p), list(pen),
                  list(hists), list(u))


@pytest.mark.parametrize("offset", [0, 1, 3])
def test_value_stream_matches_the_oracle(oracle, cuda, offset):
    """offset 0: rows on 16-byte boundaries (vector loads); 1 and 3: rows
    that start inside a vector (the element-by-element loop)."""
    w = _workload(900 + offset)
    say(f"[value-stream] B={w.B} V={w.V} row offset {offset} floats")
    dev = torch.device("cuda", 0)
    d = w.to_device(dev)
    if offset:
        big = torch.empty((w.B, w.V + 4), dtype=torch.float32, device=dev)
        big[:, offset:offset + w.V] = d["logits"]
        d["logits"] = big[:, offset:offset + w.V]
    out = torch.zeros((w.B, w.V), dtype=torch.float32, device=dev)
    tok, st = sample_batch(**d, out_probs=out, return_status=True)
    torch.cuda.synchronize()
    ref = run_oracle(oracle, w)
    check(w, ref, tok.cpu().numpy(), st.cpu().numpy(), out.cpu().numpy())
