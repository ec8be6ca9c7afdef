"""Pins each stage of the oracle's chain (oracle/sampler_oracle.c, restating
mini_engine/sampling.py:30-69) against an independent restatement:

  penalty      numpy fp32 closed form; duplicate-id known answers    (:38-45)
  greedy       numpy.argmax (first occurrence, NaN wins)             (:47-48)
  temperature  numpy fp32 IEEE division                               (:50)
  top-k        np.partition threshold, ties kept                      (:52-54)
  top-p        stable argsort + fp64 exp/cumsum cut; torch's own fp32
               chain (oracle/torch_chain.py, stable sort) away from the
               cut's rounding margin                                  (:56-66)
  softmax      fp64 closed form within 1e-6                           (:68)
  draw         u = 0 / u -> 1 end points, brute force over a u grid,
               chi-square of many draws against the probabilities     (:69)
  invariants   kept within top-k, nucleus mass >= top_p, keep set
               monotone in top_p, top_p -> 0 keeps the stable first
"""

import math

import numpy as np
import pytest
import torch

from oracle import margins
from oracle.torch_chain import cpu_ref


def run(oracle, x, T, k=0, p=1.0, pen=1.0, hist=(), u=0.5, probs=True):
    """One row through the oracle; returns (token, status, info, probs)."""
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32)[None, :])
    off = np.array([0, len(hist)], np.int32)
    ids = np.asarray(list(hist), np.int32)
    r = oracle.sample_rows(x, [T], [k], [p], [pen], off, ids, [u], want_probs=probs)
    return int(r.tokens[0]), int(r.status[0]), r.info[0], (r.probs[0] if probs else None)


def run_many(oracle, X, T, k, p, pen, hists, u, probs=True):
    X = np.ascontiguousarray(X, dtype=np.float32)
    B = X.shape[0]
    bc = lambda v, dt: np.broadcast_to(np.asarray(v, dtype=dt), (B,)).copy()
    off = np.zeros(B + 1, np.int32)
    off[1:] = np.cumsum([len(h) for h in hists])
    ids = np.asarray([i for h in hists for i in h], np.int32)
    return oracle.sample_rows(X, bc(T, np.float32), bc(k, np.int32), bc(p, np.float32),
                              bc(pen, np.float32), off, ids, bc(u, np.float32), want_probs=probs)


def np_penalize(x, hist, pen):
    y = x.astype(np.float32).copy()
    pen = np.float32(pen)
    for i in sorted(set(hist)):
        y[i] = y[i] / pen if y[i] > 0 else y[i] * pen
    return y


def np_tempered(x, T):
    return (x.astype(np.float32) / np.float32(T)).astype(np.float32)


def np_kth(l, k):
    V = l.size
    kk = min(k, V)
    return np.partition(l, V - kk)[V - kk]


def fp64_chain(x, T, k, p, pen, hist):
    """Independent fp64 restatement: kept mask (index order) and probs."""
    l = np_tempered(np_penalize(x, hist, pen), T)
    V = l.size
    keep = np.ones(V, bool)
    if k > 0:
        keep &= ~(l < np_kth(l, k))
    m = float(l[keep].max())
    w = np.where(keep, np.exp(l.astype(np.float64) - m), 0.0)
    if p < 1.0:
        order = np.argsort(-l, kind="stable")
        order = order[keep[order]]
        ws = w[order]
        excl = np.cumsum(ws) - ws
        drop = excl >= np.float64(np.float32(p)) * ws.sum()
        keep[order[drop]] = False
        w[order[drop]] = 0.0
    return keep, w / w.sum()


# ---------------------------------------------------------------- penalty

def test_penalty_known_answers(oracle):
    # applied once per unique id: 4/1.2 = 3.33 > 3 keeps id 0; twice would not
    assert run(oracle, [4.0, 3.0], 0.0, pen=1.2, hist=[0, 0, 0])[0] == 0
    assert run(oracle, [4.0, 3.0], 0.0, pen=1.2 * 1.2, hist=[0])[0] == 1
    # negative logits are multiplied, not divided
    assert run(oracle, [-1.0, -1.1], 0.0, pen=1.2, hist=[0])[0] == 1
    # penalty below one rewards history ids
    assert run(oracle, [1.0, 1.5], 0.0, pen=0.5, hist=[0])[0] == 0
    # penalty 1.0 leaves the row alone even with a history
    assert run(oracle, [1.0, 1.0 + 2**-20], 0.0, pen=1.0, hist=[1])[0] == 1


def test_penalty_matches_numpy(oracle):
    rng = np.random.default_rng(21)
    B, V = 300, 64
    X = rng.standard_normal((B, V)).astype(np.float32)
    pens = rng.uniform(0.5, 2.0, B).astype(np.float32)
    hists = [list(rng.integers(0, V, rng.integers(0, 40))) for _ in range(B)]
    r = run_many(oracle, X, 0.0, 0, 1.0, pens, hists, 0.0, probs=False)
    want = [int(np.argmax(np_penalize(X[b], hists[b], pens[b]))) for b in range(B)]
    assert list(r.tokens) == want


# ---------------------------------------------------------------- greedy

def test_greedy_first_index_and_nan(oracle):
    rng = np.random.default_rng(2)
    X = np.round(rng.standard_normal((200, 1000)) * 2).astype(np.float32)   # many ties
    X[5, 17] = np.nan
    X[5, 900] = np.nan
    X[6, :] = -np.inf
    X[7, 3] = np.inf
    r = run_many(oracle, X, 0.0, 0, 1.0, 1.0, [[]] * 200, 0.0, probs=False)
    assert list(r.tokens) == [int(np.argmax(row)) for row in X]
    assert r.tokens[5] == 17 and r.tokens[6] == 0 and r.tokens[7] == 3
    assert np.all(r.status == 0)


# ------------------------------------------------------ temperature and top-k

@pytest.mark.parametrize("T", [0.3, 0.7, 1.0, 1.37, -0.9, 1e-3])
def test_topk_threshold_and_count(oracle, T):
    rng = np.random.default_rng(int(abs(T) * 1000))
    B, V = 40, 5000
    X = (rng.standard_normal((B, V)) * 3).astype(np.float32)
    X[::3] = np.round(X[::3])                   # coarse values: ties at the threshold
    ks = rng.integers(1, 1500, B).astype(np.int32)
    r = run_many(oracle, X, T, ks, 1.0, 1.0, [[]] * B, 0.5, probs=True)
    for b in range(B):
        l = np_tempered(X[b], T)
        kth = np_kth(l, int(ks[b]))
        assert np.float32(r.info["kth"][b]) == kth
        n = int(np.count_nonzero(l >= kth))
        assert r.info["n_topk"][b] == n
        assert n >= ks[b]
        assert np.array_equal(r.probs[b] > 0, (l >= kth) & (np.exp(l.astype(np.float64) - l.max()) * 2.0**44 >= 1))


def test_topk_edges(oracle):
    x = np.float32([1.0, 3.0, 2.0, 3.0, 2.0, 2.0, 0.5, -1.0])
    assert run(oracle, x, 1.0, k=3)[2]["n_topk"] == 5      # 3, 3, 2, 2, 2: ties kept
    assert run(oracle, x, 1.0, k=8)[2]["n_topk"] == 8      # k = V keeps all
    assert run(oracle, x, 1.0, k=50)[2]["n_topk"] == 8     # k > V keeps all
    assert run(oracle, x, 1.0, k=1)[2]["n_topk"] == 2      # k = 1 keeps the tied maxima


# ---------------------------------------------------------------- top-p

def _rows(seed, B, V):
    rng = np.random.default_rng(seed)
    X = (rng.standard_normal((B, V)) * rng.uniform(0.5, 4.0, (B, 1))).astype(np.float32)
    T = rng.uniform(0.3, 1.5, B).astype(np.float32)
    k = np.where(rng.random(B) < 0.5, 0, rng.integers(1, 600, B)).astype(np.int32)
    p = rng.uniform(0.05, 0.999, B).astype(np.float32)
    pen = rng.uniform(1.0, 1.3, B).astype(np.float32)
    hists = [list(rng.integers(0, V, 64)) for _ in range(B)]
    u = rng.random(B).astype(np.float32)
    return X, T, k, p, pen, hists, u


def test_topp_and_softmax_vs_fp64(oracle):
    X, T, k, p, pen, hists, u = _rows(31, 48, 3000)
    r = run_many(oracle, X, T, k, p, pen, hists, u)
    checked = 0
    for b in range(X.shape[0]):
        keep, probs = fp64_chain(X[b], T[b], int(k[b]), float(p[b]), float(pen[b]), hists[b])
        # the cut compares integer masses; fp64 exp differs by < 1e-7 relative,
        # so only a cut within margins.FP64_BAND of a token's edge may differ
        if r.info["p_margin"][b] > margins.FP64_BAND:
            assert np.array_equal(r.probs[b] > 0, keep), b
            assert np.abs(r.probs[b] - probs).max() <= 1e-6, b
            checked += 1
        else:
            assert ((r.probs[b] > 0) != keep).sum() <= 1, b
    assert checked >= 40


def test_topp_vs_torch_chain(oracle):
    """torch's fp32 softmax/cumsum (sampling.py:58-62) with a stable sort keeps
    the same set whenever the exact cut is clear of fp32 rounding."""
    X, T, k, p, pen, hists, u = _rows(32, 32, 20000)
    r = run_many(oracle, X, T, k, p, pen, hists, u)

    class P:
        pass
    checked = 0
    for b in range(X.shape[0]):
        prm = P()
        prm.temperature, prm.top_k = float(T[b]), int(k[b])
        prm.top_p, prm.repetition_penalty = float(p[b]), float(pen[b])
        hist = [int(i) for i in hists[b]]
        tr = cpu_ref(torch.from_numpy(X[b].copy()), prm, hist, stable=True, draw="none")
        assert r.info["n_topk"][b] == tr.n_topk
        if r.info["p_margin"][b] > margins.BAND:
            assert np.array_equal(r.probs[b] > 0, tr.kept.numpy()), b
            assert np.abs(r.probs[b] - tr.probs.numpy()).max() <= 1e-6, b
            checked += 1
        # every row, margin rows included: tokens that only one side keeps lie
        # within margins.BAND of top_p in prefix mass, and probabilities
        # agree within 1e-6 on every other token
        c = margins.compare_row(X[b], prm, hist, r.probs[b], r.info["p_margin"][b], r.info["n_kept"][b])
        assert margins.holds(c), (b, c)
    assert checked >= 25


def test_topp_exact_boundary(oracle):
    # four equal logits: every mass is exactly 2^44, the cut at top_p = 0.5
    # falls exactly on position 2 (cumsum - probs = 0, .25, .5, .75, all exact
    # in fp32), so positions 2 and 3 go, as in sampling.py:62
    x = np.zeros(4, np.float32)
    assert run(oracle, x, 1.0, p=0.5)[2]["n_kept"] == 2
    assert run(oracle, x, 1.0, p=0.25)[2]["n_kept"] == 1
    assert run(oracle, x, 1.0, p=np.float32(0.5) + np.float32(2**-24))[2]["n_kept"] == 3


def test_topp_invariants(oracle):
    X, T, k, _, pen, hists, u = _rows(33, 16, 4000)
    ps = [1e-7, 0.1, 0.3, 0.5, 0.8, 0.95, 0.999]
    prev = None
    for p in ps:
        r = run_many(oracle, X, T, k, p, pen, hists, u)
        kept = r.probs > 0
        for b in range(X.shape[0]):
            l = np_tempered(np_penalize(X[b], hists[b], pen[b]), T[b])
            if k[b] > 0:
                assert not np.any(kept[b] & (l < np_kth(l, int(k[b]))))   # within top-k
            if p == 1e-7:
                first = int(np.argsort(-l, kind="stable")[0])
                assert kept[b].sum() == 1 and kept[b, first]
            # kept mass reaches top_p of the top-k mass (fp64, from the logits)
            w = np.exp(l.astype(np.float64) - l.max())
            tk = ~(l < np_kth(l, int(k[b]))) if k[b] > 0 else np.ones_like(kept[b])
            assert w[kept[b]].sum() >= p * w[tk].sum() * (1 - 1e-6)
            assert kept[b, r.tokens[b]]
        if prev is not None:
            assert np.all(kept[prev]), "keep set must grow with top_p"
        prev = kept.copy()
    assert np.allclose(r.probs.sum(axis=1), 1.0, atol=1e-5)


# ---------------------------------------------------------------- draw

def _sorted_kept(probs_row, l):
    order = np.argsort(-l, kind="stable")
    return [int(i) for i in order if probs_row[i] > 0]


def test_draw_end_points(oracle):
    rng = np.random.default_rng(41)
    x = rng.standard_normal(12).astype(np.float32)
    below_one = float(np.nextafter(np.float32(1.0), np.float32(0.0)))
    for T, k, p in [(1.0, 0, 1.0), (0.7, 5, 1.0), (1.3, 0, 0.8), (0.9, 8, 0.6)]:
        _, _, _, probs = run(oracle, x, T, k, p, u=0.0)
        order = _sorted_kept(probs, np_tempered(x, T))
        assert run(oracle, x, T, k, p, u=0.0)[0] == order[0]
        assert run(oracle, x, T, k, p, u=below_one)[0] == order[-1]
        assert run(oracle, x, T, k, p, u=2.0)[0] == order[-1]       # clamped
        assert run(oracle, x, T, k, p, u=-1.0)[0] == order[0]       # clamped
    # tied values: the sorted order puts the lower index first
    y = np.float32([1.0, 3.0, 2.0, 3.0, 3.0])
    assert run(oracle, y, 1.0, p=1e-7)[0] == 1
    assert run(oracle, y, 1.0, p=0.5, u=0.0)[0] == 1
    assert run(oracle, y, 1.0, p=0.5, u=below_one)[0] == 3


def test_draw_half_open_intervals(oracle):
    # equal masses: token i owns u in [i/4, (i+1)/4); u on a boundary belongs
    # to the token that starts there
    x = np.zeros(4, np.float32)
    for u, want in [(0.0, 0), (0.2499999, 0), (0.25, 1), (0.5, 2), (0.75, 3), (0.9999999, 3)]:
        assert run(oracle, x, 1.0, u=u)[0] == want, u


def test_draw_brute_force_small_vocab(oracle):
    rng = np.random.default_rng(42)
    grid = (np.arange(2000, dtype=np.float64) + 0.5) / 2000
    for trial in range(6):
        V = int(rng.integers(2, 17))
        x = (rng.standard_normal(V) * 1.5).astype(np.float32)
        T, k, p = float(rng.uniform(0.4, 1.5)), int(rng.integers(0, V + 1)), float(rng.uniform(0.3, 1.0))
        _, _, _, probs = run(oracle, x, T, k, p)
        order = _sorted_kept(probs, np_tempered(x, T))
        cum = np.cumsum(probs[order].astype(np.float64))
        us = grid.astype(np.float32)
        r = run_many(oracle, np.repeat(x[None], len(us), 0), T, k, p, 1.0, [[]] * len(us), us,
                     probs=False)
        for u, tok in zip(us.astype(np.float64), r.tokens):
            j = int(np.searchsorted(cum, u, side="right"))
            if np.min(np.abs(cum - u)) < 1e-6:
                continue                                  # on a boundary
            assert tok == order[min(j, len(order) - 1)], (trial, u)


def test_draw_chi_square(oracle):
    from scipy.stats import chisquare
    rng = np.random.default_rng(43)
    x = (rng.standard_normal(10) * 0.8).astype(np.float32)
    N = 200000
    us = rng.random(N).astype(np.float32)
    r = run_many(oracle, np.repeat(x[None], N, 0), 0.9, 0, 0.9, 1.0, [[]] * N, us, probs=False)
    _, _, _, probs = run(oracle, x, 0.9, 0, 0.9)
    kept = np.nonzero(probs > 0)[0]
    counts = np.array([np.count_nonzero(r.tokens == i) for i in kept])
    assert counts.sum() == N
    stat = chisquare(counts, probs[kept].astype(np.float64) * N / probs[kept].sum())
    assert stat.pvalue > 1e-3, stat


# ---------------------------------------------------------------- statuses

def test_row_statuses(oracle):
    x = np.zeros(16, np.float32)
    assert run(oracle, x, 0.8, pen=1.2, hist=[16])[:2] == (-1, 1)       # id >= V
    assert run(oracle, x, 0.8, pen=1.2, hist=[-1])[:2] == (-1, 1)       # negative id
    assert run(oracle, x, 0.8, pen=1.0, hist=[99])[1] == 0              # penalty off: ids unread
    assert run(oracle, x, float("nan"))[:2] == (-1, 2)
    y = x.copy(); y[3] = np.inf
    assert run(oracle, y, 0.8)[:2] == (-1, 3)                            # inf after temperature
    assert run(oracle, y, 0.0)[:2] == (3, 0)                             # greedy takes the inf
    assert run(oracle, y, float("inf"))[:2] == (-1, 3)                   # inf / inf is NaN
    z = x.copy(); z[5] = -1.0
    assert run(oracle, z, float("inf"))[1] == 0                          # finite / inf is 0
    n = x.copy(); n[9] = np.frombuffer(np.uint32(0xFFC00000).tobytes(), np.float32)[0]
    assert run(oracle, n, 0.8)[:2] == (-1, 3)                            # a NaN of either sign
    assert run(oracle, n, 0.8, k=2)[:2] == (-1, 3)
    assert run(oracle, x, 0.8, p=0.0)[:2] == (-1, 4)                     # top_p <= 0 keeps nothing
    assert run(oracle, x, 0.8, p=-1.0)[:2] == (-1, 4)
