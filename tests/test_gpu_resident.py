"""Histories resident on the device (HistoryStore, mxs_sample_ranges): a
decode loop that keeps each request's generated ids in a device buffer
samples exactly what the per-step repacking of req.output_ids samples
(mini_engine/scheduler.py:268-290), and ranges match the oracle fed the same
histories.
"""

import sys

import numpy as np
import pytest
import torch

from mi355x_sampler import (HistoryStore, SamplingParams, sample_batch_ranges, sample_requests,
                            sample_requests_resident)
from mi355x_sampler.workloads import VOCAB

pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def request_params(rng, n):
    out = []
    for i in range(n):
        kind = i % 4
        if kind == 0:
            out.append(SamplingParams(temperature=0.0, repetition_penalty=1.2))
        elif kind == 1:
            out.append(SamplingParams(temperature=0.8, top_k=50, top_p=0.9, repetition_penalty=1.1))
        elif kind == 2:
            out.append(SamplingParams(temperature=float(rng.uniform(0.3, 1.5)), top_k=0,
                                      top_p=0.95, repetition_penalty=1.05))
        else:
            out.append(SamplingParams(temperature=0.7, top_k=int(rng.integers(1, 1000)),
                                      top_p=float(rng.uniform(0.5, 1.0)), repetition_penalty=1.3))
    return out


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_resident_decode_loop_equals_repacking(cuda, dtype):
    """Eight decode steps over a changing subset of 12 requests: the same
    tokens from the resident store as from Python lists, and the store ends
    holding the lists."""
    rng = np.random.default_rng(3)
    S, V, steps = 12, VOCAB, 8
    params = request_params(rng, S)
    lists = [[int(t) for t in rng.integers(0, V, int(rng.integers(0, 40)))] for _ in range(S)]
    store = HistoryStore(S, 64, cuda)
    for s in range(S):
        store.reset(s, lists[s])
    gen_a = [torch.Generator().manual_seed(100 + s) for s in range(S)]
    gen_b = [torch.Generator().manual_seed(100 + s) for s in range(S)]
    for step in range(steps):
        active = sorted(rng.choice(S, int(rng.integers(3, S + 1)), replace=False).tolist())
        rng.shuffle(active)
        say(f"[resident] {dtype} step {step} rows {len(active)}")
        base = torch.from_numpy((2.0 * rng.standard_normal((len(active), V))).astype(np.float32))
        # favour some already generated ids, so the penalty changes tokens
        for r, s in enumerate(active):
            if lists[s]:
                base[r, torch.tensor(lists[s][-5:])] += 6.0
        logits = base.to(dtype).to(cuda)
        want = sample_requests(logits, [params[s] for s in active], [lists[s] for s in active],
                               [gen_a[s] for s in active])
        got = sample_requests_resident(logits, [params[s] for s in active], store, active,
                                       [gen_b[s] for s in active])
        assert got == want, (step, got, want)
        for s, t in zip(active, want):
            lists[s].append(t)
    for s in range(S):
        assert store.history(s) == lists[s], s


def test_ranges_match_the_oracle(oracle, cuda):
    """Overlapping, out-of-order and empty ranges, with probabilities."""
    rng = np.random.default_rng(9)
    V, B = VOCAB, 6
    x = (3.0 * rng.standard_normal((B, V))).astype(np.float32)
    ids = rng.integers(0, V, 400).astype(np.int32)
    top = np.argsort(-x, axis=1)[:, :4]
    ids[:8] = top[:2].reshape(-1)          # the maxima of rows 0 and 1 in the shared prefix
    begin = np.array([0, 0, 300, 50, 120, 10], np.int32)
    end = np.array([8, 200, 400, 50, 90, 399], np.int32)   # rows 3 and 4 empty
    T = np.array([0.0, 0.8, 1.1, 0.7, 0.9, 0.6], np.float32)
    K = np.array([0, 50, 0, 20, 1000, 0], np.int32)
    Pp = np.array([1.0, 0.9, 0.95, 0.8, 0.7, 0.5], np.float32)
    pen = np.array([1.3, 1.1, 1.05, 1.2, 0.8, 1.25], np.float32)
    u = rng.random(B).astype(np.float32)
    off = [0]
    flat = []
    for r in range(B):
        h = ids[begin[r]:end[r]].tolist() if end[r] > begin[r] else []
        flat += h
        off.append(len(flat))
    ref = oracle.sample_rows(x, T, K, Pp, pen, np.asarray(off, np.int32), np.asarray(flat, np.int32), u,
                             want_probs=True)
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(cuda)
    probs = torch.zeros((B, V), dtype=torch.float32, device=cuda)
    say(f"[resident] ranges B={B}")
    tok, st = sample_batch_ranges(d(x), d(T), d(K), d(Pp), d(pen), d(begin), d(end), d(ids), d(u),
                                  out_probs=probs, return_status=True)
    torch.cuda.synchronize()
    assert np.array_equal(st.cpu().numpy(), ref.status)
    assert np.array_equal(tok.cpu().numpy(), ref.tokens)
    assert np.abs(probs.cpu().numpy() - ref.probs).max() <= 1e-6
