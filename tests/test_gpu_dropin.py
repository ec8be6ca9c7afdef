"""The drop-in `sample()` (same signature as mini_engine/sampling.py:30-35)
and the batched `sample_requests` on the GPU, against the CPU oracle fed the
same uniform the drop-in draws from the caller's generator.
"""

import sys

import numpy as np
import pytest
import torch

from mi355x_sampler import SamplingParams, sample, sample_batch, sample_requests
from mi355x_sampler.workloads import make_workload

pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def oracle_token(oracle, row, prm, hist, u):
    x = np.asarray(row, dtype=np.float32)[None, :]
    V = x.shape[1]
    h = [i + V if i < 0 else i for i in hist] if prm.repetition_penalty != 1.0 else []
    r = oracle.sample_rows(x, [prm.temperature], [prm.top_k], [prm.top_p],
                           [prm.repetition_penalty], [0, len(h)], np.asarray(h, np.int32), [u])
    return int(r.tokens[0]), int(r.status[0])


def params_of(w, r):
    return SamplingParams(temperature=float(w.temperature[r]), top_k=int(w.top_k[r]),
                          top_p=float(w.top_p[r]), repetition_penalty=float(w.penalty[r]))


@pytest.mark.parametrize("where", ["cpu", "gpu"])
@pytest.mark.parametrize("name", ["single", "zipf", "flat16", "greedy"])
def test_sample_matches_oracle(oracle, cuda, name, where):
    w = make_workload(name, B=3)
    say(f"[dropin] {name} logits on {where}")
    for r in range(w.B):
        prm = params_of(w, r)
        hist = w.hist_ids[w.hist_offsets[r]:w.hist_offsets[r + 1]].tolist()
        row = torch.from_numpy(w.logits[r].copy())
        if where == "gpu":
            row = row.to(cuda)
        for seed in (0, 1, 2):
            g = torch.Generator().manual_seed(seed)
            tok = sample(row, prm, hist, g)
            u = 0.0 if prm.greedy else torch.rand((), generator=torch.Generator().manual_seed(seed)).item()
            assert (tok, 0) == oracle_token(oracle, w.logits[r], prm, hist, u), (r, seed)
            # the generator advanced by exactly one draw (none for greedy)
            g2 = torch.Generator().manual_seed(seed)
            if not prm.greedy:
                torch.rand((), generator=g2)
            assert g.get_state().equal(g2.get_state())


def test_sample_leaves_caller_logits_alone(cuda):
    x = torch.randn(5000, device=cuda)
    before = x.clone()
    sample(x, SamplingParams(temperature=0.9, repetition_penalty=1.5), list(range(0, 5000, 3)))
    torch.cuda.synchronize()
    assert torch.equal(x, before)


def test_sample_other_dtypes_are_upcast(oracle, cuda):
    x = torch.randn(3000, dtype=torch.bfloat16)
    prm = SamplingParams(temperature=0.8, top_k=40, top_p=0.9, repetition_penalty=1.2)
    g = torch.Generator().manual_seed(5)
    tok = sample(x.to(cuda), prm, [1, 2, 3], g)
    u = torch.rand((), generator=torch.Generator().manual_seed(5)).item()
    assert (tok, 0) == oracle_token(oracle, x.float().numpy(), prm, [1, 2, 3], u)


def test_sample_raises_like_the_reference(cuda):
    x = torch.randn(1000, device=cuda)
    with pytest.raises(IndexError):
        sample(x, SamplingParams(repetition_penalty=1.2), [1000])
    with pytest.raises(RuntimeError):
        sample(x, SamplingParams(top_p=0.0), [])
    y = x.clone()
    y[7] = float("inf")
    with pytest.raises(RuntimeError):
        sample(y, SamplingParams(), [])
    assert sample(y, SamplingParams(temperature=0.0), []) == 7
    with pytest.raises(RuntimeError):
        sample(x, SamplingParams(temperature=float("nan")), [])
    with pytest.raises(ValueError):
        sample(x.view(10, 100), SamplingParams(), [])
    # negative history ids wrap once, as torch indexing does
    z = torch.zeros(1000, device=cuda)
    z[999] = 2.0
    z[5] = 1.9
    assert sample(z, SamplingParams(temperature=0.0, repetition_penalty=2.0), [-1]) == 5


def test_sample_requests_equals_per_row_sample(oracle, cuda):
    w = make_workload("zipf", B=12)
    logits = torch.from_numpy(w.logits).to(cuda)
    params = [params_of(w, r) for r in range(w.B)]
    params[3] = SamplingParams(temperature=0.0, repetition_penalty=1.4)   # a greedy row in the batch
    hists = [w.hist_ids[w.hist_offsets[r]:w.hist_offsets[r + 1]].tolist() for r in range(w.B)]
    say("[dropin] sample_requests vs sample")
    gens = [torch.Generator().manual_seed(100 + r) for r in range(w.B)]
    batched = sample_requests(logits, params, hists, gens)
    single = [sample(logits[r], params[r], hists[r], torch.Generator().manual_seed(100 + r))
              for r in range(w.B)]
    assert batched == single


def test_strided_and_unaligned_rows(oracle, cuda):
    """Rows with a leading dimension above V, including rows that do not start
    on a 16-byte boundary (read element by element)."""
    w = make_workload("zipf", B=6, V=40001)
    d = w.to_device(cuda)
    for ld in (40001, 40004, 40003, 50000):
        say(f"[strided] ld={ld}")
        big = torch.zeros((w.B, ld), dtype=torch.float32, device=cuda)
        big[:, :w.V] = d["logits"]
        d2 = dict(d, logits=big[:, :w.V])
        tok, st = sample_batch(**d2, return_status=True)
        ref = oracle.sample_rows(w.logits, w.temperature, w.top_k, w.top_p, w.penalty,
                                 w.hist_offsets, w.hist_ids, w.uniforms)
        assert np.array_equal(tok.cpu().numpy(), ref.tokens), ld
        assert np.array_equal(st.cpu().numpy(), ref.status), ld


def test_fp16_unaligned_rows(oracle, cuda):
    w = make_workload("flat16", B=4, V=30011)
    d = w.to_device(cuda)
    big = torch.zeros((w.B, 30013), dtype=torch.float16, device=cuda)
    big[:, :w.V] = d["logits"]
    tok, st = sample_batch(**dict(d, logits=big[:, :w.V]), return_status=True)
    ref = oracle.sample_rows(w.logits, w.temperature, w.top_k, w.top_p, w.penalty,
                             w.hist_offsets, w.hist_ids, w.uniforms)
    assert np.array_equal(tok.cpu().numpy(), ref.tokens)
    assert np.array_equal(st.cpu().numpy(), ref.status)
