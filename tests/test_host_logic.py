"""Host-side logic of the Python layer, on the CPU: the drop-in's dataclass,
request packing (parameters, CSR history, one uniform per stochastic row from
that row's generator), history index rules, the workloads and the loud
failure without a GPU.
"""

import dataclasses
import math
import os
import subprocess
import sys

import numpy as np
import pytest
import torch

from mi355x_sampler import SamplingParams, sample
from mi355x_sampler.batch import _normalize_history, pack_requests, raise_row_status
from mi355x_sampler.workloads import VOCAB, make_workload

ROOT = os.path.abspath(os.path.join(os.path.dirname(__file__), ".."))


def test_sampling_params_matches_reference_fields():
    # mini_engine/sampling.py:15-27
    f = {x.name: x for x in dataclasses.fields(SamplingParams)}
    assert list(f) == ["temperature", "top_k", "top_p", "repetition_penalty",
                       "max_new_tokens", "stop_token_ids", "seed"]
    p = SamplingParams()
    assert (p.temperature, p.top_k, p.top_p, p.repetition_penalty, p.max_new_tokens,
            p.stop_token_ids, p.seed) == (0.7, 0, 1.0, 1.0, 256, set(), None)
    assert SamplingParams(temperature=0.0).greedy and not p.greedy
    assert SamplingParams().stop_token_ids is not SamplingParams().stop_token_ids


def test_normalize_history_follows_torch_indexing():
    assert _normalize_history([0, 5, -1, -10], 10) == [0, 5, 9, 0]
    with pytest.raises(IndexError):
        _normalize_history([10], 10)
    with pytest.raises(IndexError):
        _normalize_history([-11], 10)


def test_pack_requests_layout_and_draws():
    V = 1000
    params = [SamplingParams(temperature=0.8, top_k=50, top_p=0.9, repetition_penalty=1.1),
              SamplingParams(temperature=0.0, repetition_penalty=1.3),
              SamplingParams(temperature=1.2, top_k=2**40, top_p=1.0),
              SamplingParams(temperature=0.5, repetition_penalty=1.0)]
    hists = [[1, 2, 2, -1], [7], [3, 4], [5, 6]]
    gens = [torch.Generator().manual_seed(s) for s in (11, 12, 13, 14)]
    d = pack_requests(params, hists, V, "cpu", gens)
    assert d["temperature"].tolist() == [np.float32(0.8), 0.0, np.float32(1.2), 0.5]
    assert d["top_k"].tolist() == [50, 0, 2**31 - 1, 0]
    assert d["top_p"].tolist() == [np.float32(0.9), 1.0, 1.0, 1.0]
    assert d["penalty"].tolist() == [np.float32(1.1), np.float32(1.3), 1.0, 1.0]
    # penalty 1.0 rows carry no history (sampling.py:38 skips it)
    assert d["hist_offsets"].tolist() == [0, 4, 5, 5, 5]
    assert d["hist_ids"].tolist() == [1, 2, 2, 999, 7]
    # one uniform per stochastic row from its own generator; greedy rows draw nothing
    ref = [torch.rand((), generator=torch.Generator().manual_seed(s)).item() for s in (11, 13, 14)]
    u = d["uniforms"].tolist()
    assert u[1] == 0.0 and [u[0], u[2], u[3]] == ref
    assert gens[1].get_state().equal(torch.Generator().manual_seed(12).get_state())


def test_temperatures_that_vanish_in_float32_become_row_errors():
    # sampling.py:47 tests the Python float, :50 divides by a float32 zero
    from mi355x_sampler.batch import device_temperature
    assert device_temperature(0.0) == 0.0 and device_temperature(-0.0) == 0.0
    assert math.isnan(device_temperature(1e-50)) and math.isnan(device_temperature(-1e-50))
    assert device_temperature(1e-40) == 1e-40 and device_temperature(0.7) == 0.7
    d = pack_requests([SamplingParams(temperature=1e-50), SamplingParams(temperature=0.0)],
                      [[], []], 10, "cpu")
    t = d["temperature"].tolist()
    assert math.isnan(t[0]) and t[1] == 0.0


def test_pack_requests_without_history():
    d = pack_requests([SamplingParams()] * 3, [[], [], []], 50, "cpu")
    assert d["hist_offsets"].tolist() == [0, 0, 0, 0] and d["hist_ids"].numel() == 0


def test_raise_row_status_maps_to_reference_exceptions():
    with pytest.raises(IndexError):
        raise_row_status(1)
    for s in (2, 3, 4, 9):
        with pytest.raises(RuntimeError):
            raise_row_status(s)


def test_workloads_are_deterministic_and_sized():
    a, b = make_workload("zipf", B=4), make_workload("zipf", B=4)
    assert np.array_equal(a.logits, b.logits) and np.array_equal(a.hist_ids, b.hist_ids)
    full = make_workload("zipf", B=2)
    assert full.V == VOCAB == 151936
    # per row: V*4 logits + 4*1024 history + 16 parameter bytes + 4 uniform + 8 token
    assert full.algorithmic_bytes() == 2 * (151936 * 4 + 4 * 1024 + 16 + 4 + 8)
    g = make_workload("greedy", B=3)
    assert g.algorithmic_bytes() == 3 * (151936 * 4 + 16 + 8)
    f = make_workload("flat16", B=2)
    assert f.logits.dtype == np.float16
    assert f.algorithmic_bytes() == 2 * (151936 * 2 + 4 * 2048 + 16 + 4 + 8)
    # rows are independent streams: row r is the same whatever B is
    assert np.array_equal(make_workload("peaked", B=2).logits[1], make_workload("peaked", B=5).logits[1])


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the no-GPU failure")
def test_sample_fails_loudly_without_a_gpu():
    with pytest.raises(Exception):
        sample(torch.zeros(16), SamplingParams(), [])
    from mi355x_sampler import sample_batch
    with pytest.raises(RuntimeError, match="HIP"):
        sample_batch(torch.zeros(1, 16), torch.ones(1), torch.zeros(1, dtype=torch.int32),
                     torch.ones(1), torch.ones(1))


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2 and "one GPU" in r.stderr
