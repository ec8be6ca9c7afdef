"""Replays tests/golden/reference_tokens.json, the token ids the reference's
own sample() (mini_engine/sampling.py:30-69) returned for seeded rows and
generator seeds (written by tests/golden/make_golden.py).

  * oracle/torch_chain.cpu_ref (unstable sort, torch.multinomial, the same
    generator seeds) must return the reference's token for every case and
    seed: this fixes the restatement's op order, history dedup, greedy exit,
    top-k tie rule and top-p cut against the reference itself.
  * the exact oracle must return the reference's token on greedy rows, and
    every token the reference drew must be one the oracle keeps (the oracle's
    draw consumes one uniform instead of V exponentials, so its realized
    token differs; its keep set must not).
  * the oracle's probabilities match torch's stable-sort chain within 1e-6,
    and its keep set is torch's, except tokens whose prefix mass lies within
    the fp32 chain's rounding window of top_p (oracle/margins.py).
"""

import json
import os

import numpy as np
import pytest
import torch

from mi355x_sampler.workloads import make_workload
from oracle import margins
from oracle.torch_chain import cpu_ref

HERE = os.path.dirname(os.path.abspath(__file__))
with open(os.path.join(HERE, "golden", "reference_tokens.json")) as f:
    GOLDEN = json.load(f)

_WL = {}


class Params:
    def __init__(self, T, k, p, pen):
        self.temperature, self.top_k, self.top_p, self.repetition_penalty = T, k, p, pen


def case_inputs(case):
    """(logits row as float32/float16 numpy, Params, history list)."""
    if case["kind"] == "inline":
        row = np.asarray(case["logits"], dtype=np.float32)
        return row, Params(float(np.float32(case["temperature"])), case["top_k"],
                           float(np.float32(case["top_p"])), float(np.float32(case["penalty"]))), \
            list(case["history"])
    key = (case["name"], case["B"])
    if key not in _WL:
        _WL[key] = make_workload(case["name"], B=case["B"])
    w = _WL[key]
    r = case["row"]
    hist = w.hist_ids[w.hist_offsets[r]:w.hist_offsets[r + 1]].tolist()
    return w.logits[r], Params(float(w.temperature[r]), int(w.top_k[r]), float(w.top_p[r]),
                               float(w.penalty[r])), hist


def case_id(case):
    if case["kind"] == "inline":
        return f"inline-{len(case['logits'])}-T{case['temperature']}-k{case['top_k']}"
    return f"{case['name']}-row{case['row']}"


CASES = GOLDEN["cases"]


@pytest.mark.parametrize("case", CASES, ids=[case_id(c) for c in CASES])
def test_torch_chain_reproduces_reference_tokens(case):
    row, prm, hist = case_inputs(case)
    got = []
    for s in case["gen_seeds"]:
        g = torch.Generator().manual_seed(s)
        got.append(cpu_ref(torch.from_numpy(row.copy()), prm, hist, g).token)
    assert got == case["tokens"]


@pytest.mark.parametrize("case", CASES, ids=[case_id(c) for c in CASES])
def test_oracle_keeps_reference_tokens(oracle, case):
    row, prm, hist = case_inputs(case)
    x = np.asarray(row, dtype=np.float32)[None, :]
    r = oracle.sample_rows(x, [prm.temperature], [prm.top_k], [prm.top_p],
                           [prm.repetition_penalty], [0, len(hist)],
                           np.asarray(hist, np.int32), [0.5], want_probs=True)
    assert r.status[0] == 0
    kept = r.probs[0] > 0
    if prm.temperature == 0.0:
        assert all(int(r.tokens[0]) == t for t in case["tokens"])
        return
    assert all(kept[t] for t in case["tokens"]), \
        [t for t in case["tokens"] if not kept[t]]
    # the oracle's probabilities against torch's fp32 chain with a stable sort
    # and against the same chain in float64 (oracle/margins.py): away from
    # the cut's rounding window the keep sets are identical and every
    # probability agrees within 1e-6; a row whose exact cut lies within
    # margins.BAND of a token's edge (the flat16 rows: one token there holds
    # about 1.8e-6 of the mass, and torch's fp32 prefix moves by up to
    # 2.5e-6) may keep or drop only tokens inside that window
    c = margins.compare_row(row, prm, hist, r.probs[0], r.info["p_margin"][0], r.info["n_kept"][0])
    assert margins.holds(c), c
    if r.info["p_margin"][0] > margins.BAND:
        assert c.keep_diff_fp32 == 0 and c.max_dprob <= 1e-6, c
