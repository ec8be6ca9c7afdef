"""The oracle's exact top-p cut against the reference's fp32 chain, row by
row, on rows of every benchmark shape (CPU only).

mini_engine/sampling.py:57-62 cuts where torch's fp32 prefix of the sorted
softmax reaches top_p.  On the flat16 rows one token near the cut holds
about 1.8e-6 of the mass while torch's fp32 prefix there deviates from the
exact one by up to 2.5e-6, so the reference's own last kept token depends on
the rounding of its CPU kernels.  The statement every row is held to
(oracle/margins.holds):

  * the same chain with float64 softmax and cumsum keeps exactly the
    oracle's tokens, except tokens within FP64_BAND (2e-7) of top_p in
    prefix mass;
  * torch's fp32 chain (stable sort) keeps exactly the oracle's tokens,
    except tokens within BAND (1e-5) of top_p in prefix mass;
  * post-filter probabilities agree within 1e-6 on every other token, and on
    such a boundary token by at most its own probability (+1e-6).

python -m oracle.margins prints the same comparison over every row of the
five benchmark batches.
"""

import numpy as np
import pytest

from mi355x_sampler.workloads import make_workload
from oracle import margins


@pytest.mark.parametrize("name,rows", [("single", 1), ("peaked", 12), ("zipf", 40), ("flat16", 24)])
def test_every_row_holds(oracle, name, rows):
    w = make_workload(name, B=rows)
    ref = oracle.sample_rows(w.logits, w.temperature, w.top_k, w.top_p, w.penalty,
                             w.hist_offsets, w.hist_ids, w.uniforms, want_probs=True)
    cmp = margins.compare_workload(w, range(rows), ref)
    assert len(cmp) == rows
    for r, c in cmp.items():
        assert margins.holds(c), (name, r, c)
        if c.p_margin > margins.BAND:
            assert c.keep_diff_fp32 == 0 and c.max_dprob <= margins.PROB_TOL, (name, r, c)
    s = margins.summarize(cmp, rows)
    assert s["all_rows_hold"]
    if name == "flat16":
        # every flat16 cut lies within one small token of an edge
        assert s["margin_rows"] == rows
    if name in ("single", "peaked"):
        # cuts far from every edge (p_margin >= 1e-3): nothing may differ
        assert s["margin_rows"] == 0 and s["keep_diff_rows_vs_torch_chain"] == 0


def test_holds_rejects_what_it_should():
    """A plausible mistake fails the statement: a differing token far from
    the cut, a probability off by more than the tolerance, a disagreement
    with the fp64 chain outside its window."""
    ok = margins.RowCompare(p_margin=3e-7, n_kept=10, keep_diff_fp32=1, fp32_diff_window=2e-6,
                            keep_diff_fp64=0, fp64_diff_window=0.0, max_dprob=1.8e-6,
                            max_dprob_off_cut=2e-8, cut_token_prob=1.8e-6)
    assert margins.holds(ok)
    bad = [
        dict(fp32_diff_window=3e-5),                       # a dropped token far from the cut
        dict(max_dprob_off_cut=2e-6),                      # a probability off elsewhere
        dict(keep_diff_fp64=1, fp64_diff_window=1e-6),     # the exact cut itself misplaced
        dict(max_dprob=5e-6),                              # more than the boundary token's mass
        dict(keep_diff_fp32=0, max_dprob=1.8e-6),          # same keep set, probabilities off
    ]
    for change in bad:
        c = margins.RowCompare(**{**ok.__dict__, **change})
        assert not margins.holds(c), change


def test_fp64_chain_matches_the_oracle_on_a_known_cut(oracle):
    """Four equal logits with top_p = 0.5: the exclusive prefixes are exactly
    0, .25, .5, .75, so both the oracle and the fp64 chain keep two tokens."""
    x = np.zeros(4, np.float32)

    class P:
        temperature, top_k, top_p, repetition_penalty = 1.0, 0, 0.5, 1.0
    keep, prefix = margins.fp64_chain(x, P(), [])
    assert keep.tolist() == [True, True, False, False]
    assert prefix.tolist() == [0.0, 0.25, 0.5, 0.75]
    r = oracle.sample_rows(x[None, :], [1.0], [0], [0.5], [1.0], [0, 0], np.zeros(0, np.int32), [0.3],
                           want_probs=True)
    assert ((r.probs[0] > 0) == keep).all()
