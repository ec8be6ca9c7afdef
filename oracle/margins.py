"""Where the oracle's exact top-p cut and the reference's fp32 cut can differ.

TEST INFRASTRUCTURE ONLY: used by tests/ and by bench.py's parity block, as
the checker.  The product never imports it.

The reference cuts the sorted row where fl32(cumsum(p) - p) >= top_p
(mini_engine/sampling.py:57-62), p being torch's fp32 softmax of the sorted
logits.  That fp32 softmax is normalised by an fp32 sum whose rounding
moves every prefix by up to a few 1e-6 of the total mass (measured at the
cut: up to 2.5e-6 on the flat16 rows, 5.3e-7 on the Zipf rows), and the
amount depends on the summation order of torch's CPU kernels: the AVX512
and AVX2 builds of the same torch keep different boundary tokens on most
flat16 rows.  The oracle evaluates the cut exactly (integer masses), which
is the limit the fp32 chain approximates: the same chain with its softmax
and cumsum in float64 keeps exactly the oracle's tokens.

compare_row() measures one row three ways:

  oracle      the exact restatement (sampler_oracle.c), whose results the
              GPU reproduces bit for bit
  fp32 chain  oracle/torch_chain.cpu_ref with stable=True: the reference's
              torch ops with the lowest-index tie rule
  fp64 chain  the same ops on the same fp32 tempered logits (penalty, x / T
              and top-k as in fp32), softmax and cumsum in float64

and reports the keep-set differences, where they sit (the tokens next to
the oracle's cut in the sorted order), and the probability differences.
The bounds the tests hold it to are BAND and PROB_TOL below.
"""

from __future__ import annotations

import os
import sys
from dataclasses import dataclass

import numpy as np
import torch

from oracle.torch_chain import cpu_ref

# A token the fp32 chain keeps and the oracle drops (or the reverse) has its
# exclusive prefix mass within BAND of top_p (prefixes as fractions of the
# total): BAND is four times the largest deviation of the fp32 prefix
# measured at a cut.  Against the fp64 chain the window is FP64_BAND: the
# oracle's fp32 exp polynomial is within 1.2e-7 of exp relative to each
# mass, which moves a prefix fraction by at most about half that.
BAND = 1e-5
FP64_BAND = 2e-7
PROB_TOL = 1e-6


class _Params:
    def __init__(self, T, k, p, pen):
        self.temperature, self.top_k, self.top_p, self.repetition_penalty = T, k, p, pen


def row_params(w, r):
    return _Params(float(w.temperature[r]), int(w.top_k[r]), float(w.top_p[r]), float(w.penalty[r]))


def row_history(w, r):
    return w.hist_ids[w.hist_offsets[r]:w.hist_offsets[r + 1]].tolist()


@dataclass
class RowCompare:
    p_margin: float            # the oracle's distance from the cut to its boundary token's edges / W
    n_kept: int                # tokens the oracle keeps
    keep_diff_fp32: int        # tokens kept by exactly one of the oracle and the fp32 chain
    fp32_diff_window: float    # the largest |prefix - top_p| of those tokens (0: none)
    keep_diff_fp64: int        # tokens kept by exactly one of the oracle and the fp64 chain
    fp64_diff_window: float    # the largest |prefix - top_p| of those tokens (0: none)
    max_dprob: float           # max |oracle prob - fp32 chain prob| over the row
    max_dprob_off_cut: float   # the same without the tokens in keep_diff_fp32
    cut_token_prob: float      # the largest probability (either side) of a differing token


def fp64_chain(row: np.ndarray, prm, hist):
    """(kept bool[V], prefix float64[V]): mini_engine/sampling.py:36-66 with
    the penalty, temperature and top-k threshold in fp32 as the reference
    computes them, then a stable sort and the softmax and cumsum of the cut
    in float64; prefix[i] is token i's exclusive prefix mass (a fraction of
    the total over the top-k survivors) in that sorted order."""
    x = torch.from_numpy(np.asarray(row, dtype=np.float32).copy())
    if prm.repetition_penalty != 1.0 and hist:
        prev = torch.tensor(sorted(set(hist)))
        sc = x[prev]
        x[prev] = torch.where(sc > 0, sc / prm.repetition_penalty, sc * prm.repetition_penalty)
    l = x / prm.temperature
    if prm.top_k > 0:
        kth = torch.topk(l, min(prm.top_k, l.shape[0])).values[-1]
        l[l < kth] = float("-inf")
    order = torch.sort(l, descending=True, stable=True).indices
    l64 = l.double()
    sl = l64[order]
    pr = torch.softmax(sl, -1)
    excl = torch.cumsum(pr, -1) - pr
    prefix = torch.empty_like(excl).scatter(0, order, excl)
    if prm.top_p < 1.0:
        cut = excl >= float(np.float32(prm.top_p))
        sl[cut] = float("-inf")
        l64 = torch.full_like(l64, float("-inf")).scatter(0, order, sl)
    return (l64 > float("-inf")).numpy(), prefix.numpy()


def compare_row(row, prm, hist, oracle_probs: np.ndarray, p_margin: float, n_kept: int) -> RowCompare:
    """One stochastic row: the oracle's post-filter probabilities (a [V]
    row, as the GPU writes them) against the fp32 and fp64 chains."""
    kept_o = oracle_probs > 0
    tr = cpu_ref(torch.from_numpy(np.asarray(row).copy()), prm, hist, stable=True, draw="none")
    kept_t, probs_t = tr.kept.numpy(), tr.probs.numpy()
    kept_64, prefix = fp64_chain(row, prm, hist)
    top_p = float(np.float32(prm.top_p))
    diff = np.nonzero(kept_o != kept_t)[0]
    diff64 = np.nonzero(kept_o != kept_64)[0]
    window = lambda idx: float(np.abs(prefix[idx] - top_p).max()) if idx.size else 0.0
    dp = np.abs(oracle_probs.astype(np.float64) - probs_t.astype(np.float64))
    off = np.ones(dp.shape, bool)
    off[diff] = False
    return RowCompare(
        p_margin=float(p_margin), n_kept=int(n_kept),
        keep_diff_fp32=int(diff.size), fp32_diff_window=window(diff),
        keep_diff_fp64=int(diff64.size), fp64_diff_window=window(diff64),
        max_dprob=float(dp.max()), max_dprob_off_cut=float(dp[off].max()) if off.any() else 0.0,
        cut_token_prob=float(max([max(oracle_probs[i], probs_t[i]) for i in diff], default=0.0)))


def holds(c: RowCompare) -> bool:
    """The statement the tests hold every row to:
      * the fp64 chain keeps the oracle's tokens, except tokens whose prefix
        lies within FP64_BAND of top_p (the oracle's own resolution);
      * the fp32 chain keeps the oracle's tokens, except tokens whose prefix
        lies within BAND of top_p (the fp32 chain's rounding);
      * probabilities agree within PROB_TOL on every other token, and on a
        differing token by at most its own probability plus PROB_TOL."""
    if c.keep_diff_fp64 and not c.fp64_diff_window < FP64_BAND:
        return False
    if c.keep_diff_fp32 and not c.fp32_diff_window < BAND:
        return False
    if c.max_dprob_off_cut > PROB_TOL:
        return False
    return c.max_dprob <= (c.cut_token_prob if c.keep_diff_fp32 else 0.0) + PROB_TOL


def compare_workload(w, rows, oracle_result):
    """compare_row for the given rows of a workload (stochastic, status-ok
    rows with top-p on; others are skipped), with the oracle's probabilities."""
    out = {}
    for r in rows:
        if w.temperature[r] == 0.0 or not (w.top_p[r] < 1.0) or oracle_result.status[r] != 0:
            continue
        out[r] = compare_row(w.logits[r], row_params(w, r), row_history(w, r), oracle_result.probs[r],
                             oracle_result.info["p_margin"][r], oracle_result.info["n_kept"][r])
    return out


def summarize(cmp: dict, B: int) -> dict:
    cs = list(cmp.values())
    return {
        "rows": B, "rows_compared": len(cs),
        "margin_rows": int(sum(c.p_margin < BAND for c in cs)),
        "keep_diff_rows_vs_torch_chain": int(sum(c.keep_diff_fp32 > 0 for c in cs)),
        "max_keep_diff_vs_torch_chain": int(max([c.keep_diff_fp32 for c in cs], default=0)),
        "keep_diff_rows_vs_fp64_chain": int(sum(c.keep_diff_fp64 > 0 for c in cs)),
        "max_prefix_window_of_diffs_vs_torch_chain": float(max([c.fp32_diff_window for c in cs], default=0.0)),
        "max_dprob_vs_torch_chain": float(max([c.max_dprob for c in cs], default=0.0)),
        "max_dprob_off_cut_vs_torch_chain": float(max([c.max_dprob_off_cut for c in cs], default=0.0)),
        "all_rows_hold": bool(all(holds(c) for c in cs)),
    }


def _one(args):
    name, B, lo, hi = args
    torch.set_num_threads(1)
    from mi355x_sampler.workloads import make_workload
    from oracle import oracle as orc
    w = make_workload(name, B=B)
    sub = slice(lo, hi)
    ref = orc.sample_rows(w.logits[sub], w.temperature[sub], w.top_k[sub], w.top_p[sub], w.penalty[sub],
                          w.hist_offsets[lo:hi + 1] - w.hist_offsets[lo],
                          w.hist_ids[w.hist_offsets[lo]:w.hist_offsets[hi]], w.uniforms[sub], want_probs=True)
    out = {}
    for i, r in enumerate(range(lo, hi)):
        if w.temperature[r] == 0.0 or not (w.top_p[r] < 1.0) or ref.status[i] != 0:
            continue
        out[r] = compare_row(w.logits[r], row_params(w, r), row_history(w, r), ref.probs[i],
                             ref.info["p_margin"][i], ref.info["n_kept"][i])
    return out


def main():
    """Prints the per-workload table (every row of each benchmark shape):
    python -m oracle.margins, from the repository root."""
    from concurrent.futures import ProcessPoolExecutor

    from mi355x_sampler.workloads import SHAPES
    jobs = int(os.environ.get("MAX_JOBS", os.cpu_count() or 1))
    print("| workload | B | rows with top-p | margin rows (p_margin < 1e-5) | rows whose keep set differs "
          "from the fp32 chain (tokens) | largest \\|prefix - top_p\\| of a differing token | "
          "rows differing from the fp64 chain | max \\|dprob\\| | off the differing tokens | holds |")
    print("|---|---|---|---|---|---|---|---|---|---|")
    for name, (_, B, _, _) in SHAPES.items():
        step = 16
        parts = [(name, B, lo, min(B, lo + step)) for lo in range(0, B, step)]
        cmp = {}
        with ProcessPoolExecutor(min(jobs, len(parts))) as ex:
            for d in ex.map(_one, parts):
                cmp.update(d)
        s = summarize(cmp, B)
        print(f"| {name} | {B} | {s['rows_compared']} | {s['margin_rows']} | "
              f"{s['keep_diff_rows_vs_torch_chain']} (at most {s['max_keep_diff_vs_torch_chain']}) | "
              f"{s['max_prefix_window_of_diffs_vs_torch_chain']:.3g} | "
              f"{s['keep_diff_rows_vs_fp64_chain']} | {s['max_dprob_vs_torch_chain']:.3g} | "
              f"{s['max_dprob_off_cut_vs_torch_chain']:.3g} | {s['all_rows_hold']} |", flush=True)


if __name__ == "__main__":
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    for p in (root, os.path.join(root, "llm-inference-scheduler_amd")):
        if p not in sys.path:
            sys.path.insert(0, p)
    print(f"torch {torch.__version__}, CPU capability {torch.backends.cpu.get_cpu_capability()}")
    main()
