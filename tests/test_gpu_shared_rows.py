"""Top-k-off rows shared with helper workgroups (batches above 64 rows).

With the flag MXS_FLAG_SHARE_ROWS (share_rows=True; sample_requests sets it
from the requests' parameters, mi355x_sampler.shares_rows), in an fp32
batch of more than 64 rows that mixes rows with top-k off
(sampling.py:56-69 over the whole row) and other rows, the first 16 rows
with top-k off (by row order) open their two passes to the workgroups that
finished their own rows; those take slices from the back of each pass and
hand their counts, sums and listed elements over through the workspace.
Whatever the split, every token and status must equal the oracle's:

  * the mixed Zipf batch with 8 such rows (the zipf_k0 workload);
  * more than 16 such rows (the later ones run alone), with penalties over
    histories, negative temperatures, tiny and ordinary top-p, NaN rows;
  * a batch of more than 512 rows (rows take the job slot r mod 16);
  * one Sampler, whose workspace carries the previous calls' records, run
    on several batches in turn (each call's records carry its own tag);
  * rows whose vectors are not 16-byte aligned (they are never shared);
  * the batch's rows all with top-k off (nothing is shared).
"""

import sys

import numpy as np
import pytest
import torch

from mi355x_sampler import Sampler, sample_batch
from mi355x_sampler.workloads import VOCAB, Workload, make_workload

pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def mixed(seed, V, B, frac_off):
    """B rows of varied logits; about frac_off of them with top-k off."""
    rng = np.random.default_rng(seed)
    x = np.empty((B, V), np.float32)
    for r in range(B):
        kind = rng.integers(0, 4)
        if kind == 0:
            x[r] = rng.standard_normal(V) * rng.choice([0.5, 1.0, 3.0])
        elif kind == 1:
            x[r] = -1.1 * np.log(rng.permutation(V) + 1.0) + 0.1 * rng.standard_normal(V)
        elif kind == 2:
            x[r] = rng.standard_normal(V)
            x[r, rng.choice(V, 5, replace=False)] += 12.0
        else:
            x[r] = 2.0 * rng.standard_normal(V)
            if rng.random() < 0.2:
                x[r, int(rng.integers(0, V))] = np.nan
    T = rng.uniform(0.3, 1.5, B).astype(np.float32)
    T[rng.random(B) < 0.1] *= -1.0
    T[rng.random(B) < 0.1] = 0.0
    off_rows = rng.random(B) < frac_off
    k = np.where(off_rows, 0, rng.integers(1, 1100, B)).astype(np.int32)
    k[off_rows & (rng.random(B) < 0.3)] = V    # k >= V is top-k off too
    p = np.where(rng.random(B) < 0.4, 1.0, rng.uniform(0.05, 0.99, B)).astype(np.float32)
    p[rng.random(B) < 0.05] = 1e-6
    pen = np.where(rng.random(B) < 0.5, 1.0, rng.uniform(0.7, 1.4, B)).astype(np.float32)
    hists = [rng.integers(0, V, int(rng.choice([0, 40, 1024]))).astype(np.int32) for _ in range(B)]
    off = np.zeros(B + 1, np.int32)
    off[1:] = np.cumsum([len(h) for h in hists])
    ids = np.concatenate(hists).astype(np.int32)
    u = rng.random(B).astype(np.float32)
    return Workload(f"shared{seed}", x, T, k, p, pen, off, ids, u)


def check(oracle, w, tok, st):
    ref = oracle.sample_rows(w.logits, w.temperature, w.top_k, w.top_p, w.penalty,
                             w.hist_offsets, w.hist_ids, w.uniforms)
    st = st.cpu().numpy()
    tok = tok.cpu().numpy()
    bad = np.nonzero(st != ref.status)[0]
    assert bad.size == 0, f"rows {bad[:8]}: status gpu {st[bad[:8]]} oracle {ref.status[bad[:8]]}"
    bad = np.nonzero(tok != ref.tokens)[0]
    assert bad.size == 0, f"rows {bad[:8]}: gpu {tok[bad[:8]]} oracle {ref.tokens[bad[:8]]}"


def test_mixed_zipf_batch(oracle, cuda):
    w = make_workload("zipf_k0")
    say(f"[shared] zipf_k0 B={w.B} rows with top-k off: {int((w.top_k <= 0).sum())}")
    tok, st = sample_batch(**w.to_device(cuda), return_status=True, share_rows=True)
    torch.cuda.synchronize()
    check(oracle, w, tok, st)


@pytest.mark.parametrize("seed,V,B,frac", [
    (1, VOCAB, 96, 0.3),      # about 29 rows with top-k off: 16 shared, the rest alone
    (2, 40000, 200, 0.05),    # a few shared rows, many helpers
    (3, 65536, 130, 0.5),     # half the rows
    (4, 32768, 600, 0.1),     # more than 512 rows: slots r mod 16, rows not all resident
])
def test_mixed_batches(oracle, cuda, seed, V, B, frac):
    w = mixed(seed, V, B, frac)
    say(f"[shared] seed={seed} V={V} B={B} rows with top-k off: {int(((w.top_k <= 0) | (w.top_k >= V)).sum())}")
    d = w.to_device(cuda)
    tok, st = sample_batch(**d, return_status=True, share_rows=True)
    torch.cuda.synchronize()
    check(oracle, w, tok, st)
    # the launch without the flag (no sharing code) gives the same tokens
    tok2, st2 = sample_batch(**d, return_status=True)
    assert torch.equal(tok, tok2) and torch.equal(st, st2)


def test_one_sampler_many_calls(oracle, cuda):
    """The workspace keeps the earlier calls' job records: each call's own
    tag keeps them apart (no reset between calls)."""
    B, V = 80, 50000
    s = Sampler(B, V, cuda)
    for seed in (11, 12, 13, 14):
        w = mixed(seed, V, B, 0.2 + 0.1 * (seed % 3))
        say(f"[shared] sampler call seed={seed}")
        d = w.to_device(cuda)
        s.run(d["logits"], d["temperature"], d["top_k"], d["top_p"], d["penalty"], d["hist_offsets"],
              d["hist_ids"], d["uniforms"], share_rows=True)
        torch.cuda.synchronize()
        check(oracle, w, s.tokens, s.status)


def test_unaligned_rows(oracle, cuda):
    """Rows that start off a 16-byte boundary (a row stride of V + 1) are
    not shared; the batch still matches."""
    B, V = 72, 30001
    w = mixed(21, V, B, 0.3)
    d = w.to_device(cuda)
    big = torch.zeros((B, V + 1), dtype=torch.float32, device=cuda)
    big[:, :V] = d["logits"]
    d["logits"] = big[:, :V]
    say("[shared] unaligned rows")
    tok, st = sample_batch(**d, return_status=True, share_rows=True)
    torch.cuda.synchronize()
    check(oracle, w, tok, st)


def test_all_rows_top_k_off(oracle, cuda):
    w = mixed(31, 20000, 70, 1.0)
    say("[shared] every row with top-k off")
    tok, st = sample_batch(**w.to_device(cuda), return_status=True, share_rows=True)
    torch.cuda.synchronize()
    check(oracle, w, tok, st)

