"""GPU sampler vs the CPU oracle: identical token ids and row statuses,
post-filter probabilities within 1e-6 absolute (the
kernels use the oracle's arithmetic, so they are normally bit-identical).

Every launch goes through mi355x_sampler.sample_batch -> torch extension ->
mxs_sample (C ABI) -> gfx950 kernels.
"""

import sys

import numpy as np
import pytest
import torch

from mi355x_sampler import sample_batch
from mi355x_sampler.workloads import VOCAB, Workload, make_workload

pytestmark = pytest.mark.gpu

PROB_TOL = 1e-6


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def run_gpu(w: Workload, device, probs=True):
    d = w.to_device(device)
    out = torch.zeros((w.B, w.V), dtype=torch.float32, device=device) if probs else None
    tok, st = sample_batch(**d, out_probs=out, return_status=True)
    torch.cuda.synchronize()
    return tok.cpu().numpy(), st.cpu().numpy(), (out.cpu().numpy() if probs else None)


def run_oracle(oracle, w: Workload, probs=True):
    return oracle.sample_rows(w.logits, w.temperature, w.top_k, w.top_p, w.penalty,
                              w.hist_offsets, w.hist_ids, w.uniforms, want_probs=probs)


def check(w, ref, tok, st, probs):
    assert np.array_equal(st, ref.status), f"status gpu {st[:16]} oracle {ref.status[:16]}"
    bad = np.nonzero(tok != ref.tokens)[0]
    assert bad.size == 0, (f"{w.name}: token mismatch in {bad.size} rows, first {bad[:8]}: "
                           f"gpu {tok[bad[:8]]} oracle {ref.tokens[bad[:8]]}")
    if probs is not None:
        err = np.abs(probs - ref.probs)
        worst = np.unravel_index(int(err.argmax()), err.shape)
        assert err.max() <= PROB_TOL, f"{w.name}: |dprob| {err.max()} at {worst}"


def custom(name, logits, T, k, p, pen, hists, u):
    x = np.ascontiguousarray(np.atleast_2d(logits))
    B = x.shape[0]
    bc = lambda v, dt: np.broadcast_to(np.asarray(v, dtype=dt), (B,)).copy()
    off = np.zeros(B + 1, np.int32)
    off[1:] = np.cumsum([len(h) for h in hists])
    ids = np.asarray([i for h in hists for i in h], dtype=np.int32)
    return Workload(name, x, bc(T, np.float32), bc(k, np.int32), bc(p, np.float32),
                    bc(pen, np.float32), off, ids, bc(u, np.float32))


@pytest.mark.parametrize("name,B", [("single", 1), ("greedy", 16), ("peaked", 16),
                                    ("zipf", 24), ("flat16", 3), ("default", 8), ("default", 96),
                                    ("zipf_k0", 70)])
def test_parity_small_batches(oracle, cuda, name, B):
    w = make_workload(name, B=B)
    say(f"[parity-small] {name} B={B} V={w.V}")
    ref = run_oracle(oracle, w)
    tok, st, probs = run_gpu(w, cuda)
    check(w, ref, tok, st, probs)


@pytest.mark.parametrize("name", ["greedy", "peaked", "zipf", "default", "zipf_k0"])
def test_parity_full_batches(oracle, cuda, name):
    w = make_workload(name)
    say(f"[parity-full] {name} B={w.B} V={w.V}")
    ref = run_oracle(oracle, w, probs=False)
    tok, st, _ = run_gpu(w, cuda, probs=False)
    check(w, ref, tok, st, None)


def test_parity_full_flat16(oracle, cuda):
    w = make_workload("flat16", B=64)
    say(f"[parity-full] flat16 B={w.B} V={w.V}")
    ref = run_oracle(oracle, w, probs=False)
    tok, st, _ = run_gpu(w, cuda, probs=False)
    check(w, ref, tok, st, None)


def test_parity_flat16_benchmark_batch(oracle, cuda):
    """The flat16 benchmark shape itself, B = 1024 (one workgroup per row,
    the instance without the small-batch hand-over), with the post-filter
    probabilities of every row."""
    w = make_workload("flat16")
    assert w.B == 1024
    say(f"[parity-full] flat16 B={w.B} V={w.V} with probabilities")
    ref = run_oracle(oracle, w, probs=True)
    tok, st, probs = run_gpu(w, cuda, probs=True)
    check(w, ref, tok, st, probs)


def _edge_rows(V, seed=7):
    rng = np.random.default_rng(seed)
    base = (2.0 * rng.standard_normal(V)).astype(np.float32)
    rows = []
    #          T      k     p      pen   hist                      u
    rows.append((0.8, 1, 1.0, 1.0, [], 0.3))                  # k = 1
    rows.append((0.8, V, 1.0, 1.0, [], 0.3))                  # k = V keeps all
    rows.append((0.8, V + 5, 0.5, 1.0, [], 0.7))              # k > V
    rows.append((1.3, 0, 1e-7, 1.0, [], 0.9))                 # tiny top_p keeps the argmax
    rows.append((-0.9, 20, 0.8, 1.0, [], 0.5))                # negative temperature
    rows.append((0.6, 0, 1.0, 0.7, [3, 3, 5, 9, 9, 9], 0.2))  # penalty < 1, duplicates
    rows.append((2.5, 700, 0.97, 1.2, list(range(0, V, 7)), 0.999))
    rows.append((0.05, 40, 0.9, 1.0, [], 0.0))                # u = 0
    rows.append((1.0, 1024, 0.99, 1.0, [], 0.61))             # k = KMAX
    rows.append((1.0, 1025, 0.99, 1.0, [], 0.61))             # k just above KMAX
    top = [int(i) for i in np.argsort(-base, kind="stable")[:100]]
    rows.append((0.9, 50, 0.9, 5.0, top, 0.42))                # heavy penalty on the row's top ids
    rows.append((0.9, 30, 0.9, 0.8, top[:40] + [1, 2], 0.77))  # penalty < 1 on a top-k row
    rows.append((-0.7, 25, 0.95, 1.3, top + [3, 4], 0.33))     # negative temperature with a penalty
    rows.append((1.1, 1000, 0.97, 1.15, list(range(0, V, 3)), 0.5))   # a third of the row penalized
    return base, rows


@pytest.mark.parametrize("V", [1000, 4099, VOCAB])
def test_parity_edge_parameters(oracle, cuda, V):
    base, rows = _edge_rows(V)
    x = np.stack([base] * len(rows))
    T, k, p, pen, h, u = (list(c) for c in zip(*rows))
    w = custom("edge", x, T, k, p, pen, h, u)
    say(f"[edge-params] V={V} rows={w.B}")
    ref = run_oracle(oracle, w)
    tok, st, probs = run_gpu(w, cuda)
    check(w, ref, tok, st, probs)


def test_parity_ties_and_infinities(oracle, cuda):
    V = VOCAB
    rows, params = [], []
    rows.append(np.zeros(V, np.float32)); params.append((0.7, 0, 0.5, 1.0, [], 0.37))      # all tied
    rows.append(np.zeros(V, np.float32)); params.append((0.7, 50, 1.0, 1.0, [], 0.37))     # tied top-k
    r = np.full(V, -np.inf, np.float32); r[[5, 77, 150000]] = [1.0, 2.0, 2.0]
    rows.append(r); params.append((1.0, 0, 1.0, 1.0, [], 0.8))                             # -inf mask
    rows.append(r.copy()); params.append((1.0, 10, 1.0, 1.0, [], 0.8))                     # kth is -inf
    q = np.round(np.random.default_rng(3).standard_normal(V) * 4).astype(np.float32)
    rows.append(q); params.append((0.9, 300, 0.9, 1.1, [1, 2, 3], 0.55))                   # coarse ties
    rows.append(q.copy()); params.append((float("inf"), 0, 0.3, 1.0, [], 0.5))             # T = inf
    qi = q.copy(); qi[1234] = -np.inf
    rows.append(qi); params.append((float("inf"), 20, 0.9, 1.0, [], 0.5))                  # inf / inf
    qn = q.copy(); qn[777] = np.frombuffer(np.uint32(0xFFC00000).tobytes(), np.float32)[0]
    rows.append(qn); params.append((0.8, 20, 0.9, 1.0, [], 0.5))                           # negative NaN
    T, k, p, pen, h, u = (list(c) for c in zip(*params))
    w = custom("ties", np.stack(rows), T, k, p, pen, h, u)
    say(f"[ties] rows={w.B}")
    ref = run_oracle(oracle, w)
    tok, st, probs = run_gpu(w, cuda)
    check(w, ref, tok, st, probs)


def test_row_status_errors(oracle, cuda):
    V = 5000
    x = np.random.default_rng(1).standard_normal((5, V)).astype(np.float32)
    x[3, 17] = np.inf
    w = custom("errors", x, [0.8, float("nan"), 0.8, 0.8, 0.8], [0, 0, 0, 0, 0],
               [1.0, 1.0, 0.0, 1.0, 0.9], [1.2, 1.0, 1.0, 1.0, 1.0],
               [[V + 3], [], [], [], []], [0.5] * 5)
    say("[errors]")
    ref = run_oracle(oracle, w)
    tok, st, _ = run_gpu(w, cuda, probs=False)
    assert list(ref.status) == [1, 2, 4, 3, 0]
    check(w, ref, tok, st, None)


def test_greedy_nan_and_ties(oracle, cuda):
    V = 70000
    x = np.zeros((3, V), np.float32)
    x[0, [10, 20]] = 5.0                       # tie: lowest index
    x[1, 30] = np.nan; x[1, 40] = np.nan       # NaN is the max, first one
    x[2, :] = -1.0; x[2, 69999] = -0.5
    w = custom("greedy-edge", x, 0.0, 0, 1.0, [1.0, 1.0, 2.0], [[], [], [69999]], 0.0)
    ref = run_oracle(oracle, w)
    tok, st, _ = run_gpu(w, cuda, probs=False)
    assert list(ref.tokens) == [10, 30, 0]
    check(w, ref, tok, st, None)


def test_repeat_calls_leave_workspace_clean(oracle, cuda):
    w = make_workload("zipf", B=8)
    ref = run_oracle(oracle, w, probs=False)
    for _ in range(3):
        tok, st, _ = run_gpu(w, cuda, probs=False)
        check(w, ref, tok, st, None)


def test_workspace_reuse_across_batch_sizes(oracle, cuda):
    """Candidate lists of one batch size land where another batch size keeps
    its row counters; changing B between calls must still give exact rows."""
    for name, B in [("peaked", 64), ("zipf", 256), ("zipf", 8), ("peaked", 64), ("zipf", 256)]:
        w = make_workload(name, B=B)
        say(f"[ws-reuse] {name} B={B}")
        ref = run_oracle(oracle, w, probs=False)
        tok, st, _ = run_gpu(w, cuda, probs=False)
        check(w, ref, tok, st, None)


def test_parity_one_workgroup_per_row_fallbacks(oracle, cuda):
    """A batch large enough for one workgroup per row, with rows built to
    defeat the sampled first bound: sampled positions that overstate the top
    values (the estimate fails its check and the row is streamed again with a
    compacted buffer), top values hidden between the sampled positions, a
    20000-way tie that overflows every buffer (multi-pass path), and rows
    that apply the penalty while streaming (T < 0, penalty < 1, greedy)."""
    V = VOCAB
    stride = V // 512
    rng = np.random.default_rng(11)
    rows, params = [], []
    r = (2.0 * rng.standard_normal(V)).astype(np.float32)
    r[np.arange(512) * stride] = 50.0
    rows.append(r); params.append((1.0, 700, 0.9, 1.0, [], 0.3))         # estimate too high
    r = (2.0 * rng.standard_normal(V)).astype(np.float32)
    r[np.arange(512) * stride + 8] = 30.0 + rng.random(512).astype(np.float32)
    rows.append(r); params.append((0.8, 300, 0.95, 1.1, list(range(0, V, 97)), 0.6))   # hidden top values
    r = (2.0 * rng.standard_normal(V)).astype(np.float32)
    r[rng.choice(V, 20000, replace=False)] = 5.0
    rows.append(r); params.append((1.0, 100, 0.9, 1.0, [], 0.45))        # ties overflow the buffer
    r = (2.0 * rng.standard_normal(V)).astype(np.float32)
    rows.append(r); params.append((-0.6, 40, 0.9, 1.4, list(range(5, V, 11)), 0.8))   # T < 0, penalty
    r = (2.0 * rng.standard_normal(V)).astype(np.float32)
    rows.append(r); params.append((0.7, 60, 0.85, 0.6, list(range(7, V, 13)), 0.1))   # penalty < 1
    r = (2.0 * rng.standard_normal(V)).astype(np.float32)
    top = [int(i) for i in np.argsort(-r)[:3]]
    rows.append(r); params.append((0.0, 0, 1.0, 3.0, top, 0.0))           # greedy with a penalty
    r = (2.0 * rng.standard_normal(V)).astype(np.float32)
    r[99] = np.inf
    rows.append(r); params.append((float("inf"), 50, 0.9, 1.0, [], 0.5))  # inf / inf: non-finite
    r = (2.0 * rng.standard_normal(V)).astype(np.float32)
    r[4242] = np.frombuffer(np.uint32(0xFFC00000).tobytes(), np.float32)[0]
    rows.append(r); params.append((0.9, 50, 0.9, 1.2, [4242, 7], 0.5))   # a negative NaN
    # top-k off: the whole row takes part in the top-p cut and the draw
    for T, kq, pq, pen, u in [(0.7, 0, 0.95, 1.05, 0.31), (1.3, 0, 0.5, 1.0, 0.77),
                              (0.9, 0, 1.0, 1.2, 0.05), (0.8, V, 0.8, 1.0, 0.99),
                              (-0.8, 0, 0.9, 1.1, 0.5)]:
        r = rng.standard_normal(V).astype(np.float32)
        rows.append(r); params.append((T, kq, pq, pen, list(range(3, V, 71)), u))
    z = make_workload("zipf", B=128 - len(rows))
    x = np.concatenate([np.stack(rows), z.logits])
    T = [p[0] for p in params] + z.temperature.tolist()
    k = [p[1] for p in params] + z.top_k.tolist()
    pp = [p[2] for p in params] + z.top_p.tolist()
    pen = [p[3] for p in params] + z.penalty.tolist()
    hists = [p[4] for p in params] + [z.hist_ids[z.hist_offsets[i]:z.hist_offsets[i + 1]].tolist()
                                      for i in range(z.B)]
    u = [p[5] for p in params] + z.uniforms.tolist()
    w = custom("fused-fallbacks", x, T, k, pp, pen, hists, u)
    say(f"[fused-fallbacks] rows={w.B}")
    ref = run_oracle(oracle, w, probs=False)
    tok, st, _ = run_gpu(w, cuda, probs=False)
    check(w, ref, tok, st, None)


@pytest.mark.parametrize("V", [1, 2, 7, 33, 1000])
def test_parity_tiny_vocabularies(oracle, cuda, V):
    """Rows shorter than one tile (element-by-element loads only), in every
    row mode."""
    rng = np.random.default_rng(V)
    rows, params = [], []
    for T, k, p, pen in [(0.0, 0, 1.0, 1.0), (0.0, 0, 1.0, 1.5), (0.8, 0, 0.9, 1.2), (0.8, 1, 1.0, 1.0),
                         (1.1, 3, 0.7, 1.0), (0.9, V, 0.5, 0.8), (-0.5, 2, 0.9, 1.3), (0.7, 0, 1e-7, 1.0)]:
        rows.append(rng.standard_normal(V).astype(np.float32))
        params.append((T, k, p, pen, [0, V - 1, 0], float(rng.random())))
    T, k, p, pen, h, u = (list(c) for c in zip(*params))
    w = custom("tiny", np.stack(rows), T, k, p, pen, h, u)
    say(f"[tiny] V={V} rows={w.B}")
    ref = run_oracle(oracle, w)
    tok, st, probs = run_gpu(w, cuda)
    check(w, ref, tok, st, probs)


@pytest.mark.parametrize("V", [7, 1000, 4099, 8192])
def test_parity_constant_rows_top_p_only(oracle, cuda, V):
    """Rows whose values are all equal, with top-k off: every element falls
    into one mass bin, and no key lies in a higher one (regression: the
    search for a bin's key interval must end when nothing lies above)."""
    rows, params = [], []
    rows.append(np.zeros(V, np.float32)); params.append((0.7, 0, 0.5, 1.0, [], 0.37))
    rows.append(np.zeros(V, np.float32)); params.append((1.3, 0, 1.0, 1.0, [], 0.91))
    rows.append(np.full(V, -2.5, np.float32)); params.append((0.9, V, 0.9, 1.0, [], 0.05))
    rows.append(np.ones(V, np.float32)); params.append((0.8, 0, 0.7, 1.2, [0, V // 2], 0.66))
    T, k, p, pen, h, u = (list(c) for c in zip(*params))
    w = custom("constant", np.stack(rows), T, k, p, pen, h, u)
    say(f"[constant] V={V} rows={w.B}")
    ref = run_oracle(oracle, w)
    tok, st, probs = run_gpu(w, cuda)
    check(w, ref, tok, st, probs)


def test_parity_fp16_top_k_rows(oracle, cuda):
    """fp16 rows through the top-k path (the fp16 workload itself has top-k
    off): 128-bit loads of eight halves, converted in registers."""
    w = make_workload("zipf", B=24)
    w16 = Workload("zipf16", w.logits.astype(np.float16), w.temperature, w.top_k, w.top_p,
                   w.penalty, w.hist_offsets, w.hist_ids, w.uniforms)
    say(f"[fp16-topk] B={w16.B} V={w16.V}")
    ref = run_oracle(oracle, w16)
    tok, st, probs = run_gpu(w16, cuda)
    check(w16, ref, tok, st, probs)


def test_parity_history_and_row_extremes(oracle, cuda):
    """Greedy and top-k-off rows take the row's extremes from a raw pass and
    fold in the penalized history afterwards; rows whose raw maximum is a
    history id stream again with the penalty applied."""
    V = VOCAB
    rng = np.random.default_rng(11)
    base = (2.0 * rng.standard_normal(V)).astype(np.float32)
    top = [int(i) for i in np.argsort(-base, kind="stable")[:8]]
    rows, params = [], []
    #               T     k     p     pen   hist                       u
    rows.append(base); params.append((0.0, 0, 1.0, 1.3, top[:1] + [5, 6], 0.0))     # greedy, max penalized
    rows.append(base); params.append((0.0, 0, 1.0, 1.3, [5, 6, 7], 0.0))            # greedy, max not in history
    rows.append(base); params.append((0.0, 0, 1.0, 0.5, [5, 6, 7], 0.0))            # greedy, penalty raises
    rows.append(base); params.append((0.8, 0, 0.9, 1.3, top[:2], 0.3))             # top-p, max penalized
    rows.append(base); params.append((0.8, 0, 0.9, 1.3, [9, 10, 11], 0.7))          # top-p, max not in history
    rows.append(base); params.append((0.8, 0, 0.9, 0.6, list(range(0, V, 5)), 0.5))  # top-p, penalty raises
    rows.append(base); params.append((-0.7, 0, 0.8, 1.2, top[:3] + [1], 0.4))      # top-p, T < 0
    rows.append(base); params.append((0.9, 2000, 0.95, 1.1, top[:4], 0.8))         # k above the candidate cap
    rn = base.copy(); rn[top[0]] = np.nan
    rows.append(rn); params.append((0.8, 0, 0.9, 1.2, top[:1], 0.5))               # NaN among the history ids
    rows.append(rn.copy()); params.append((0.0, 0, 1.0, 1.2, top[:1], 0.0))        # greedy, NaN in history
    T, k, p, pen, h, u = (list(c) for c in zip(*params))
    w = custom("extremes", np.stack(rows), T, k, p, pen, h, u)
    say(f"[extremes] rows={w.B}")
    ref = run_oracle(oracle, w)
    tok, st, probs = run_gpu(w, cuda)
    check(w, ref, tok, st, probs)


def _counted_rows(V, seed=23):
    """fp16 rows with top-k off, long enough for the value-count path, and
    the cases its ranks and history placement have to get right."""
    rng = np.random.default_rng(seed)
    f16 = lambda a: np.asarray(a, dtype=np.float16)
    base = f16(rng.standard_normal(V))
    top = [int(i) for i in np.argsort(-base.astype(np.float32), kind="stable")[:16]]
    hist2k = [int(i) for i in rng.choice(V, 2048, replace=False)]
    rows, params = [], []
    #                    T     k  p      pen   hist         u
    rows.append(base); params.append((0.7, 0, 0.95, 1.05, hist2k, 0.37))        # the fp16 workload's row
    rows.append(base); params.append((0.7, 0, 0.95, 1.05, hist2k, 0.0))
    rows.append(base); params.append((0.7, 0, 0.95, 1.05, hist2k, 0.99999994))
    rows.append(base); params.append((0.7, V, 1.0, 1.0, [], 0.61))             # k >= V, no cut, no history
    rows.append(base); params.append((-0.8, 0, 0.9, 1.2, top[:3] + [1], 0.4))  # T < 0
    rows.append(base); params.append((1.3, 0, 0.5, 0.7, top[:8] + hist2k[:500], 0.8))  # penalty raises values
    rows.append(base); params.append((0.9, 0, 0.8, 1.3, top[:1], 0.05))        # the maximum is a history id
    rows.append(base); params.append((0.9, 0, 0.8, 1.3, top[:16], 0.02))       # ... and the next fifteen
    rows.append(base); params.append((0.9, 0, 1e-6, 1.1, hist2k[:64], 0.9))    # the cut at the first element
    # penalized history values equal to raw values (pen 2: 2.0 -> 1.0): the
    # tie groups interleave history and raw ids by index
    tie = f16(rng.standard_normal(V) - 4.0)
    ones = rng.choice(V, 300, replace=False)
    twos = rng.choice(np.setdiff1d(np.arange(V), ones), 200, replace=False)
    tie[ones] = 1.0
    tie[twos] = 2.0
    for u in (0.1, 0.5, 0.93):
        rows.append(tie); params.append((1.0, 0, 1.0, 2.0, [int(i) for i in twos], u))
    rows.append(tie); params.append((1.0, 0, 0.6, 2.0, [int(i) for i in twos[:150]], 0.7))
    # penalized history values strictly between ranks: fifty equal ones on top
    btw = f16(rng.standard_normal(V) - 3.0)
    hb = rng.choice(V, 50, replace=False)
    btw[hb] = 5.0
    for u in (0.0, 0.45, 0.999):
        rows.append(btw); params.append((0.8, 0, 1.0, 1.3, [int(i) for i in hb], u))
    # more than 256 history ids placed in one chunk: the general path
    many = f16(rng.standard_normal(V) - 3.0)
    hm = rng.choice(V, 300, replace=False)
    many[hm] = 5.0
    rows.append(many); params.append((0.8, 0, 0.9, 1.3, [int(i) for i in hm], 0.3))
    # heavy ties: four levels
    lv = f16(rng.integers(0, 4, V) * 0.5)
    rows.append(lv); params.append((0.5, 0, 0.7, 1.1, hist2k[:100], 0.66))
    # +0 and -0 on top, mixed signs in index order
    z = f16(np.full(V, -12.0))
    zi = rng.choice(V, 400, replace=False)
    z[zi] = np.where(rng.random(400) < 0.5, 0.0, -0.0)
    for u in (0.2, 0.8):
        rows.append(z); params.append((1.0, 0, 1.0, 1.0, [], u))
    rows.append(z); params.append((-1.0, 0, 0.5, 1.5, [int(i) for i in zi[:10]], 0.4))
    # masked rows: -inf below, and a rank holding 65536 or more elements
    msk = base.copy()
    msk[rng.choice(V, V // 3, replace=False)] = -np.inf
    rows.append(msk); params.append((0.7, 0, 0.95, 1.05, hist2k, 0.5))
    msk2 = base.copy()
    msk2[: 70000] = -np.inf
    rows.append(msk2); params.append((0.7, 0, 0.95, 1.05, hist2k, 0.5))
    big = base.copy()
    big[rng.choice(V, 70000, replace=False)] = 0.25
    rows.append(big); params.append((0.7, 0, 0.9, 1.0, [], 0.5))
    # non-finite rows
    for bits in (0x7E00, 0xFE00, 0x7C00):   # NaN, NaN with the sign bit, +inf
        b = base.copy(); b.view(np.uint16)[V // 2] = bits
        rows.append(b); params.append((0.7, 0, 0.9, 1.05, hist2k[:10], 0.5))
    b = base.copy(); b[V // 3] = -np.inf
    rows.append(b); params.append((-0.7, 0, 0.9, 1.05, hist2k[:10], 0.5))        # -inf / T, T < 0: +inf
    b = base.copy(); b[V // 3] = -np.inf
    rows.append(b); params.append((0.7, 0, 0.0, 1.0, [], 0.5))                 # an empty nucleus
    return rows, params


def test_parity_fp16_value_counts(oracle, cuda):
    """fp16 rows with top-k off finish from per-value counts: ranks, the
    penalized history placed between or tied with them, the drawn element's
    index found by a second pass; and the rows that fall back."""
    V = VOCAB
    rows, params = _counted_rows(V)
    T, k, p, pen, h, u = (list(c) for c in zip(*params))
    w = custom("counts16", np.stack(rows), T, k, p, pen, h, u)
    say(f"[counts16] rows={w.B} V={V}")
    ref = run_oracle(oracle, w)
    tok, st, probs = run_gpu(w, cuda)
    check(w, ref, tok, st, probs)
    say("[counts16] no probabilities")
    tok2, st2, _ = run_gpu(w, cuda, probs=False)
    check(w, ref, tok2, st2, None)


def test_parity_fp16_value_counts_unaligned(oracle, cuda):
    """Odd row lengths: every other row is not 16-byte aligned and is
    counted element by element."""
    V = 40001
    rng = np.random.default_rng(5)
    x = rng.standard_normal((3, V)).astype(np.float16)
    hists = [[int(i) for i in rng.choice(V, 300, replace=False)] for _ in range(3)]
    w = custom("counts16-odd", x, [0.7, -0.9, 1.1], 0, [0.95, 0.5, 1.0], [1.05, 1.2, 0.8], hists, [0.3, 0.6, 0.9])
    say(f"[counts16-odd] rows={w.B} V={V}")
    ref = run_oracle(oracle, w)
    tok, st, probs = run_gpu(w, cuda)
    check(w, ref, tok, st, probs)
