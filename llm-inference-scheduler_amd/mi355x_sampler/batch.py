"""Batched sampling: one kernel launch for a whole [B, V] batch of logits.

`sample_batch` is the device-array entry (per-row parameters as tensors, the
history as CSR); `sample_requests` packs a scheduler's per-request
SamplingParams, output ids and generators into that form (the batched
counterpart of the per-row loop at mini_engine/scheduler.py:268-275).
`HistoryStore` keeps the requests' generated ids on the device across steps,
and `sample_requests_resident` / `sample_batch_ranges` read them there.
"""

from __future__ import annotations

import math
from typing import Optional, Sequence

import numpy as np
import torch

from . import _native

ROW_OK = 0
ROW_BAD_HISTORY = 1
ROW_BAD_PARAM = 2
ROW_NONFINITE = 3
ROW_EMPTY_NUCLEUS = 4
MAX_VOCAB = 262144


def sample_batch(logits: torch.Tensor, temperature: torch.Tensor, top_k: torch.Tensor,
                 top_p: torch.Tensor, penalty: torch.Tensor,
                 hist_offsets: Optional[torch.Tensor] = None,
                 hist_ids: Optional[torch.Tensor] = None,
                 uniforms: Optional[torch.Tensor] = None,
                 out_probs: Optional[torch.Tensor] = None,
                 return_status: bool = False,
                 row_best: Optional[torch.Tensor] = None,
                 share_rows: bool = False):
    """Sample one token per row of `logits` ([B, V], float32 or float16).

    temperature f32[B] (0 = greedy), top_k i32[B] (<= 0 off), top_p f32[B]
    (>= 1 off), penalty f32[B] (1 off), hist_offsets i32[B+1] / hist_ids i32[N]
    (CSR history of generated ids), uniforms f32[B] in [0, 1).  All tensors on
    the logits' device.  Returns int64[B] token ids on the device (-1 for rows
    whose status is not ok), plus int32[B] row statuses if return_status.
    out_probs, if given, is filled with the post-filter probabilities [B, V].
    row_best, if given, holds the row maxima that `head.lm_head` wrote with
    these logits: greedy rows without a penalty take their token from it.
    share_rows: the batch may mix rows with top-k off and other rows
    (MXS_FLAG_SHARE_ROWS: the former share their passes with the
    workgroups that finished their own rows; see `shares_rows`).  The
    tokens are the same either way.  The launch is asynchronous on the
    current stream.
    """
    _native.require_gpu(logits.device)
    ext = _native.extension()
    B, V = logits.shape
    dev = logits.device
    tokens = torch.empty(B, dtype=torch.int64, device=dev)
    status = torch.empty(B, dtype=torch.int32, device=dev)
    ws = _native.workspace(dev, B, V)
    flags = ext.FLAG_SHARE_ROWS if share_rows else 0
    if row_best is None:
        ext.sample(logits, temperature, top_k, top_p, penalty, hist_offsets, hist_ids, uniforms,
                   tokens, status, out_probs, ws, flags)
    else:
        ext.sample_head(logits, temperature, top_k, top_p, penalty, hist_offsets, hist_ids, uniforms,
                        tokens, status, out_probs, row_best, ws, flags)
    return (tokens, status) if return_status else tokens


def shares_rows(params_list, V: int) -> bool:
    """Whether a batch of these SamplingParams mixes rows with top-k off
    (sampling.py:52: top_k <= 0, or top_k >= V, with a temperature) and
    other rows: then its top-k-off rows are worth sharing (share_rows)."""
    off = [p.temperature != 0.0 and (int(p.top_k) <= 0 or int(p.top_k) >= V) for p in params_list]
    return any(off) and not all(off)


class Sampler:
    """Preallocated outputs and workspace for repeated [B, V] launches.

    For serving loops: `run()` is one asynchronous launch on the current
    stream with no allocation, so back-to-back steps keep the GPU busy.
    """

    def __init__(self, B: int, V: int, device, with_probs: bool = False):
        self.device = torch.device(device)
        _native.require_gpu(self.device)
        self.ext = _native.extension()
        self.B, self.V = B, V
        self.tokens = torch.empty(B, dtype=torch.int64, device=self.device)
        self.status = torch.empty(B, dtype=torch.int32, device=self.device)
        self.probs = (torch.zeros((B, V), dtype=torch.float32, device=self.device)
                      if with_probs else None)
        self.workspace = torch.zeros(max(int(self.ext.workspace_bytes(B, V)), 256),
                                     dtype=torch.uint8, device=self.device)   # (zero-filled once)

    def run(self, logits, temperature, top_k, top_p, penalty, hist_offsets=None,
            hist_ids=None, uniforms=None, share_rows: bool = False):
        self.ext.sample(logits, temperature, top_k, top_p, penalty, hist_offsets, hist_ids,
                        uniforms, self.tokens, self.status, self.probs, self.workspace,
                        self.ext.FLAG_SHARE_ROWS if share_rows else 0)
        return self.tokens


def device_temperature(t: float) -> float:
    """The float32 temperature a row is sampled with.  sampling.py:47 tests
    the Python float (T == 0 is greedy) and :50 divides by it as a float32
    scalar, so a non-zero T that is 0 in float32 (|T| < 2^-150) divides by
    zero there, and torch.multinomial then rejects the row; such a row gets
    NaN here, which the kernels report as a row error, instead of turning
    greedy."""
    t = float(t)
    if t != 0.0 and np.float32(t) == 0.0:
        return math.nan
    return t


def _normalize_history(ids: Sequence[int], V: int) -> list:
    """torch indexing rules of sampling.py:39-40: negative ids wrap once,
    anything else out of range raises IndexError."""
    out = []
    for i in ids:
        i = int(i)
        if i < 0:
            i += V
        if i < 0 or i >= V:
            raise IndexError(f"index {i} is out of bounds for dimension 0 with size {V}")
        out.append(i)
    return out


def pack_requests(params_list, histories, V: int, device, generators=None):
    """Device tensors for sample_batch from per-request SamplingParams.

    One host buffer is filled and copied to the device in a single transfer.
    Uniforms are drawn on the host, one per stochastic row, from that row's
    generator (or torch's default generator when None), in row order; greedy
    rows draw nothing, as sampling.py:47-48 returns before any draw.
    """
    B = len(params_list)
    gens = generators if generators is not None else [None] * B
    hists = []
    for p, h in zip(params_list, histories):
        use = p.repetition_penalty != 1.0 and len(h) > 0
        hists.append(_normalize_history(h, V) if use else [])
    total = sum(len(h) for h in hists)
    # layout (int32 words): T[B] K[B] P[B] PEN[B] U[B] OFF[B+1] IDS[total]
    buf = torch.empty(5 * B + B + 1 + max(total, 1), dtype=torch.int32)
    f = buf.view(torch.float32)
    off = 0
    for r, (p, g) in enumerate(zip(params_list, gens)):
        f[r] = device_temperature(p.temperature)
        buf[B + r] = int(p.top_k) if -2**31 <= int(p.top_k) < 2**31 else (2**31 - 1)
        f[2 * B + r] = float(p.top_p)
        f[3 * B + r] = float(p.repetition_penalty)
        f[4 * B + r] = 0.0 if p.temperature == 0.0 else float(torch.rand((), generator=g))
        buf[5 * B + r] = off
        off += len(hists[r])
    buf[6 * B] = off
    if total:
        buf[6 * B + 1: 6 * B + 1 + total] = torch.tensor([i for h in hists for i in h], dtype=torch.int32)
    d = buf.to(device, non_blocking=False)
    df = d.view(torch.float32)
    return dict(temperature=df[0:B], top_k=d[B:2 * B], top_p=df[2 * B:3 * B],
                penalty=df[3 * B:4 * B], uniforms=df[4 * B:5 * B],
                hist_offsets=d[5 * B:6 * B + 1], hist_ids=d[6 * B + 1:6 * B + 1 + total])


def sample_requests(logits: torch.Tensor, params_list, histories, generators=None,
                    out_probs: Optional[torch.Tensor] = None) -> list:
    """Per-request tokens for a [B, V] batch in one launch; raises like the
    reference would for the first failing row."""
    B, V = logits.shape
    packed = pack_requests(params_list, histories, V, logits.device, generators)
    tokens, status = sample_batch(logits, out_probs=out_probs, return_status=True,
                                  share_rows=shares_rows(params_list, V), **packed)
    st = status.cpu().tolist()
    for r, s in enumerate(st):
        if s != ROW_OK:
            raise_row_status(s, r)
    return tokens.cpu().tolist()


def sample_batch_ranges(logits: torch.Tensor, temperature: torch.Tensor, top_k: torch.Tensor,
                        top_p: torch.Tensor, penalty: torch.Tensor, hist_begin: torch.Tensor,
                        hist_end: torch.Tensor, hist_ids: torch.Tensor,
                        uniforms: Optional[torch.Tensor] = None,
                        out_probs: Optional[torch.Tensor] = None,
                        return_status: bool = False, share_rows: bool = False):
    """sample_batch with row r's history at hist_ids[hist_begin[r], hist_end[r])
    (i32[B] each, on the device): hist_ids can stay on the device across
    steps (HistoryStore).  The launch is asynchronous on the current stream."""
    _native.require_gpu(logits.device)
    ext = _native.extension()
    B, V = logits.shape
    dev = logits.device
    tokens = torch.empty(B, dtype=torch.int64, device=dev)
    status = torch.empty(B, dtype=torch.int32, device=dev)
    ws = _native.workspace(dev, B, V)
    ext.sample_ranges(logits, temperature, top_k, top_p, penalty, hist_begin, hist_end, hist_ids,
                      uniforms, tokens, status, out_probs, ws, ext.FLAG_SHARE_ROWS if share_rows else 0)
    return (tokens, status) if return_status else tokens


class HistoryStore:
    """Generated token ids of up to `slots` requests, resident on the device
    across decode steps; their lengths are mirrored on the host.

    The reference rebuilds each request's history from its Python list at
    every step (req.output_ids, mini_engine/scheduler.py:43, appended at :276
    and read by sampling.py:38-45).  Here request slot s owns
    ids[s * max_len, (s + 1) * max_len); `append` writes a step's sampled
    tokens there on the device, so a step sends only each row's range.
    """

    def __init__(self, slots: int, max_len: int, device):
        if slots <= 0 or max_len <= 0:
            raise ValueError("slots and max_len must be positive")
        if slots * max_len >= 2**31:
            raise ValueError("slots * max_len must stay below 2^31 (int32 ranges)")
        self.slots, self.max_len = int(slots), int(max_len)
        self.device = torch.device(device)
        self.ids = torch.zeros(self.slots * self.max_len, dtype=torch.int32, device=self.device)
        self.lens = [0] * self.slots

    def _check_slot(self, slot: int) -> int:
        slot = int(slot)
        if not 0 <= slot < self.slots:
            raise IndexError(f"slot {slot} outside [0, {self.slots})")
        return slot

    def reset(self, slot: int, ids: Sequence[int] = (), V: Optional[int] = None) -> None:
        """Start slot `slot` with `ids` (ids it generated before; normalized
        like sampling.py:39-40 when V is given)."""
        slot = self._check_slot(slot)
        ids = _normalize_history(ids, V) if V is not None else [int(i) for i in ids]
        if len(ids) > self.max_len:
            raise ValueError(f"{len(ids)} ids exceed max_len {self.max_len}")
        if ids:
            b = slot * self.max_len
            self.ids[b:b + len(ids)] = torch.tensor(ids, dtype=torch.int32).to(self.device)
        self.lens[slot] = len(ids)

    def append(self, slots: Sequence[int], tokens) -> None:
        """Append tokens[i] to slot slots[i] (tokens: a device tensor, as
        returned by the sampler, or a sequence of ints).  Device-side copy;
        no synchronization."""
        slots = [self._check_slot(s) for s in slots]
        if len(set(slots)) != len(slots):
            raise ValueError("a slot appears twice in one append")
        pos = []
        for s in slots:
            if self.lens[s] >= self.max_len:
                raise ValueError(f"slot {s} is full ({self.max_len} ids)")
            pos.append(s * self.max_len + self.lens[s])
        if not pos:
            return
        idx = torch.tensor(pos, dtype=torch.int64).to(self.device)
        tok = torch.as_tensor(tokens).to(device=self.device, dtype=torch.int32).reshape(-1)
        if tok.numel() != len(pos):
            raise ValueError(f"{tok.numel()} tokens for {len(pos)} slots")
        self.ids.index_copy_(0, idx, tok)
        for s in slots:
            self.lens[s] += 1

    def ranges(self, slots: Sequence[int]):
        """Host lists (begin, end) of the given slots' histories in `ids`."""
        slots = [self._check_slot(s) for s in slots]
        return ([s * self.max_len for s in slots],
                [s * self.max_len + self.lens[s] for s in slots])

    def history(self, slot: int) -> list:
        """Slot `slot`'s ids, read back (for checks; synchronizes)."""
        slot = self._check_slot(slot)
        b = slot * self.max_len
        return self.ids[b:b + self.lens[slot]].cpu().tolist()


def pack_resident(params_list, store: HistoryStore, slots: Sequence[int], device, generators=None):
    """Device tensors for sample_batch_ranges: the per-row parameters, one
    uniform per stochastic row (as pack_requests draws them) and each row's
    history range in store.ids, in one host buffer and one transfer."""
    B = len(params_list)
    if len(slots) != B:
        raise ValueError(f"{len(slots)} slots for {B} rows")
    gens = generators if generators is not None else [None] * B
    begin, end = store.ranges(slots)
    # layout (int32 words): T[B] K[B] P[B] PEN[B] U[B] BEGIN[B] END[B]
    buf = torch.empty(7 * B, dtype=torch.int32)
    f = buf.view(torch.float32)
    for r, (p, g) in enumerate(zip(params_list, gens)):
        f[r] = device_temperature(p.temperature)
        buf[B + r] = int(p.top_k) if -2**31 <= int(p.top_k) < 2**31 else (2**31 - 1)
        f[2 * B + r] = float(p.top_p)
        f[3 * B + r] = float(p.repetition_penalty)
        f[4 * B + r] = 0.0 if p.temperature == 0.0 else float(torch.rand((), generator=g))
        buf[5 * B + r] = begin[r]
        buf[6 * B + r] = end[r]
    d = buf.to(device, non_blocking=False)
    df = d.view(torch.float32)
    return dict(temperature=df[0:B], top_k=d[B:2 * B], top_p=df[2 * B:3 * B],
                penalty=df[3 * B:4 * B], uniforms=df[4 * B:5 * B],
                hist_begin=d[5 * B:6 * B], hist_end=d[6 * B:7 * B])


def sample_requests_resident(logits: torch.Tensor, params_list, store: HistoryStore,
                             slots: Sequence[int], generators=None,
                             out_probs: Optional[torch.Tensor] = None, append: bool = True) -> list:
    """sample_requests with the histories resident in `store`: row r is the
    request in slot slots[r].  The sampled tokens are appended to their slots
    on the device (mini_engine/scheduler.py:276) unless append is False;
    raises like the reference would for the first failing row, before
    appending anything."""
    packed = pack_resident(params_list, store, slots, logits.device, generators)
    tokens, status = sample_batch_ranges(logits, hist_ids=store.ids, out_probs=out_probs,
                                         return_status=True, share_rows=shares_rows(params_list, logits.shape[1]),
                                         **packed)
    st = status.cpu().tolist()
    for r, s in enumerate(st):
        if s != ROW_OK:
            raise_row_status(s, r)
    if append:
        store.append(slots, tokens)
    return tokens.cpu().tolist()


def raise_row_status(s: int, row: int = 0) -> None:
    if s == ROW_BAD_HISTORY:
        raise IndexError(f"row {row}: a history id is outside the vocabulary")
    if s == ROW_BAD_PARAM:
        raise RuntimeError(f"row {row}: temperature is NaN")
    if s == ROW_NONFINITE:
        raise RuntimeError(f"row {row}: probability tensor contains either inf, nan or element < 0")
    if s == ROW_EMPTY_NUCLEUS:
        raise RuntimeError(f"row {row}: invalid multinomial distribution (sum of probabilities <= 0)")
    raise RuntimeError(f"row {row}: sampler status {s}")
