"""Batched sampling: one kernel launch for a whole [B, V] batch of logits.

`sample_batch` is the device-array entry (per-row parameters as tensors, the
history as CSR); `sample_requests` packs a scheduler's per-request
SamplingParams, output ids and generators into that form (the batched
counterpart of the per-row loop at mini_engine/scheduler.py:268-275).
"""

from __future__ import annotations

from typing import Optional, Sequence

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
                 return_status: bool = False):
    """Sample one token per row of `logits` ([B, V], float32 or float16).

    temperature f32[B] (0 = greedy), top_k i32[B] (<= 0 off), top_p f32[B]
    (>= 1 off), penalty f32[B] (1 off), hist_offsets i32[B+1] / hist_ids i32[N]
    (CSR history of generated ids), uniforms f32[B] in [0, 1).  All tensors on
    the logits' device.  Returns int64[B] token ids on the device (-1 for rows
    whose status is not ok), plus int32[B] row statuses if return_status.
    out_probs, if given, is filled with the post-filter probabilities [B, V].
    The launch is asynchronous on the current stream.
    """
    _native.require_gpu(logits.device)
    ext = _native.extension()
    B, V = logits.shape
    dev = logits.device
    tokens = torch.empty(B, dtype=torch.int64, device=dev)
    status = torch.empty(B, dtype=torch.int32, device=dev)
    ws = _native.workspace(dev, B, V)
    ext.sample(logits, temperature, top_k, top_p, penalty, hist_offsets, hist_ids, uniforms,
               tokens, status, out_probs, ws)
    return (tokens, status) if return_status else tokens


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
        self.workspace = torch.empty(max(int(self.ext.workspace_bytes(B, V)), 256),
                                     dtype=torch.uint8, device=self.device)

    def run(self, logits, temperature, top_k, top_p, penalty, hist_offsets=None,
            hist_ids=None, uniforms=None):
        self.ext.sample(logits, temperature, top_k, top_p, penalty, hist_offsets, hist_ids,
                        uniforms, self.tokens, self.status, self.probs, self.workspace)
        return self.tokens


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
        f[r] = float(p.temperature)
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
    tokens, status = sample_batch(logits, out_probs=out_probs, return_status=True, **packed)
    st = status.cpu().tolist()
    for r, s in enumerate(st):
        if s != ROW_OK:
            raise_row_status(s, r)
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
