"""The model's LM head feeding the sampler: logits = hidden . weight^T in
fp32 on MFMA, with each row's maximum reduced in the same kernel.

Replaces `logits = F.linear(h[last_idx], self.lm_head)` of
mini_engine/model/qwen2.py:176-183 (lm_head is the tied embedding,
qwen2.py:92-96; the engine runs fp32, mini_engine/engine.py:29).  The
maxima let the sampler finish greedy rows without reading their logits
again (sample_batch(..., row_best=best)).
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch

from . import _native


def lm_head(hidden: torch.Tensor, weight: torch.Tensor,
            out_logits: Optional[torch.Tensor] = None,
            out_best: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """(logits f32[B, V], best i64[B]) for hidden f32[B, D] and weight
    f32[V, D] (rows contiguous, 16-byte aligned).  best[r] packs the row's
    maximum as (key << 32) | ~index with key the order-preserving key of
    the value (NaN above everything): the greedy token is
    best_token(best).  Sums are fp32 in the kernel's own order: a logit is
    within D * 2^-23 * sum_k |hidden[r, k] weight[v, k]| of the exact sum.
    Asynchronous on the current stream."""
    _native.require_gpu(hidden.device)
    ext = _native.extension()
    B, V = hidden.shape[0], weight.shape[0]
    if out_logits is None:
        out_logits = torch.empty((B, V), dtype=torch.float32, device=hidden.device)
    if out_best is None:
        out_best = torch.empty(B, dtype=torch.int64, device=hidden.device)
    ext.lm_head(hidden, weight, out_logits, out_best)
    return out_logits, out_best


def best_token(best: torch.Tensor) -> torch.Tensor:
    """The first index of each row's maximum from lm_head's packed maxima."""
    return 0xFFFFFFFF - (best & 0xFFFFFFFF)
