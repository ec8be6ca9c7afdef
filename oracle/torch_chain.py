"""Torch-CPU restatement of the reference sampler chain, op for op.

TEST INFRASTRUCTURE ONLY: used by tests/ to pin the exact oracle
(sampler_oracle.c) against the reference's own composition, and by bench.py's
cpu_baseline leg as the timed CPU path (it runs the same torch CPU ops, in the
same order, as mini_engine/sampling.py:30-69, so it costs what the reference
costs).  The product never imports it.

Differences from the reference are switches, all off by default except the
copy at the top:
  stable=True        torch.sort(..., stable=True): lowest index first on ties
                     (the reference's sampling.py:57 uses stable=False)
  draw="multinomial" torch.multinomial(probs, 1, generator), as sampling.py:69
  draw="none"        stop after the softmax at sampling.py:68
The caller's fp32 logits are cloned, so unlike sampling.py:36/45 the penalty
does not write into the caller's tensor.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass
class ChainTrace:
    token: int | None
    probs: torch.Tensor            # [V] post-filter probabilities (sampling.py:68)
    kept: torch.Tensor             # [V] bool, tokens still finite after top-k/top-p
    n_topk: int                    # survivors of top-k (V when off)


def cpu_ref(logits: torch.Tensor, params, generated_ids, generator=None, *,
            stable: bool = False, draw: str = "multinomial") -> ChainTrace:
    """Restates mini_engine/sampling.py:30-69 (see the module docstring)."""
    logits = logits.float().clone()                                        # :36

    if params.repetition_penalty != 1.0 and generated_ids:                # :38
        prev = torch.tensor(sorted(set(generated_ids)), device=logits.device)   # :39
        scores = logits[prev]                                              # :40
        scores = torch.where(                                              # :42-44
            scores > 0, scores / params.repetition_penalty,
            scores * params.repetition_penalty)
        logits[prev] = scores                                              # :45

    if params.temperature == 0.0:                                          # :47 (greedy)
        tok = int(torch.argmax(logits).item())                             # :48
        probs = torch.zeros_like(logits)
        probs[tok] = 1.0
        return ChainTrace(tok, probs, probs > 0, 1)

    logits = logits / params.temperature                                   # :50

    n_topk = logits.shape[-1]
    if params.top_k > 0:                                                   # :52
        kth = torch.topk(logits, min(params.top_k, logits.shape[-1])).values[-1]   # :53
        logits[logits < kth] = float("-inf")                               # :54
        n_topk = int((logits > float("-inf")).sum().item())

    if params.top_p < 1.0:                                                 # :56
        sorted_logits, sorted_idx = torch.sort(logits, descending=True,
                                               stable=stable)              # :57
        probs = torch.softmax(sorted_logits, dim=-1)                       # :58
        cumulative = torch.cumsum(probs, dim=-1)                           # :59
        cutoff = cumulative - probs >= params.top_p                        # :62
        sorted_logits[cutoff] = float("-inf")                              # :63
        logits = torch.full_like(logits, float("-inf")).scatter(          # :64-66
            0, sorted_idx, sorted_logits)

    kept = logits > float("-inf")
    probs = torch.softmax(logits, dim=-1)                                  # :68
    tok = None
    if draw == "multinomial":
        tok = int(torch.multinomial(probs, 1, generator=generator).item())   # :69
    elif draw != "none":
        raise ValueError(f"unknown draw mode {draw!r}")
    return ChainTrace(tok, probs, kept, n_topk)


def cpu_ref_token(logits, params, generated_ids, generator=None) -> int:
    """Token only, exactly as the reference computes it (stable=False)."""
    return cpu_ref(logits, params, generated_ids, generator).token
