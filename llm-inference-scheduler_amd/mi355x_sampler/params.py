"""SamplingParams at the API edge.

`params_from_request` builds SamplingParams from a chat-completion request
body with the keys and defaults of server/worker.py:54-62; `check_params`
rejects values the sampler cannot serve as asked, before they reach a batch.
The reference validates nothing there: a bad value surfaces later as a
torch error from inside its sampler (for example multinomial on an all-zero
distribution when top_p <= 0), one request at a time.  Here each rule names
the row status (mxs_row_status, include/mxs_sampler.h) or behaviour it
prevents, so an HTTP front end can answer 400 instead of failing a batch.
"""

from __future__ import annotations

import math

import numpy as np

from .sampling import SamplingParams


def _f32(v):
    """v as a float32 value (a Python float), or None if v is not a real number."""
    if isinstance(v, bool) or not isinstance(v, (int, float)):
        return None
    with np.errstate(over="ignore"):
        return float(np.float32(v))


def params_from_request(body: dict) -> SamplingParams:
    """server/worker.py:54-62: the same keys, defaults and conversions,
    then check_params."""
    p = SamplingParams(
        temperature=float(body.get("temperature", 0.7)),
        top_p=float(body.get("top_p", 1.0)),
        top_k=int(body.get("top_k", 0)),
        repetition_penalty=float(body.get("repetition_penalty", 1.0)),
        max_new_tokens=int(body.get("max_tokens", 256)),
        seed=body.get("seed"),
    )
    check_params(p)
    return p


def check_params(p: SamplingParams) -> None:
    """Raise ValueError naming every field out of range:

    temperature         0, or finite and > 0 (NaN: MXS_ROW_BAD_PARAM; a negative
                        value reverses the order of the logits; inf makes
                        every row non-finite, MXS_ROW_NONFINITE)
    top_p               in (0, 1] (<= 0: MXS_ROW_EMPTY_NUCLEUS; NaN or > 1
                        would silently turn top-p off)
    top_k               >= 0 (a negative value would silently turn top-k off)
    repetition_penalty  finite and > 0 (0 or inf turn penalized logits into
                        inf or NaN: MXS_ROW_NONFINITE; a negative one flips
                        their signs)
    max_new_tokens      >= 1
    seed                an int or None

    The sampler computes in float32, as the reference's tensor arithmetic
    does (sampling.py:42-44, 50, 62 use the Python floats as float32
    scalars), so the ranges are checked on the float32 values: a temperature
    of 1e-50 is 0 in float32 (greedy, where the reference would divide by
    zero), a top_p of 1e-50 is 0 (an empty nucleus), a penalty of 1e39 is
    inf; all are rejected here.
    """
    bad = []
    t = p.temperature
    t32 = _f32(t)
    if not (t32 is not None and math.isfinite(t32) and (t32 > 0.0 or t == 0.0)):
        bad.append(f"temperature must be 0 or a number > 0 that stays finite and non-zero "
                   f"in float32, got {t!r}")
    tp = p.top_p
    tp32 = _f32(tp)
    if not (tp32 is not None and 0.0 < tp32 and tp <= 1.0):
        bad.append(f"top_p must be in (0, 1] and non-zero in float32, got {tp!r}")
    if not (isinstance(p.top_k, int) and p.top_k >= 0):
        bad.append(f"top_k must be an integer >= 0, got {p.top_k!r}")
    rp = p.repetition_penalty
    rp32 = _f32(rp)
    if not (rp32 is not None and math.isfinite(rp32) and rp32 > 0.0):
        bad.append(f"repetition_penalty must be a number > 0 that stays finite and non-zero "
                   f"in float32, got {rp!r}")
    if not (isinstance(p.max_new_tokens, int) and p.max_new_tokens >= 1):
        bad.append(f"max_tokens must be an integer >= 1, got {p.max_new_tokens!r}")
    if p.seed is not None and not (isinstance(p.seed, int) and not isinstance(p.seed, bool)):
        bad.append(f"seed must be an integer or null, got {p.seed!r}")
    if bad:
        raise ValueError("; ".join(bad))
