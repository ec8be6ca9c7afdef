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

from .sampling import SamplingParams


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

    temperature         finite and >= 0 (NaN: MXS_ROW_BAD_PARAM; a negative
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
    """
    bad = []
    t = p.temperature
    if not (isinstance(t, (int, float)) and math.isfinite(t) and t >= 0.0):
        bad.append(f"temperature must be a finite number >= 0, got {t!r}")
    tp = p.top_p
    if not (isinstance(tp, (int, float)) and 0.0 < tp <= 1.0):
        bad.append(f"top_p must be in (0, 1], got {tp!r}")
    if not (isinstance(p.top_k, int) and p.top_k >= 0):
        bad.append(f"top_k must be an integer >= 0, got {p.top_k!r}")
    rp = p.repetition_penalty
    if not (isinstance(rp, (int, float)) and math.isfinite(rp) and rp > 0.0):
        bad.append(f"repetition_penalty must be a finite number > 0, got {rp!r}")
    if not (isinstance(p.max_new_tokens, int) and p.max_new_tokens >= 1):
        bad.append(f"max_tokens must be an integer >= 1, got {p.max_new_tokens!r}")
    if p.seed is not None and not (isinstance(p.seed, int) and not isinstance(p.seed, bool)):
        bad.append(f"seed must be an integer or null, got {p.seed!r}")
    if bad:
        raise ValueError("; ".join(bad))
