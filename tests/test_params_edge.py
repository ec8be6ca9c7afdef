"""SamplingParams at the API edge, on the CPU: the request body's keys and
defaults of server/worker.py:54-62, and the range checks that keep values
the sampler would turn into row errors (or silently ignore) out of a batch.
"""

import math

import pytest

from mi355x_sampler import SamplingParams, check_params, params_from_request


def test_defaults_and_keys_follow_the_worker():
    p = params_from_request({})
    assert (p.temperature, p.top_p, p.top_k, p.repetition_penalty, p.max_new_tokens, p.seed) == \
        (0.7, 1.0, 0, 1.0, 256, None)
    p = params_from_request({"temperature": "0", "top_p": 0.9, "top_k": "50",
                             "repetition_penalty": 1.1, "max_tokens": 8, "seed": 3})
    assert p.greedy and (p.top_p, p.top_k, p.repetition_penalty, p.max_new_tokens, p.seed) == \
        (0.9, 50, 1.1, 8, 3)
    assert isinstance(p, SamplingParams)


@pytest.mark.parametrize("field,value", [
    ("temperature", -0.1), ("temperature", math.nan), ("temperature", math.inf),
    ("top_p", 0.0), ("top_p", -1.0), ("top_p", 1.5), ("top_p", math.nan),
    ("top_k", -1),
    ("repetition_penalty", 0.0), ("repetition_penalty", -1.2), ("repetition_penalty", math.inf),
    ("repetition_penalty", math.nan),
    ("max_tokens", 0),
    ("seed", "abc"), ("seed", 1.5),
    # values that the float32 arithmetic of the chain turns into 0 or inf
    ("temperature", 1e-50), ("temperature", 1e39),
    ("top_p", 1e-50),
    ("repetition_penalty", 1e-50), ("repetition_penalty", 1e39),
])
def test_out_of_range_values_are_rejected(field, value):
    with pytest.raises(ValueError, match=field):
        params_from_request({field: value})


def test_every_bad_field_is_named():
    with pytest.raises(ValueError) as e:
        check_params(SamplingParams(temperature=-1.0, top_p=0.0, top_k=-5))
    msg = str(e.value)
    assert "temperature" in msg and "top_p" in msg and "top_k" in msg


def test_edge_values_pass():
    for body in ({"temperature": 0.0}, {"top_p": 1.0}, {"top_p": 1e-6}, {"top_k": 0},
                 {"top_k": 10**6}, {"repetition_penalty": 1e-3}, {"max_tokens": 1}, {"seed": 0},
                 {"temperature": 1e-40}, {"top_p": 1e-40}, {"repetition_penalty": 3e38}):
        params_from_request(body)   # (1e-40 is a float32 subnormal, not 0)
