"""The host-side rule that sets MXS_FLAG_SHARE_ROWS (no GPU needed).

sample_requests and sample_requests_resident set the flag when the batch's
SamplingParams mix rows with top-k off (sampling.py:52: top_k <= 0 or
top_k >= V, with a temperature) and other rows."""

from mi355x_sampler import SamplingParams, shares_rows


def test_shares_rows_rule():
    """The host-side rule sample_requests uses to set the flag."""
    V = 1000
    assert shares_rows([SamplingParams(temperature=0.7, top_k=0), SamplingParams(temperature=0.7, top_k=50)], V)
    assert shares_rows([SamplingParams(temperature=0.7, top_k=V), SamplingParams(temperature=0.0)], V)
    assert not shares_rows([SamplingParams(temperature=0.7, top_k=0)] * 3, V)
    assert not shares_rows([SamplingParams(temperature=0.7, top_k=50)] * 3, V)
    assert not shares_rows([SamplingParams(temperature=0.0, top_k=0), SamplingParams(temperature=0.7, top_k=5)], V)
