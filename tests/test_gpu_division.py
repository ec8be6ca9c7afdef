"""The quotient pass 2 of a top-k-off row computes: fl32(x * RN64(1 / T)).

mini_engine/sampling.py:50 divides the logits by the temperature in fp32
(an IEEE quotient).  The kernel's mass pass forms the same quotient as the
binary64 product of x and the binary64 reciprocal of T, rounded to
binary32.  Checked here bit for bit against the IEEE fp32 quotient, on the
GPU (torch's fp32 division and binary64 multiply are IEEE operations):

  * every one of the 2^32 binary32 values of x, for T = 0.7 and T = -1.3;
  * 2^24 random bit patterns of x for each of 64 temperatures spread over
    2^-40 .. 2^40 (both signs), and for T a power of two;
  * every normal, zero, infinite or NaN quotient must match exactly; a
    subnormal quotient may differ by one unit in its last place only (the
    kernel falls back to the IEEE path for rows whose maximum m could make
    that visible, 0 < |m| < 2^-101).
"""

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

TINY = 2.0 ** -126


def compare(x: torch.Tensor, T: float):
    q = x / torch.tensor(T, dtype=torch.float32, device=x.device)
    r = 1.0 / float(np.float64(np.float32(T)))          # RN64(1 / T) of the fp32 temperature
    p = (x.double() * r).float()
    qi, pi = q.view(torch.int32), p.view(torch.int32)
    nan = torch.isnan(q)
    assert bool((torch.isnan(p) == nan).all())
    sub = (q.abs() < TINY) & (q != 0)
    bad = (qi != pi) & ~nan
    assert not bool((bad & ~sub).any()), (T, x[bad & ~sub][:4].tolist())
    # a subnormal quotient: at most one unit in the last place
    assert bool(((qi.long() - pi.long()).abs()[bad] <= 1).all())
    return int(bad.sum())


@pytest.mark.parametrize("T", [0.7, -1.3])
def test_every_binary32_value(cuda, T):
    step = 1 << 28
    off = 0
    for start in range(-(1 << 31), 1 << 31, step):
        bits = torch.arange(start, start + step, dtype=torch.int64, device=cuda).to(torch.int32)
        off += compare(bits.view(torch.float32), T)
    print(f"T={T}: {off} subnormal quotients off by one unit", flush=True)


def test_random_values_many_temperatures(cuda):
    g = torch.Generator(device=cuda).manual_seed(5)
    rng = np.random.default_rng(7)
    temps = list(np.float32(np.exp2(rng.uniform(-40, 40, 60)) * rng.choice([-1, 1], 60)))
    temps += [np.float32(1.0), np.float32(0.5), np.float32(-8.0), np.float32(3.0)]
    for T in temps:
        bits = torch.randint(-(1 << 31), 1 << 31, (1 << 24,), generator=g, device=cuda, dtype=torch.int64)
        compare(bits.to(torch.int32).view(torch.float32), float(T))
