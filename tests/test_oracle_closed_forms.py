"""Pins the oracle's arithmetic primitives (oracle/sampler_oracle.c) against
what mathematics fixes, independently of how the oracle computes them:

  orc_mass(d)        floor(exp(d) * 2^44), checked against fp64 exp within the
                     fp32 polynomial's error, exactly at d = 0 and exact powers
                     of two, monotone over the whole fp32 range it accepts
  orc_ceil_mul/floor_mul   ceil/floor of the exact rational p*W (Fractions)
  orc_vkey           order-preserving on sorted floats, +0 and -0 share a key
  orc_clamp_uniform  [0, 1) clamp: NaN and negatives read 0, >= 1 reads 1-2^-24
"""

import math
from fractions import Fraction

import numpy as np
import pytest

MASS_ONE = 1 << 44


def test_mass_at_zero_and_powers_of_two(oracle):
    assert oracle.mass(0.0) == MASS_ONE
    assert oracle.mass(-0.0) == MASS_ONE
    # d = -n*ln2 rounds to n exactly and leaves r ~ 0: the mass is 2^(44-n)
    # up to the polynomial's rounding near 1
    for n in range(1, 40):
        d = float(np.float32(-n * math.log(2.0)))
        exact = math.exp(d) * MASS_ONE
        assert abs(oracle.mass(d) - exact) <= 2.0 ** (44 - n) * 4e-7 + 1


def test_mass_special_inputs(oracle):
    assert oracle.mass(float("-inf")) == 0
    assert oracle.mass(float("nan")) == 0
    assert oracle.mass(-200.0) == 0
    assert oracle.mass(-104.5) == 0


def test_mass_matches_fp64_exp(oracle):
    rng = np.random.default_rng(11)
    d = np.concatenate([
        -rng.random(4000).astype(np.float32) * 2.0,     # near the maximum
        -rng.random(4000).astype(np.float32) * 30.0,     # the bulk of a row
        -np.float32(np.log(2.0)) * np.arange(1, 30, dtype=np.float32) / 2,   # half-way points
    ]).astype(np.float32)
    worst = 0.0
    for v in d:
        exact = math.exp(float(v)) * MASS_ONE
        got = oracle.mass(float(v))
        if exact < 2.0 ** 24:           # small masses: the floor dominates
            assert abs(got - exact) <= exact * 1e-6 + 1.0
            continue
        worst = max(worst, abs(got - exact) / exact)
    # the degree-7 polynomial in fp32 with fma stays within ~7e-8 of exp on
    # these inputs.  A dropped r^7/5040 term adds up to 1.2e-7 at |r| = ln2/2,
    # a dropped r^6/720 term 2.4e-6, a wrong ln2 split far more.
    assert worst < 1e-7, worst


def test_mass_monotone(oracle):
    # every fp32 value of d in [-20, 0] at a stride, plus a dense patch near 0
    vals = np.unique(np.concatenate([
        np.linspace(-20.0, 0.0, 20001, dtype=np.float32),
        -np.arange(0, 5000, dtype=np.float32) * np.float32(2.0 ** -20),
    ]))
    m = np.array([oracle.mass(float(v)) for v in vals], dtype=np.float64)
    assert np.all(np.diff(m) >= 0), "mass must not decrease as d grows"


def _exact(p):
    return Fraction(float(np.float32(p)))


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_ceil_floor_mul_exact(oracle, seed):
    rng = np.random.default_rng(seed)
    ps = np.concatenate([rng.random(300).astype(np.float32),
                         np.float32([0.0, 1e-30, 1e-7, 0.5, 0.9999999, 2.0 ** -24, 0.75])])
    Ws = [1, 2, 3, 7, 1 << 44, (1 << 44) + 12345, (1 << 62) + 98765, (1 << 63) - 1,
          int(rng.integers(1, 1 << 62))]
    for p in ps:
        for W in Ws:
            prod = _exact(p) * W
            assert oracle.ceil_mul(float(p), W) == math.ceil(prod), (p, W)
            assert oracle.floor_mul(float(p), W) == math.floor(prod), (p, W)


def test_vkey_order_preserving(oracle):
    rng = np.random.default_rng(5)
    x = np.concatenate([rng.standard_normal(500).astype(np.float32) * 100,
                        np.float32([np.inf, -np.inf, 0.0, -0.0, 1e-45, -1e-45,
                                    3.4e38, -3.4e38, 1.0, -1.0])])
    xs = np.sort(x)
    keys = [oracle.vkey(float(v)) for v in xs]
    for a, b, ka, kb in zip(xs[:-1], xs[1:], keys[:-1], keys[1:]):
        if a < b:
            assert ka < kb, (a, b)
        else:
            assert ka == kb, (a, b)
    assert oracle.vkey(0.0) == oracle.vkey(-0.0)


def test_clamp_uniform(oracle):
    L = oracle.lib()
    below_one = float(np.nextafter(np.float32(1.0), np.float32(0.0)))
    assert L.orc_clamp_uniform(float("nan")) == 0.0
    assert L.orc_clamp_uniform(-0.25) == 0.0
    assert L.orc_clamp_uniform(0.0) == 0.0
    assert L.orc_clamp_uniform(0.3) == float(np.float32(0.3))
    assert L.orc_clamp_uniform(1.0) == below_one
    assert L.orc_clamp_uniform(7.0) == below_one
