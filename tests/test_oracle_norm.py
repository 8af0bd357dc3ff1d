"""Pins the oracle's layer-boundary restatement (oracle/q35_oracle_norm.c):
Ops.AddInPlace + Qwen35Ops.RmsNormZeroCentered (Qwen35Ops.cs:22-64).

The reference has no tests for it, so the restatement is pinned by:
  - hand-built rows whose sum of squares depends on the order: 2^24 in lane 0
    and ones elsewhere, where a sequential sum loses every +1 but the 8-lane
    FMA order with the VecDotQ4K.HorizontalSum pairing keeps them (sum
    2^24 + 14 for dim 16), and a 12-wide row whose 4 tail elements are added
    after the horizontal sum;
  - the fp64 value of (h / rms) * (1 + w) on random rows, within fp32 rounding;
  - the residual add being the exact fp32 sum, and w = None equal to w = 0.
"""
from __future__ import annotations

import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "oracle"))

import oracle  # noqa: E402

F = np.float32


def _expected_from_sum(row, s, eps):
    scale = F(1.0) / np.sqrt(F(F(s) / F(row.size)) + F(eps), dtype=F)
    return (row * scale).astype(F)


def test_lane_order_keeps_small_squares():
    row = np.ones(16, F)
    row[0] = 4096.0                       # square 2^24: one more ulp is 2
    _, y = oracle.add_rmsnorm(row[None], None, None, 16, eps=0.0)
    # lane 0: fma(1, 1, 2^24) rounds back to 2^24; lanes 1-7 hold 2 each;
    # ((a0 + a4) + (a2 + a6)) + ((a1 + a5) + (a3 + a7)) = 2^24 + 14 exactly
    assert np.array_equal(y[0], _expected_from_sum(row, 2.0 ** 24 + 14, 0.0))
    # a sequential sum would give 2^24: the outputs differ
    assert not np.array_equal(y[0], _expected_from_sum(row, 2.0 ** 24, 0.0))


def test_tail_after_horizontal_sum():
    row = np.ones(12, F)
    row[0] = 4096.0
    _, y = oracle.add_rmsnorm(row[None], None, None, 12, eps=0.0)
    # lanes: a0 = 2^24, a1..a7 = 1; (2^24 + 1 -> 2^24) + 2, + 4 = 2^24 + 6;
    # tail +1 four times: 2^24 + 7 -> 2^24 + 8 (ties to even), then each +1
    # ties back to 2^24 + 8
    assert np.array_equal(y[0], _expected_from_sum(row, 2.0 ** 24 + 8, 0.0))


@pytest.mark.parametrize("dim", [2560, 4096, 200])
def test_against_fp64(dim):
    rng = np.random.default_rng(dim)
    h = (rng.standard_normal((5, dim)) * rng.uniform(0.1, 30, (5, 1))).astype(F)
    d = rng.standard_normal((5, dim)).astype(F)
    w = (rng.standard_normal(dim) * 0.1).astype(F)
    hout, y = oracle.add_rmsnorm(h, d, w, dim, eps=1e-6)
    assert np.array_equal(hout, (h + d).astype(F))
    h64 = hout.astype(np.float64)
    want = h64 / np.sqrt((h64 ** 2).mean(1, keepdims=True) + 1e-6) * (1.0 + w.astype(np.float64))
    assert np.all(np.abs(y - want) <= 3e-7 * np.abs(want) + 1e-30)


def test_null_weight_is_zero_weight():
    rng = np.random.default_rng(3)
    h = rng.standard_normal((3, 64)).astype(F)
    _, y0 = oracle.add_rmsnorm(h, None, None, 64)
    _, y1 = oracle.add_rmsnorm(h, None, np.zeros(64, F), 64)
    assert np.array_equal(y0, y1)
