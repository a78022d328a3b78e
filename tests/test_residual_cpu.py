"""Pins of the residual sidecar oracle (oracle/residual.py) on the CPU.

The reference ships no vectors for these operators.  Exact-integer inputs make every
summation order give the float64 value exactly, so an index, sign or bit-order mistake
cannot hide behind rounding; a planted bit-order reversal must be caught, and an
out-of-range index must poison only its own row.
"""

from __future__ import annotations

import numpy as np

from oracle import residual as R
from tests.helpers import rng


def test_sparse_exact_integer_inputs():
    g = rng(31)
    rows, terms, cols = 50, 150, 700
    values = g.integers(-4, 5, size=(rows, terms)).astype(np.float32)
    idx = g.integers(0, cols, size=(rows, terms))
    x = g.integers(-8, 9, size=cols).astype(np.float32)
    want = np.array([sum(float(values[m, k]) * float(x[idx[m, k]]) for k in range(terms)) for m in range(rows)])
    assert np.array_equal(R.sparse_residual(values, idx, x).astype(np.float64), want)


def test_sparse_bad_index_poisons_only_its_row():
    g = rng(32)
    values = g.standard_normal((4, 10)).astype(np.float32)
    idx = g.integers(0, 20, size=(4, 10))
    idx[1, 3] = 20
    idx[2, 0] = -1
    got = R.sparse_residual(values, idx, g.standard_normal(20).astype(np.float32))
    assert np.isnan(got[1]) and np.isnan(got[2]) and not np.isnan(got[0]) and not np.isnan(got[3])


def test_binary_exact_integer_inputs_and_bit_order():
    g = rng(33)
    rows, cols = 20, 2880
    signs = g.integers(0, 256, size=(rows, cols // 8)).astype(np.uint8)
    scales = g.integers(1, 4, size=(rows, cols // 32)).astype(np.float32)
    x = g.integers(-5, 6, size=cols).astype(np.float32)
    bits = np.unpackbits(signs, axis=1, bitorder="little").astype(np.float64)
    w = (2.0 * bits - 1.0) * np.repeat(scales.astype(np.float64), 32, axis=1)
    want = w @ x.astype(np.float64)
    assert np.array_equal(R.binary_residual(signs, scales, x).astype(np.float64), want)
    # a planted bit-order reversal (MSB first) must change the result
    flipped = np.packbits(np.unpackbits(signs, axis=1, bitorder="little"), axis=1, bitorder="big")
    assert not np.array_equal(R.binary_residual(flipped, scales, x).astype(np.float64), want)
