"""Pins of the ternary expert oracle (oracle/ternary.py) on the CPU.

The reference ships no vectors for this format, so each check is one the mathematics
fixes, chosen so that a digit-order, power, sign or bit-position mistake fails it:

* base-3 identity of the digit table (every byte below 243 is the sum of its digits
  times 1, 3, 9, 27, 81);
* exact round trip: MXFP4 blocks whose values are already {-a, 0, +a} for one of the
  seven magnitudes pack and dequantise to exactly the MXFP4 values;
* optimality by brute force: on random MXFP4 blocks the packer's magnitude has the
  least mean squared error (first index on ties) and every digit is a nearest point;
* selector bits read back through numpy's little-endian bit unpacking;
* the ordered GEMV against float64 on exact-integer inputs (every summation order
  gives the same float), and against float64 at the tolerance otherwise;
* a planted selector-bit mistake in the oracle's own dequantiser is caught.
"""

from __future__ import annotations


import numpy as np
import pytest

from oracle import ref
from oracle import ternary as T
from tests.helpers import rng


def _mxfp4_codes_for(values: np.ndarray) -> np.ndarray:
    """float values that are e2m1 numbers -> their 4-bit codes (sign in bit 3)."""
    mags = np.abs(values)
    table = ref.E2M1[:8]
    code = np.argmin(np.abs(mags[..., None] - table), axis=-1)
    assert np.all(table[code] == mags)
    return (code | np.where(values < 0, 8, 0)).astype(np.uint8)


def _blocks_from_codes(codes: np.ndarray) -> np.ndarray:
    """codes [..., G, 32] -> MXFP4 blocks [..., G, 16] (element 2j = low nibble)."""
    return (codes[..., 0::2] | (codes[..., 1::2] << 4)).astype(np.uint8)


def test_digit_table_is_base3():
    lut = T.digit_lut().astype(np.int64)
    digits = (lut[:, None] >> (2 * np.arange(5))) & 3
    assert digits.max() <= 2
    b = np.arange(256)
    assert np.array_equal((digits[:243] * np.array(T.POWERS)).sum(axis=1), b[:243])
    # bytes 243..255: the fifth digit is (b // 81) % 3 = 0, as the reference's loop gives
    assert np.all(digits[243:, 4] == 0)


@pytest.mark.parametrize("rows,groups", [(3, 1), (5, 3), (4, 90), (2, 160)])
def test_ternary_exact_round_trip(rows, groups):
    g = rng(100 + groups)
    experts = 2
    mag_idx = g.integers(0, 7, size=(experts, rows, groups))
    a = T.MAGNITUDES[mag_idx]
    digit = g.integers(0, 3, size=(experts, rows, groups, 32))
    vals = (digit - 1) * a[..., None]
    codes = _mxfp4_codes_for(vals)
    blocks = _blocks_from_codes(codes)
    scales = g.integers(110, 140, size=(experts, rows, groups)).astype(np.uint8)
    packed, s2 = T.pack_mxfp4_to_ternary(blocks, scales)
    tg, tb, mb = T.ternary_geometry(groups * 32)
    assert packed.shape == (experts, rows, tb + mb)
    assert np.array_equal(s2, scales)
    want = ref.mxfp4_dequant(blocks, scales)
    got = T.ternary_dequant(packed, scales)
    assert np.array_equal(got, want)


def test_packer_choice_is_least_squares():
    g = rng(7)
    experts, rows, groups = 2, 6, 12
    codes = g.integers(0, 16, size=(experts, rows, groups, 32)).astype(np.uint8)
    # a few all-zero blocks: every magnitude ties at zero error, the first is kept
    codes[0, 0, :3] = 0
    blocks = _blocks_from_codes(codes)
    scales = np.full((experts, rows, groups), 127, dtype=np.uint8)
    packed, _ = T.pack_mxfp4_to_ternary(blocks, scales)
    v = ref.E2M1[codes]
    got = T.ternary_dequant(packed, scales).reshape(experts, rows, groups, 32)
    # every element is a nearest point of {-a, 0, +a} for its group's magnitude
    tg, tb, _ = T.ternary_geometry(groups * 32)
    bits = np.unpackbits(packed[..., tb:], axis=-1, bitorder="little")
    sel = np.zeros((experts, rows, groups), dtype=np.int64)
    for b in range(3):
        sel |= bits[..., 3 * np.arange(groups) + b].astype(np.int64) << b
    assert sel.max() <= 6
    a = T.MAGNITUDES[sel][..., None]
    cand = np.stack([-a + 0 * v, 0 * v, a + 0 * v])
    best = np.min(np.abs(cand - v), axis=0)
    assert np.array_equal(np.abs(got - v), best)
    # the magnitude minimises the block's squared error (brute force over the seven)
    errs = []
    for m in T.MAGNITUDES:
        rec = np.where(np.abs(v) > m / 2, np.sign(v) * m, 0.0)
        errs.append(np.square(v - rec).mean(axis=-1))
    errs = np.stack(errs, axis=-1)
    assert np.array_equal(sel, np.argmin(errs, axis=-1))
    assert np.all(sel[0, 0, :3] == 0)


def test_ordered_gemv_exact_integer_inputs():
    g = rng(11)
    experts, rows, groups = 3, 40, 33          # 1056 columns: a partial last chunk
    cols = groups * 32
    _, tb, mb = T.ternary_geometry(cols)
    packed = g.integers(0, 256, size=(experts, rows, tb + mb)).astype(np.uint8)
    scales = g.integers(127, 130, size=(experts, rows, groups)).astype(np.uint8)
    x = g.integers(-3, 4, size=(2, cols)).astype(np.float32)
    idx = np.array([2, 0])
    got = T.ternary_selected_gemv(packed, scales, x, idx)
    w = T.ternary_dequant(packed, scales)
    want = np.stack([w[e] @ x[i].astype(np.float64) for i, e in enumerate(idx)])
    assert np.array_equal(got.astype(np.float64), want)


def test_ordered_gemv_tolerance_and_invalid_expert():
    g = rng(12)
    experts, rows, groups = 2, 16, 90
    cols = groups * 32
    _, tb, mb = T.ternary_geometry(cols)
    packed = g.integers(0, 256, size=(experts, rows, tb + mb)).astype(np.uint8)
    scales = g.integers(119, 124, size=(experts, rows, groups)).astype(np.uint8)
    x = g.standard_normal(cols).astype(np.float16).astype(np.float32)
    got = T.ternary_selected_gemv(packed, scales, x, np.array([1, 5]))
    want = T.ternary_dequant(packed, scales)[1] @ x.astype(np.float64)
    assert ref.max_rel_err(got[0], want) < 1e-5
    assert np.all(np.isnan(got[1]))


def test_planted_selector_mistake_is_caught():
    """Reading the selector one bit off must break the exact round trip."""
    g = rng(3)
    mag_idx = g.integers(0, 7, size=(1, 2, 8))
    digit = g.integers(0, 3, size=(1, 2, 8, 32))
    vals = (digit - 1) * T.MAGNITUDES[mag_idx][..., None]
    blocks = _blocks_from_codes(_mxfp4_codes_for(vals))
    scales = np.full((1, 2, 8), 127, dtype=np.uint8)
    packed, _ = T.pack_mxfp4_to_ternary(blocks, scales)
    _, tb, _ = T.ternary_geometry(256)
    shifted = packed.copy()
    sel = shifted[..., tb:].astype(np.uint32)
    shifted[..., tb:] = ((sel << 1) & 0xFF).astype(np.uint8)
    assert not np.array_equal(T.ternary_dequant(shifted, scales), ref.mxfp4_dequant(blocks, scales))
