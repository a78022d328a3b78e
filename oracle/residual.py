"""Residual sidecar corrections in the HIP kernels' order -- TEST INFRASTRUCTURE ONLY.

CPU restatement, used only to check the HIP kernels, of the reference's sparse and
binary residual matvecs (triton_kernels.py:2335-2419, wrappers :5429-5487):

* sparse: correction[m] = sum_k values[m, k] * x[indices[m, k]];
* binary: correction[m] = sum_k (bit ? +1 : -1) * scale[m, k // 32] * x[k], sign bit k
  at byte k // 8, bit k % 8.

Both return float32 corrections in the kernels' documented order (one 64-lane wave per
row, lane l taking terms / groups l, l + 64, ..., then the pairwise butterfly over the
lanes); the caller adds them to the previous output and rounds to the output dtype.
"""

from __future__ import annotations

import numpy as np


def _butterfly(lanes: np.ndarray) -> np.ndarray:
    while lanes.shape[1] > 1:
        lanes = lanes[:, 0::2] + lanes[:, 1::2]
    return lanes[:, 0]


def sparse_residual(values: np.ndarray, indices: np.ndarray, x: np.ndarray) -> np.ndarray:
    v = np.asarray(values, dtype=np.float32)
    idx = np.asarray(indices, dtype=np.int64)
    x = np.asarray(x, dtype=np.float32)
    rows, terms = v.shape
    bad = np.any((idx < 0) | (idx >= x.size), axis=1)
    xv = x[np.where((idx >= 0) & (idx < x.size), idx, 0)]
    lanes = np.zeros((rows, 64), dtype=np.float32)
    for k in range(terms):
        lanes[:, k % 64] = lanes[:, k % 64] + v[:, k] * xv[:, k]
    out = _butterfly(lanes)
    out[bad] = np.nan
    return out


def binary_residual(signs: np.ndarray, scales: np.ndarray, x: np.ndarray) -> np.ndarray:
    s = np.asarray(scales, dtype=np.float32)
    x = np.asarray(x, dtype=np.float32)
    rows = s.shape[0]
    cols = x.size
    k = np.arange(cols)
    bit = (np.asarray(signs, dtype=np.uint8)[:, k // 8] >> (k % 8)) & 1
    term = np.where(bit != 0, x[None, :], -x[None, :]).astype(np.float32)
    lanes = np.zeros((rows, 64), dtype=np.float32)
    for g in range(cols // 32):
        p = np.zeros(rows, dtype=np.float32)
        for c in range(32 * g, 32 * g + 32):
            p = p + term[:, c]
        lanes[:, g % 64] = lanes[:, g % 64] + s[:, g] * p
    return _butterfly(lanes)
