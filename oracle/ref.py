"""Float64 closed forms of the reference's dequantise-then-matmul semantics.

TEST INFRASTRUCTURE ONLY.  Each dequantiser restates the reference directly from
its source (file:line cited) and is written independently of the product's packers
and kernels: it reads the packed bytes the way the reference kernels do.
"""

from __future__ import annotations

import numpy as np

# e2m1 magnitudes, sign in bit 3 (triton_kernels.py:249-276; gpu_runtime.py:12876-12897)
E2M1 = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0, -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0])
# q2 codebook and q1 signs (triton_kernels.py:1181-1188)
Q2_LUT = np.array([-1.5, -0.5, 0.5, 1.5])


def int4_codes(packed: np.ndarray) -> np.ndarray:
    """uint8 [..., cols/2] -> stored codes c in [0, 15]: low nibble = k even
    (triton_kernels.py:1606-1610 / 1461-1462)."""
    p = np.asarray(packed, dtype=np.uint8)
    c = np.empty(p.shape[:-1] + (p.shape[-1] * 2,), dtype=np.int64)
    c[..., 0::2] = p & 0x0F
    c[..., 1::2] = (p >> 4) & 0x0F
    return c


def int4_dequant(packed: np.ndarray, scales: np.ndarray, group_size: int) -> np.ndarray:
    """w = (c - 8) * s (symmetric, triton_kernels.py:1466-1467) or, for scales of
    shape [rows, groups, 2], w = c * s + m (affine, triton_kernels.py:1633-1649)."""
    c = int4_codes(packed).astype(np.float64)
    rows, cols = c.shape
    s = np.asarray(scales, dtype=np.float64)
    if s.ndim == 3:
        grp = np.arange(cols) // group_size
        return c * s[:, grp, 0] + s[:, grp, 1]
    if group_size >= cols:
        return (c - 8.0) * s.reshape(rows, -1)[:, :1]
    grp = np.arange(cols) // group_size
    return (c - 8.0) * s[:, grp]


def fp8_e4m3fn(bits: np.ndarray) -> np.ndarray:
    """float8_e4m3fn decode from the format definition (OCP FP8 E4M3, finite-only)."""
    b = np.asarray(bits, dtype=np.int64)
    s = np.where(b >> 7, -1.0, 1.0)
    e = (b >> 3) & 15
    m = b & 7
    v = np.where(e == 0, m * 2.0 ** -9, (8 + m) * np.exp2(e.astype(np.float64) - 10))
    v = np.where((e == 15) & (m == 7), np.nan, v)
    return s * v


def mxfp4_dequant(blocks: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """blocks uint8 [..., G, 16], scales uint8 [..., G] -> float64 [..., G*32]
    (triton_kernels.py:444-470: element 2j = low nibble of byte j, times 2^(e-127))."""
    b = np.asarray(blocks, dtype=np.uint8)
    lo = E2M1[b & 0x0F]
    hi = E2M1[b >> 4]
    vals = np.empty(b.shape[:-1] + (32,), dtype=np.float64)
    vals[..., 0::2] = lo
    vals[..., 1::2] = hi
    vals = vals * np.exp2(np.asarray(scales, dtype=np.float64) - 127.0)[..., None]
    return vals.reshape(vals.shape[:-2] + (-1,))


def lowbit_e8_dequant(packed: np.ndarray, scales: np.ndarray, bits: int) -> np.ndarray:
    """packed uint8 [..., G, 32*bits/8], scales uint8 [..., G] (triton_kernels.py:1163-1199)."""
    p = np.asarray(packed, dtype=np.uint8).astype(np.int64)
    i = np.arange(32)
    if bits == 2:
        code = (p[..., i // 4] >> (2 * (i % 4))) & 3
        val = Q2_LUT[code]
    else:
        code = (p[..., i // 8] >> (i % 8)) & 1
        val = np.where(code != 0, 1.0, -1.0)
    val = val * np.exp2(np.asarray(scales, dtype=np.float64) - 127.0)[..., None]
    return val.reshape(val.shape[:-2] + (-1,))


def lowbit_affine_dequant(packed: np.ndarray, scale_zero: np.ndarray, bits: int, group_size: int, cols: int) -> np.ndarray:
    """Affine q2/q1 (BASELINE cfg2 definition): w = (c - z) * s per group."""
    p = np.asarray(packed, dtype=np.uint8).astype(np.int64)
    i = np.arange(cols)
    per = 8 // bits
    code = (p[:, i // per] >> (bits * (i % per))) & ((1 << bits) - 1)
    sz = np.asarray(scale_zero, dtype=np.float64)
    g = i // group_size
    return (code - sz[:, g, 1]) * sz[:, g, 0]


def gemv64(w: np.ndarray, x: np.ndarray) -> np.ndarray:
    return np.asarray(w, dtype=np.float64) @ np.asarray(x, dtype=np.float64)


def max_rel_err(got: np.ndarray, want: np.ndarray) -> float:
    """max |got - want| / max |want| (the north-star tolerance metric)."""
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    denom = max(float(np.max(np.abs(want))), 1e-30)
    return float(np.max(np.abs(got - want)) / denom)
