"""Ternary expert weights: packer, dequantiser and ordered GEMV -- TEST INFRASTRUCTURE ONLY.

CPU restatement of the reference's ternary expert format, used only to check the HIP
kernel (tests) and never by the product:

* ``digit_lut`` -- the 256-entry base-3 digit table the reference backend builds at
  construction (triton_kernels.py:3613-3624);
* ``pack_mxfp4_to_ternary`` -- ``quantize_mxfp4_to_ternary_cpu``
  (gpu_runtime.py:494-583): per 32-element MXFP4 block, the magnitude of
  {0.5, 1, 1.5, 2, 3, 4, 6} with the least mean squared error (strictly smaller
  error replaces, so ties keep the first), digits by |v| > a/2, five digits per byte
  (powers 1, 3, 9, 27, 81), 3-bit selectors at bit 3g LSB-first, E8M0 scales kept;
* ``ternary_dequant`` -- what the reference kernel reads (triton_kernels.py:1044-1104):
  LUT digits, selector bits (crossing bytes), nibble = 0 for digit 1, else
  (m + 1) | 8 * (digit == 0), value e2m1(nibble) * 2^(e - 127);
* ``ternary_selected_gemv`` -- the HIP kernel's documented summation order in binary32
  (per-group digit*x chain minus the group's x sum, groups in order per 160-column
  chunk, chunks in order), so GPU results can be compared bit for bit.
"""

from __future__ import annotations

import numpy as np

from .ref import E2M1

MAGNITUDES = np.array([0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0])
POWERS = (1, 3, 9, 27, 81)


def digit_lut() -> np.ndarray:
    """int16 [256]: digit i of byte b in bits 2i..2i+1, each (b // 3^i) % 3."""
    lut = np.zeros(256, dtype=np.int16)
    for packed in range(256):
        value, expanded = packed, 0
        for digit in range(5):
            expanded |= (value % 3) << (2 * digit)
            value //= 3
        lut[packed] = expanded
    return lut


def ternary_geometry(cols: int) -> tuple[int, int, int]:
    """(groups, digit bytes, selector bytes) of one row (gpu_runtime.py:513-516)."""
    groups = cols // 32
    return groups, (cols + 4) // 5, (groups * 3 + 7) // 8


def pack_mxfp4_to_ternary(blocks: np.ndarray, scales: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """blocks uint8 [E, rows, G, 16], scales uint8 [E, rows, G] -> (packed uint8
    [E, rows, T + M], scales)."""
    blocks = np.asarray(blocks, dtype=np.uint8)
    experts, rows, groups = scales.shape
    cols = groups * 32
    _, tbytes, mbytes = ternary_geometry(cols)
    flat = blocks.reshape(experts * rows, groups, 16)
    nib = np.empty((experts * rows, groups, 32), dtype=np.uint8)
    nib[..., 0::2] = flat & 0x0F
    nib[..., 1::2] = flat >> 4
    v = E2M1.astype(np.float32)[nib]
    best_err = best_dig = best_mag = None
    for index, a in enumerate(MAGNITUDES.astype(np.float32)):
        dig = np.where(np.abs(v) > a / 2, np.where(v < 0, 0, 2), 1).astype(np.uint8)
        rec = np.where(dig == 1, np.float32(0), np.where(dig == 0, -a, a)).astype(np.float32)
        err = np.square(v - rec).mean(axis=2, dtype=np.float32)
        if best_err is None:
            best_err, best_dig, best_mag = err, dig, np.full(err.shape, index, dtype=np.uint8)
        else:
            take = err < best_err
            best_err = np.where(take, err, best_err)
            best_dig = np.where(take[..., None], dig, best_dig)
            best_mag = np.where(take, np.uint8(index), best_mag)
    digits = best_dig.reshape(experts * rows, cols).astype(np.int64)
    out = np.zeros((experts * rows, tbytes + mbytes), dtype=np.uint8)
    tern = np.zeros((experts * rows, tbytes), dtype=np.int64)
    for d, power in enumerate(POWERS):
        vals = digits[:, d::5]
        tern[:, : vals.shape[1]] += vals * power
    out[:, :tbytes] = tern.astype(np.uint8)
    for g in range(groups):
        bit = 3 * g
        byte, shift = bit // 8, bit & 7
        vals = best_mag[:, g].astype(np.int64)
        out[:, tbytes + byte] |= ((vals << shift) & 0xFF).astype(np.uint8)
        if shift > 5:
            out[:, tbytes + byte + 1] |= (vals >> (8 - shift)).astype(np.uint8)
    return out.reshape(experts, rows, tbytes + mbytes), np.asarray(scales, dtype=np.uint8)


def ternary_dequant(packed: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """packed uint8 [..., rows, T + M], scales uint8 [..., rows, G] -> float64 [..., rows, 32 G]."""
    p = np.asarray(packed, dtype=np.uint8).astype(np.int64)
    s = np.asarray(scales, dtype=np.int64)
    groups = s.shape[-1]
    cols = groups * 32
    _, tbytes, _ = ternary_geometry(cols)
    k = np.arange(cols)
    lut = digit_lut().astype(np.int64)
    digits = (lut[p[..., k // 5]] >> (2 * (k % 5))) & 3
    g = k // 32
    mbit = g * 3
    mbyte = tbytes + mbit // 8
    mshift = mbit % 8
    row_bytes = p.shape[-1]
    low = p[..., mbyte]
    cross = (mshift > 5) & (mbyte + 1 < row_bytes)
    high = np.where(cross, p[..., np.minimum(mbyte + 1, row_bytes - 1)], 0)
    mcode = ((low >> mshift) | (high << (8 - mshift))) & 7
    nibble = np.where(digits == 1, 0, (mcode + 1) | np.where(digits == 0, 8, 0)) & 0x0F
    return E2M1[nibble] * np.exp2(s[..., g].astype(np.float64) - 127.0)


def _digits(packed_rows: np.ndarray, cols: int) -> np.ndarray:
    k = np.arange(cols)
    b = packed_rows[:, k // 5].astype(np.int64)
    return (b // np.array(POWERS, dtype=np.int64)[k % 5]) % 3


def ternary_selected_gemv(packed: np.ndarray, scales: np.ndarray, x: np.ndarray, experts: np.ndarray) -> np.ndarray:
    """float32 [selected, rows] in the HIP kernel's order; x is [cols] or [selected, cols]
    (values as float32); ids outside [0, E) give NaN rows.  Order, all binary32:
    A_g = column-order chain of A + digit * x (exact products), B_g = column-order sum
    of x, p_g = A_g - B_g; chunk = sum over the 160-column chunk's groups in order of
    v_g * p_g with v_g = |w|_g * 2^(e_g - 127); row = sum of the chunks in order."""
    packed = np.asarray(packed, dtype=np.uint8)
    n_exp, rows, _ = packed.shape
    groups = scales.shape[-1]
    cols = groups * 32
    _, tbytes, _ = ternary_geometry(cols)
    chunks = -(-cols // 160)
    sel = len(experts)
    xs = np.asarray(x, dtype=np.float32)
    if xs.ndim == 1:
        xs = np.broadcast_to(xs, (sel, cols))
    out = np.full((sel, rows), np.nan, dtype=np.float32)
    for si, e in enumerate(experts):
        if not 0 <= int(e) < n_exp:
            continue
        pr = packed[int(e)]
        digit = _digits(pr, cols).astype(np.float32)
        mbits = np.arange(groups) * 3
        mb = tbytes + mbits // 8
        word = pr[:, mb].astype(np.int64) | (pr[:, np.minimum(mb + 1, pr.shape[1] - 1)].astype(np.int64) << 8)
        word = np.where((mb + 1 < pr.shape[1])[None, :], word, pr[:, mb].astype(np.int64))
        mcode = (word >> (mbits % 8)) & 7
        mag = np.where(mcode == 7, 0.0, MAGNITUDES[np.minimum(mcode, 6)])
        v = mag.astype(np.float32) * np.exp2(np.asarray(scales[int(e)], dtype=np.float64) - 127.0).astype(np.float32)
        xrow = xs[si]
        A = np.zeros((rows, groups), dtype=np.float32)
        B = np.zeros(groups, dtype=np.float32)
        for k in range(cols):
            A[:, k // 32] = A[:, k // 32] + digit[:, k] * xrow[k]
            B[k // 32] = B[k // 32] + xrow[k]
        p = A - B[None, :]
        row = np.zeros(rows, dtype=np.float32)
        for c in range(chunks):
            chunk = np.zeros(rows, dtype=np.float32)
            for g in range(5 * c, min(5 * c + 5, groups)):
                chunk = chunk + v[:, g] * p[:, g]
            row = row + chunk
        out[si] = row
    return out
