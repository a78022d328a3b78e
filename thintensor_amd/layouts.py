"""Packed weight layouts of the reference runtime, produced from integer codes.

These are the on-device formats the kernels read, identical to the reference's
packers so that packed pages are interchangeable:

* int4: ``uint8 [rows, cols/2]``, k = 2b in the low nibble of byte b, k = 2b + 1
  in the high nibble; stored code c = q + 8 (gpu_runtime.py:296-304, 6671-6674).
  Reinterpreted little-endian it is ``uint32 [rows, cols/8]`` with nibble j of a
  word holding k = 8w + j.
* q2 (E8M0 experts): ``uint8 [E, rows, cols/32, 8]``, element i of a 32-block at
  byte i//4, bits 2*(i%4) (gpu_runtime.py:384-395; kernel triton_kernels.py:1166-1171).
* q1 (E8M0 experts): ``uint8 [E, rows, cols/32, 4]``, element i at byte i//8, bit
  i%8 (gpu_runtime.py:474-488).
* MXFP4 (gpt-oss): blocks ``uint8 [E, rows, cols/32, 16]``, element 2j of a block
  in the low nibble of byte j (triton_kernels.py:444-459), scales ``uint8
  [E, rows, cols/32]`` E8M0 (bias 127).
* affine q2/q1 with group g (no reference packer): the same bit order as the E8M0
  formats, packed along each row, with fp16 ``[rows, cols/g, 2]`` (scale, zero).

All functions take and return numpy arrays; nothing here runs on the GPU.
"""

from __future__ import annotations

import numpy as np


def pack_int4(codes: np.ndarray) -> np.ndarray:
    """codes uint8 in [0, 15], shape [..., cols] (cols even) -> uint8 [..., cols/2]."""
    codes = np.asarray(codes, dtype=np.uint8)
    if codes.shape[-1] % 2:
        raise ValueError("int4 packing needs an even number of columns")
    if codes.size and codes.max() > 15:
        raise ValueError("int4 codes must lie in [0, 15]")
    return (codes[..., 0::2] | (codes[..., 1::2] << 4)).astype(np.uint8)


def unpack_int4(packed: np.ndarray) -> np.ndarray:
    packed = np.asarray(packed, dtype=np.uint8)
    out = np.empty(packed.shape[:-1] + (packed.shape[-1] * 2,), dtype=np.uint8)
    out[..., 0::2] = packed & 15
    out[..., 1::2] = packed >> 4
    return out


def pack_bits(codes: np.ndarray, bits: int) -> np.ndarray:
    """Pack 1- or 2-bit codes along the last axis: element i at byte i*bits//8,
    bit (i*bits) % 8 (the E8M0 and affine low-bit orders)."""
    if bits not in (1, 2):
        raise ValueError("bits must be 1 or 2")
    codes = np.asarray(codes, dtype=np.uint8)
    per_byte = 8 // bits
    if codes.shape[-1] % per_byte:
        raise ValueError(f"{bits}-bit packing needs a multiple of {per_byte} columns")
    if codes.size and codes.max() >= (1 << bits):
        raise ValueError(f"codes must fit in {bits} bits")
    c = codes.reshape(codes.shape[:-1] + (codes.shape[-1] // per_byte, per_byte)).astype(np.uint32)
    shifts = (np.arange(per_byte, dtype=np.uint32) * bits)
    return (c << shifts).sum(axis=-1).astype(np.uint8)


def unpack_bits(packed: np.ndarray, bits: int, count: int | None = None) -> np.ndarray:
    packed = np.asarray(packed, dtype=np.uint8)
    per_byte = 8 // bits
    shifts = (np.arange(per_byte, dtype=np.uint8) * bits)
    out = (packed[..., None] >> shifts) & ((1 << bits) - 1)
    out = out.reshape(packed.shape[:-1] + (packed.shape[-1] * per_byte,))
    return out if count is None else out[..., :count]


def pack_lowbit_blocks(codes: np.ndarray, bits: int) -> np.ndarray:
    """codes [E, rows, cols] -> reference expert layout [E, rows, cols/32, 32*bits/8]."""
    codes = np.asarray(codes, dtype=np.uint8)
    if codes.shape[-1] % 32:
        raise ValueError("low-bit expert columns must be a multiple of 32")
    blocks = codes.reshape(codes.shape[:-1] + (codes.shape[-1] // 32, 32))
    return pack_bits(blocks, bits)


def pack_mxfp4_blocks(codes: np.ndarray) -> np.ndarray:
    """e2m1 codes [E, rows, cols] -> blocks uint8 [E, rows, cols/32, 16]."""
    codes = np.asarray(codes, dtype=np.uint8)
    if codes.shape[-1] % 32:
        raise ValueError("MXFP4 columns must be a multiple of 32")
    blocks = codes.reshape(codes.shape[:-1] + (codes.shape[-1] // 32, 32))
    return pack_int4(blocks)


def int4_as_u32(packed: np.ndarray) -> np.ndarray:
    """Reinterpret the uint8 int4 layout as little-endian uint32 (8 codes per word)."""
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    if packed.shape[-1] % 4:
        raise ValueError("row bytes must be a multiple of 4")
    return packed.view("<u4")
