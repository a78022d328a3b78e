"""CPU oracle for the decode hot path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import this package, and only as the checker.  The product
(``thintensor_amd``) never imports it.

Two layers:

* ``emul``: ctypes binding of ``tt_oracle.c``, a binary32 restatement of each
  operator in the kernels' documented reduction order (bit-exact target);
* ``ref``: numpy float64 closed forms that restate the reference's dequantise-
  then-matmul semantics (tolerance target), see ``oracle/ref.py``.
"""

from __future__ import annotations

import ctypes
from functools import lru_cache

import numpy as np

from . import build as _build
from . import ref  # noqa: F401  (re-export)

F16, BF16, F32 = 0, 1, 2
FMT = dict(int4_sym=0, int4_aff=1, fp8=2, f16w=3, bf16w=4, mxfp4=5, q2e8=6, q1e8=7, q2aff=8, q1aff=9)
SMODE = dict(none=0, row=1, group=2, group_aff=3, block_e8=4)

_P = ctypes.c_void_p
_I = ctypes.c_int
_L = ctypes.c_int64


@lru_cache(maxsize=1)
def lib() -> ctypes.CDLL:
    path = _build.ensure_built()
    L = ctypes.CDLL(str(path))
    L.tto_gemv.argtypes = [_I, _I, _P, _L, _P, _I, _L, _L, _L, _I, _P, _I, _P, _I, _L, _I, _I, _I]
    L.tto_gemv.restype = _I
    L.tto_f32_to_f16.argtypes = [ctypes.c_float]
    L.tto_f32_to_f16.restype = ctypes.c_uint16
    L.tto_exp_f32.argtypes = [ctypes.c_float]
    L.tto_exp_f32.restype = ctypes.c_float
    _register_extra(L)
    return L


def _register_extra(L: ctypes.CDLL) -> None:
    """Signatures of the non-GEMV operators."""
    for name, argtypes in EXTRA_SIGNATURES.items():
        fn = getattr(L, name)
        fn.argtypes = argtypes
        fn.restype = _I
    L.tto_argmax.argtypes = [_P, _I, _L]
    L.tto_argmax.restype = _L


_F = ctypes.c_float

EXTRA_SIGNATURES: dict[str, list] = {
    "tto_rms_norm": [_P, _I, _P, _I, _P, _I, _I, ctypes.c_float, ctypes.c_float],
    "tto_add_rms_norm": [_P, _P, _P, _I, _P, _I, _P, _I, _I, ctypes.c_float],
    "tto_silu_mul": [_P, _P, _P, _I, _I],
    "tto_interleaved_swiglu": [_P, _P, _I, _I, _I, ctypes.c_float, ctypes.c_float],
    "tto_weighted_expert_sum": [_P, _I, _P, _I, _P, _I, _I],
    "tto_rope": [_P, _P, _I, _P, _P, _I, _I, _I],
    "tto_attention": [_P, _P, _P, _I, _L, _L, _L, _L, _P, _I, _I, _I, _I, _I, _P],
    "tto_router": [_P, _I, _L, _P, _I, _I, _P, _I, _I, _I, _I, _P, _P, _I],
    "tto_topk": [_P, _I, _I, _I, _I, _P, _P, _I],
    "tto_swiglu": [_I, _I, _P, _L, _L, _P, _L, _L, _P, _I, _L, _P, _I, _P, _I, _L, ctypes.c_float, ctypes.c_float,
                   _P, _I, _L, _I, _I, _I],
    "tto_weighted_down": [_I, _I, _P, _L, _L, _P, _L, _L, _P, _I, _L, _P, _P, _I, _I, _P, _I, _L, _P, _I, _I, _I,
                          _I],
}


def _ptr(a: np.ndarray | None) -> int | None:
    return None if a is None else a.ctypes.data


def dtype_code(a: np.ndarray) -> int:
    if a.dtype == np.float16:
        return F16
    if a.dtype == np.float32:
        return F32
    if a.dtype == np.uint16:  # raw bfloat16 bits
        return BF16
    raise TypeError(f"unsupported oracle dtype {a.dtype}")


def out_array(rows: int, odtype: int) -> np.ndarray:
    if odtype == F16:
        return np.empty(rows, dtype=np.float16)
    if odtype == BF16:
        return np.empty(rows, dtype=np.uint16)
    return np.empty(rows, dtype=np.float32)


def gemv(fmt: str, smode: str, w: np.ndarray, scales: np.ndarray | None, x: np.ndarray, *, cols: int, lpr: int,
         L: int = 1, s_row: int = 0, s_grp: int = 0, s_pair: int = 0, aff_zero: int = 0,
         odtype: int = F16, sdtype: int | None = None) -> np.ndarray:
    """Bit-exact restatement of one GEMV launch.  ``w`` is uint8 [rows, row_bytes]."""
    w = np.ascontiguousarray(w)
    wb = w.view(np.uint8).reshape(w.shape[0], -1)
    x = np.ascontiguousarray(x)
    rows = wb.shape[0]
    out = out_array(rows, odtype)
    if scales is not None:
        scales = np.ascontiguousarray(scales)
        if sdtype is None:
            sdtype = F32 if scales.dtype == np.float32 else (F16 if scales.dtype == np.float16 else F32)
    else:
        sdtype = F32
    rc = lib().tto_gemv(FMT[fmt], SMODE[smode], _ptr(wb), wb.strides[0], _ptr(scales), sdtype, s_row, s_grp, s_pair,
                        aff_zero, _ptr(x), dtype_code(x), _ptr(out), odtype, rows, cols, L, lpr)
    if rc != 0:
        raise ValueError(f"oracle gemv rejected the configuration ({rc})")
    return out


def f32_to_f16_bits(v: float) -> int:
    return int(lib().tto_f32_to_f16(v))


def exp_f32(v: float) -> float:
    return float(lib().tto_exp_f32(v))
