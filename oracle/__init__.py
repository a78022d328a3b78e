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
FMT = dict(int4_sym=0, int4_aff=1, fp8=2, f16w=3, bf16w=4, mxfp4=5, q2e8=6, q1e8=7, q2aff=8, q1aff=9, int8=10)
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
    "tto_head_rms_norm": [_P, _I, _P, _I, _P, _I, _I, ctypes.c_float],
    "tto_qk_head_rope": [_P, _P, _I, _P, _P, _I, _P, _P, _I, _I, _I, ctypes.c_float],
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


# ---------------------------------------------------------------- operator wrappers
# Convenience wrappers over the binary32 restatement (fp16 activations unless noted);
# each returns fresh numpy arrays.

def _c(a):
    return np.ascontiguousarray(a)


def rms_norm(x, w, eps: float, offset: float = 0.0) -> np.ndarray:
    x, w = _c(x), _c(w)
    out = np.empty(x.shape[0], dtype=np.float16)
    lib().tto_rms_norm(_ptr(x), dtype_code(x), _ptr(w), dtype_code(w), _ptr(out), F16, x.shape[0], eps, offset)
    return out


def add_rms_norm(left, right, w, eps: float):
    left, right, w = _c(left), _c(right), _c(w)
    n = left.shape[0]
    res = np.empty(n, dtype=left.dtype)
    out = np.empty(n, dtype=np.float16)
    lib().tto_add_rms_norm(_ptr(left), _ptr(right), _ptr(res), dtype_code(left), _ptr(w), dtype_code(w), _ptr(out),
                           F16, n, eps)
    return res, out


def silu_mul(gate, up) -> np.ndarray:
    gate, up = _c(gate), _c(up)
    out = np.empty_like(gate)
    lib().tto_silu_mul(_ptr(gate), _ptr(up), _ptr(out), dtype_code(gate), gate.shape[0])
    return out


def interleaved_swiglu(gate_up, alpha: float, limit: float) -> np.ndarray:
    gu = _c(gate_up)
    rows, n2 = gu.reshape(-1, gu.shape[-1]).shape
    out = np.empty((rows, n2 // 2), dtype=gu.dtype)
    lib().tto_interleaved_swiglu(_ptr(gu), _ptr(out), dtype_code(gu), rows, n2 // 2, alpha, limit)
    return out


def weighted_expert_sum(experts, scores) -> np.ndarray:
    ex, sc = _c(experts), _c(scores)
    out = np.empty(ex.shape[1], dtype=ex.dtype)
    lib().tto_weighted_expert_sum(_ptr(ex), dtype_code(ex), _ptr(sc), dtype_code(sc), _ptr(out), ex.shape[1],
                                  ex.shape[0])
    return out


def rope(q, k, cos_row, sin_row, heads: int, kv_heads: int, head_dim: int):
    q, k = _c(q).copy(), _c(k).copy()
    c, s = _c(cos_row), _c(sin_row)
    lib().tto_rope(_ptr(q), _ptr(k), dtype_code(q), _ptr(c), _ptr(s), heads, kv_heads, head_dim)
    return q, k


def attention(q, keys, values, tokens: int, heads: int, kv_heads: int, head_dim: int, sinks=None) -> np.ndarray:
    """keys/values [kv_heads, capacity, head_dim] (contiguous); q [heads * head_dim]."""
    q, keys, values = _c(q), _c(keys), _c(values)
    cap = keys.shape[1]
    sk = None if sinks is None else _c(sinks)
    out = np.empty(heads * head_dim, dtype=q.dtype)
    lib().tto_attention(_ptr(q), _ptr(keys), _ptr(values), dtype_code(q), cap * head_dim, head_dim, cap * head_dim,
                        head_dim, _ptr(sk), F16 if sk is None else dtype_code(sk), tokens, heads, kv_heads, head_dim,
                        _ptr(out))
    return out


def router(weight, hidden, bias, k: int, renormalize: bool):
    w, x = _c(weight), _c(hidden)
    b = None if bias is None else _c(bias)
    idx = np.empty(k, dtype=np.int32)
    sc = np.empty(k, dtype=np.float16)
    lib().tto_router(_ptr(w), dtype_code(w), w.shape[1], _ptr(x), dtype_code(x), x.shape[0], _ptr(b),
                     F16 if b is None else dtype_code(b), w.shape[0], k, int(renormalize), _ptr(idx), _ptr(sc), F16)
    return idx, sc


def topk(logits, k: int, renormalize: bool):
    lg = _c(logits)
    idx = np.empty(k, dtype=np.int32)
    sc = np.empty(k, dtype=np.float16)
    lib().tto_topk(_ptr(lg), dtype_code(lg), lg.shape[0], k, int(renormalize), _ptr(idx), _ptr(sc), F16)
    return idx, sc


def expert_swiglu(fmt: str, packed, scales, x, experts, bias, alpha: float, limit: float, *, lpr: int,
                  x_per_slot: bool = False) -> np.ndarray:
    """Fused selected-expert gate/up GEMV + SwiGLU.  packed [E, 2I, K*b/8 ...], scales
    E8M0 [E, 2I, K/32]; q2/q1 round through bf16, MXFP4 through the activation dtype."""
    pw, sw, x, ex = _c(packed), _c(scales), _c(x), _c(np.asarray(experts, dtype=np.int32))
    rows2 = pw.shape[1]
    cols = sw.shape[2] * 32
    inter = rows2 // 2
    top_k = ex.shape[0]
    rt = F16 if fmt == "mxfp4" else BF16
    b = None if bias is None else _c(bias)
    out = np.empty((top_k, inter), dtype=np.float16)
    rc = lib().tto_swiglu(FMT[fmt], rt, _ptr(pw), pw.strides[0], pw.strides[1], _ptr(sw), sw.strides[0],
                          sw.strides[1], _ptr(x), dtype_code(x), cols if x_per_slot else 0, _ptr(ex), top_k, _ptr(b),
                          F16 if b is None else dtype_code(b), rows2, alpha, limit, _ptr(out), F16, inter, inter, cols,
                          lpr)
    if rc != 0:
        raise ValueError("oracle swiglu rejected the configuration")
    return out


def weighted_down(fmt: str, packed, scales, x, experts, scores, bias, *, lpr: int) -> np.ndarray:
    """Fused selected-expert down GEMV + router-weighted sum in slot order."""
    pw, sw, x, ex, sc = _c(packed), _c(scales), _c(x), _c(np.asarray(experts, dtype=np.int32)), _c(scores)
    rows = pw.shape[1]
    cols = sw.shape[2] * 32
    rt = F16 if fmt == "mxfp4" else BF16
    b = None if bias is None else _c(bias)
    out = np.empty(rows, dtype=np.float16)
    rc = lib().tto_weighted_down(FMT[fmt], rt, _ptr(pw), pw.strides[0], pw.strides[1], _ptr(sw), sw.strides[0],
                                 sw.strides[1], _ptr(x), dtype_code(x), cols, _ptr(ex), _ptr(sc), dtype_code(sc),
                                 ex.shape[0], _ptr(b), F16 if b is None else dtype_code(b), rows, _ptr(out), F16,
                                 rows, cols, lpr)
    if rc != 0:
        raise ValueError("oracle weighted_down rejected the configuration")
    return out


def head_rms_norm(x, w, heads: int, head_dim: int, eps: float) -> np.ndarray:
    x, w = _c(x), _c(w)
    out = np.empty_like(x)
    lib().tto_head_rms_norm(_ptr(x), dtype_code(x), _ptr(w), dtype_code(w), _ptr(out), heads, head_dim, eps)
    return out


def qk_head_rmsnorm_rope(q, k, q_weight, k_weight, cos_row, sin_row, heads: int, kv_heads: int, head_dim: int,
                         eps: float):
    q, k = _c(q).copy(), _c(k).copy()
    qw, kw = _c(q_weight), _c(k_weight)
    c, s = _c(cos_row), _c(sin_row)
    lib().tto_qk_head_rope(_ptr(q), _ptr(k), dtype_code(q), _ptr(qw), _ptr(kw), dtype_code(qw), _ptr(c), _ptr(s),
                           heads, kv_heads, head_dim, eps)
    return q, k


def split_k_gemv(fmt: str, w: np.ndarray, x: np.ndarray, split_k: int, scales=None, odtype: int = F16) -> np.ndarray:
    """Split-K GEMV restated: slices of q = ceil(K/32/split_k) whole chunks (last one
    shorter or absent), each the single-matrix binary32 row sum of its width, added in
    slice order from +0, times the per-row scale, rounded once.  ``w`` is uint8
    [rows, row_bytes] of dense fp16/bf16, fp8 or int8 weights."""
    from .decode_ref import lanes

    esz = 1 if fmt in ("fp8", "int8") else 2
    wb = np.ascontiguousarray(w).view(np.uint8).reshape(w.shape[0], -1)
    cols = x.shape[0]
    nchunks = cols // 32
    q = -(-nchunks // split_k)
    acc = np.zeros(wb.shape[0], dtype=np.float32)
    for c0 in range(0, nchunks, q):
        c1 = min(nchunks, c0 + q)
        width = (c1 - c0) * 32
        part = gemv(fmt, "none", wb[:, c0 * 32 * esz:c1 * 32 * esz], None, np.ascontiguousarray(x[c0 * 32:c1 * 32]),
                    cols=width, lpr=lanes(width), odtype=F32)
        acc = (acc + part).astype(np.float32)
    if scales is not None:
        acc = (acc * np.asarray(scales, dtype=np.float32)).astype(np.float32)
    if odtype == F16:
        return acc.astype(np.float16)
    if odtype == BF16:
        u = acc.view(np.uint32).astype(np.uint64)
        return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return acc
