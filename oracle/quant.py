"""CPU restatement of the load-time quantizers -- TEST INFRASTRUCTURE ONLY.

Each function restates one reference quantizer (thinruntime/gpu_runtime.py, lines
cited per function) in the arithmetic of the HIP kernels in
thintensor_amd/csrc/quantize.hip, so the GPU results are compared bit for bit:

* every elementwise step is the reference's binary32 operation in the reference's
  order (numpy float32 arithmetic is IEEE binary32 with round-to-nearest-even;
  ``np.rint`` is torch.round's half-to-even);
* every sum over a group (the reference's ``.sum``/``.mean`` in binary32, whose
  order torch leaves to the CPU's vector width) is taken in binary64 in the
  kernels' fixed order -- element partials per lane in index order starting from
  +0, then a halving tree over the 64 lanes -- and rounded once to binary32, which
  agrees with the reference except where its own binary32 order decides a code
  or a candidate (a near-tie; the golden vectors in tests/golden pin the rest);
* ``ceil(log2(v))`` / ``floor(log2(v))`` of a binary32 ``v`` are taken exactly
  (from the binary exponent), where the reference's float log2 may round an input a
  few ulps above (below) a power of two onto the integer.

The reference outputs themselves are recorded by tests/golden/make_quant_vectors.py.
"""

from __future__ import annotations

import numpy as np

from .ternary import pack_mxfp4_to_ternary  # noqa: F401  (MXFP4 -> ternary packer)

F32 = np.float32
TINY = F32(1e-12)
FP8_MAX = F32(448.0)
E2M1 = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0], dtype=np.float32)


# ----------------------------------------------------------------------------- helpers
def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (bits.astype(np.uint32) << 16).view(np.float32)


def f16_to_f32(bits: np.ndarray) -> np.ndarray:
    return bits.astype(np.uint16).view(np.float16).astype(np.float32)


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """binary32 -> bfloat16 bits, round to nearest even (NaN kept quiet)."""
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(np.asarray(x, dtype=np.float32))
    return np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), r)


def lane_sum(terms: np.ndarray, present: np.ndarray | None = None) -> np.ndarray:
    """Sum over the last axis (one quantization group of G elements) in the kernels'
    order: lane l holds elements [l*G/64, (l+1)*G/64) for G >= 64 (element l for
    G < 64), adds them in binary64 from +0 in index order, then the 64 lane partials
    are folded in halves (lanes l and l + n/2).  Absent elements add nothing."""
    t = np.asarray(terms, dtype=np.float64)
    if present is not None:
        t = np.where(present, t, 0.0)
    G = t.shape[-1]
    lead = t.shape[:-1]
    if G >= 64:
        epl = G // 64
        assert G == 64 * epl
        t = t.reshape(lead + (64, epl))
        p = np.zeros(lead + (64,), dtype=np.float64)
        for k in range(epl):
            p = p + t[..., k]
    else:
        p = np.zeros(lead + (64,), dtype=np.float64)
        p[..., :G] = 0.0 + t
    n = 64
    while n > 1:
        n //= 2
        p = p[..., :n] + p[..., n:2 * n]
    return p[..., 0].astype(np.float32)


def half_sum32(terms: np.ndarray) -> np.ndarray:
    """Sum of 32 elements (one MX group) in the kernels' order: lane l holds element
    l (binary64 from +0), folded in halves over 32 lanes, rounded once."""
    t = np.asarray(terms, dtype=np.float64)
    assert t.shape[-1] == 32
    p = 0.0 + t
    n = 32
    while n > 1:
        n //= 2
        p = p[..., :n] + p[..., n:2 * n]
    return p[..., 0].astype(np.float32)


def ceil_log2(v: np.ndarray) -> np.ndarray:
    """Exact ceil(log2(v)) of positive normal binary32 values."""
    m, e = np.frexp(np.asarray(v, dtype=np.float64))   # v = m * 2^e, m in [0.5, 1)
    return np.where(m == 0.5, e - 1, e).astype(np.int32)


def floor_log2(v: np.ndarray) -> np.ndarray:
    m, e = np.frexp(np.asarray(v, dtype=np.float64))
    return (e - 1).astype(np.int32)


def exp2i(e: np.ndarray) -> np.ndarray:
    """2^e as binary32 for integer e in [-149, 127] (subnormal below -126)."""
    return np.ldexp(np.float32(1.0), np.asarray(e, dtype=np.int32)).astype(np.float32)


def _groups(x: np.ndarray, G: int) -> tuple[np.ndarray, np.ndarray]:
    """[rows, cols] -> [rows, groups, G] padded with zeros, and the presence mask."""
    rows, cols = x.shape
    groups = -(-cols // G)
    pad = groups * G - cols
    xp = np.concatenate([x, np.zeros((rows, pad), np.float32)], axis=1) if pad else x
    present = (np.arange(groups * G) < cols).reshape(groups, G)
    return xp.reshape(rows, groups, G).astype(np.float32), np.broadcast_to(present, (rows, groups, G))


def _pack_nibbles(codes: np.ndarray) -> np.ndarray:
    c = codes.astype(np.uint8)
    return (c[:, 0::2] | (c[:, 1::2] << 4)).astype(np.uint8)


# ------------------------------------------------------------------------------- INT4
def int4_lsq(x: np.ndarray, group_size: int) -> tuple[np.ndarray, np.ndarray]:
    """quantize_to_int4_cpu, symmetric (gpu_runtime.py:237-253 and the ragged branch
    :254-272): scale = amax/7, codes round(x/scale) in [-8, 7], one least-squares
    refinement scale = |sum(x q) / max(sum(q^2), 1)|, codes again; fp16 scales."""
    rows, cols = x.shape
    g, present = _groups(x, group_size)
    amax = np.max(np.where(present, np.abs(g), 0), axis=2).astype(np.float32)
    s0 = (np.maximum(amax, TINY) / F32(7.0)).astype(np.float32)
    q = np.clip(np.rint(g / s0[..., None]), -8, 7).astype(np.float32)
    num = lane_sum((g * q).astype(np.float32), present)
    den = np.maximum(lane_sum((q * q).astype(np.float32), present), F32(1.0))
    s = np.maximum(np.abs((num / den).astype(np.float32)), TINY).astype(np.float32)
    codes = (np.clip(np.rint(g / s[..., None]), -8, 7) + 8).astype(np.uint8)
    codes = codes.reshape(rows, -1)[:, :cols]
    return _pack_nibbles(codes), s.astype(np.float16)


def _affine_fit(g, q, w, present):
    """One regression of the affine line on the assigned codes (gpu_runtime.py:165-
    199): means (weighted by w when given), slope, clamped, intercept."""
    G = g.shape[-1]
    if w is None:
        q_mean = (lane_sum(q, present) / F32(G)).astype(np.float32)
        x_mean = (lane_sum(g, present) / F32(G)).astype(np.float32)
        rw = None
    else:
        wsum = lane_sum(np.broadcast_to(w, g.shape), present)
        q_mean = (lane_sum((q * w).astype(np.float32), present) / wsum).astype(np.float32)
        x_mean = (lane_sum((g * w).astype(np.float32), present) / wsum).astype(np.float32)
        rw = w
    qc = (q - q_mean[..., None]).astype(np.float32)
    t = ((g - x_mean[..., None]).astype(np.float32) * qc).astype(np.float32)
    d = (qc * qc).astype(np.float32)
    if rw is not None:
        t = (t * rw).astype(np.float32)
        d = (d * rw).astype(np.float32)
    num = lane_sum(t, present)
    den = np.maximum(lane_sum(d, present), TINY)
    s = np.maximum((num / den).astype(np.float32), TINY).astype(np.float32)
    mn = (x_mean - (s * q_mean).astype(np.float32)).astype(np.float32)
    return s, mn


def int4_lsq_affine(x: np.ndarray, group_size: int, input_rms: np.ndarray | None = None,
                    gptq_factors: np.ndarray | None = None):
    """quantize_to_int4_cpu with THINTENSOR_AFFINE_INT4=1 (gpu_runtime.py:155-236,
    cols divisible by the group): min/max line, two refits each followed by a
    requantization, then a final refit of (scale, minimum); codes in [0, 15];
    optional column importance max(rms^2, 1e-8).  With ``gptq_factors`` (binary32
    [groups, 32, 32] upper factors U, groups of 32) two GPTQ passes follow
    (:217-262): column c of each group is rounded on the current line from its
    adjusted value, (value - code * scale - minimum) / U[c, c] is taken out of columns
    c.. along U[c, c..] (product, then difference), and the line is refitted after the
    first pass.  fp16 [scale, minimum] pairs."""
    rows, cols = x.shape
    assert cols % group_size == 0
    g, present = _groups(x, group_size)
    w = None
    if input_rms is not None:
        imp = np.maximum((input_rms.astype(np.float32) * input_rms.astype(np.float32)).astype(np.float32), F32(1e-8))
        w = imp.reshape(1, cols // group_size, group_size).astype(np.float32)
    mn = np.min(g, axis=2)
    mx = np.max(g, axis=2)
    s = (np.maximum((mx - mn).astype(np.float32), TINY) / F32(15.0)).astype(np.float32)
    q = np.clip(np.rint(((g - mn[..., None]).astype(np.float32) / s[..., None]).astype(np.float32)), 0, 15).astype(np.float32)
    for _ in range(2):
        s, mn = _affine_fit(g, q, w, present)
        q = np.clip(np.rint(((g - mn[..., None]).astype(np.float32) / s[..., None]).astype(np.float32)), 0, 15).astype(np.float32)
    s, mn = _affine_fit(g, q, w, present)
    if gptq_factors is not None:
        assert group_size == 32
        U = np.asarray(gptq_factors, dtype=np.float32)
        for gptq_pass in range(2):
            adj = g.copy()
            for c in range(group_size):
                cur = adj[:, :, c].copy()
                code = np.clip(np.rint(((cur - mn).astype(np.float32) / s).astype(np.float32)), 0, 15).astype(np.float32)
                q[:, :, c] = code
                qv = ((code * s).astype(np.float32) + mn).astype(np.float32)
                err = ((cur - qv).astype(np.float32) / U[None, :, c, c]).astype(np.float32)
                adj[:, :, c:] = (adj[:, :, c:] - (err[..., None] * U[None, :, c, c:]).astype(np.float32)).astype(np.float32)
            if gptq_pass == 0:
                s, mn = _affine_fit(g, q, w, present)
    codes = q.astype(np.uint8).reshape(rows, cols)
    scales = np.stack([s, mn], axis=-1).astype(np.float16)
    return _pack_nibbles(codes), scales


def int4_rows(x: np.ndarray, group_size: int, affine: bool = False):
    """ThinGpuCausalLMRuntime._quantize_int4_rows (gpu_runtime.py:6609-6700): per group
    scale = amax/7 with codes round(x/scale) in [-7, 7] (+8), or the min/max affine
    line with codes in [0, 15]; fp32 scales ([scale, minimum] when affine)."""
    rows, cols = x.shape
    g, present = _groups(x, group_size)
    if affine:
        mn = np.min(np.where(present, g, np.inf), axis=2).astype(np.float32)
        mx = np.max(np.where(present, g, -np.inf), axis=2).astype(np.float32)
        s = (np.maximum((mx - mn).astype(np.float32), TINY) / F32(15.0)).astype(np.float32)
        q = np.clip(np.rint(((g - mn[..., None]).astype(np.float32) / s[..., None]).astype(np.float32)), 0, 15)
        codes = q.astype(np.uint8).reshape(rows, -1)[:, :cols]
        return _pack_nibbles(codes), np.stack([s, mn], axis=-1).astype(np.float32)
    amax = np.max(np.where(present, np.abs(g), 0), axis=2).astype(np.float32)
    s = (np.maximum(amax, TINY) / F32(7.0)).astype(np.float32)
    q = np.clip(np.rint((g / s[..., None]).astype(np.float32)), -7, 7) + 8
    codes = q.astype(np.uint8).reshape(rows, -1)[:, :cols]
    return _pack_nibbles(codes), s


# -------------------------------------------------------------------------------- FP8
def f32_to_e4m3(v: np.ndarray) -> np.ndarray:
    """binary32 -> float8_e4m3fn bits, round to nearest even on the e4m3 grid
    (quantum 2^(max(e, -6) - 3) for |v| in [2^e, 2^(e+1))); magnitudes that round
    past 448, and NaN/inf, give the NaN pattern 0x7f (torch's conversion)."""
    with np.errstate(invalid="ignore"):
        return _f32_to_e4m3(np.asarray(v, dtype=np.float32))


def _f32_to_e4m3(v: np.ndarray) -> np.ndarray:
    sign = (np.signbit(v).astype(np.uint8) << 7).astype(np.uint8)
    a = np.abs(v).astype(np.float64)
    finite = np.isfinite(a)
    a0 = np.where(finite & (a > 0), a, 1.0)
    _, fe = np.frexp(a0)
    step = np.ldexp(1.0, np.maximum(fe - 1, -6) - 3)
    r = np.where(finite, np.rint(a0 / step) * step, np.inf)
    r = np.where(a == 0, 0.0, r)
    _, fr = np.frexp(np.where(r > 0, r, 1.0))
    ee = fr - 1
    mant = np.rint((np.where(r > 0, r, 1.0) / np.ldexp(1.0, ee) - 1.0) * 8).astype(np.int64)
    code = np.where(r >= 2.0 ** -6, ((ee + 7).astype(np.int64) << 3) | mant, np.rint(r / 2.0 ** -9).astype(np.int64))
    code = np.where(r > 448.0, 0x7F, code)
    return (code.astype(np.uint8) | sign).astype(np.uint8)


def fp8_rows(x: np.ndarray, block: int = 0, via_bf16: bool = False, src_bf16_bits: np.ndarray | None = None):
    """_quantize_fp8_rows (gpu_runtime.py:6551-6607) and, with via_bf16,
    quantize_to_fp8_via_gpu (:40-88; the source is taken as bfloat16 and x/scale is
    rounded to bfloat16 before e4m3).  scale = max(amax, 1e-12)/448 per row or per
    block of columns (fp32); e4m3(x / scale)."""
    rows, cols = x.shape
    nb = -(-cols // block) if block > 0 else 1
    bs = block if block > 0 else cols
    scales = np.empty((rows, nb), dtype=np.float32)
    q = np.empty((rows, cols), dtype=np.uint8)
    for b in range(nb):
        c0, c1 = b * bs, min(cols, (b + 1) * bs)
        v = x[:, c0:c1].astype(np.float32)
        s = (np.maximum(np.max(np.abs(v), axis=1).astype(np.float32), TINY) / FP8_MAX).astype(np.float32)
        y = (v / s[:, None]).astype(np.float32)
        if via_bf16:
            y = bf16_to_f32(f32_to_bf16(y))
        q[:, c0:c1] = f32_to_e4m3(y)
        scales[:, b] = s
    return q, (scales if block > 0 else scales[:, 0])


# ------------------------------------------------------------------------------- MXFP4
def fwht(x: np.ndarray, T: int, signs: np.ndarray | None = None) -> np.ndarray:
    """Blockwise Walsh-Hadamard transform as the reference's loop (gpu_runtime.py:
    6745-6762): optional sign flip, butterflies (l + r, l - r) at strides 1, 2, 4,
    ..., then times fp32(T^-0.5)."""
    rows, cols = x.shape
    t = x.astype(np.float32)
    if signs is not None:
        t = (t * signs.astype(np.float32)[None, :]).astype(np.float32)
    t = t.reshape(-1, T)
    s = 1
    while s < T:
        p = t.reshape(-1, T // (2 * s), 2, s)
        l, r = p[:, :, 0, :], p[:, :, 1, :]
        t = np.stack(((l + r).astype(np.float32), (l - r).astype(np.float32)), axis=2).reshape(-1, T)
        s *= 2
    return (t * F32(T ** -0.5)).astype(np.float32).reshape(rows, cols)


def mxfp4_rows(x: np.ndarray, hadamard_size: int = 0, signs: np.ndarray | None = None,
               binary_residual: bool = False):
    """_quantize_mxfp4_rows (gpu_runtime.py:6702-6812): per 32-group exponent
    e0 = ceil(log2(max(amax, 2^-126) / 6)), candidates e0 - 1 and e0 (clamped to
    [-127, 127]); codes by the E2M1 thresholds, the candidate with the smaller sum of
    squared residuals (the binary-residual variant first removes +-2^round(log2(mean
    |r|)))); ties keep e0 - 1.  Packed nibbles (low first) and E8M0 scales."""
    rows, cols = x.shape
    assert cols % 32 == 0
    b = fwht(x, hadamard_size, signs) if hadamard_size else x.astype(np.float32)
    b = b.reshape(rows, cols // 32, 32)
    amax = np.max(np.abs(b), axis=2).astype(np.float32)
    base = np.clip(ceil_log2((np.maximum(amax, F32(2.0 ** -126)) / F32(6.0)).astype(np.float32)), -127, 127)
    best_err = best_e = best_c = None
    thr = np.array([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0], dtype=np.float32)
    for bias in (-1, 0):
        e = np.clip(base + bias, -127, 127)
        f = exp2i(e)
        nrm = (b / f[..., None]).astype(np.float32)
        mag = np.abs(nrm)
        code = np.zeros(nrm.shape, dtype=np.uint8)
        for t in thr:
            code = code + (mag >= t).astype(np.uint8)
        code = code | (np.signbit(nrm).astype(np.uint8) << 3)
        rec = (E2M1[code & 7] * np.where((code & 8) != 0, F32(-1.0), F32(1.0))).astype(np.float32)
        rec = (rec * f[..., None]).astype(np.float32)
        res = (b - rec).astype(np.float32)
        if binary_residual:
            mean = (half_sum32(np.abs(res)) / F32(32.0)).astype(np.float32)
            mean = np.maximum(mean, F32(2.0 ** -126))
            re = np.clip(np.rint(np.log2(mean.astype(np.float64))), -127, 127).astype(np.int32)
            rs = exp2i(re)
            res = (res - np.where(res >= 0, rs[..., None], -rs[..., None])).astype(np.float32)
        err = half_sum32((res * res).astype(np.float32))
        if best_err is None:
            best_err, best_e, best_c = err, e, code
        else:
            take = err < best_err
            best_err = np.where(take, err, best_err)
            best_e = np.where(take, e, best_e)
            best_c = np.where(take[..., None], code, best_c)
    codes = best_c.reshape(rows, cols)
    return _pack_nibbles(codes), (best_e + 127).astype(np.uint8)


# ------------------------------------------------------------------ MXFP4 -> Q2 / Q1
def _mx_nibbles(blocks: np.ndarray) -> np.ndarray:
    n = np.empty(blocks.shape[:-1] + (32,), dtype=np.uint8)
    n[..., 0::2] = blocks & 0x0F
    n[..., 1::2] = blocks >> 4
    return n


def mxfp4_to_lowbit(blocks: np.ndarray, scales: np.ndarray, bits: int):
    """quantize_mxfp4_to_lowbit_cpu (gpu_runtime.py:306-395): per MXFP4 group, the
    exponent offset d in -2..3 whose Q2 {+-0.5, +-1.5} * 2^d (Q1 +-2^d) codes give the
    smallest mean squared error against the E2M1 values (ties keep the earlier d);
    scale byte clamp(s - 127 + d, -127, 127) + 127.  All errors are sums of
    multiples of 1/4, exact in binary32 in any order."""
    nib = _mx_nibbles(blocks)
    vals = np.concatenate([E2M1, -E2M1])[nib]
    neg = (nib & 8) != 0
    q2 = np.array([-1.5, -0.5, 0.5, 1.5], dtype=np.float32)
    best_err = best_c = best_d = None
    for d in (-2, -1, 0, 1, 2, 3):
        f = F32(2.0 ** d)
        if bits == 2:
            outer = np.abs(vals) >= f
            codes = np.where(neg, np.where(outer, 0, 1), np.where(outer, 3, 2)).astype(np.uint8)
            rec = (q2[codes] * f).astype(np.float32)
        else:
            codes = (~neg).astype(np.uint8)
            rec = np.where(neg, -f, f).astype(np.float32)
        err = (half_sum32(((vals - rec) ** 2).astype(np.float32)) / F32(32.0)).astype(np.float32)
        if best_err is None:
            best_err, best_c, best_d = err, codes, np.full(err.shape, d, np.int16)
        else:
            take = err < best_err
            best_err = np.where(take, err, best_err)
            best_c = np.where(take[..., None], codes, best_c)
            best_d = np.where(take, d, best_d)
    adj = (np.clip(scales.astype(np.int16) - 127 + best_d, -127, 127) + 127).astype(np.uint8)
    if bits == 2:
        packed = (best_c[..., 0::4] | (best_c[..., 1::4] << 2) | (best_c[..., 2::4] << 4) | (best_c[..., 3::4] << 6))
    else:
        packed = best_c[..., 0::8].copy()
        for bit in range(1, 8):
            packed = packed | (best_c[..., bit::8] << bit)
    return packed.astype(np.uint8), adj


def dense_to_lowbit(x: np.ndarray, bits: int):
    """quantize_dense_to_mxfp_lowbit_cpu (gpu_runtime.py:398-491): per 32-group base
    exponent floor(log2(max(amax, 2^-126) / L)) (L = 1.5 for Q2, 1 for Q1), offsets
    -2..2 (clamped to [-127, 127]), the candidate with the smallest mean squared
    error (ties keep the earlier offset); scale byte clamp(e + 127, 0, 254)."""
    rows, cols = x.shape
    v = x.astype(np.float32).reshape(rows, cols // 32, 32)
    amax = np.maximum(np.max(np.abs(v), axis=2).astype(np.float32), F32(2.0 ** -126))
    L = F32(1.5) if bits == 2 else F32(1.0)
    base = floor_log2((amax / L).astype(np.float32))
    best_err = best_c = best_e = None
    for off in (-2, -1, 0, 1, 2):
        e = np.clip(base + off, -127, 127)
        f = exp2i(e)[..., None]
        nrm = (v / f).astype(np.float32)
        if bits == 2:
            outer = np.abs(nrm) >= 1.0
            neg = nrm < 0
            codes = np.where(neg, np.where(outer, 0, 1), np.where(outer, 3, 2)).astype(np.uint8)
            mag = np.where(outer, F32(1.5), F32(0.5))
            rec = (np.copysign(mag, nrm).astype(np.float32) * f).astype(np.float32)
        else:
            codes = (nrm >= 0).astype(np.uint8)
            rec = np.where(codes.astype(bool), f, -f).astype(np.float32)
        d = (v - rec).astype(np.float32)
        err = (half_sum32((d * d).astype(np.float32)) / F32(32.0)).astype(np.float32)
        if best_err is None:
            best_err, best_c, best_e = err, codes, e
        else:
            take = err < best_err
            best_err = np.where(take, err, best_err)
            best_c = np.where(take[..., None], codes, best_c)
            best_e = np.where(take, e, best_e)
    sc = np.clip(best_e + 127, 0, 254).astype(np.uint8)
    if bits == 2:
        packed = (best_c[..., 0::4] | (best_c[..., 1::4] << 2) | (best_c[..., 2::4] << 4) | (best_c[..., 3::4] << 6))
    else:
        packed = np.zeros(best_c.shape[:-1] + (4,), dtype=np.uint8)
        for bit in range(8):
            packed = packed | (best_c[..., bit::8] << bit)
    return packed.astype(np.uint8), sc
