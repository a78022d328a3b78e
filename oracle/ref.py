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
    """float64 W x, converting W in row blocks so a large matrix is never copied whole."""
    x64 = np.asarray(x, dtype=np.float64)
    w = np.asarray(w)
    if w.ndim == 2 and w.size > (1 << 24):
        step = max(1, (1 << 24) // w.shape[1])
        return np.concatenate([w[i:i + step].astype(np.float64) @ x64 for i in range(0, w.shape[0], step)])
    return np.asarray(w, dtype=np.float64) @ x64


def max_rel_err(got: np.ndarray, want: np.ndarray) -> float:
    """max |got - want| / max |want| (the north-star tolerance metric)."""
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    denom = max(float(np.max(np.abs(want))), 1e-30)
    return float(np.max(np.abs(got - want)) / denom)


# ---------------------------------------------------------------- decode-step operators
#
# Float64 statements of the reference's elementwise, norm, RoPE, attention and router
# semantics.  They are written as plain mathematics (vectorised numpy, a stable sort,
# complex multiplication, a whole-vector softmax), not in the kernels' reduction order,
# so they pin the binary32 restatement in tt_oracle.c rather than repeat it.  Rounding
# points that the reference fixes (bf16 residuals, bf16 router logits, bf16 expert
# dot products) are applied with an exact float64 round-to-nearest-even below.


def f64(a) -> np.ndarray:
    a = np.asarray(a)
    if a.dtype == np.uint16:  # raw bfloat16 bits
        return (a.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    return a.astype(np.float64)


def round_bits64(v, bits: int) -> np.ndarray:
    """Round float64 values to `bits` significant bits, ties to even (no subnormals:
    the values here lie far inside the binary32 exponent range)."""
    v = np.asarray(v, dtype=np.float64)
    m, e = np.frexp(v)
    return np.ldexp(np.rint(np.ldexp(m, bits)), e - bits)


def bf16_round64(v) -> np.ndarray:
    """float64 -> nearest bfloat16 value (8 significant bits), as float64."""
    return round_bits64(v, 8)


def f16_round64(v) -> np.ndarray:
    """float64 -> nearest IEEE binary16 value (numpy's correctly rounded conversion)."""
    return np.asarray(v, dtype=np.float64).astype(np.float16).astype(np.float64)


def rms_norm64(x, w, eps: float, offset: float = 0.0) -> np.ndarray:
    """_rms_norm_kernel (triton_kernels.py:2562-2577): x * rsqrt(mean(x^2) + eps) * (w + offset)."""
    x = f64(x)
    return x / np.sqrt(np.mean(x * x) + eps) * (f64(w) + offset)


def add_rms_norm64(left, right, w, eps: float):
    """_add_rms_norm_kernel (triton_kernels.py:2581-2614): the residual left + right is
    rounded through bfloat16 and stored; the RMS is taken over the rounded residual.
    Returns (residual, normed)."""
    r = bf16_round64(f64(left) + f64(right))
    return r, r / np.sqrt(np.mean(r * r) + eps) * f64(w)


def silu_mul64(gate, up) -> np.ndarray:
    """_silu_mul_kernel (triton_kernels.py:2761-2774): gate / (1 + e^-gate) * up."""
    g = f64(gate)
    return g / (1.0 + np.exp(-g)) * f64(up)


def gptoss_swiglu64(gate, up, alpha: float, limit: float) -> np.ndarray:
    """gpt-oss SwiGLU (triton_kernels.py:2790-2793, 1334-1338):
    g = min(gate, L), u = clamp(up, -L, L), (u + 1) * g * sigmoid(alpha * g)."""
    g = np.minimum(f64(gate), limit)
    u = np.clip(f64(up), -limit, limit)
    return (u + 1.0) * g / (1.0 + np.exp(-alpha * g))


def interleaved_swiglu64(gate_up, alpha: float, limit: float) -> np.ndarray:
    """_interleaved_swiglu_kernel (triton_kernels.py:2778-2793): gate = even columns,
    up = odd columns of each row."""
    gu = f64(gate_up)
    return gptoss_swiglu64(gu[..., 0::2], gu[..., 1::2], alpha, limit)


def weighted_expert_sum64(experts, scores) -> np.ndarray:
    """_weighted_expert_sum_kernel (triton_kernels.py:2797-2817): sum_e scores[e] * experts[e]."""
    return f64(scores) @ f64(experts)


def rope64(first, second, cos, sin):
    """Rotation of the (first, second) halves of a head (triton_kernels.py:2638-2687,
    gpu_runtime.py:8696-8705) as the complex product (first + i second)(cos + i sin)."""
    z = (f64(first) + 1j * f64(second)) * (f64(cos) + 1j * f64(sin))
    return z.real, z.imag


def attention64(q, keys, values, kv_heads: int, sinks=None) -> np.ndarray:
    """Single-token GQA attention (triton_kernels.py:15-109): query head h reads KV head
    h // (heads / kv_heads); scores q.k * head_dim^-0.5; a sink adds one more logit to
    the softmax that carries no value (:52-57).  q [heads, D], keys/values
    [kv_heads, tokens, D]; returns [heads, D]."""
    q = f64(q)
    k = f64(keys)
    v = f64(values)
    heads, D = q.shape
    group = heads // kv_heads
    out = np.empty((heads, D))
    for h in range(heads):
        kv = h // group
        s = k[kv] @ q[h] / np.sqrt(D)
        logits = s if sinks is None else np.concatenate([[float(f64(sinks)[h])], s])
        p = np.exp(logits - logits.max())
        p /= p.sum()
        out[h] = (p if sinks is None else p[1:]) @ v[kv]
    return out


def topk_softmax64(logits, k: int, renormalize: bool):
    """_moe_router_topk_kernel (triton_kernels.py:2821-2851): top-k by value with the
    lowest index first among equal values (a stable sort), then
    p = e^(v - max_all) / D with D over the selected (renormalize) or all logits."""
    lg = f64(logits)
    order = np.argsort(-lg, kind="stable")[:k]
    e = np.exp(lg - lg.max())
    den = e[order].sum() if renormalize else e.sum()
    return order.astype(np.int32), e[order] / den


def router64(weight, hidden, bias, k: int, renormalize: bool):
    """_moe_router_matvec_topk_kernel (triton_kernels.py:2855-2921): logits = bf16(W h),
    then bf16(logits + bias), then top-k and softmax as topk_softmax64."""
    lg = bf16_round64(f64(weight) @ f64(hidden))
    if bias is not None:
        lg = bf16_round64(lg + f64(bias))
    return topk_softmax64(lg, k, renormalize)


def expert_swiglu64(w_gate_up, x, bias, alpha: float, limit: float, rnd) -> np.ndarray:
    """Fused gate/up expert GEMV + SwiGLU (triton_kernels.py:1214-1343): rows 2a (gate)
    and 2a+1 (up) of the dequantised matrix w_gate_up [2I, K]; the dot products and the
    bias sums pass through `rnd` (bfloat16 for q2/q1, :1319-1333; the activation dtype
    for the MXFP4 operator chain, gpu_runtime.py:9647-9704)."""
    y = rnd(f64(w_gate_up) @ f64(x))
    if bias is not None:
        y = rnd(y + f64(bias))
    return gptoss_swiglu64(y[0::2], y[1::2], alpha, limit)


def weighted_down64(w_down_per_slot, x_per_slot, scores, biases, rnd) -> np.ndarray:
    """Fused down GEMV + router-weighted sum (triton_kernels.py:1347-1435):
    sum_s score_s * rnd(rnd(W_s x_s) + bias_s)."""
    out = 0.0
    for s, (w, x) in enumerate(zip(w_down_per_slot, x_per_slot)):
        y = rnd(f64(w) @ f64(x))
        if biases is not None:
            y = rnd(y + f64(biases[s]))
        out = out + float(f64(scores)[s]) * y
    return out


def ulp16(v) -> np.ndarray:
    """Spacing of binary16 values at |v| (normal range; 2^-24 below it)."""
    a = np.abs(np.asarray(v, dtype=np.float64))
    e = np.floor(np.log2(np.maximum(a, 2.0 ** -14)))
    return np.exp2(e - 10)


def err_ulp16(got, want) -> np.ndarray:
    """|got - want| in units of the binary16 spacing at want."""
    return np.abs(f64(got) - f64(want)) / ulp16(want)
