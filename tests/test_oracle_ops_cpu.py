"""CPU checks that pin the oracle's decode-step operators to the reference semantics.

Each binary32 restatement in oracle/tt_oracle.c (norms, SiLU/SwiGLU, weighted sums,
RoPE, attention with sinks, router top-k and softmax, the fused expert SwiGLU and
weighted-down) is compared with an independent float64 statement of the reference
formula (oracle/ref.py: whole-vector numpy, a stable sort, complex rotation), on:

* random inputs, within one binary16 ulp of the correctly rounded float64 value;
* exact inputs (dyadic values, integer activations, one-token attention, position 0)
  where every evaluation order gives the same float, so the outputs must be equal;
* a planted mistake per operator (swapped gate/up interleave, a dropped sink, the
  wrong softmax denominator, a missing bf16 rounding point, ...) that the same check
  must reject, so a plausible error in the restatement cannot pass unseen.
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle
from oracle import ref
from oracle.decode_ref import lanes
from tests.helpers import f16_normal, rng
from thintensor_amd import layouts


def within_ulp(got, want64, ulps: float = 1.0, exact_frac: float = 0.95) -> bool:
    """got (binary16) is within `ulps` of the float64 value everywhere and equal to its
    correctly rounded binary16 value for at least `exact_frac` of the outputs."""
    got = np.asarray(got, dtype=np.float16).reshape(-1)
    want64 = np.asarray(want64, dtype=np.float64).reshape(-1)
    err = ref.err_ulp16(got, want64)
    exact = np.mean(got.astype(np.float64) == ref.f16_round64(want64))
    return bool(np.max(err) <= ulps and exact >= exact_frac)


def dyadic_f16(g, shape, lo=-16, hi=17, denom=8.0):
    return (g.integers(lo, hi, size=shape) / denom).astype(np.float16)


# ---------------------------------------------------------------- RMSNorm


@pytest.mark.parametrize("n,offset", [(2048, 0.0), (2880, 1.0), (5120, 0.0), (100, 0.0)])
def test_rms_norm_vs_float64(n, offset):
    g = rng(100 + n)
    x, w = f16_normal(g, n, 3.0), f16_normal(g, n, 0.1)
    got = oracle.rms_norm(x, w, 1e-5, offset)
    want = ref.rms_norm64(x, w, 1e-5, offset)
    assert within_ulp(got, want)
    if offset:
        # planted: the (w + offset) term dropped
        assert not within_ulp(oracle.rms_norm(x, w, 1e-5, 0.0), want)


def test_rms_norm_exact_when_mean_square_is_a_power_of_four():
    g = rng(101)
    n = 2048
    x = np.where(g.integers(0, 2, n) == 1, 2.0, -2.0).astype(np.float16)  # mean(x^2) = 4, rsqrt = 1/2
    w = dyadic_f16(g, n)
    got = oracle.rms_norm(x, w, 0.0)
    assert np.array_equal(got.astype(np.float64), ref.rms_norm64(x, w, 0.0))


@pytest.mark.parametrize("n", [2048, 2880, 5120])
def test_add_rms_norm_rounding_point(n):
    g = rng(200 + n)
    left, right, w = f16_normal(g, n), f16_normal(g, n, 0.5), f16_normal(g, n, 0.1)
    res, out = oracle.add_rms_norm(left, right, w, 1e-5)
    want_res, want = ref.add_rms_norm64(left, right, w, 1e-5)
    # the stored residual is exactly the bf16-rounded sum (triton_kernels.py:2603-2606)
    assert np.array_equal(res.astype(np.float64), want_res)
    assert within_ulp(out, want)
    # planted: residual rounded to the activation dtype instead of bfloat16
    r16 = ref.f16_round64(ref.f64(left) + ref.f64(right))
    assert not np.array_equal(r16, want_res)
    bad = ref.f16_round64(r16 / np.sqrt(np.mean(r16 * r16) + 1e-5) * ref.f64(w))
    assert not within_ulp(bad, want)


# ---------------------------------------------------------------- SiLU / SwiGLU / weighted sum


def test_silu_mul_vs_float64_and_swap_caught():
    g = rng(300)
    n = 8192
    gate, up = f16_normal(g, n, 3.0), f16_normal(g, n)
    gate[:4] = [0.0, -0.0, -30.0, 30.0]
    got = oracle.silu_mul(gate, up)
    assert within_ulp(got, ref.silu_mul64(gate, up))
    assert got[0] == 0 and got[1] == 0
    assert not within_ulp(oracle.silu_mul(up, gate), ref.silu_mul64(gate, up))


@pytest.mark.parametrize("rows,n", [(4, 2880), (1, 64)])
def test_interleaved_swiglu_vs_float64_and_swap_caught(rows, n):
    g = rng(301 + n)
    gu = f16_normal(g, (rows, 2 * n), 6.0)  # |values| above the limit 7 exercise both clamps
    got = oracle.interleaved_swiglu(gu, 1.702, 7.0)
    want = ref.interleaved_swiglu64(gu, 1.702, 7.0)
    assert within_ulp(got, want)
    assert np.mean(np.abs(gu[:, 0::2]) > 7.0) > 0.1
    swapped = gu.reshape(rows, n, 2)[:, :, ::-1].reshape(rows, 2 * n)  # planted: up/gate interleave swapped
    assert not within_ulp(oracle.interleaved_swiglu(swapped, 1.702, 7.0), want)


def test_weighted_expert_sum_exact_and_order_caught():
    g = rng(302)
    ex = dyadic_f16(g, (4, 2880))
    sc = np.array([0.5, 0.25, 0.125, 0.125], dtype=np.float16)
    got = oracle.weighted_expert_sum(ex, sc)
    assert np.array_equal(got.astype(np.float64), ref.f16_round64(ref.weighted_expert_sum64(ex, sc)))
    exr = f16_normal(g, (4, 2880))
    assert within_ulp(oracle.weighted_expert_sum(exr, sc), ref.weighted_expert_sum64(exr, sc))
    assert not within_ulp(oracle.weighted_expert_sum(exr, sc[::-1].copy()), ref.weighted_expert_sum64(exr, sc))


# ---------------------------------------------------------------- RoPE


def _rope_table(positions: int, D: int, theta: float = 500000.0):
    inv = (theta ** (-np.arange(0, D, 2, dtype=np.float32) / D)).astype(np.float32)
    ang = np.arange(positions, dtype=np.float32)[:, None] * inv[None, :]
    return np.cos(ang).astype(np.float16), np.sin(ang).astype(np.float16)


def test_rope_rotation_identity_and_fp16_arithmetic():
    heads, kv_heads, D = 32, 8, 64
    half = D // 2
    g = rng(400)
    cos, sin = _rope_table(600, D)
    q, k = f16_normal(g, heads * D), f16_normal(g, kv_heads * D)
    # position 0: cos = 1, sin = 0 -> identity
    q0, k0 = oracle.rope(q, k, cos[0], sin[0], heads, kv_heads, D)
    assert np.array_equal(q0, q) and np.array_equal(k0, k)
    p = 517
    qr, kr = oracle.rope(q, k, cos[p], sin[p], heads, kv_heads, D)
    for src, got in ((q, qr), (k, kr)):
        a, b = src.reshape(-1, D)[:, :half], src.reshape(-1, D)[:, half:]
        first, second = ref.rope64(a, b, cos[p], sin[p])
        # per-op binary16 rounding (gpu_runtime.py:8696-8705): numpy's float16 arithmetic
        c16, s16 = cos[p], sin[p]
        assert np.array_equal(got.reshape(-1, D)[:, :half], (a * c16) - (b * s16))
        assert np.array_equal(got.reshape(-1, D)[:, half:], (b * c16) + (a * s16))
        # and the rotation itself, within the rounding of three binary16 operations
        scale = ref.ulp16(np.abs(ref.f64(a)) + np.abs(ref.f64(b)))
        assert np.max(np.abs(ref.f64(got.reshape(-1, D)[:, :half]) - first) / scale) <= 1.5
        assert np.max(np.abs(ref.f64(got.reshape(-1, D)[:, half:]) - second) / scale) <= 1.5
    # planted: the sine's sign flipped (rotation the wrong way)
    qb, _ = oracle.rope(q, k, cos[p], (-sin[p]).astype(np.float16), heads, kv_heads, D)
    a, b = q.reshape(-1, D)[:, :half], q.reshape(-1, D)[:, half:]
    first, _ = ref.rope64(a, b, cos[p], sin[p])
    assert np.max(np.abs(ref.f64(qb.reshape(-1, D)[:, :half]) - first)) > 0.1


# ---------------------------------------------------------------- attention


def _attention_inputs(g, heads, kv_heads, cap, D=64):
    return (f16_normal(g, heads * D), f16_normal(g, (kv_heads, cap, D)), f16_normal(g, (kv_heads, cap, D)))


def _attn_close(got, want, values) -> bool:
    got = ref.f64(got).reshape(want.shape)
    tol = ref.ulp16(want) + 1e-5 * np.max(np.abs(ref.f64(values)))
    return bool(np.all(np.abs(got - want) <= tol))


@pytest.mark.parametrize("heads,kv_heads,tokens,sinks", [(8, 2, 5, False), (8, 2, 513, True), (64, 8, 1025, True),
                                                         (32, 8, 64, False), (4, 4, 130, True)])
def test_attention_vs_float64(heads, kv_heads, tokens, sinks):
    D, cap = 64, 1100
    g = rng(500 + tokens + heads)
    q, keys, vals = _attention_inputs(g, heads, kv_heads, cap)
    sk = f16_normal(g, heads, 2.0) if sinks else None
    got = oracle.attention(q, keys, vals, tokens, heads, kv_heads, D, sinks=sk)
    want = ref.attention64(q.reshape(heads, D), keys[:, :tokens], vals[:, :tokens], kv_heads, sinks=sk)
    assert _attn_close(got, want, vals)
    if sinks:  # planted: the sink dropped
        assert not _attn_close(oracle.attention(q, keys, vals, tokens, heads, kv_heads, D), want, vals)
    # planted: the head_dim^-1/2 scale left out (q * 8 for head_dim 64)
    q8 = (q.astype(np.float32) * 8).astype(np.float16)
    assert not _attn_close(oracle.attention(q8, keys, vals, tokens, heads, kv_heads, D, sinks=sk), want, vals)


def test_attention_single_token_returns_value_and_sink_shrinks_it():
    heads, kv_heads, D, cap = 8, 2, 64, 64
    g = rng(501)
    q, keys, vals = _attention_inputs(g, heads, kv_heads, cap)
    got = oracle.attention(q, keys, vals, 1, heads, kv_heads, D).reshape(heads, D)
    for h in range(heads):  # softmax over one token is 1: the output is that token's value
        assert np.array_equal(got[h], vals[h // (heads // kv_heads), 0])
    sk = f16_normal(g, heads, 1.0)
    got_s = oracle.attention(q, keys, vals, 1, heads, kv_heads, D, sinks=sk).reshape(heads, D)
    for h in range(heads):
        kv = h // (heads // kv_heads)
        s = float(ref.f64(q.reshape(heads, D)[h]) @ ref.f64(keys[kv, 0])) / 8.0
        want = ref.f64(vals[kv, 0]) / (1.0 + np.exp(float(sk[h]) - s))
        assert _attn_close(got_s[h], want, vals)


# ---------------------------------------------------------------- router top-k / softmax


@pytest.mark.parametrize("E,k,renorm", [(32, 4, True), (32, 4, False), (128, 8, True), (8, 1, False), (64, 64, True)])
def test_topk_vs_stable_sort_and_float64_softmax(E, k, renorm):
    g = rng(600 + E + k)
    lg = (np.round(g.standard_normal(E) * 4) / 4).astype(np.float16)  # coarse: many equal values
    lg[:3] = [np.float16(-0.0), np.float16(0.0), np.float16(-np.inf)]
    idx, sc = oracle.topk(lg, k, renorm)
    widx, wsc = ref.topk_softmax64(lg, k, renorm)
    assert np.array_equal(idx, widx)
    assert within_ulp(sc, wsc, exact_frac=0.75)
    # planted: the other denominator
    _, bad = oracle.topk(lg, k, not renorm)
    if k < E:
        assert not within_ulp(bad, wsc, exact_frac=0.75)
    # planted: highest index first among equal values (oracle run on the reversed logits)
    ridx, _ = oracle.topk(lg[::-1].copy(), k, renorm)
    if len(set(lg[widx].tolist())) < k or np.sum(lg == lg[widx[-1]]) > 1:
        assert not np.array_equal(E - 1 - ridx, widx)


def test_topk_equal_values_lowest_index_first():
    lg = np.array([1.0, 3.0, 3.0, -2.0, 3.0, 0.5, 2.0, 2.0], dtype=np.float16)
    idx, _ = oracle.topk(lg, 4, True)
    assert idx.tolist() == [1, 2, 4, 6] == ref.topk_softmax64(lg, 4, True)[0].tolist()


@pytest.mark.parametrize("renorm,with_bias", [(True, True), (False, True), (True, False)])
def test_router_exact_inputs(renorm, with_bias):
    """Dyadic weights and integer activations: every dot product is exact in binary32,
    so the bf16 logits are fixed and the indices must equal the float64 brute force."""
    E, H, k = 32, 2880, 4
    g = rng(700 + renorm + 2 * with_bias)
    w = (g.integers(-8, 9, size=(E, H)) / 64.0).astype(np.float16)
    x = g.integers(-3, 4, size=H).astype(np.float16)
    b = dyadic_f16(g, E, -8, 9, 4.0) if with_bias else None
    idx, sc = oracle.router(w, x, b, k, renorm)
    widx, wsc = ref.router64(w, x, b, k, renorm)
    assert np.array_equal(idx, widx)
    assert within_ulp(sc, wsc, exact_frac=0.75)


def test_router_random_and_missing_bf16_rounding_caught():
    E, H, k = 32, 2880, 4
    fails = 0
    for seed in range(8):
        g = rng(710 + seed)
        w, x, b = f16_normal(g, (E, H), 0.02), f16_normal(g, H), f16_normal(g, E, 0.1)
        idx, sc = oracle.router(w, x, b, k, True)
        widx, wsc = ref.router64(w, x, b, k, True)
        assert np.array_equal(idx, widx)
        assert within_ulp(sc, wsc, exact_frac=0.75)
        # planted: logits kept in binary32 (no bf16 rounding point)
        lg = ref.f64(w) @ ref.f64(x) + ref.f64(b)
        e = np.exp(lg - lg.max())
        bad = e[widx] / e[widx].sum()
        fails += not within_ulp(bad, wsc, exact_frac=0.75)
    assert fails >= 6


# ---------------------------------------------------------------- fused expert SwiGLU / weighted down


def _expert_weights(g, fmt, experts, rows, cols):
    if fmt == "mxfp4":
        codes = g.integers(0, 16, size=(experts, rows, cols), dtype=np.uint8)
        packed = layouts.pack_mxfp4_blocks(codes)
        scales = g.integers(119, 124, size=(experts, rows, cols // 32), dtype=np.uint8)
        dq = ref.mxfp4_dequant(packed, scales)
    else:
        bits = 2 if fmt == "q2e8" else 1
        codes = g.integers(0, 1 << bits, size=(experts, rows, cols), dtype=np.uint8)
        packed = layouts.pack_lowbit_blocks(codes, bits)
        scales = g.integers(118, 123, size=(experts, rows, cols // 32), dtype=np.uint8)
        dq = ref.lowbit_e8_dequant(packed, scales, bits)
    return packed, scales, dq


def _rnd(fmt):
    return ref.f16_round64 if fmt == "mxfp4" else ref.bf16_round64


@pytest.mark.parametrize("fmt", ["q2e8", "q1e8", "mxfp4"])
@pytest.mark.parametrize("exact", [True, False])
def test_expert_swiglu_vs_float64(fmt, exact):
    E, inter, cols = 3, 96, 320
    g = rng(800 + exact + len(fmt))
    packed, scales, dq = _expert_weights(g, fmt, E, 2 * inter, cols)
    x = g.integers(-4, 5, size=cols).astype(np.float16) if exact else f16_normal(g, cols)
    bias = dyadic_f16(g, (E, 2 * inter), -8, 9, 4.0) if exact else f16_normal(g, (E, 2 * inter), 0.5)
    experts = [2, 0, 1]
    lpr = lanes(cols)
    got = oracle.expert_swiglu(fmt, packed, scales, x, experts, bias, 1.702, 7.0, lpr=lpr)
    want = np.stack([ref.expert_swiglu64(dq[e], x, bias[e], 1.702, 7.0, _rnd(fmt)) for e in experts])
    if exact:
        assert within_ulp(got, want)
    else:
        assert ref.max_rel_err(got, want) < 1e-2 and within_ulp(got, want, ulps=16, exact_frac=0.9)
    # planted: gate and up rows swapped in the interleave
    sw_p = packed.copy()
    sw_p[:, 0::2], sw_p[:, 1::2] = packed[:, 1::2], packed[:, 0::2]
    sw_s = scales.copy()
    sw_s[:, 0::2], sw_s[:, 1::2] = scales[:, 1::2], scales[:, 0::2]
    sw_b = bias.copy()
    sw_b[:, 0::2], sw_b[:, 1::2] = bias[:, 1::2], bias[:, 0::2]
    bad = oracle.expert_swiglu(fmt, sw_p, sw_s, x, experts, sw_b, 1.702, 7.0, lpr=lpr)
    assert not within_ulp(bad, want, ulps=16, exact_frac=0.5)


def test_expert_swiglu_bf16_rounding_point_caught():
    """q2: gate/up pass through bfloat16 (triton_kernels.py:1319-1333); a float64 path
    without those rounding points is rejected by the same check."""
    E, inter, cols = 2, 128, 320
    g = rng(810)
    packed, scales, dq = _expert_weights(g, "q2e8", E, 2 * inter, cols)
    x = g.integers(-4, 5, size=cols).astype(np.float16)
    bias = dyadic_f16(g, (E, 2 * inter), -8, 9, 4.0)
    got = oracle.expert_swiglu("q2e8", packed, scales, x, [1, 0], bias, 1.702, 7.0, lpr=lanes(cols))
    want = np.stack([ref.expert_swiglu64(dq[e], x, bias[e], 1.702, 7.0, ref.bf16_round64) for e in (1, 0)])
    unrounded = np.stack([ref.expert_swiglu64(dq[e], x, bias[e], 1.702, 7.0, lambda v: v) for e in (1, 0)])
    assert within_ulp(got, want)
    assert not within_ulp(got, unrounded)


@pytest.mark.parametrize("fmt", ["q2e8", "q1e8", "mxfp4"])
def test_weighted_down_exact_and_slot_order_caught(fmt):
    E, rows, cols, k = 4, 160, 288, 4
    g = rng(900 + len(fmt))
    packed, scales, dq = _expert_weights(g, fmt, E, rows, cols)
    x = g.integers(-4, 5, size=(k, cols)).astype(np.float16)
    bias = dyadic_f16(g, (E, rows), -8, 9, 4.0)
    experts = [3, 1, 0, 2]
    scores = np.array([0.5, 0.25, 0.125, 0.125], dtype=np.float16)
    got = oracle.weighted_down(fmt, packed, scales, x, experts, scores, bias, lpr=lanes(cols))
    want = ref.weighted_down64([dq[e] for e in experts], x, scores, [bias[e] for e in experts], _rnd(fmt))
    assert np.array_equal(got.astype(np.float64), ref.f16_round64(want))
    # random activations: within tolerance
    xr = f16_normal(g, (k, cols))
    gotr = oracle.weighted_down(fmt, packed, scales, xr, experts, scores, bias, lpr=lanes(cols))
    wantr = ref.weighted_down64([dq[e] for e in experts], xr, scores, [bias[e] for e in experts], _rnd(fmt))
    assert ref.max_rel_err(gotr, wantr) < 1e-2
    # planted: router scores applied in reverse slot order
    bad = oracle.weighted_down(fmt, packed, scales, x, experts, scores[::-1].copy(), bias, lpr=lanes(cols))
    assert not np.array_equal(bad.astype(np.float64), ref.f16_round64(want))


# ---------------------------------------------------------------- per-head RMSNorm and QK norm + RoPE


@pytest.mark.parametrize("heads,D", [(32, 128), (8, 64), (4, 256)])
def test_head_rms_norm_vs_float64(heads, D):
    g = rng(1000 + heads + D)
    x, w = f16_normal(g, heads * D, 2.0), f16_normal(g, D, 0.5)
    got = oracle.head_rms_norm(x, w, heads, D, 1e-6)
    want = np.concatenate([ref.rms_norm64(x[h * D:(h + 1) * D], w, 1e-6) for h in range(heads)])
    assert within_ulp(got, want)
    # planted: one norm over all heads instead of one per head
    assert not within_ulp(got, ref.rms_norm64(x, np.tile(w, heads), 1e-6))


def _qk_norm_rope64(x, w, heads, D, c, s, eps):
    out = []
    for h in range(heads):
        n = ref.rms_norm64(x[h * D:(h + 1) * D], w, eps)
        first, second = ref.rope64(n[:D // 2], n[D // 2:], c, s)
        out.append(np.concatenate([first, second]))
    return np.concatenate(out)


def test_qk_head_rmsnorm_rope_vs_float64_and_planted_sign():
    heads, kv_heads, D = 16, 4, 128
    g = rng(1100)
    cos, sin = _rope_table(700, D, 1000000.0)
    q, k = f16_normal(g, heads * D, 2.0), f16_normal(g, kv_heads * D)
    qw, kw = f16_normal(g, D, 0.5), f16_normal(g, D, 0.5)
    p = 613
    qo, ko = oracle.qk_head_rmsnorm_rope(q, k, qw, kw, cos[p], sin[p], heads, kv_heads, D, 1e-6)
    for x, w, n, got in ((q, qw, heads, qo), (k, kw, kv_heads, ko)):
        want = _qk_norm_rope64(x, w, n, D, cos[p], sin[p], 1e-6)
        # binary32 rotation rounded once: within one binary16 ulp of the operands' scale
        norm = np.concatenate([np.abs(ref.rms_norm64(x[h * D:(h + 1) * D], w, 1e-6)) for h in range(n)])
        scale = ref.ulp16(np.maximum(norm, np.roll(norm.reshape(n, 2, D // 2), 1, axis=1).reshape(-1)))
        assert np.max(np.abs(ref.f64(got) - want) / scale) <= 1.0
    # position 0 is the per-head RMSNorm alone (cos 1, sin 0)
    q0, _ = oracle.qk_head_rmsnorm_rope(q, k, qw, kw, cos[0], sin[0], heads, kv_heads, D, 1e-6)
    assert within_ulp(q0, np.concatenate([ref.rms_norm64(q[h * D:(h + 1) * D], qw, 1e-6) for h in range(heads)]))
    # planted: rotation the wrong way
    qb, _ = oracle.qk_head_rmsnorm_rope(q, k, qw, kw, cos[p], (-sin[p]).astype(np.float16), heads, kv_heads, D, 1e-6)
    assert np.max(np.abs(ref.f64(qb) - _qk_norm_rope64(q, qw, heads, D, cos[p], sin[p], 1e-6))) > 0.1


def test_split_k_restatement_vs_float64_and_exact():
    """Split-K composition of the GEMV restatement: exact on integer inputs whatever
    the split, close to float64 otherwise, and a dropped slice is caught."""
    g = rng(1200)
    rows, cols = 64, 2880
    w_int = g.integers(-4, 5, size=(rows, cols)).astype(np.float16)
    x_int = g.integers(-3, 4, size=cols).astype(np.float16)
    for sk in (2, 4, 8):
        got = oracle.split_k_gemv("f16w", w_int, x_int, sk, odtype=oracle.F32)
        assert np.array_equal(got.astype(np.float64), ref.gemv64(w_int, x_int))
    w, x = f16_normal(g, (rows, cols), 0.05), f16_normal(g, cols)
    sc = np.abs(g.standard_normal(rows)).astype(np.float32)
    got = oracle.split_k_gemv("f16w", w, x, 8, scales=sc)
    want = ref.gemv64(w, x) * sc
    assert within_ulp(got, want, ulps=1.0, exact_frac=0.9)
    # planted: the last (shorter) slice left out
    nchunks, q = cols // 32, -(-(cols // 32) // 8)
    last = (nchunks // q) * q * 32
    bad = oracle.split_k_gemv("f16w", w[:, :last], x[:last], 8, scales=sc)
    assert not within_ulp(bad, want, ulps=1.0, exact_frac=0.9)
