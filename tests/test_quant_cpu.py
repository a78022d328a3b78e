"""Load-time quantizer oracle (oracle/quant.py) pinned to the reference's outputs.

tests/golden/quant_vectors.npz holds seeded inputs and the outputs of the reference's
own torch quantizers (written by tests/golden/make_quant_vectors.py, which imports
them from the reference tree in the build container).  Every oracle function must
reproduce them bit for bit, and each planted mistake below must be caught.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import quant as Q

GOLDEN = Path(__file__).resolve().parent / "golden" / "quant_vectors.npz"


@pytest.fixture(scope="module")
def V():
    return np.load(GOLDEN)


def src(V, name):
    bits = V[name + ".source"]
    return Q.f16_to_f32(bits) if name == "fp8_rows_f16" else Q.bf16_to_f32(bits)


def same(got, want):
    got = np.asarray(got)
    if got.dtype == np.float16:
        got = got.view(np.uint16)
    return got.shape == want.shape and np.array_equal(got, want)


@pytest.mark.parametrize("name", ["int4_lsq", "int4_lsq_ragged", "int4_lsq_g32"])
def test_int4_lsq_matches_reference(V, name):
    p, s = Q.int4_lsq(src(V, name), int(V[name + ".group_size"]))
    assert same(p, V[name + ".packed"]) and same(s, V[name + ".scales"])


@pytest.mark.parametrize("name,rms", [("int4_affine", False), ("int4_affine_rms", True)])
def test_int4_affine_matches_reference(V, name, rms):
    p, s = Q.int4_lsq_affine(src(V, name), 128, V[name + ".input_rms"] if rms else None)
    assert same(p, V[name + ".packed"]) and same(s, V[name + ".scales"])


def gptq_factors(V, name):
    """The upper Cholesky factors of the damped inverse covariances, from the host-side
    set-up the product uses (thintensor_amd.quantize.gptq_inverse_cholesky)."""
    from thintensor_amd.quantize import gptq_inverse_cholesky

    return gptq_inverse_cholesky(torch.from_numpy(V[name + ".covariance"])).numpy()


@pytest.mark.parametrize("name,rms", [("int4_affine_gptq", False), ("int4_affine_gptq_rms", True)])
def test_int4_affine_gptq_matches_reference(V, name, rms):
    x = src(V, name)
    U = gptq_factors(V, name)
    p, s = Q.int4_lsq_affine(x, 32, V[name + ".input_rms"] if rms else None, gptq_factors=U)
    assert same(p, V[name + ".packed"]) and same(s, V[name + ".scales"])
    # the passes change the result (the vectors pin them, not just the plain affine fit)
    p0, s0 = Q.int4_lsq_affine(x, 32, V[name + ".input_rms"] if rms else None)
    assert not same(p0, V[name + ".packed"])
    # planted mistake: the factor transposed (error spread down column c instead of along row c)
    bad = np.ascontiguousarray(np.swapaxes(U, 1, 2))
    pb, _ = Q.int4_lsq_affine(x, 32, V[name + ".input_rms"] if rms else None, gptq_factors=bad)
    assert not same(pb, V[name + ".packed"])


def test_int4_lsq_ignores_covariance(V):
    """The symmetric fit computes the factors and leaves them unused (gpu_runtime.py:237-253)."""
    name = "int4_lsq_gptq_unused"
    p, s = Q.int4_lsq(src(V, name), 32)
    assert same(p, V[name + ".packed"]) and same(s, V[name + ".scales"])


def test_gptq_factors_properties(V):
    """U is upper triangular with a positive diagonal and U^T U inverts the damped
    covariance (float64 check of the host set-up)."""
    cov = V["int4_affine_gptq.covariance"].astype(np.float64)
    U = gptq_factors(V, "int4_affine_gptq").astype(np.float64)
    assert np.all(np.tril(U, -1) == 0) and np.all(np.diagonal(U, axis1=1, axis2=2) > 0)
    damp = np.maximum(np.diagonal(cov, axis1=1, axis2=2).mean(axis=1) * 0.01, 1e-6)
    H = cov + damp[:, None, None] * np.eye(32)
    # inv(H) = U^T U  <=>  U H U^T = I
    eye = U @ H @ np.swapaxes(U, 1, 2)
    assert np.max(np.abs(eye - np.eye(32))) < 1e-3


@pytest.mark.parametrize("name,affine", [("int4_rows", False), ("int4_rows_ragged", False), ("int4_rows_affine", True)])
def test_int4_rows_matches_reference(V, name, affine):
    p, s = Q.int4_rows(src(V, name), int(V[name + ".group_size"]), affine=affine)
    assert same(p, V[name + ".packed"]) and same(s, V[name + ".scales"])


@pytest.mark.parametrize("name,via", [("fp8_rows", False), ("fp8_rows_f16", False), ("fp8_block", False),
                                      ("fp8_block_ragged", False), ("fp8_via_bf16", True),
                                      ("fp8_via_bf16_block", True)])
def test_fp8_matches_reference(V, name, via):
    q, s = Q.fp8_rows(src(V, name), int(V[name + ".block"]), via_bf16=via)
    assert same(q, V[name + ".quantized"]) and same(s, V[name + ".scales"])


@pytest.mark.parametrize("name,kw", [("mxfp4_rows", {}), ("mxfp4_rows_h32", {"hadamard_size": 32}),
                                     ("mxfp4_rows_h64s", {"hadamard_size": 64, "signs": True}),
                                     ("mxfp4_rows_resid", {"binary_residual": True})])
def test_mxfp4_rows_matches_reference(V, name, kw):
    kw = dict(kw)
    if kw.pop("signs", False):
        kw["signs"] = Q.bf16_to_f32(V[name + ".signs"])
    p, s = Q.mxfp4_rows(src(V, name), **kw)
    assert same(p, V[name + ".packed"]) and same(s, V[name + ".scales"])


@pytest.mark.parametrize("bits", [2, 1])
def test_lowbit_requant_and_dense_match_reference(V, bits):
    n = f"lowbit_q{bits}"
    p, s = Q.mxfp4_to_lowbit(V[n + ".blocks"], V[n + ".scales"], bits)
    assert same(p, V[n + ".packed"]) and same(s, V[n + ".out_scales"])
    n = f"dense_q{bits}"
    p, s = Q.dense_to_lowbit(src(V, n), bits)
    assert same(p, V[n + ".packed"]) and same(s, V[n + ".out_scales"])


def test_ternary_matches_reference(V):
    p, s = Q.pack_mxfp4_to_ternary(V["ternary.blocks"], V["ternary.scales"])
    assert same(p, V["ternary.packed"]) and same(s, V["ternary.out_scales"])


def test_e4m3_conversion_matches_torch():
    vals = np.concatenate([
        np.linspace(-500, 500, 100001, dtype=np.float32),
        (np.arange(-3000, 3000, dtype=np.float32) * 2.0 ** -13).astype(np.float32),
        np.array([0.0, -0.0, 448, 463.99, 464, 464.01, 479.9, 480, np.inf, -np.inf, np.nan, 2 ** -9, 2 ** -10,
                  3 * 2 ** -11, 2 ** -6, 2 ** -6 * (1 - 2 ** -20)], dtype=np.float32),
    ])
    want = torch.from_numpy(vals).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    got = Q.f32_to_e4m3(vals)
    nan = np.isnan(vals)
    assert np.array_equal(got[~nan], want[~nan])
    assert np.all((got[nan] & 0x7F) == 0x7F) and np.all((want[nan] & 0x7F) == 0x7F)


def test_lane_sum_is_exact_on_integers_and_order_fixed():
    rng = np.random.default_rng(0)
    x = rng.integers(-1000, 1000, size=(7, 128)).astype(np.float32)
    assert np.array_equal(Q.lane_sum(x), x.sum(axis=1).astype(np.float32))
    # binary64 accumulation: 2^24 + 1 + 1 is exact before the single rounding
    y = np.zeros((1, 64), np.float32)
    y[0, 0], y[0, 1], y[0, 2] = 2.0 ** 24, 1.0, 1.0
    assert Q.lane_sum(y)[0] == np.float32(2.0 ** 24 + 2)


def test_log2_helpers_are_exact_at_powers_of_two():
    v = np.array([2.0 ** -140, 2.0 ** -126, 0.75, 1.0, 1.0000001, 6.0, 2.0 ** 100], dtype=np.float32)
    assert list(Q.ceil_log2(v)) == [-140, -126, 0, 0, 1, 3, 100]
    assert list(Q.floor_log2(v)) == [-140, -126, -1, 0, 0, 2, 100]


# ----------------------------------------------------------------- planted mistakes
def test_planted_mistakes_are_caught(V, monkeypatch):
    # 1. LSQ without its least-squares refit: the first-pass scale amax/7
    x = src(V, "int4_lsq")
    g, present = Q._groups(x, 128)
    amax = np.max(np.abs(g), axis=2).astype(np.float32)
    s0 = (np.maximum(amax, Q.TINY) / np.float32(7.0)).astype(np.float32)
    assert not same(s0.astype(np.float16), V["int4_lsq.scales"])
    # 2. body INT4 rows with codes offset by 7 instead of 8
    p, s = Q.int4_rows(src(V, "int4_rows"), 128)
    low, high = p & 15, p >> 4
    wrong = (((low - 1) & 15) | (((high - 1) & 15) << 4)).astype(np.uint8)
    assert not same(wrong, V["int4_rows.packed"])
    # 3. e4m3 by truncation instead of round-to-nearest-even
    y = (src(V, "fp8_rows") / V["fp8_rows.scales"][:, None]).astype(np.float32)
    trunc = np.sign(y) * np.ldexp(np.floor(np.ldexp(np.abs(y), 3 - np.floor(np.log2(np.maximum(np.abs(y), 2 ** -6))).astype(int))),
                                  np.floor(np.log2(np.maximum(np.abs(y), 2 ** -6))).astype(int) - 3)
    assert not same(Q.f32_to_e4m3(trunc.astype(np.float32)), V["fp8_rows.quantized"])
    # 4. MXFP4 exponent from floor instead of ceil of log2(amax / 6)
    monkeypatch.setattr(Q, "ceil_log2", lambda v: Q.floor_log2(v))
    p, s = Q.mxfp4_rows(src(V, "mxfp4_rows"))
    assert not same(s, V["mxfp4_rows.scales"])
    monkeypatch.undo()
    # 5. Q2 requantization with the tie rule reversed (later offset wins ties)
    n = "lowbit_q2"
    orig = Q.mxfp4_to_lowbit

    def reversed_ties(blocks, scales, bits):
        nib = Q._mx_nibbles(blocks)
        vals = np.concatenate([Q.E2M1, -Q.E2M1])[nib]
        neg = (nib & 8) != 0
        q2 = np.array([-1.5, -0.5, 0.5, 1.5], dtype=np.float32)
        best_err = best_d = None
        for d in (-2, -1, 0, 1, 2, 3):
            f = np.float32(2.0 ** d)
            outer = np.abs(vals) >= f
            codes = np.where(neg, np.where(outer, 0, 1), np.where(outer, 3, 2))
            err = (((vals - q2[codes] * f) ** 2).sum(axis=-1) / 32).astype(np.float32)
            if best_err is None:
                best_err, best_d = err, np.full(err.shape, d)
            else:
                take = err <= best_err
                best_err, best_d = np.where(take, err, best_err), np.where(take, d, best_d)
        return (np.clip(scales.astype(np.int16) - 127 + best_d, -127, 127) + 127).astype(np.uint8)

    assert orig(V[n + ".blocks"], V[n + ".scales"], 2)[1].shape == V[n + ".out_scales"].shape
    assert not same(reversed_ties(V[n + ".blocks"], V[n + ".scales"], 2), V[n + ".out_scales"])
    # 6. dense Q2 with the Q1 level (base exponent from amax / 1 instead of amax / 1.5)
    x = src(V, "dense_q2")
    amax = np.maximum(np.max(np.abs(x.reshape(16, 8, 32)), axis=2), np.float32(2.0 ** -126))
    assert not np.array_equal(Q.floor_log2(amax), Q.floor_log2((amax / np.float32(1.5)).astype(np.float32)))
    p1, s1 = Q.dense_to_lowbit(x, 1)
    assert not same(s1, V["dense_q2.out_scales"])
