"""GPU parity of the load-time quantizers (csrc/quantize.hip via thintensor_amd.quantize).

Three checks per quantizer:
* the reference's own outputs (tests/golden/quant_vectors.npz), bit for bit;
* the oracle restatement (oracle/quant.py, pinned to those outputs) on larger seeded
  inputs, bit for bit;
* at full layer sizes, properties fixed by the formats themselves: every INT4 code
  reconstructs its weight within half a scale step, e4m3 keeps 3 significant bits, and
  the MXFP4 -> Q1/Q2 -> ternary packers agree with the oracle on every group.
"""

from __future__ import annotations

import os
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import quant as Q
from thintensor_amd import quantize as TQ

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden" / "quant_vectors.npz"


@pytest.fixture(scope="module")
def V():
    return np.load(GOLDEN)


def src_t(V, name):
    bits = torch.from_numpy(V[name + ".source"].astype(np.int16))
    return bits.view(torch.float16 if name == "fp8_rows_f16" else torch.bfloat16)


def as_np(t):
    t = t.cpu()
    if t.dtype in (torch.float16, torch.bfloat16):
        return t.view(torch.int16).numpy().view(np.uint16)
    if t.dtype == torch.float8_e4m3fn:
        return t.view(torch.uint8).numpy()
    return t.numpy()


def eq(got, want, what):
    g = as_np(got)
    assert g.shape == want.shape, f"{what}: shape {g.shape} vs {want.shape}"
    bad = np.nonzero(g.reshape(-1) != want.reshape(-1))[0]
    assert bad.size == 0, f"{what}: {bad.size} of {want.size} differ (first at {bad[:5]})"


@pytest.fixture
def affine_env(monkeypatch):
    def set_(on: bool):
        monkeypatch.setenv("THINTENSOR_AFFINE_INT4", "1" if on else "0")
    return set_


# ------------------------------------------------------------------- reference vectors
@pytest.mark.parametrize("name", ["int4_lsq", "int4_lsq_ragged", "int4_lsq_g32"])
def test_int4_lsq_reference_vectors(V, affine_env, name):
    affine_env(False)
    p, s = TQ.quantize_to_int4_cpu(src_t(V, name), group_size=int(V[name + ".group_size"]))
    assert p.device.type == "cpu" and s.dtype == torch.float16
    eq(p, V[name + ".packed"], name + " packed")
    eq(s, V[name + ".scales"], name + " scales")


def test_int4_affine_reference_vectors(V, affine_env):
    affine_env(True)
    p, s = TQ.quantize_to_int4_cpu(src_t(V, "int4_affine"), group_size=128)
    eq(p, V["int4_affine.packed"], "affine packed")
    eq(s, V["int4_affine.scales"], "affine scales")
    rms = torch.from_numpy(V["int4_affine_rms.input_rms"])
    p, s = TQ.quantize_to_int4_cpu(src_t(V, "int4_affine_rms"), group_size=128, input_rms=rms)
    eq(p, V["int4_affine_rms.packed"], "affine+rms packed")
    eq(s, V["int4_affine_rms.scales"], "affine+rms scales")


@pytest.mark.parametrize("name,rms", [("int4_affine_gptq", False), ("int4_affine_gptq_rms", True)])
def test_int4_affine_gptq_reference_vectors(V, affine_env, name, rms):
    """GPTQ passes with a calibration covariance (gpu_runtime.py:130-150, :217-262)."""
    affine_env(True)
    cov = torch.from_numpy(V[name + ".covariance"])
    kw = {"input_rms": torch.from_numpy(V[name + ".input_rms"])} if rms else {}
    p, s = TQ.quantize_to_int4_cpu(src_t(V, name), group_size=32, input_covariance32=cov, **kw)
    assert p.device.type == "cpu"
    eq(p, V[name + ".packed"], name + " packed")
    eq(s, V[name + ".scales"], name + " scales")


def test_int4_gptq_covariance_contract(V, affine_env):
    """The symmetric fit leaves the factors unused; group sizes other than 32 and
    mismatched covariance shapes raise the reference's errors."""
    affine_env(False)
    name = "int4_lsq_gptq_unused"
    cov = torch.from_numpy(V[name + ".covariance"])
    p, s = TQ.quantize_to_int4_cpu(src_t(V, name), group_size=32, input_covariance32=cov)
    eq(p, V[name + ".packed"], "symmetric packed")
    eq(s, V[name + ".scales"], "symmetric scales")
    with pytest.raises(ValueError, match="require INT4 group size 32"):
        TQ.quantize_to_int4_cpu(src_t(V, name), group_size=64, input_covariance32=cov)
    with pytest.raises(ValueError, match="covariance shape"):
        TQ.quantize_to_int4_cpu(src_t(V, name), group_size=32, input_covariance32=cov[:4])


@pytest.mark.parametrize("name,affine", [("int4_rows", False), ("int4_rows_ragged", False), ("int4_rows_affine", True)])
def test_int4_rows_reference_vectors(V, affine_env, device, name, affine):
    affine_env(affine)
    x = src_t(V, name).to(device)
    p, s = TQ.quantize_int4_rows(x, group_size=int(V[name + ".group_size"]))
    assert p.device.type == "cuda" and s.dtype == torch.float32
    eq(p, V[name + ".packed"], name + " packed")
    eq(s, V[name + ".scales"], name + " scales")


@pytest.mark.parametrize("name", ["fp8_rows", "fp8_rows_f16", "fp8_block", "fp8_block_ragged"])
def test_fp8_rows_reference_vectors(V, device, name):
    q, s = TQ.quantize_fp8_rows(src_t(V, name).to(device), scale_block_size=int(V[name + ".block"]))
    assert q.dtype == torch.float8_e4m3fn
    eq(q, V[name + ".quantized"], name + " codes")
    eq(s, V[name + ".scales"], name + " scales")


@pytest.mark.parametrize("name", ["fp8_via_bf16", "fp8_via_bf16_block"])
def test_fp8_via_gpu_reference_vectors(V, device, name):
    q, s = TQ.quantize_to_fp8_via_gpu(src_t(V, name), device=device, scale_block_size=int(V[name + ".block"]))
    assert q.device.type == "cpu"
    eq(q, V[name + ".quantized"], name + " codes")
    eq(s, V[name + ".scales"], name + " scales")


@pytest.mark.parametrize("name,kw", [("mxfp4_rows", {}), ("mxfp4_rows_h32", {"hadamard": True}),
                                     ("mxfp4_rows_h64s", {"hadamard_size": 64, "signs": True}),
                                     ("mxfp4_rows_resid", {"binary_residual": True})])
def test_mxfp4_rows_reference_vectors(V, device, name, kw):
    kw = dict(kw)
    if kw.pop("signs", False):
        kw["signs"] = torch.from_numpy(V[name + ".signs"].astype(np.int16)).view(torch.bfloat16)
    p, s = TQ.quantize_mxfp4_rows(src_t(V, name).to(device), **kw)
    eq(p, V[name + ".packed"], name + " packed")
    eq(s, V[name + ".scales"], name + " scales")


@pytest.mark.parametrize("bits", [2, 1])
def test_lowbit_reference_vectors(V, bits):
    n = f"lowbit_q{bits}"
    out, sc = TQ.quantize_mxfp4_to_lowbit_cpu(torch.from_numpy(V[n + ".blocks"]), torch.from_numpy(V[n + ".scales"]),
                                              bits=bits)
    eq(out, V[n + ".packed"], n + " packed")
    eq(sc, V[n + ".out_scales"], n + " scales")
    n = f"dense_q{bits}"
    out, sc = TQ.quantize_dense_to_mxfp_lowbit_cpu(src_t(V, n), bits=bits)
    eq(out, V[n + ".packed"], n + " packed")
    eq(sc, V[n + ".out_scales"], n + " scales")


def test_ternary_reference_vectors(V):
    out, sc = TQ.quantize_mxfp4_to_ternary_cpu(torch.from_numpy(V["ternary.blocks"]),
                                               torch.from_numpy(V["ternary.scales"]))
    eq(out, V["ternary.packed"], "ternary packed")
    eq(sc, V["ternary.out_scales"], "ternary scales")


# -------------------------------------------------------------- oracle, larger inputs
def seeded(seed, rows, cols, dtype=torch.bfloat16, scale=0.05):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(rows, cols, generator=g) * scale
    x[:, ::97] *= 40.0      # outliers in every row
    return x.to(dtype)


def f32(t):
    return t.float().numpy()


@pytest.mark.parametrize("gs,dtype", [(32, torch.bfloat16), (64, torch.float16), (128, torch.bfloat16),
                                      (256, torch.float32), (512, torch.bfloat16)])
def test_int4_lsq_matches_oracle(affine_env, gs, dtype):
    affine_env(False)
    x = seeded(gs, 96, 2048 + 64, dtype)      # ragged last group for gs > 64
    p, s = TQ.quantize_to_int4_cpu(x, group_size=gs)
    wp, ws = Q.int4_lsq(f32(x), gs)
    eq(p, wp, "packed")
    eq(s, ws.view(np.uint16), "scales")


@pytest.mark.parametrize("with_rms", [False, True])
def test_int4_affine_matches_oracle(affine_env, with_rms):
    affine_env(True)
    x = seeded(5, 128, 4096)
    rms = (torch.rand(4096, generator=torch.Generator().manual_seed(6)) * 3 + 0.01) if with_rms else None
    p, s = TQ.quantize_to_int4_cpu(x, group_size=128, input_rms=rms)
    wp, ws = Q.int4_lsq_affine(f32(x), 128, rms.numpy() if with_rms else None)
    eq(p, wp, "packed")
    eq(s, ws.view(np.uint16), "scales")


@pytest.mark.parametrize("with_rms", [False, True])
def test_int4_affine_gptq_matches_oracle(affine_env, with_rms):
    """GPTQ passes at a projection-sized width against the oracle, bit for bit."""
    affine_env(True)
    rows, cols = 96, 2048
    x = seeded(8, rows, cols)
    g = torch.Generator().manual_seed(9)
    calib = torch.randn(256, cols, generator=g)
    calib = calib + 0.5 * torch.roll(calib, 1, dims=1)
    blocks = calib.reshape(256, cols // 32, 32).permute(1, 2, 0).contiguous()
    cov = torch.matmul(blocks, blocks.transpose(1, 2).contiguous()) / 256.0
    rms = (torch.rand(cols, generator=g) * 3 + 0.01) if with_rms else None
    p, s = TQ.quantize_to_int4_cpu(x, group_size=32, input_rms=rms, input_covariance32=cov)
    U = TQ.gptq_inverse_cholesky(cov).numpy()
    wp, ws = Q.int4_lsq_affine(f32(x), 32, rms.numpy() if with_rms else None, gptq_factors=U)
    eq(p, wp, "packed")
    eq(s, ws.view(np.uint16), "scales")


@pytest.mark.parametrize("block,via", [(0, False), (128, False), (96, False), (0, True), (128, True)])
def test_fp8_matches_oracle(device, block, via):
    x = seeded(7 + block, 64, 2880)
    if via:
        q, s = TQ.quantize_to_fp8_via_gpu(x, device=device, scale_block_size=block)
    else:
        q, s = TQ.quantize_fp8_rows(x.to(device), scale_block_size=block)
    wq, ws = Q.fp8_rows(f32(x), block, via_bf16=via)
    eq(q, wq, "codes")
    eq(s, ws, "scales")


@pytest.mark.parametrize("kw", [{}, {"hadamard_size": 32}, {"hadamard_size": 128, "signs": True},
                                {"hadamard_size": 512}, {"binary_residual": True}])
def test_mxfp4_rows_matches_oracle(device, kw):
    kw = dict(kw)
    x = seeded(9, 48, 2048)
    np_kw = {k: v for k, v in kw.items() if k != "signs"}
    if kw.pop("signs", False):
        sg = torch.where(torch.rand(2048, generator=torch.Generator().manual_seed(3)) < 0.5, -1.0, 1.0).to(torch.bfloat16)
        kw["signs"] = sg
        np_kw["signs"] = f32(sg)
    p, s = TQ.quantize_mxfp4_rows(x.to(device), **kw)
    wp, ws = Q.mxfp4_rows(f32(x), **np_kw)
    eq(p, wp, "packed")
    eq(s, ws, "scales")


@pytest.mark.parametrize("bits", [2, 1])
def test_lowbit_and_ternary_match_oracle(bits):
    g = torch.Generator().manual_seed(11)
    blocks = torch.randint(0, 256, (4, 360, 90, 16), generator=g, dtype=torch.int64).to(torch.uint8)
    scales = torch.randint(100, 150, (4, 360, 90), generator=g, dtype=torch.int64).to(torch.uint8)
    out, sc = TQ.quantize_mxfp4_to_lowbit_cpu(blocks, scales, bits=bits)
    wo, ws = Q.mxfp4_to_lowbit(blocks.numpy(), scales.numpy(), bits)
    eq(out, wo, "lowbit packed")
    eq(sc, ws, "lowbit scales")
    x = seeded(12 + bits, 80, 2880)
    out, sc = TQ.quantize_dense_to_mxfp_lowbit_cpu(x, bits=bits)
    wo, ws = Q.dense_to_lowbit(f32(x), bits)
    eq(out, wo, "dense packed")
    eq(sc, ws, "dense scales")
    if bits == 2:
        out, sc = TQ.quantize_mxfp4_to_ternary_cpu(blocks, scales)
        wo, _ = Q.pack_mxfp4_to_ternary(blocks.numpy(), scales.numpy())
        eq(out, wo, "ternary packed")
        assert torch.equal(sc, scales)


# -------------------------------------------------------- full layer sizes, properties
def test_int4_rows_full_size_reconstruction_bound(device, affine_env):
    """Every symmetric body-INT4 code reconstructs its weight within half a scale step
    (|x / s| <= 7 by construction, so no code is clamped), at a 14336 x 4096 layer."""
    affine_env(False)
    torch.manual_seed(0)
    x = (torch.randn(14336, 4096, device=device) * 0.02).to(torch.bfloat16)
    p, s = TQ.quantize_int4_rows(x, group_size=128)
    lo = (p & 15).to(torch.float32) - 8
    hi = (p >> 4).to(torch.float32) - 8
    codes = torch.stack([lo, hi], dim=-1).reshape(14336, 4096)
    rec = codes.reshape(14336, 32, 128) * s[:, :, None]
    err = (rec - x.float().reshape(14336, 32, 128)).abs()
    assert bool((err <= s[:, :, None] * 0.5000001).all())
    assert int(codes.abs().max()) == 7


def test_fp8_full_size_relative_error(device):
    """e4m3 keeps three significant bits: |e4m3(x/s) - x/s| <= 2^-4 |x/s| above the
    subnormal range, at a 201088 x 2880 lm_head."""
    torch.manual_seed(1)
    x = (torch.randn(201088, 2880, device=device) * 0.02).to(torch.bfloat16)
    q, s = TQ.quantize_fp8_rows(x, scale_block_size=0)
    y = x.float() / s[:, None]
    d = q.float()
    normal = y.abs() >= 2.0 ** -6
    assert bool(((d - y).abs() <= y.abs() * 2.0 ** -4 + 1e-30)[normal].all())
    assert float(d.abs().max()) == 448.0
