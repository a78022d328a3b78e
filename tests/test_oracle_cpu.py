"""CPU checks that pin the oracle: conversions against library routines, decoders
against the reference tables, binary32 restatements against float64 closed forms
and exact (order-independent) cases, and the int4 path against torch's CPU int4 op
that the reference's CPU path calls (gpu_runtime.py:3204-3230)."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import oracle
from oracle import ref
from tests.helpers import bf16_bits, f16_normal, rng
from thintensor_amd import layouts


def test_f16_conversion_matches_numpy():
    g = rng(0)
    vals = np.concatenate([
        g.standard_normal(200000).astype(np.float32) * np.float32(2.0) ** g.integers(-30, 20, 200000).astype(np.float32),
        np.array([65504, 65519.99, 65520, 65536, 1e-8, 5.96e-8, 2.98e-8, 2.99e-8, -0.0, 0.0, np.inf, -np.inf],
                 dtype=np.float32),
    ])
    # halfway cases between neighbouring fp16 values
    h = np.arange(0, 0x7bff, dtype=np.uint16).view(np.float16).astype(np.float32)
    mid = ((h[:-1].astype(np.float64) + h[1:].astype(np.float64)) / 2).astype(np.float32)
    vals = np.concatenate([vals, mid, -mid])
    got = np.array([oracle.f32_to_f16_bits(float(v)) for v in vals[::7]], dtype=np.uint16)
    want = vals[::7].astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


def test_fp8_decoder_matches_torch():
    bits = np.arange(256, dtype=np.uint8)
    t = torch.from_numpy(bits).view(torch.float8_e4m3fn).to(torch.float32).numpy()
    mine = ref.fp8_e4m3fn(bits)
    assert np.array_equal(np.isnan(t), np.isnan(mine))
    ok = ~np.isnan(t)
    assert np.array_equal(t[ok].astype(np.float64), mine[ok])


@pytest.mark.parametrize("smode", ["row", "group"])
def test_int8_emulation_exact_on_integer_inputs(smode):
    """int8 rows (the reference reads them with .to(fp32), triton_kernels.py:554-560):
    integer activations and power-of-two scales make every partial sum exact, so the
    binary32 restatement must equal the float64 closed form over torch's own int8
    conversion; reading the bytes as unsigned (a plausible decode mistake) must not."""
    from oracle.decode_ref import lanes

    g = rng(11)
    rows, cols, block = 40, 1024, 128
    q = g.integers(-128, 128, size=(rows, cols), dtype=np.int8)
    x = g.integers(-4, 5, size=cols).astype(np.float16)
    w64 = torch.from_numpy(q).to(torch.float64).numpy()
    if smode == "row":
        s = (2.0 ** g.integers(-8, 0, size=rows)).astype(np.float32)
        got = oracle.gemv("int8", "row", q.view(np.uint8), s, x, cols=cols, lpr=lanes(cols), s_row=1,
                          odtype=oracle.F32)
        scale = s[:, None].astype(np.float64)
    else:
        s = (2.0 ** g.integers(-8, 0, size=(rows, cols // block))).astype(np.float32)
        L = block // 32
        got = oracle.gemv("int8", "group", q.view(np.uint8), s, x, cols=cols, lpr=lanes(cols, L), L=L,
                          s_row=cols // block, s_grp=1, odtype=oracle.F32)
        scale = np.repeat(s.astype(np.float64), block, axis=1)
    assert np.array_equal(got.astype(np.float64), ref.gemv64(w64 * scale, x))
    unsigned = q.view(np.uint8).astype(np.float64)
    assert not np.array_equal(got.astype(np.float64), ref.gemv64(unsigned * scale, x))


def test_e2m1_and_lowbit_tables():
    # e2m1: value = (-1)^s * 2^(e-1) * (1 + m/2) for e > 0, m/2 for e == 0 (OCP MX v1.0)
    for code in range(16):
        s, e, m = code >> 3, (code >> 1) & 3, code & 1
        v = (m * 0.5) if e == 0 else (2.0 ** (e - 1)) * (1 + m / 2)
        assert ref.E2M1[code] == (-v if s else v)
    assert list(ref.Q2_LUT) == [-1.5, -0.5, 0.5, 1.5]


def test_packers_roundtrip_and_bit_positions():
    g = rng(1)
    c4 = g.integers(0, 16, size=(3, 64), dtype=np.uint8)
    p = layouts.pack_int4(c4)
    assert np.array_equal(layouts.unpack_int4(p), c4)
    assert p[0, 0] == (c4[0, 0] | (c4[0, 1] << 4))
    # uint32 view: nibble j of word w is element 8w + j
    u = layouts.int4_as_u32(p)
    assert all(((int(u[1, 2]) >> (4 * j)) & 15) == c4[1, 16 + j] for j in range(8))
    for bits in (1, 2):
        c = g.integers(0, 1 << bits, size=(2, 96), dtype=np.uint8)
        pb = layouts.pack_bits(c, bits)
        assert np.array_equal(layouts.unpack_bits(pb, bits), c)
        i = 37
        assert (pb[1, i * bits // 8] >> ((i * bits) % 8)) & ((1 << bits) - 1) == c[1, i]


@pytest.mark.parametrize("cols,group,lpr", [(256, 128, 64), (512, 64, 32), (2048, 2048, 64), (160 * 32, 128, 32)])
def test_int4_emulation_exact_on_integer_inputs(cols, group, lpr):
    """Integer activations and power-of-two scales make every partial sum exact, so
    the binary32 emulation must equal the float64 closed form whatever the order."""
    g = rng(cols + group)
    rows = 40
    codes = g.integers(0, 16, size=(rows, cols), dtype=np.uint8)
    packed = layouts.pack_int4(codes)
    groups = max(cols // group, 1)
    scales = (2.0 ** g.integers(-6, 0, size=(rows, groups))).astype(np.float16)
    x = g.integers(-4, 5, size=cols).astype(np.float16)
    L = 1 if group >= cols else group // 32
    got = oracle.gemv("int4_sym", "row" if group >= cols else "group", packed, scales, x, cols=cols, lpr=lpr, L=L,
                      s_row=groups, s_grp=1, odtype=oracle.F32)
    want = ref.gemv64(ref.int4_dequant(packed, scales, group), x)
    assert np.array_equal(got.astype(np.float64), want)


def test_int4_emulation_close_to_closed_form_and_planted_error_caught():
    g = rng(3)
    rows, cols, group = 64, 2048, 128
    codes = g.integers(0, 16, size=(rows, cols), dtype=np.uint8)
    packed = layouts.pack_int4(codes)
    scales = (np.abs(g.standard_normal((rows, cols // group))) * 0.02).astype(np.float16)
    x = f16_normal(g, cols)
    got = oracle.gemv("int4_sym", "group", packed, scales, x, cols=cols, lpr=64, L=4, s_row=16, s_grp=1,
                      odtype=oracle.F32)
    want = ref.gemv64(ref.int4_dequant(packed, scales, group), x)
    assert ref.max_rel_err(got, want) < 1e-5
    # a wrong nibble order (a plausible packing mistake) must be visible to this check
    swapped = ((packed >> 4) | (packed << 4)).astype(np.uint8)
    bad = oracle.gemv("int4_sym", "group", swapped, scales, x, cols=cols, lpr=64, L=4, s_row=16, s_grp=1,
                      odtype=oracle.F32)
    assert ref.max_rel_err(bad, want) > 1e-2


def test_int4_closed_form_matches_reference_cpu_op():
    """The reference's CPU path: torch.ops.aten._weight_int4pack_mm_for_cpu with
    scale_zeros bf16 [G, N, 2] = (s, 0) and w = (q - 8) * s + z (gpu_runtime.py:3107-3149)."""
    g = rng(4)
    rows, cols, group = 64, 256, 128
    codes = g.integers(0, 16, size=(rows, cols), dtype=np.uint8)
    packed = layouts.pack_int4(codes)
    scales = (np.abs(g.standard_normal((rows, cols // group))) * 0.02).astype(np.float16)
    x = f16_normal(g, cols)
    w_int = torch.from_numpy(codes.astype(np.int32))
    packed_cpu = torch.ops.aten._convert_weight_to_int4pack_for_cpu(w_int, 1)
    sz = torch.zeros((cols // group, rows, 2), dtype=torch.bfloat16)
    sz[:, :, 0] = torch.from_numpy(scales.astype(np.float32)).t().to(torch.bfloat16)
    xb = torch.from_numpy(x.astype(np.float32)).to(torch.bfloat16).reshape(1, cols)
    y_ref = torch.ops.aten._weight_int4pack_mm_for_cpu(xb, packed_cpu, group, sz).float().numpy().reshape(-1)
    s_bf = sz[:, :, 0].t().float().numpy()
    w64 = ref.int4_dequant(packed, s_bf, group)
    y64 = ref.gemv64(w64, xb.float().numpy().reshape(-1))
    assert ref.max_rel_err(y_ref, y64) < 1e-2


def test_mxfp4_and_lowbit_emulation_vs_closed_form():
    g = rng(6)
    rows, cols = 48, 2880
    codes = g.integers(0, 16, size=(1, rows, cols), dtype=np.uint8)
    blocks = layouts.pack_mxfp4_blocks(codes)[0]
    scales = g.integers(119, 124, size=(rows, cols // 32), dtype=np.uint8)
    x = f16_normal(g, cols)
    got = oracle.gemv("mxfp4", "block_e8", blocks.reshape(rows, -1), scales, x, cols=cols, lpr=32, s_row=cols // 32,
                      odtype=oracle.F32)
    assert ref.max_rel_err(got, ref.gemv64(ref.mxfp4_dequant(blocks, scales), x)) < 1e-5
    for bits in (1, 2):
        c = g.integers(0, 1 << bits, size=(1, rows, cols), dtype=np.uint8)
        pk = layouts.pack_lowbit_blocks(c, bits)[0]
        got = oracle.gemv("q2e8" if bits == 2 else "q1e8", "block_e8", pk.reshape(rows, -1), scales, x, cols=cols,
                          lpr=32, s_row=cols // 32, odtype=oracle.F32)
        assert ref.max_rel_err(got, ref.gemv64(ref.lowbit_e8_dequant(pk, scales, bits), x)) < 1e-5


def test_affine_lowbit_emulation_vs_closed_form():
    g = rng(7)
    rows, cols, group = 32, 1024, 64
    for bits in (1, 2):
        codes = g.integers(0, 1 << bits, size=(rows, cols), dtype=np.uint8)
        packed = layouts.pack_bits(codes, bits)
        sz = np.stack([np.abs(g.standard_normal((rows, cols // group))) * 0.05,
                       g.uniform(0, (1 << bits) - 1, size=(rows, cols // group))], axis=-1).astype(np.float16)
        x = f16_normal(g, cols)
        got = oracle.gemv("q2aff" if bits == 2 else "q1aff", "group_aff", packed, sz, x, cols=cols, lpr=32, L=2,
                          s_row=sz.shape[1] * 2, s_grp=2, s_pair=1, aff_zero=1, odtype=oracle.F32)
        assert ref.max_rel_err(got, ref.gemv64(ref.lowbit_affine_dequant(packed, sz, bits, group, cols), x)) < 1e-4


def test_exp_restatement_accuracy():
    xs = np.linspace(-87.0, 88.0, 20011)
    worst = 0.0
    for v in xs[::3]:
        f = float(np.float32(v))
        got = oracle.exp_f32(f)
        want = math.exp(f)
        worst = max(worst, abs(got - want) / want)
    assert worst < 3 * 2.0 ** -23
    assert oracle.exp_f32(-100.0) == 0.0 and math.isinf(oracle.exp_f32(100.0))
