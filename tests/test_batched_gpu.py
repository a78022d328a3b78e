"""Batched small-M GEMM (M activation rows): below the MFMA threshold (int4 M < 4, fp8
M < 16) rows must equal the single-row operators (and the oracle) bit for bit; from
there the GEMM runs on MFMA and must match the
float64 dequantise-then-matmul reference within the north-star tolerance (max
relative error 1e-2, fp16 out, fp32 accumulate).  The M-row lm_head argmax must give
every row's token exactly."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from oracle import ref
from oracle.decode_ref import lanes
from tests.helpers import f16_normal, from_torch_bits, rng, to_torch
from tests.test_gemv_gpu import TOL, assert_bits_equal
from thintensor_amd import layouts

pytestmark = pytest.mark.gpu


def _int4_case(g, rows, cols):
    codes = g.integers(0, 16, size=(rows, cols), dtype=np.uint8)
    packed = layouts.pack_int4(codes)
    scales = (np.abs(g.standard_normal((rows, cols // 128))) * 0.02).astype(np.float16)
    return packed, scales


@pytest.mark.parametrize("m", [1, 2, 3, 4, 7, 16, 33, 64])
def test_int4_batched(backend, device, m):
    g = rng(100 + m)
    rows, cols = 1000, 5120
    packed, scales = _int4_case(g, rows, cols)
    x = f16_normal(g, (m, cols))
    out = torch.empty((m, rows), device=device, dtype=torch.float16)
    backend.int4_batched_matvec(to_torch(packed, device), to_torch(scales, device), to_torch(x, device), out)
    got = from_torch_bits(out)
    w64 = ref.int4_dequant(packed, scales, 128)
    for r in range(m):
        y64 = ref.gemv64(w64, x[r].astype(np.float64))
        assert ref.max_rel_err(got[r], y64) < TOL, f"row {r}"
        if m < 4:
            want = oracle.gemv("int4_sym", "group", packed, scales, x[r], cols=cols, lpr=lanes(cols, 4), L=4,
                               s_row=cols // 128, s_grp=1)
            assert_bits_equal(got[r], want, f"int4 batched row {r}")


def test_int4_batched_decode_shape_mfma(backend, device):
    """cfg4a shape at M = 64 through MFMA: tolerance against float64 on sampled rows,
    and close to the bit-exact single-row engine."""
    g = rng(7)
    rows, cols, m = 17920, 5120, 64
    packed, scales = _int4_case(g, rows, cols)
    x = f16_normal(g, (m, cols))
    pd, sd, xd = to_torch(packed, device), to_torch(scales, device), to_torch(x, device)
    out = torch.empty((m, rows), device=device, dtype=torch.float16)
    backend.int4_batched_matvec(pd, sd, xd, out)
    got = from_torch_bits(out)
    w64 = ref.int4_dequant(packed, scales, 128)
    for r in (0, 17, 63):
        assert ref.max_rel_err(got[r], ref.gemv64(w64, x[r].astype(np.float64))) < TOL
    one = torch.empty(rows, device=device, dtype=torch.float16)
    backend.int4_scaled_matvec(pd, sd, xd[5], one, rows=rows, cols=cols, group_size=128)
    diff = np.abs(got[5].astype(np.float64) - from_torch_bits(one).astype(np.float64))
    assert diff.max() / np.abs(from_torch_bits(one).astype(np.float64)).max() < 2e-3


@pytest.mark.parametrize("fmt,rows,cols,m", [
    ("int4", 64, 256, 16),        # two K steps over four waves: two waves hold no columns; one row per tile
    ("int4", 100, 768, 20),       # six K steps: waves take 1, 2, 1, 2 of them; ragged activation tile
    ("int4", 4000, 2048, 48),     # one 16-row tile per workgroup
    ("int4", 17920, 5120, 16),    # five tiles of 14 rows on each of 256 workgroups
    ("int4", 40000, 1024, 64),    # six full tiles per workgroup, more workgroups than CUs
    ("fp8", 100, 768, 17),
    ("fp8", 3001, 1024, 33),      # 12-row tiles, the last workgroup holding one row
    ("fp8", 9000, 4096, 64),      # three tiles of 12 rows
])
def test_batched_mfma_blocks(backend, device, fmt, rows, cols, m):
    """The MFMA path gives each workgroup a block of weight rows cut into tiles of up to
    16 rows (padding rows computed and dropped) and splits K over its four waves, whose
    partial tiles are summed in LDS.  Every output row is checked against float64, and
    a second call with 16 activation rows follows on the same buffers."""
    g = rng(rows + cols + m)
    if fmt == "int4":
        packed, scales = _int4_case(g, rows, cols)
        w64 = ref.int4_dequant(packed, scales, 128)
        wd, sd = to_torch(packed, device), to_torch(scales, device)
        call = backend.int4_batched_matvec
    else:
        bits, scales = _fp8_case(g, rows, cols)
        w64 = ref.fp8_e4m3fn(bits) * scales[:, None].astype(np.float64)
        wd, sd = torch.from_numpy(bits).to(device).view(torch.float8_e4m3fn), to_torch(scales, device)
        call = backend.scaled_batched_matvec
    for mm in (m, 16):
        x = f16_normal(g, (mm, cols))
        out = torch.empty((mm, rows), device=device, dtype=torch.float16)
        call(wd, sd, to_torch(x, device), out)
        got = from_torch_bits(out)
        y64 = x.astype(np.float64) @ w64.T
        for r in range(mm):
            assert ref.max_rel_err(got[r], y64[r]) < TOL, f"{fmt} {rows}x{cols} m={mm} row {r}"


def _fp8_case(g, rows, cols):
    bits = g.integers(0, 256, size=(rows, cols), dtype=np.uint8)
    bits[(bits & 0x7F) == 0x7F] = 0x3C          # no NaN encodings
    scales = (np.abs(g.standard_normal(rows)) * 0.01 + 1e-3).astype(np.float32)
    return bits, scales


@pytest.mark.parametrize("m", [1, 2, 4, 16, 64])
def test_fp8_batched(backend, device, m):
    g = rng(200 + m)
    rows, cols = 777, 5120
    bits, scales = _fp8_case(g, rows, cols)
    x = f16_normal(g, (m, cols))
    w = torch.from_numpy(bits).to(device).view(torch.float8_e4m3fn)
    out = torch.empty((m, rows), device=device, dtype=torch.float16)
    backend.scaled_batched_matvec(w, to_torch(scales, device), to_torch(x, device), out)
    got = from_torch_bits(out)
    w64 = ref.fp8_e4m3fn(bits) * scales[:, None].astype(np.float64)
    for r in range(m):
        assert ref.max_rel_err(got[r], ref.gemv64(w64, x[r].astype(np.float64))) < TOL, f"row {r}"
        if m < 16:
            want = oracle.gemv("fp8", "row", bits, scales, x[r], cols=cols, lpr=lanes(cols), s_row=1)
            assert_bits_equal(got[r], want, f"fp8 batched row {r}")


@pytest.mark.parametrize("m", [1, 4, 6, 8, 9, 15])
def test_lm_head_argmax_batched(backend, device, m):
    g = rng(300 + m)
    rows, cols = 20000, 5120
    w = f16_normal(g, (rows, cols), 0.02)
    x = f16_normal(g, (m, cols))
    # plant an exact tie in row 2: two identical weight rows, the lower index must win
    w[12345] = w[777]
    wd = to_torch(w, device)
    logits = torch.empty((m, rows), device=device, dtype=torch.float16)
    idx = backend.matvec_argmax_batched(wd, to_torch(x, device), logits).cpu().numpy()
    for r in range(m):
        want_logits = oracle.gemv("f16w", "none", w.view(np.uint8).reshape(rows, -1), None, x[r], cols=cols,
                                  lpr=lanes(cols))
        assert_bits_equal(from_torch_bits(logits[r]), want_logits, f"logits row {r}")
        assert idx[r] == int(oracle.lib().tto_argmax(want_logits.ctypes.data, oracle.F16, rows)), f"row {r}"
        one = int(backend.matvec_argmax_tensor(wd, to_torch(x[r], device)))
        assert idx[r] == one


def test_batched_rejects_bad_shapes(backend, device):
    g = rng(1)
    packed, scales = _int4_case(g, 64, 256)
    x = torch.zeros((65, 256), device=device, dtype=torch.float16)
    out = torch.empty((65, 64), device=device, dtype=torch.float16)
    with pytest.raises(ValueError):
        backend.int4_batched_matvec(to_torch(packed, device), to_torch(scales, device), x, out)
