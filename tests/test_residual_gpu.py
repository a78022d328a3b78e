"""Residual sidecar corrections on the GPU against the oracle (oracle/residual.py).

Bit-exact against the oracle's restatement of the kernels' order, applied on top of a
previous output in fp16/bf16/fp32, and within 1e-2 of the float64 sum; int32 and
int64 indices, a strided values view, more than 64 terms, rows that are not a
multiple of four, an out-of-range index (NaN row), fp16/fp32 scales, K = 32, 2880 and
5120, and the reference's shape errors.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import ref
from oracle import residual as R
from tests.helpers import bf16_bits, bf16_to_f32, from_torch_bits, rng, to_torch

pytestmark = pytest.mark.gpu


def _out(device, prev32, out_dtype):
    import torch

    if out_dtype == "f16":
        return to_torch(prev32.astype(np.float16), device), prev32.astype(np.float16).astype(np.float32)
    if out_dtype == "bf16":
        b = bf16_bits(prev32)
        return to_torch(b.view(np.int16), device, bf16=True), bf16_to_f32(b)
    return to_torch(prev32.astype(np.float32), device), prev32.astype(np.float32)


def _check(out_t, base32, corr32, out_dtype):
    want = base32 + corr32
    if out_dtype == "f16":
        assert np.array_equal(from_torch_bits(out_t).view(np.uint16), want.astype(np.float16).view(np.uint16))
    elif out_dtype == "bf16":
        assert np.array_equal(from_torch_bits(out_t), bf16_bits(want))
    else:
        got = out_t.cpu().numpy()
        assert np.array_equal(got.view(np.uint32), want.astype(np.float32).view(np.uint32))


@pytest.mark.parametrize("rows,terms,cols,idx_dtype,vdt,out_dtype,strided", [
    (2880, 16, 2880, "int64", "f16", "f16", False),
    (77, 150, 5120, "int32", "f32", "f32", True),
    (5, 1, 32, "int64", "bf16", "bf16", False),
    (5120, 32, 17920, "int16", "f16", "f16", False),  # the reference runtime's int16 sidecar indices
    (300, 70, 2880, "int16", "bf16", "f32", True),
])
def test_sparse_residual_matches_oracle(backend, device, rows, terms, cols, idx_dtype, vdt, out_dtype, strided):
    import torch

    g = rng(rows + terms)
    vals = g.standard_normal((rows, terms)).astype(np.float32) * 0.1
    idx = g.integers(0, cols, size=(rows, terms))
    x = g.standard_normal(cols).astype(np.float16)
    if vdt == "f16":
        v16 = vals.astype(np.float16)
        vt, v32 = to_torch(v16, device), v16.astype(np.float32)
    elif vdt == "bf16":
        b = bf16_bits(vals)
        vt, v32 = to_torch(b.view(np.int16), device, bf16=True), bf16_to_f32(b)
    else:
        vt, v32 = to_torch(vals, device), vals
    if strided:
        big = torch.zeros((rows, 2 * terms), device=device, dtype=vt.dtype)
        big[:, ::2] = vt
        vt = big[:, ::2]
    it = torch.from_numpy(idx.astype({"int16": np.int16, "int32": np.int32, "int64": np.int64}[idx_dtype])).to(device)
    out_t, base = _out(device, g.standard_normal(rows).astype(np.float32), out_dtype)
    print(f"sparse residual rows={rows} terms={terms} cols={cols}", flush=True)
    backend.sparse_residual_matvec(vt, it, to_torch(x, device), out_t)
    torch.cuda.synchronize()
    corr = R.sparse_residual(v32, idx, x.astype(np.float32))
    _check(out_t, base, corr, out_dtype)
    exact = np.array([np.dot(v32[m].astype(np.float64), x.astype(np.float64)[idx[m]]) for m in range(rows)])
    assert ref.max_rel_err(corr, exact) < 1e-2


def test_sparse_residual_bad_index_is_nan(backend, device):
    import torch

    g = rng(41)
    vals = g.standard_normal((9, 8)).astype(np.float32)
    idx = g.integers(0, 64, size=(9, 8))
    idx[4, 7] = 64
    out = torch.zeros(9, device=device, dtype=torch.float32)
    backend.sparse_residual_matvec(to_torch(vals, device), torch.from_numpy(idx).to(device),
                                   to_torch(g.standard_normal(64).astype(np.float16), device), out)
    got = out.cpu().numpy()
    assert np.isnan(got[4]) and not np.any(np.isnan(np.delete(got, 4)))


@pytest.mark.parametrize("rows,cols,sdt,out_dtype", [
    (2880, 2880, "f16", "f16"), (301, 5120, "f32", "f32"), (3, 32, "f16", "bf16"), (64, 8192, "bf16", "f32"),
])
def test_binary_residual_matches_oracle(backend, device, rows, cols, sdt, out_dtype):
    import torch

    g = rng(rows + cols + 7)
    signs = g.integers(0, 256, size=(rows, cols // 8)).astype(np.uint8)
    sc = np.abs(g.standard_normal((rows, cols // 32))).astype(np.float32) * 0.01
    if sdt == "f16":
        s16 = sc.astype(np.float16)
        st, s32 = to_torch(s16, device), s16.astype(np.float32)
    elif sdt == "bf16":
        b = bf16_bits(sc)
        st, s32 = to_torch(b.view(np.int16), device, bf16=True), bf16_to_f32(b)
    else:
        st, s32 = to_torch(sc, device), sc
    x = g.standard_normal(cols).astype(np.float16)
    out_t, base = _out(device, g.standard_normal(rows).astype(np.float32), out_dtype)
    print(f"binary residual rows={rows} cols={cols}", flush=True)
    backend.binary_residual_matvec(to_torch(signs, device), st, to_torch(x, device), out_t)
    torch.cuda.synchronize()
    corr = R.binary_residual(signs, s32, x.astype(np.float32))
    _check(out_t, base, corr, out_dtype)
    bits = np.unpackbits(signs, axis=1, bitorder="little").astype(np.float64)
    w = (2.0 * bits - 1.0) * np.repeat(s32.astype(np.float64), 32, axis=1)
    assert ref.max_rel_err(corr, w @ x.astype(np.float64)) < 1e-2


def test_residual_shape_errors(backend, device):
    import torch

    x = torch.zeros(64, device=device, dtype=torch.float16)
    out = torch.zeros(4, device=device, dtype=torch.float16)
    with pytest.raises(ValueError, match="sparse residual values/indices shape mismatch"):
        backend.sparse_residual_matvec(torch.zeros((4, 3), device=device, dtype=torch.float16),
                                       torch.zeros((4, 2), device=device, dtype=torch.int64), x, out)
    with pytest.raises(ValueError, match="binary residual sign plane shape mismatch"):
        backend.binary_residual_matvec(torch.zeros((4, 7), device=device, dtype=torch.uint8),
                                       torch.zeros((4, 2), device=device, dtype=torch.float16), x, out)
    with pytest.raises(ValueError, match="binary residual scale shape mismatch"):
        backend.binary_residual_matvec(torch.zeros((4, 8), device=device, dtype=torch.uint8),
                                       torch.zeros((4, 3), device=device, dtype=torch.float16), x, out)
