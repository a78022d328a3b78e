"""Ternary selected-expert GEMV on the GPU against the oracle.

Bit-exact against the oracle's restatement of the kernel's summation order
(oracle/ternary.py), and within the north-star tolerance (max relative error 1e-2)
of the reference's dequantise-then-matmul in float64.  Cases: the gpt-oss expert
shapes (gate/up 5760 x 2880, down 2880 x 2880), one 32-column group (rows of eight
bytes, reads clamped at the buffer end), a partial last 160-column chunk, K = 5120
and 8192 (52 chunks per row), per-slot activations, bf16 inputs, fp16/bf16/fp32
outputs, weights packed from MXFP4 by the reference's packer, and ids outside the
expert range (NaN rows).
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import ref
from oracle import ternary as T
from tests.helpers import bf16_bits, bf16_to_f32, from_torch_bits, rng, to_torch

pytestmark = pytest.mark.gpu


def _random_packed(g, experts, rows, cols):
    groups, tb, mb = T.ternary_geometry(cols)
    packed = g.integers(0, 256, size=(experts, rows, tb + mb)).astype(np.uint8)
    scales = g.integers(118, 128, size=(experts, rows, groups)).astype(np.uint8)
    return packed, scales


def _run(backend, device, packed, scales, x_vals, idx, *, x_bf16=False, out_dtype="f16"):
    import torch

    if x_bf16:
        xb = bf16_bits(x_vals)
        xt = to_torch(xb.view(np.int16), device, bf16=True)
        x32 = bf16_to_f32(xb)
    else:
        xh = x_vals.astype(np.float16)
        xt = to_torch(xh, device)
        x32 = xh.astype(np.float32)
    rows = packed.shape[1]
    tdt = {"f16": torch.float16, "bf16": torch.bfloat16, "f32": torch.float32}[out_dtype]
    out = torch.empty((len(idx), rows), device=device, dtype=tdt)
    ids = torch.tensor(np.asarray(idx, dtype=np.int32), device=device)
    backend.mxfp_ternary_selected_tensorcore_matvec(to_torch(packed, device), to_torch(scales, device), xt, ids, out)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    want32 = T.ternary_selected_gemv(packed, scales, x32, np.asarray(idx))
    if out_dtype == "f16":
        want_bits = want32.astype(np.float16)
        assert np.array_equal(from_torch_bits(out).view(np.uint16), want_bits.view(np.uint16))
    elif out_dtype == "bf16":
        assert np.array_equal(from_torch_bits(out), bf16_bits(want32))
    else:
        assert np.array_equal(got.view(np.uint32), want32.view(np.uint32))
    return got, x32


def _check_tolerance(got, packed, scales, x32, idx):
    cols = scales.shape[-1] * 32
    xs = np.broadcast_to(x32, (len(idx), cols)) if x32.ndim == 1 else x32
    for i, e in enumerate(idx):
        if 0 <= e < packed.shape[0]:
            w = T.ternary_dequant(packed[e], scales[e])
            assert ref.max_rel_err(got[i], w @ xs[i].astype(np.float64)) < 1e-2


@pytest.mark.parametrize(
    "experts,rows,cols,sel,per_slot,x_bf16,out_dtype",
    [
        (8, 5760, 2880, 4, False, False, "f16"),     # gpt-oss gate/up, shared x
        (8, 2880, 2880, 4, True, False, "f16"),      # gpt-oss down, per-slot x
        (2, 3, 32, 2, False, False, "f32"),          # one group, eight-byte rows
        (3, 77, 1056, 3, True, True, "f32"),         # partial last chunk, bf16 x
        (2, 300, 5120, 2, False, True, "bf16"),      # 32 chunks
        (2, 64, 8192, 2, True, False, "f16"),        # 52 chunks per row
    ],
)
def test_ternary_selected_matches_oracle(backend, device, experts, rows, cols, sel, per_slot, x_bf16, out_dtype):
    g = rng(rows + cols)
    packed, scales = _random_packed(g, experts, rows, cols)
    idx = g.permutation(experts)[:sel].tolist()
    shape = (sel, cols) if per_slot else (cols,)
    x = g.standard_normal(shape).astype(np.float32)
    print(f"ternary case E={experts} rows={rows} cols={cols} sel={sel}", flush=True)
    got, x32 = _run(backend, device, packed, scales, x, idx, x_bf16=x_bf16, out_dtype=out_dtype)
    _check_tolerance(got, packed, scales, x32, idx)


def test_ternary_from_mxfp4_packer(backend, device):
    """Weights packed from MXFP4 by the reference's packer (restated in the oracle)."""
    g = rng(21)
    experts, rows, groups = 4, 256, 90
    codes = g.integers(0, 16, size=(experts, rows, groups, 32)).astype(np.uint8)
    blocks = (codes[..., 0::2] | (codes[..., 1::2] << 4)).astype(np.uint8)
    scales = g.integers(120, 126, size=(experts, rows, groups)).astype(np.uint8)
    packed, scales = T.pack_mxfp4_to_ternary(blocks, scales)
    x = g.standard_normal(groups * 32).astype(np.float32)
    got, x32 = _run(backend, device, packed, scales, x, [3, 1], out_dtype="f32")
    _check_tolerance(got, packed, scales, x32, [3, 1])


def test_ternary_exact_integer_inputs(backend, device):
    """Integer activations and scales >= 1: every order gives the float64 sum exactly."""
    g = rng(22)
    experts, rows, cols = 3, 129, 2880
    packed, _ = _random_packed(g, experts, rows, cols)
    scales = g.integers(127, 130, size=(experts, rows, cols // 32)).astype(np.uint8)
    x = g.integers(-4, 5, size=cols).astype(np.float32)
    got, _ = _run(backend, device, packed, scales, x, [2, 0, 1], out_dtype="f32")
    for i, e in enumerate([2, 0, 1]):
        w = T.ternary_dequant(packed[e], scales[e])
        assert np.array_equal(got[i].astype(np.float64), w @ x.astype(np.float64))


def test_ternary_invalid_expert_rows_are_nan(backend, device):
    g = rng(23)
    packed, scales = _random_packed(g, 2, 50, 320)
    x = g.standard_normal(320).astype(np.float32)
    got, _ = _run(backend, device, packed, scales, x, [1, 7, -1], out_dtype="f32")
    assert np.all(np.isnan(got[1])) and np.all(np.isnan(got[2])) and not np.any(np.isnan(got[0]))


def test_ternary_shape_errors(backend, device):
    import torch

    g = rng(24)
    packed, scales = _random_packed(g, 2, 8, 320)
    p = to_torch(packed, device)
    s = to_torch(scales, device)
    x = torch.zeros(320, device=device, dtype=torch.float16)
    ids = torch.zeros(1, device=device, dtype=torch.int32)
    with pytest.raises(ValueError, match="ternary weight shape mismatch"):
        backend.mxfp_ternary_selected_tensorcore_matvec(p[:, :, :-1], s, x, ids, torch.empty((1, 8), device=device, dtype=torch.float16))
    with pytest.raises(ValueError, match="ternary output must be"):
        backend.mxfp_ternary_selected_tensorcore_matvec(p, s, x, ids, torch.empty((2, 8), device=device, dtype=torch.float16))
    with pytest.raises(ValueError, match="ternary input must be"):
        backend.mxfp_ternary_selected_tensorcore_matvec(p, s, x[:100], ids, torch.empty((1, 8), device=device, dtype=torch.float16))
