"""GPU parity of the int8 weight rows of the scaled GEMV family: scaled_matvec (per-row
and per-block scales), multi_scaled_tensorcore_matvec, split_k_matvec and
fused_scaled_gate_up_silu.  The reference kernels read int8 rows with .to(fp32)
(triton_kernels.py:539-592, :1958-2071, :3023-3100, :3113-3152, :3243-3350), and the
runtime quantises rowwise int8 pages as round(w / s) clamped to +-127 with
s = amax / 127 (gpu_runtime.py:1037-1078).  Each output is checked bit for bit against
the CPU oracle and within TOL = 1e-2 (max relative error) of the float64 closed form."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from oracle import ref
from oracle.decode_ref import lanes
from tests.helpers import bf16_bits, bf16_to_f32, from_torch_bits, rng, to_torch
from tests.test_fp8_ops_gpu import act
from tests.test_gemv_gpu import assert_bits_equal

pytestmark = pytest.mark.gpu

TOL = 1e-2
ODT = {"f16": (torch.float16, oracle.F16), "bf16": (torch.bfloat16, oracle.BF16), "f32": (torch.float32, oracle.F32)}


def int8_weights(g, rows, cols, block=0):
    """Rowwise (or per row block) int8 codes and fp32 scales as the reference loader makes
    them: s = max(amax, 1e-12) / 127, q = clamp(round(w / s), -127, 127)."""
    src = torch.from_numpy((g.standard_normal((rows, cols)) * 0.05).astype(np.float32))
    width = block or cols
    nb = -(-cols // width)
    scales = torch.empty((rows, nb), dtype=torch.float32)
    q = torch.empty((rows, cols), dtype=torch.int8)
    for b in range(nb):
        blk = src[:, b * width:(b + 1) * width]
        s = blk.abs().amax(dim=1).clamp_min(1e-12) / 127.0
        scales[:, b] = s
        q[:, b * width:(b + 1) * width] = torch.round(blk / s[:, None]).clamp(-127, 127).to(torch.int8)
    if not block:
        scales = scales[:, 0].contiguous()
    return q.numpy(), scales.numpy()


def deq64(q, s, block=0):
    w = q.astype(np.float64)
    if s.ndim == 1:
        return w * s[:, None].astype(np.float64)
    return w * np.repeat(s.astype(np.float64), block, axis=1)[:, :q.shape[1]]


def dev_i8(q, device):
    return torch.from_numpy(q).to(device)


@pytest.mark.parametrize("rows,cols,bf16,odt", [
    (1000, 5120, False, "f16"),
    (4096, 2048, True, "bf16"),
    (130, 2880, False, "f32"),
])
def test_int8_scaled_matvec(backend, device, rows, cols, bf16, odt):
    g = rng(rows + cols + 8)
    q, s = int8_weights(g, rows, cols)
    xb, x32 = act(g, cols, bf16)
    out = torch.empty(rows, device=device, dtype=ODT[odt][0])
    backend.scaled_matvec(dev_i8(q, device), to_torch(s, device), to_torch(xb, device, bf16=bf16), out)
    got = from_torch_bits(out)
    want = oracle.gemv("int8", "row", q.view(np.uint8), s, xb, cols=cols, lpr=lanes(cols), s_row=1,
                       odtype=ODT[odt][1])
    assert_bits_equal(got, want, f"int8 scaled {rows}x{cols}")
    assert ref.max_rel_err(ref.f64(got), ref.gemv64(deq64(q, s), x32)) < TOL


@pytest.mark.parametrize("rows,cols,block,bf16", [
    (2880, 2880, 128, False),   # ragged last block
    (1000, 2048, 32, True),
    (512, 4096, 1024, False),   # generic engine
    (768, 2048, 2048, True),    # one block per row
])
def test_int8_block_scaled_matvec(backend, device, rows, cols, block, bf16):
    g = rng(rows + cols + block + 8)
    q, s = int8_weights(g, rows, cols, block)
    xb, x32 = act(g, cols, bf16)
    out = torch.empty(rows, device=device, dtype=torch.bfloat16 if bf16 else torch.float16)
    backend.scaled_matvec(dev_i8(q, device), to_torch(s, device), to_torch(xb, device, bf16=bf16), out)
    got = from_torch_bits(out)
    odt = oracle.BF16 if bf16 else oracle.F16
    if block >= cols:
        want = oracle.gemv("int8", "row", q.view(np.uint8), s[:, 0].copy(), xb, cols=cols, lpr=lanes(cols), s_row=1,
                           odtype=odt)
    else:
        L = block // 32
        want = oracle.gemv("int8", "group", q.view(np.uint8), s, xb, cols=cols, lpr=lanes(cols, L), L=L,
                           s_row=s.shape[1], s_grp=1, odtype=odt)
    assert_bits_equal(got, want, f"int8 block-scaled {rows}x{cols}/{block}")
    assert ref.max_rel_err(ref.f64(got), ref.gemv64(deq64(q, s, block), x32)) < TOL


@pytest.mark.parametrize("cols,bf16", [(2048, True), (5120, False)])
def test_int8_multi_scaled_tensorcore_matvec(backend, device, cols, bf16):
    """The runtime's int8 QKV / gate-up call (gpu_runtime.py:11851-11873)."""
    g = rng(cols + 9)
    rows = (2048, 512, 512)
    mats = [int8_weights(g, r, cols) for r in rows]
    xb, x32 = act(g, cols, bf16)
    out = torch.empty(sum(rows), device=device, dtype=torch.bfloat16 if bf16 else torch.float16)
    backend.multi_scaled_tensorcore_matvec(tuple(dev_i8(q, device) for q, _ in mats),
                                           tuple(to_torch(s, device) for _, s in mats), rows, cols,
                                           to_torch(xb, device, bf16=bf16), out)
    got = from_torch_bits(out)
    r0 = 0
    for (q, s), r in zip(mats, rows):
        want = oracle.gemv("int8", "row", q.view(np.uint8), s, xb, cols=cols, lpr=lanes(cols), s_row=1,
                           odtype=oracle.BF16 if bf16 else oracle.F16)
        assert_bits_equal(got[r0:r0 + r], want, f"int8 matrix at row {r0}")
        assert ref.max_rel_err(ref.f64(got[r0:r0 + r]), ref.gemv64(deq64(q, s), x32)) < TOL
        r0 += r
    # one dtype for all matrices, as the reference requires
    fp8 = torch.zeros((rows[1], cols), device=device, dtype=torch.float8_e4m3fn)
    with pytest.raises(ValueError, match="share one dtype"):
        backend.multi_scaled_tensorcore_matvec((dev_i8(mats[0][0], device), fp8),
                                               tuple(to_torch(s, device) for _, s in mats[:2]), rows[:2], cols,
                                               to_torch(xb, device, bf16=bf16), out)


@pytest.mark.parametrize("rows,cols,split_k", [(2048, 8192, 2), (1024, 5120, 4)])
def test_int8_split_k_matvec(backend, device, rows, cols, split_k):
    """The runtime's split-K down projection with a rowwise int8 page (gpu_runtime.py:12292-12309)."""
    g = rng(rows + cols + split_k + 8)
    q, s = int8_weights(g, rows, cols)
    xb, x32 = act(g, cols, False)
    out = torch.empty(rows, device=device, dtype=torch.float16)
    backend.split_k_matvec(dev_i8(q, device), to_torch(xb, device), out, scales=to_torch(s, device), split_k=split_k)
    got = from_torch_bits(out)
    want = oracle.split_k_gemv("int8", q.view(np.uint8), xb, split_k, scales=s, odtype=oracle.F16)
    assert_bits_equal(got, want, f"int8 split-K {rows}x{cols}/{split_k}")
    assert ref.max_rel_err(ref.f64(got), ref.gemv64(deq64(q, s), x32)) < TOL


@pytest.mark.parametrize("rows,cols,bf16", [(8192, 2048, True), (100, 2880, False)])
def test_int8_fused_scaled_gate_up_silu(backend, device, rows, cols, bf16):
    """The adaptive int8 body's fused MLP (gate_up_fp8 covers int8 bodies, gpu_runtime.py:4990-4996, 11642)."""
    g = rng(rows + cols + 10)
    qg, sg = int8_weights(g, rows, cols)
    qu, su = int8_weights(g, rows, cols)
    xb, x32 = act(g, cols, bf16)
    out = torch.empty(rows, device=device, dtype=torch.bfloat16 if bf16 else torch.float16)
    backend.fused_scaled_gate_up_silu(dev_i8(qg, device), to_torch(sg, device), dev_i8(qu, device),
                                      to_torch(su, device), to_torch(xb, device, bf16=bf16), out)
    got = from_torch_bits(out)
    gate = oracle.gemv("int8", "row", qg.view(np.uint8), sg, xb, cols=cols, lpr=lanes(cols), s_row=1,
                       odtype=oracle.F32)
    up = oracle.gemv("int8", "row", qu.view(np.uint8), su, xb, cols=cols, lpr=lanes(cols), s_row=1, odtype=oracle.F32)
    gate, up = bf16_to_f32(bf16_bits(gate)), bf16_to_f32(bf16_bits(up))
    prod = np.empty(rows, dtype=np.float32)
    oracle.lib().tto_silu_mul(gate.ctypes.data, up.ctypes.data, prod.ctypes.data, oracle.F32, rows)
    want = bf16_bits(prod) if bf16 else prod.astype(np.float16)
    assert_bits_equal(got, want, f"int8 gate/up SiLU {rows}x{cols}")
    g64 = ref.bf16_round64(ref.gemv64(qg.astype(np.float64), x32) * sg)
    u64 = ref.bf16_round64(ref.gemv64(qu.astype(np.float64), x32) * su)
    assert ref.max_rel_err(ref.f64(got), ref.silu_mul64(g64, u64)) < TOL
    with pytest.raises(ValueError, match="share a dtype"):
        backend.fused_scaled_gate_up_silu(dev_i8(qg, device), to_torch(sg, device),
                                          torch.zeros((rows, cols), device=device, dtype=torch.float8_e4m3fn),
                                          to_torch(su, device), to_torch(xb, device, bf16=bf16), out)


def test_scaled_matvec_rejects_other_byte_dtypes(backend, device):
    w = torch.zeros((64, 256), device=device, dtype=torch.uint8)
    s = torch.ones(64, device=device)
    x = torch.zeros(256, device=device, dtype=torch.float16)
    out = torch.empty(64, device=device, dtype=torch.float16)
    with pytest.raises(ValueError, match="float8_e4m3fn and int8"):
        backend.scaled_matvec(w, s, x, out)
