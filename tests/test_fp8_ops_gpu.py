"""GPU parity of the fp8 operator family beyond the per-row GEMV (block-scaled
scaled_matvec, multi_scaled_tensorcore_matvec, fused_scaled_gate_up_silu), the split-K
GEMV and the per-head norms (head_rms_norm, qk_head_rmsnorm_rope_inplace): bit for bit
against the CPU oracle and within the north-star tolerance TOL = 1e-2 (max relative
error) of the float64 closed forms in oracle/ref.py."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from oracle import ref
from oracle.decode_ref import lanes
from tests.helpers import bf16_bits, bf16_to_f32, f16_normal, from_torch_bits, rng, to_torch
from tests.test_gemv_gpu import assert_bits_equal

pytestmark = pytest.mark.gpu

TOL = 1e-2


def fp8_weights(g, rows, cols, block=0):
    """float8_e4m3fn weights quantised as the reference runtime does (amax / 448 per row
    or per row block, gpu_runtime.py:6553-6607), as (uint8 bits, fp32 scales)."""
    src = torch.from_numpy((g.standard_normal((rows, cols)) * 0.05).astype(np.float32))
    if block:
        nb = -(-cols // block)
        scales = torch.empty((rows, nb), dtype=torch.float32)
        q = torch.empty((rows, cols), dtype=torch.float8_e4m3fn)
        for b in range(nb):
            blk = src[:, b * block:(b + 1) * block]
            s = blk.abs().amax(dim=1).clamp_min(1e-12) / 448.0
            scales[:, b] = s
            q[:, b * block:(b + 1) * block] = (blk / s[:, None]).to(torch.float8_e4m3fn)
    else:
        scales = src.abs().amax(dim=1).clamp_min(1e-12) / 448.0
        q = (src / scales[:, None]).to(torch.float8_e4m3fn)
    return q.view(torch.uint8).numpy(), scales.numpy()


def act(g, n, bf16: bool):
    v = g.standard_normal(n).astype(np.float32)
    return (bf16_bits(v), bf16_to_f32(bf16_bits(v))) if bf16 else (v.astype(np.float16), v.astype(np.float16))


def dev_fp8(bits, device):
    return torch.from_numpy(bits).to(device).view(torch.float8_e4m3fn)


@pytest.mark.parametrize("rows,cols,block,bf16,odt", [
    (2880, 2880, 128, False, "f16"),    # ragged last block (22.5 blocks)
    (4096, 5120, 128, True, "bf16"),
    (1000, 2048, 32, False, "f32"),
    (512, 4096, 1024, True, "f32"),     # generic engine (blocks of 32 chunks)
    (768, 2048, 2048, False, "f16"),    # one block per row: the per-row-scale GEMV
])
def test_block_scaled_matvec(backend, device, rows, cols, block, bf16, odt):
    g = rng(rows + cols + block)
    w, sc = fp8_weights(g, rows, cols, block)
    xb, x32 = act(g, cols, bf16)
    out_dt = {"f16": torch.float16, "bf16": torch.bfloat16, "f32": torch.float32}[odt]
    out = torch.empty(rows, device=device, dtype=out_dt)
    backend.scaled_matvec(dev_fp8(w, device), to_torch(sc, device), to_torch(xb, device, bf16=bf16), out)
    got = from_torch_bits(out)
    nb = sc.shape[1]
    if block >= cols:
        want = oracle.gemv("fp8", "row", w, sc[:, 0].copy(), xb, cols=cols, lpr=lanes(cols), s_row=1,
                           odtype={"f16": oracle.F16, "bf16": oracle.BF16, "f32": oracle.F32}[odt])
    else:
        L = block // 32
        want = oracle.gemv("fp8", "group", w, sc, xb, cols=cols, lpr=lanes(cols, L), L=L, s_row=nb, s_grp=1,
                           odtype={"f16": oracle.F16, "bf16": oracle.BF16, "f32": oracle.F32}[odt])
    assert_bits_equal(got, want, f"block-scaled fp8 {rows}x{cols}/{block}")
    deq = ref.fp8_e4m3fn(w) * np.repeat(sc.astype(np.float64), block, axis=1)[:, :cols]
    y64 = ref.gemv64(deq, x32)
    assert ref.max_rel_err(ref.f64(got), y64) < TOL


@pytest.mark.parametrize("cols,bf16", [(2048, True), (5120, False)])
def test_multi_scaled_tensorcore_matvec(backend, device, cols, bf16):
    g = rng(cols + 3)
    rows = (4096, 512, 512)
    mats = [fp8_weights(g, r, cols) for r in rows]
    xb, x32 = act(g, cols, bf16)
    out = torch.empty(sum(rows), device=device, dtype=torch.bfloat16 if bf16 else torch.float16)
    backend.multi_scaled_tensorcore_matvec(tuple(dev_fp8(w, device) for w, _ in mats),
                                           tuple(to_torch(s, device) for _, s in mats), rows, cols,
                                           to_torch(xb, device, bf16=bf16), out)
    got = from_torch_bits(out)
    r0 = 0
    for (w, s), r in zip(mats, rows):
        want = oracle.gemv("fp8", "row", w, s, xb, cols=cols, lpr=lanes(cols), s_row=1,
                           odtype=oracle.BF16 if bf16 else oracle.F16)
        assert_bits_equal(got[r0:r0 + r], want, f"matrix at row {r0}")
        y64 = ref.gemv64(ref.fp8_e4m3fn(w) * s[:, None].astype(np.float64), x32)
        assert ref.max_rel_err(ref.f64(got[r0:r0 + r]), y64) < TOL
        r0 += r
    with pytest.raises(ValueError, match="divisible by 256"):
        backend.multi_scaled_tensorcore_matvec(tuple(dev_fp8(w, device)[:, :2880] for w, _ in mats[:2]),
                                               tuple(to_torch(s, device) for _, s in mats[:2]), rows[:2], 2880,
                                               to_torch(xb, device, bf16=bf16)[:2880], out)


@pytest.mark.parametrize("fmt,rows,cols,split_k,bf16", [
    ("f16w", 2048, 8192, 2, False),   # Llama down_proj shape, the reference runtime's split_k=2
    ("bf16w", 4096, 2880, 8, True),   # 90 chunks: slices of 12, the last of 6
    ("fp8", 1024, 5120, 4, False),    # scaled
    ("f16w", 300, 96, 8, False),      # three chunks: slices of one, five empty
])
def test_split_k_matvec(backend, device, fmt, rows, cols, split_k, bf16):
    g = rng(rows + cols + split_k)
    scales = None
    if fmt == "fp8":
        w, scales = fp8_weights(g, rows, cols)
        wt = dev_fp8(w, device)
        deq = ref.fp8_e4m3fn(w) * scales[:, None].astype(np.float64)
    elif fmt == "bf16w":
        w = bf16_bits(g.standard_normal((rows, cols)).astype(np.float32) * 0.02)
        wt = to_torch(w, device, bf16=True)
        deq = bf16_to_f32(w).astype(np.float64)
    else:
        w = f16_normal(g, (rows, cols), 0.02)
        wt = to_torch(w, device)
        deq = w.astype(np.float64)
    xb, x32 = act(g, cols, bf16)
    out = torch.empty(rows, device=device, dtype=torch.bfloat16 if bf16 else torch.float16)
    backend.split_k_matvec(wt, to_torch(xb, device, bf16=bf16), out,
                           scales=None if scales is None else to_torch(scales, device), split_k=split_k)
    got = from_torch_bits(out)
    want = oracle.split_k_gemv(fmt, w.view(np.uint8).reshape(rows, -1), xb, split_k, scales=scales,
                               odtype=oracle.BF16 if bf16 else oracle.F16)
    assert_bits_equal(got, want, f"split-K {fmt} {rows}x{cols}/{split_k}")
    assert ref.max_rel_err(ref.f64(got), ref.gemv64(deq, x32)) < TOL
    with pytest.raises(ValueError, match="split_k must be 2, 4, or 8"):
        backend.split_k_matvec(wt, to_torch(xb, device, bf16=bf16), out, split_k=3)


@pytest.mark.parametrize("rows,cols,bf16", [(8192, 2048, False), (17920, 5120, True), (100, 2880, False)])
def test_fused_scaled_gate_up_silu(backend, device, rows, cols, bf16):
    g = rng(rows + cols + 7)
    wg, sg = fp8_weights(g, rows, cols)
    wu, su = fp8_weights(g, rows, cols)
    xb, x32 = act(g, cols, bf16)
    out = torch.empty(rows, device=device, dtype=torch.bfloat16 if bf16 else torch.float16)
    backend.fused_scaled_gate_up_silu(dev_fp8(wg, device), to_torch(sg, device), dev_fp8(wu, device),
                                      to_torch(su, device), to_torch(xb, device, bf16=bf16), out)
    got = from_torch_bits(out)
    # the oracle composition: scaled_matvec's binary32 rows, bfloat16, SiLU * up
    gate = oracle.gemv("fp8", "row", wg, sg, xb, cols=cols, lpr=lanes(cols), s_row=1, odtype=oracle.F32)
    up = oracle.gemv("fp8", "row", wu, su, xb, cols=cols, lpr=lanes(cols), s_row=1, odtype=oracle.F32)
    gate, up = bf16_to_f32(bf16_bits(gate)), bf16_to_f32(bf16_bits(up))
    prod = np.empty(rows, dtype=np.float32)
    oracle.lib().tto_silu_mul(gate.ctypes.data, up.ctypes.data, prod.ctypes.data, oracle.F32, rows)
    want = bf16_bits(prod) if bf16 else prod.astype(np.float16)
    assert_bits_equal(got, want, f"gate/up SiLU {rows}x{cols}")
    g64 = ref.bf16_round64(ref.gemv64(ref.fp8_e4m3fn(wg), x32) * sg)
    u64 = ref.bf16_round64(ref.gemv64(ref.fp8_e4m3fn(wu), x32) * su)
    assert ref.max_rel_err(ref.f64(got), ref.silu_mul64(g64, u64)) < TOL


@pytest.mark.parametrize("heads,D,bf16", [(32, 128, False), (8, 64, True), (40, 256, False)])
def test_head_rms_norm(backend, device, heads, D, bf16):
    g = rng(heads * D)
    xb, x32 = act(g, heads * D, bf16)
    wb, w32 = act(g, D, bf16)
    out = torch.empty(heads * D, device=device, dtype=torch.bfloat16 if bf16 else torch.float16)
    backend.head_rms_norm(to_torch(xb, device, bf16=bf16), to_torch(wb, device, bf16=bf16), out, heads, D, 1e-6)
    got = from_torch_bits(out)
    assert_bits_equal(got, oracle.head_rms_norm(xb, wb, heads, D, 1e-6), "head_rms_norm")
    want64 = np.concatenate([ref.rms_norm64(x32[h * D:(h + 1) * D], w32, 1e-6) for h in range(heads)])
    assert ref.max_rel_err(ref.f64(got), want64) < TOL


@pytest.mark.parametrize("heads,kv_heads,D,device_pos", [(32, 8, 128, True), (16, 2, 64, False)])
def test_qk_head_rmsnorm_rope_inplace(backend, device, heads, kv_heads, D, device_pos):
    g = rng(heads + kv_heads + D)
    positions, p = 800, 731
    inv = (1000000.0 ** (-np.arange(0, D, 2, dtype=np.float32) / D)).astype(np.float32)
    ang = np.arange(positions, dtype=np.float32)[:, None] * inv[None, :]
    cos, sin = np.cos(ang).astype(np.float16), np.sin(ang).astype(np.float16)
    q, k = f16_normal(g, heads * D, 2.0), f16_normal(g, kv_heads * D)
    qw, kw = f16_normal(g, D, 0.5), f16_normal(g, D, 0.5)
    qt, kt = to_torch(q, device), to_torch(k, device)
    if device_pos:
        backend.qk_head_rmsnorm_rope_inplace(qt, kt, to_torch(qw, device), to_torch(kw, device), to_torch(cos, device),
                                             to_torch(sin, device), heads, kv_heads, D, 1e-6,
                                             position=torch.tensor([p], dtype=torch.int32, device=device))
    else:
        backend.qk_head_rmsnorm_rope_inplace(qt, kt, to_torch(qw, device), to_torch(kw, device),
                                             to_torch(cos[p], device), to_torch(sin[p], device), heads, kv_heads, D,
                                             1e-6)
    qo, ko = oracle.qk_head_rmsnorm_rope(q, k, qw, kw, cos[p], sin[p], heads, kv_heads, D, 1e-6)
    assert_bits_equal(from_torch_bits(qt), qo, "q")
    assert_bits_equal(from_torch_bits(kt), ko, "k")
    for x, w, n, got in ((q, qw, heads, qt), (k, kw, kv_heads, kt)):
        want = []
        for h in range(n):
            nrm = ref.rms_norm64(x[h * D:(h + 1) * D], w, 1e-6)
            first, second = ref.rope64(nrm[:D // 2], nrm[D // 2:], cos[p], sin[p])
            want.append(np.concatenate([first, second]))
        assert ref.max_rel_err(ref.f64(from_torch_bits(got)), np.concatenate(want)) < TOL
