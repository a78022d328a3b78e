"""GPU parity of the fused decode-step GEMVs against the unfused operator sequence
they replace (bit for bit): every prologue (add + RMSNorm, embedding + RMSNorm,
add then RMSNorm), every segment kind (RoPE to a buffer, RoPE to the K cache, V cache,
SiLU pair, plain with bias), the lane groupings 64 / 32 / 16, and the lm_head with
the token log and position advance in its finishing kernel."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from tests.helpers import f16_normal, rng, to_torch
from thintensor_amd import _lib
from thintensor_amd.decode import _dense_segment, _int4_segment
from thintensor_amd.synth import rope_tables

pytestmark = pytest.mark.gpu


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy()


def _int4(g, rows, cols, device):
    packed = torch.from_numpy(g.integers(0, 256, size=(rows, cols // 2), dtype=np.uint8)).to(device)
    scales = to_torch((np.abs(g.standard_normal((rows, cols // 128))) * 0.02).astype(np.float16), device)
    return packed, scales


def _prologue(d, kind, dev_inputs):
    d.prologue = kind
    if kind in (_lib.PRO_ADD_NORM, _lib.PRO_ADD_RMS_NORM):
        d.left, d.right = dev_inputs["left"].data_ptr(), dev_inputs["right"].data_ptr()
    elif kind == _lib.PRO_EMBED_NORM:
        d.embed, d.embed_row = dev_inputs["embed"].data_ptr(), dev_inputs["embed"].stride(0)
        d.vocab, d.token = int(dev_inputs["embed"].shape[0]), dev_inputs["token"].data_ptr()
    d.norm_weight, d.eps = dev_inputs["norm"].data_ptr(), 1e-5
    d.residual_out = dev_inputs["res"].data_ptr()


def _unfused_prologue(be, kind, dev_inputs, normed):
    res = dev_inputs["res"]
    if kind == _lib.PRO_ADD_NORM:
        be.add_rms_norm(dev_inputs["left"], dev_inputs["right"], res, dev_inputs["norm"], normed, 1e-5)
    elif kind == _lib.PRO_EMBED_NORM:
        be.embedding(dev_inputs["embed"], dev_inputs["token"], res)
        be.rms_norm(res, dev_inputs["norm"], normed, 1e-5)
    else:
        be.add(dev_inputs["left"], dev_inputs["right"], res)
        be.rms_norm(res, dev_inputs["norm"], normed, 1e-5)


def _inputs(g, n, device):
    return {
        "left": to_torch(f16_normal(g, n, 2.0), device),
        "right": to_torch(f16_normal(g, n, 2.0), device),
        "embed": to_torch(f16_normal(g, (97, n), 1.0), device),
        "token": torch.tensor(41, device=device, dtype=torch.int64),
        "norm": to_torch(f16_normal(g, n, 0.5), device),
        "res": torch.empty(n, device=device, dtype=torch.float16),
    }


@pytest.mark.parametrize("cols,prologue", [(2048, _lib.PRO_ADD_NORM), (2048, _lib.PRO_EMBED_NORM),
                                           (2048, _lib.PRO_ADD_RMS_NORM), (1536, _lib.PRO_ADD_NORM),
                                           (2816, _lib.PRO_ADD_RMS_NORM)])
def test_fused_int4_qkv_rope_cache(backend, device, cols, prologue):
    """cols 2048 / 1536 / 2816 give 64 / 16 / 32 lanes per row."""
    g = rng(cols + prologue)
    heads, kv_heads, D, cap, pos = 8, 2, 64, 128, 77
    qd, kd = heads * D, kv_heads * D
    Wq, Wk, Wv = _int4(g, qd, cols, device), _int4(g, kd, cols, device), _int4(g, kd, cols, device)
    inp = _inputs(g, cols, device)
    cos, sin = rope_tables(D, 10000.0, cap, device)
    position = torch.tensor([pos], device=device, dtype=torch.int32)
    kc0 = to_torch(f16_normal(g, (kv_heads, cap, D)), device)
    vc0 = to_torch(f16_normal(g, (kv_heads, cap, D)), device)
    # unfused reference sequence
    normed = torch.empty(cols, device=device, dtype=torch.float16)
    _unfused_prologue(backend, prologue, inp, normed)
    res_want = inp["res"].clone()
    qkv = torch.empty(qd + 2 * kd, device=device, dtype=torch.float16)
    backend.multi_int4_scaled_matvec((Wq[0], Wk[0], Wv[0]), (Wq[1], Wk[1], Wv[1]), (qd, kd, kd), cols, normed, qkv,
                                     group_size=128)
    q, k, v = qkv[:qd], qkv[qd:qd + kd], qkv[qd + kd:]
    backend.rope_qk_inplace(q, k, cos, sin, heads, kv_heads, D, position=position)
    kc_want, vc_want = kc0.clone(), vc0.clone()
    backend.kv_append(k, v, kc_want, vc_want, position, kv_heads, D)
    # fused
    inp["res"].fill_(0)
    kc, vc = kc0.clone(), vc0.clone()
    qout = torch.empty(qd, device=device, dtype=torch.float16)
    d = _lib.FusedGemv()
    d.weight_format, d.group_size, d.act_dtype, d.cols = _lib.FMT_INT4_G, 128, _lib.F16, cols
    _prologue(d, prologue, inp)
    d.count = 3
    _int4_segment(d.seg[0], Wq, qout, qd, _lib.SEG_ROPE_OUT)
    _int4_segment(d.seg[1], Wk, kc, kd, _lib.SEG_ROPE_CACHE)
    _int4_segment(d.seg[2], Wv, vc, kd, _lib.SEG_CACHE)
    d.position, d.capacity, d.cache_head = position.data_ptr(), cap, kc.stride(0)
    d.cos_table, d.sin_table, d.table_row, d.table_rows, d.head_dim = cos.data_ptr(), sin.data_ptr(), cos.stride(0), cap, D
    backend.fused_gemv(d)
    assert np.array_equal(_bits(qout), _bits(q))
    assert np.array_equal(_bits(kc), _bits(kc_want))
    assert np.array_equal(_bits(vc), _bits(vc_want))
    assert np.array_equal(_bits(inp["res"]), _bits(res_want))


@pytest.mark.parametrize("cols,inter", [(2048, 1024), (1536, 512)])
def test_fused_int4_gate_up_silu(backend, device, cols, inter):
    g = rng(cols + inter)
    Wg, Wu = _int4(g, inter, cols, device), _int4(g, inter, cols, device)
    inp = _inputs(g, cols, device)
    normed = torch.empty(cols, device=device, dtype=torch.float16)
    _unfused_prologue(backend, _lib.PRO_ADD_NORM, inp, normed)
    res_want = inp["res"].clone()
    gu = torch.empty(2 * inter, device=device, dtype=torch.float16)
    backend.multi_int4_scaled_matvec((Wg[0], Wu[0]), (Wg[1], Wu[1]), (inter, inter), cols, normed, gu, group_size=128)
    act_want = torch.empty(inter, device=device, dtype=torch.float16)
    backend.silu_mul(gu[:inter], gu[inter:], act_want)
    inp["res"].fill_(0)
    act = torch.empty(inter, device=device, dtype=torch.float16)
    d = _lib.FusedGemv()
    d.weight_format, d.group_size, d.act_dtype, d.cols = _lib.FMT_INT4_G, 128, _lib.F16, cols
    _prologue(d, _lib.PRO_ADD_NORM, inp)
    d.count = 1
    _int4_segment(d.seg[0], Wg, act, inter, _lib.SEG_SILU, weight2=Wu)
    backend.fused_gemv(d)
    assert np.array_equal(_bits(act), _bits(act_want))
    assert np.array_equal(_bits(inp["res"]), _bits(res_want))


@pytest.mark.parametrize("cols", [2880, 2048])
def test_fused_dense_bias_qkv_rope(backend, device, cols):
    g = rng(cols)
    heads, kv_heads, D, cap, pos = 16, 4, 64, 192, 130
    qd, kd = heads * D, kv_heads * D
    W = [to_torch(f16_normal(g, (r, cols), 0.02), device) for r in (qd, kd, kd)]
    B = [to_torch(f16_normal(g, r, 0.05), device) for r in (qd, kd, kd)]
    inp = _inputs(g, cols, device)
    cos, sin = rope_tables(D, 150000.0, cap, device)
    position = torch.tensor([pos], device=device, dtype=torch.int32)
    kc0 = to_torch(f16_normal(g, (kv_heads, cap, D)), device)
    vc0 = to_torch(f16_normal(g, (kv_heads, cap, D)), device)
    normed = torch.empty(cols, device=device, dtype=torch.float16)
    _unfused_prologue(backend, _lib.PRO_ADD_NORM, inp, normed)
    qkv = torch.empty(qd + 2 * kd, device=device, dtype=torch.float16)
    backend.multi_matvec_bias(tuple(W), tuple(B), normed, qkv)
    q, k, v = qkv[:qd], qkv[qd:qd + kd], qkv[qd + kd:]
    backend.rope_qk_inplace(q, k, cos, sin, heads, kv_heads, D, position=position)
    kc_want, vc_want = kc0.clone(), vc0.clone()
    backend.kv_append(k, v, kc_want, vc_want, position, kv_heads, D)
    kc, vc = kc0.clone(), vc0.clone()
    qout = torch.empty(qd, device=device, dtype=torch.float16)
    d = _lib.FusedGemv()
    d.weight_format, d.weight_dtype, d.act_dtype, d.cols = _lib.FMT_DENSE, _lib.F16, _lib.F16, cols
    _prologue(d, _lib.PRO_ADD_NORM, inp)
    d.count = 3
    _dense_segment(d.seg[0], W[0], B[0], qout, _lib.SEG_ROPE_OUT)
    _dense_segment(d.seg[1], W[1], B[1], kc, _lib.SEG_ROPE_CACHE)
    _dense_segment(d.seg[2], W[2], B[2], vc, _lib.SEG_CACHE)
    d.position, d.capacity, d.cache_head = position.data_ptr(), cap, kc.stride(0)
    d.cos_table, d.sin_table, d.table_row, d.table_rows, d.head_dim = cos.data_ptr(), sin.data_ptr(), cos.stride(0), cap, D
    backend.fused_gemv(d)
    assert np.array_equal(_bits(qout), _bits(q))
    assert np.array_equal(_bits(kc), _bits(kc_want))
    assert np.array_equal(_bits(vc), _bits(vc_want))


@pytest.mark.parametrize("prologue", [_lib.PRO_ADD_NORM, _lib.PRO_ADD_RMS_NORM])
def test_fused_lm_head_argmax_bookkeeping(backend, device, prologue):
    g = rng(prologue)
    rows, cols = 50000, 2048
    W = to_torch(f16_normal(g, (rows, cols), 0.02), device)
    inp = _inputs(g, cols, device)
    normed = torch.empty(cols, device=device, dtype=torch.float16)
    _unfused_prologue(backend, prologue, inp, normed)
    tok_want = int(backend.matvec_argmax_tensor(W, normed))
    logits_want = backend.logits_buffer(rows, torch.float16).clone()
    position = torch.tensor([20], device=device, dtype=torch.int32)
    base = torch.tensor([17], device=device, dtype=torch.int32)
    history = torch.full((8,), -1, device=device, dtype=torch.int64)
    logits = torch.empty(rows, device=device, dtype=torch.float16)
    d = _lib.FusedGemv()
    d.weight_format, d.weight_dtype, d.act_dtype, d.cols = _lib.FMT_DENSE, _lib.F16, _lib.F16, cols
    _prologue(d, prologue, inp)
    d.residual_out = None
    d.count = 1
    _dense_segment(d.seg[0], W, None, logits, _lib.SEG_PLAIN)
    tok = backend.fused_lm_head_argmax(d, position=position, base=base, history=history)
    assert int(tok) == tok_want
    assert np.array_equal(_bits(logits), _bits(logits_want))
    assert int(position) == 21
    assert history.cpu().tolist() == [-1, -1, -1, tok_want, -1, -1, -1, -1]


def test_fused_rejects_bad_descriptors(backend, device):
    d = _lib.FusedGemv()
    d.weight_format, d.group_size, d.act_dtype, d.cols = _lib.FMT_INT4_G, 64, _lib.F16, 2048
    d.prologue = _lib.PRO_LOAD
    with pytest.raises((ValueError, _lib.KernelLibraryError)):
        backend.fused_gemv(d)
