"""The decode step's router split across two launches: add + RMSNorm + router logits
(tt_add_rms_norm_router_logits), then the expert SwiGLU taking its own top-k from those
logits (tt_mxfp_lowbit_selected_swiglu_router).  Bit for bit the pair equals
add_rms_norm_router_topk + mxfp_lowbit_selected_swiglu(_tokens), whose parts are pinned
against the oracle elsewhere; the top-k over special logits (ties, signed zeros, -inf,
NaN) is checked against the sequential oracle scan directly."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from oracle import ref
from tests.helpers import f16_normal, from_torch_bits, rng, to_torch
from tests.test_gemv_gpu import _mxfp4_expert_weights, assert_bits_equal

pytestmark = pytest.mark.gpu


def P(a):
    return a.ctypes.data


@pytest.mark.parametrize("tokens,E,H,bias", [(1, 32, 2880, True), (8, 32, 2880, True), (3, 17, 2048, False),
                                             (2, 1, 64, True)])
def test_norm_router_logits(backend, device, tokens, E, H, bias):
    """Residual and norm outputs equal the top-k launch's; the logits rank to its
    experts and scores, and lie within 1e-2 of the float64 dot products."""
    g = rng(tokens * 31 + E + H)
    T = lambda a: to_torch(a, device)
    a, b = f16_normal(g, (tokens, H)), f16_normal(g, (tokens, H), 0.5)
    nw, w = f16_normal(g, H, 0.1), f16_normal(g, (E, H), 0.05)
    bs = T(f16_normal(g, E, 0.1)) if bias else None
    k = min(4, E)
    res, normed = (torch.empty((tokens, H), device=device, dtype=torch.float16) for _ in range(2))
    logits = torch.full((tokens, E), float("nan"), device=device, dtype=torch.float32)
    backend.add_rms_norm_router_logits(T(a), T(b), res, T(nw), normed, 1e-5, T(w), logits, bias=bs)
    r2, n2 = torch.empty_like(res), torch.empty_like(res)
    idx = torch.empty((tokens, k), device=device, dtype=torch.int32)
    sc = torch.empty((tokens, k), device=device, dtype=torch.float16)
    backend.add_rms_norm_router_topk(T(a), T(b), r2, T(nw), n2, 1e-5, T(w), idx, sc, bias=bs, renormalize=True)
    assert torch.equal(res.view(torch.int16), r2.view(torch.int16))
    assert torch.equal(normed.view(torch.int16), n2.view(torch.int16))
    for t in range(tokens):
        i1 = torch.empty(k, device=device, dtype=torch.int32)
        s1 = torch.empty(k, device=device, dtype=torch.float16)
        backend.moe_router_topk(logits[t], i1, s1, renormalize=True)
        assert torch.equal(i1, idx[t]), (t, i1, idx[t])
        assert torch.equal(s1.view(torch.int16), sc[t].view(torch.int16))
    nrm = from_torch_bits(normed).astype(np.float64)
    want = nrm @ w.astype(np.float64).T
    if bias:
        want = want + from_torch_bits(bs).astype(np.float64)[None, :]
    got = logits.cpu().numpy().astype(np.float64)
    assert np.abs(got - want).max() / np.abs(want).max() < 1e-2


def _special_logits(g, tokens, E):
    """Ties (values on a 0.5 grid); token t % 3 == 1 adds signed zeros and -inf, t % 3 == 2
    also NaN (the scan without NaN and the NaN-aware scan are different code paths)."""
    lg = (np.round(g.standard_normal((tokens, E)) * 2) / 2).astype(np.float32)
    for t in range(tokens):
        if t % 3:
            lg[t, g.integers(0, E, size=max(1, E // 8))] = 0.0
            lg[t, g.integers(0, E, size=max(1, E // 8))] = -0.0
            lg[t, g.integers(0, E, size=max(1, E // 16))] = -np.inf
        if t % 3 == 2:
            lg[t, g.integers(1, E, size=max(1, E // 16))] = np.nan
    return lg


@pytest.mark.parametrize("tokens,E,k,renorm,rows", [(1, 32, 4, True, 2880), (8, 32, 4, True, 2880),
                                                    (2, 128, 6, False, 512), (5, 65, 64, True, 192),
                                                    (3, 7, 7, False, 320)])
def test_swiglu_router(backend, device, tokens, E, k, renorm, rows):
    """Every slot's expert is the token's top-k choice: the activations equal the
    index-driven SwiGLU on moe_router_topk's experts, and the published indices and
    scores equal moe_router_topk's and the sequential oracle scan's."""
    cols = 2880 if rows == 2880 else 1024
    g = rng(tokens * 101 + E + k)
    T = lambda a: to_torch(a, device)
    gu, gus = _mxfp4_expert_weights(g, E, 2 * rows, cols)
    gub = f16_normal(g, (E, 2 * rows), 0.5)
    x = f16_normal(g, (tokens, cols))
    lg = _special_logits(g, tokens, E)
    gu_d, gus_d, gub_d, x_d, lg_d = T(gu), T(gus), T(gub), T(x), torch.from_numpy(lg).to(device)
    act = torch.empty((tokens * k, rows), device=device, dtype=torch.float16)
    idx = torch.full((tokens, k), -1, device=device, dtype=torch.int32)
    sc = torch.empty((tokens, k), device=device, dtype=torch.float16)
    backend.mxfp_lowbit_selected_swiglu_router(gu_d, gus_d, x_d, lg_d, idx, sc, act, bits=4, alpha=1.702, limit=7.0,
                                               renormalize=renorm, bias=gub_d)
    i_ref = torch.empty_like(idx)
    s_ref = torch.empty_like(sc)
    for t in range(tokens):
        backend.moe_router_topk(lg_d[t], i_ref[t], s_ref[t], renormalize=renorm)
        widx = np.empty(k, dtype=np.int32)
        wsc = np.empty(k, dtype=np.float16)
        lt = np.ascontiguousarray(lg[t])
        oracle.lib().tto_topk(P(lt), oracle.F32, E, k, int(renorm), P(widx), P(wsc), oracle.F16)
        assert np.array_equal(idx[t].cpu().numpy(), widx), (t, idx[t].cpu().numpy(), widx)
        assert_bits_equal(from_torch_bits(sc[t]), wsc, f"scores token {t}")
        if not np.isnan(lt).any() and not np.isinf(lt).any():
            i64, s64 = ref.topk_softmax64(lt, k, renorm)
            assert np.array_equal(widx, i64)
            assert np.abs(from_torch_bits(sc[t]).astype(np.float64) - s64).max() < 1e-2
    assert torch.equal(idx, i_ref)
    assert torch.equal(sc.view(torch.int16), s_ref.view(torch.int16))
    want = torch.empty_like(act)
    if tokens == 1:
        backend.mxfp_lowbit_selected_swiglu(gu_d, gus_d, x_d[0], i_ref[0], want, bits=4, alpha=1.702, limit=7.0,
                                            bias=gub_d)
    else:
        backend.mxfp_lowbit_selected_swiglu_tokens(gu_d, gus_d, x_d, i_ref, want, bits=4, alpha=1.702, limit=7.0,
                                                   bias=gub_d)
    assert torch.equal(act.view(torch.int16), want.view(torch.int16))


def test_swiglu_router_rejects_wide_rows(backend, device):
    """Rows longer than the router-mode kernels take raise instead of launching."""
    g = rng(5)
    gu, gus = _mxfp4_expert_weights(g, 4, 64, 16384)
    T = lambda a: to_torch(a, device)
    act = torch.empty((2, 32), device=device, dtype=torch.float16)
    lg = torch.zeros((1, 4), device=device, dtype=torch.float32)
    idx = torch.empty((1, 2), device=device, dtype=torch.int32)
    sc = torch.empty((1, 2), device=device, dtype=torch.float16)
    with pytest.raises(Exception):
        backend.mxfp_lowbit_selected_swiglu_router(T(gu), T(gus), T(f16_normal(g, (1, 16384))), lg, idx, sc, act,
                                                   bits=4, alpha=1.702, limit=7.0, renormalize=True)
