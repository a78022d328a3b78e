"""GPU parity of norms, elementwise ops, RoPE, attention, router and lm_head argmax
against the CPU oracle (bit for bit) and the float64 closed forms of oracle/ref.py
(max relative error below the north-star tolerance TOL = 1e-2; router indices exact)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from oracle import ref
from tests.helpers import bf16_bits, f16_normal, from_torch_bits, rng, to_torch
from tests.test_gemv_gpu import assert_bits_equal, lanes

pytestmark = pytest.mark.gpu

TOL = 1e-2  # max |got - want| / max |want| against the float64 closed form


def assert_f64(got, want64, what: str) -> None:
    err = ref.max_rel_err(ref.f64(got).reshape(-1), np.asarray(want64, dtype=np.float64).reshape(-1))
    assert err < TOL, f"{what}: max relative error {err:.3g} against float64"


def P(a):
    return a.ctypes.data


@pytest.mark.parametrize("n,offset", [(2048, 0.0), (2880, 1.0), (5120, 0.0), (100, 0.0)])
def test_rms_norm(backend, device, n, offset):
    g = rng(n)
    x = f16_normal(g, n, 3.0)
    w = f16_normal(g, n, 0.1)
    out = torch.empty(n, device=device, dtype=torch.float16)
    backend.rms_norm(to_torch(x, device), to_torch(w, device), out, 1e-5, weight_offset=offset)
    want = np.empty(n, dtype=np.float16)
    oracle.lib().tto_rms_norm(P(x), oracle.F16, P(w), oracle.F16, P(want), oracle.F16, n, 1e-5, offset)
    assert_bits_equal(from_torch_bits(out), want, "rms_norm")
    assert_f64(from_torch_bits(out), ref.rms_norm64(x, w, 1e-5, offset), "rms_norm")


@pytest.mark.parametrize("n,seed", [(2048, 0), (2880, 0), (4096, 1), (5120, 0), (5120, 2), (8192, 3)])
def test_add_rms_norm(backend, device, n, seed):
    # ~27k outputs in all: a conversion that rounds the normalized product once,
    # straight to fp16, instead of to binary32 first differs in about one output of
    # several thousand, so these sizes catch it
    g = rng(n + 1 + 1000 * seed)
    a, b = f16_normal(g, n), f16_normal(g, n, 0.5)
    w = f16_normal(g, n, 0.1)
    res = torch.empty(n, device=device, dtype=torch.float16)
    out = torch.empty(n, device=device, dtype=torch.float16)
    backend.add_rms_norm(to_torch(a, device), to_torch(b, device), res, to_torch(w, device), out, 1e-5)
    want_res = np.empty(n, dtype=np.float16)
    want = np.empty(n, dtype=np.float16)
    oracle.lib().tto_add_rms_norm(P(a), P(b), P(want_res), oracle.F16, P(w), oracle.F16, P(want), oracle.F16, n, 1e-5)
    assert_bits_equal(from_torch_bits(res), want_res, "residual")
    assert_bits_equal(from_torch_bits(out), want, "normed")
    want_res64, want64 = ref.add_rms_norm64(a, b, w, 1e-5)
    assert np.array_equal(from_torch_bits(res).astype(np.float64), want_res64)
    assert_f64(from_torch_bits(out), want64, "add_rms_norm")


@pytest.mark.parametrize("rows,n", [(8, 2880), (3, 4096), (1, 2048)])
def test_add_then_rms_norm_rows(backend, device, rows, n):
    """The batched end-of-step launch equals add then rms_norm on each row, bit for bit,
    and both equal the oracle."""
    g = rng(rows * 31 + n)
    a, b = f16_normal(g, (rows, n), 2.0), f16_normal(g, (rows, n), 0.5)
    w = f16_normal(g, n, 0.1)
    ad, bd, wd = to_torch(a, device), to_torch(b, device), to_torch(w, device)
    sums = torch.empty((rows, n), device=device, dtype=torch.float16)
    out = torch.empty((rows, n), device=device, dtype=torch.float16)
    backend.add_then_rms_norm_rows(ad, bd, sums, wd, out, 1e-5)
    got_sum, got = from_torch_bits(sums), from_torch_bits(out)
    for r in range(rows):
        want_sum = (a[r].astype(np.float32) + b[r].astype(np.float32)).astype(np.float16)
        assert_bits_equal(got_sum[r], want_sum, f"sum row {r}")
        want = np.empty(n, dtype=np.float16)
        oracle.lib().tto_rms_norm(P(want_sum), oracle.F16, P(w), oracle.F16, P(want), oracle.F16, n, 1e-5, 0.0)
        assert_bits_equal(got[r], want, f"normed row {r}")
        one_sum = torch.empty(n, device=device, dtype=torch.float16)
        one = torch.empty(n, device=device, dtype=torch.float16)
        backend.add(ad[r], bd[r], one_sum)
        backend.rms_norm(one_sum, wd, one, 1e-5)
        assert_bits_equal(got[r], from_torch_bits(one), f"unbatched row {r}")


def test_record_tokens_advance(backend, device):
    tokens = torch.tensor([5, 7, 11], device=device, dtype=torch.int64)
    history = torch.zeros((3, 4), device=device, dtype=torch.int64)
    position = torch.tensor([10], device=device, dtype=torch.int32)
    base = torch.tensor([9], device=device, dtype=torch.int32)
    backend.record_tokens_advance(tokens, position, base, history)
    backend.record_tokens_advance(tokens + 1, position, base, history)
    assert history.cpu().tolist() == [[0, 5, 6, 0], [0, 7, 8, 0], [0, 11, 12, 0]]
    assert int(position.item()) == 12
    position.fill_(13)  # outside the log: skipped, the position still moves
    backend.record_tokens_advance(tokens, position, base, history)
    assert history.cpu().tolist() == [[0, 5, 6, 0], [0, 7, 8, 0], [0, 11, 12, 0]]
    assert int(position.item()) == 14


def test_silu_swiglu_weighted_sum_add(backend, device):
    g = rng(3)
    n = 8192
    gt, up = f16_normal(g, n, 3.0), f16_normal(g, n)
    out = torch.empty(n, device=device, dtype=torch.float16)
    backend.silu_mul(to_torch(gt, device), to_torch(up, device), out)
    want = np.empty(n, dtype=np.float16)
    oracle.lib().tto_silu_mul(P(gt), P(up), P(want), oracle.F16, n)
    assert_bits_equal(from_torch_bits(out), want, "silu_mul")
    assert_f64(from_torch_bits(out), ref.silu_mul64(gt, up), "silu_mul")

    gu = f16_normal(g, (4, 2 * 2880), 6.0)
    out2 = torch.empty((4, 2880), device=device, dtype=torch.float16)
    backend.interleaved_swiglu(to_torch(gu, device), out2, alpha=1.702, limit=7.0)
    want2 = np.empty((4, 2880), dtype=np.float16)
    oracle.lib().tto_interleaved_swiglu(P(gu), P(want2), oracle.F16, 4, 2880, 1.702, 7.0)
    assert_bits_equal(from_torch_bits(out2).reshape(-1), want2.reshape(-1), "interleaved_swiglu")
    assert_f64(from_torch_bits(out2), ref.interleaved_swiglu64(gu, 1.702, 7.0), "interleaved_swiglu")

    ex = f16_normal(g, (4, 2880))
    sc = np.array([0.5, 0.25, 0.125, 0.125], dtype=np.float16)
    out3 = torch.empty(2880, device=device, dtype=torch.float16)
    backend.weighted_expert_sum(to_torch(ex, device), to_torch(sc, device), out3)
    want3 = np.empty(2880, dtype=np.float16)
    oracle.lib().tto_weighted_expert_sum(P(ex), oracle.F16, P(sc), oracle.F16, P(want3), 2880, 4)
    assert_bits_equal(from_torch_bits(out3), want3, "weighted_expert_sum")
    assert_f64(from_torch_bits(out3), ref.weighted_expert_sum64(ex, sc), "weighted_expert_sum")

    out4 = torch.empty(n, device=device, dtype=torch.float16)
    backend.add(to_torch(gt, device), to_torch(up, device), out4)
    assert_bits_equal(from_torch_bits(out4), (gt.astype(np.float32) + up.astype(np.float32)).astype(np.float16), "add")


def test_rope_table_and_device_position(backend, device):
    heads, kv_heads, D = 32, 8, 64
    g = rng(4)
    positions = 600
    inv = (500000.0 ** (-np.arange(0, D, 2, dtype=np.float32) / D)).astype(np.float32)
    ang = np.arange(positions, dtype=np.float32)[:, None] * inv[None, :]
    cos = np.cos(ang).astype(np.float16)
    sin = np.sin(ang).astype(np.float16)
    q = f16_normal(g, heads * D)
    k = f16_normal(g, kv_heads * D)
    pos = torch.tensor([517], dtype=torch.int32, device=device)
    q_t, k_t = to_torch(q, device), to_torch(k, device)
    backend.rope_qk_inplace(q_t, k_t, to_torch(cos, device), to_torch(sin, device), heads, kv_heads, D, position=pos)
    qw, kw = q.copy(), k.copy()
    oracle.lib().tto_rope(P(qw), P(kw), oracle.F16, P(cos[517]), P(sin[517]), heads, kv_heads, D)
    assert_bits_equal(from_torch_bits(q_t), qw, "rope q")
    assert_bits_equal(from_torch_bits(k_t), kw, "rope k")
    for src, got in ((q, q_t), (k, k_t)):
        h = src.reshape(-1, D)
        first, second = ref.rope64(h[:, :D // 2], h[:, D // 2:], cos[517], sin[517])
        assert_f64(from_torch_bits(got), np.concatenate([first, second], axis=1), "rope")


@pytest.mark.parametrize("cap", [1100, 1152])  # 1152: whole chunks, contiguous rows -> vector-load kernel
@pytest.mark.parametrize("heads,kv_heads,tokens,sinks", [(32, 8, 513, False), (64, 8, 1025, True), (8, 8, 5, False),
                                                         (32, 8, 64, True), (128, 8, 1100, False),
                                                         # 64 KV heads x 18 chunks: two chunks per workgroup
                                                         (256, 64, 1025, True), (512, 64, 705, False)])
def test_gqa_attention(backend, device, heads, kv_heads, tokens, sinks, cap):
    D = 64
    g = rng(heads + tokens)
    q = f16_normal(g, heads * D)
    keys = f16_normal(g, (kv_heads, cap, D))
    vals = f16_normal(g, (kv_heads, cap, D))
    sk = f16_normal(g, heads) if sinks else None
    out = torch.empty(heads * D, device=device, dtype=torch.float16)
    qd, kd, vd = to_torch(q, device), to_torch(keys, device), to_torch(vals, device)
    skd = to_torch(sk, device) if sinks else None
    # two calls in a row on the same scratch and output, the second with fewer tokens
    # (stale partials of the first call must not leak into the second)
    for n in (tokens, max(1, tokens // 2 - 3)):
        tok = torch.tensor([n], dtype=torch.int32, device=device)
        backend.single_token_gqa_attention(qd, kd, vd, out, heads, kv_heads, D, sinks=skd, active_tokens=tok)
        want = np.empty(heads * D, dtype=np.float16)
        oracle.lib().tto_attention(P(q), P(keys), P(vals), oracle.F16, cap * D, D, cap * D, D, P(sk) if sinks else None,
                                   oracle.F16, n, heads, kv_heads, D, P(want))
        assert_bits_equal(from_torch_bits(out), want, f"attention ({n} tokens)")
        want64 = ref.attention64(q.reshape(heads, D), keys[:, :n], vals[:, :n], kv_heads, sinks=sk)
        assert_f64(from_torch_bits(out), want64, f"attention ({n} tokens)")


@pytest.mark.parametrize("renorm,with_bias", [(True, True), (False, False)])
def test_router(backend, device, renorm, with_bias):
    E, H, k = 32, 2880, 4
    g = rng(7 + renorm)
    w = f16_normal(g, (E, H), 0.02)
    x = f16_normal(g, H)
    b = f16_normal(g, E, 0.1) if with_bias else None
    idx = torch.empty(k, device=device, dtype=torch.int32)
    sc = torch.empty(k, device=device, dtype=torch.float16)
    backend.moe_router_matvec_topk(to_torch(w, device), to_torch(x, device), idx, sc,
                                   bias=to_torch(b, device) if with_bias else None, renormalize=renorm)
    widx = np.empty(k, dtype=np.int32)
    wsc = np.empty(k, dtype=np.float16)
    oracle.lib().tto_router(P(w), oracle.F16, H, P(x), oracle.F16, H, P(b) if with_bias else None, oracle.F16, E, k,
                            int(renorm), P(widx), P(wsc), oracle.F16)
    assert np.array_equal(idx.cpu().numpy(), widx)
    assert_bits_equal(from_torch_bits(sc), wsc, "router scores")
    idx64, sc64 = ref.router64(w, x, b, k, renorm)
    assert np.array_equal(idx.cpu().numpy(), idx64)
    assert_f64(from_torch_bits(sc), sc64, "router scores")


@pytest.mark.parametrize("E,H,k,renorm,bias_dtype,wbf16", [
    (32, 2880, 4, True, "f16", False),    # gpt-oss router: one launch
    (8, 2048, 2, False, None, False),
    (32, 4096, 8, True, "bf16", True),    # largest one-launch hidden size, bf16 router weight
    (1, 64, 1, True, "f32", False),
    (17, 2080, 3, False, "f16", False),   # ragged second round of chunks
    (64, 2880, 4, True, "f16", False),    # more experts than one launch takes: two launches
    (32, 5120, 4, True, None, False),     # hidden above 4096: two launches
])
@pytest.mark.parametrize("split", [True, False])
def test_add_rms_norm_router(backend, device, E, H, k, renorm, bias_dtype, wbf16, split):
    """The combined launch equals add_rms_norm followed by the router on its output,
    with the router rows over ceil(E / 4) workgroups (split) or in one workgroup."""
    g = rng(E * 7 + H + k)
    a, b = f16_normal(g, H), f16_normal(g, H, 0.5)
    nw = f16_normal(g, H, 0.1)
    wf = (g.standard_normal((E, H)) * 0.05).astype(np.float32)
    w = bf16_bits(wf) if wbf16 else wf.astype(np.float16)
    bias = None
    if bias_dtype == "f16":
        bias = f16_normal(g, E, 0.1)
    elif bias_dtype == "bf16":
        bias = bf16_bits(g.standard_normal(E).astype(np.float32) * 0.1)
    elif bias_dtype == "f32":
        bias = (g.standard_normal(E) * 0.1).astype(np.float32)
    bcode = {"f16": oracle.F16, "bf16": oracle.BF16, "f32": oracle.F32, None: oracle.F16}[bias_dtype]
    res = torch.empty(H, device=device, dtype=torch.float16)
    normed = torch.empty(H, device=device, dtype=torch.float16)
    idx = torch.empty(k, device=device, dtype=torch.int32)
    sc = torch.empty(k, device=device, dtype=torch.float16)
    backend.add_rms_norm_router_topk(to_torch(a, device), to_torch(b, device), res, to_torch(nw, device), normed, 1e-5,
                                     to_torch(w, device, bf16=wbf16), idx, sc,
                                     bias=None if bias is None else to_torch(bias, device, bf16=bias_dtype == "bf16"),
                                     renormalize=renorm, split=split)
    want_res = np.empty(H, dtype=np.float16)
    want_n = np.empty(H, dtype=np.float16)
    oracle.lib().tto_add_rms_norm(P(a), P(b), P(want_res), oracle.F16, P(nw), oracle.F16, P(want_n), oracle.F16, H, 1e-5)
    widx = np.empty(k, dtype=np.int32)
    wsc = np.empty(k, dtype=np.float16)
    oracle.lib().tto_router(P(w), oracle.BF16 if wbf16 else oracle.F16, H, P(want_n), oracle.F16, H,
                            None if bias is None else P(bias), bcode, E, k, int(renorm), P(widx), P(wsc), oracle.F16)
    assert_bits_equal(from_torch_bits(res), want_res, "residual")
    assert_bits_equal(from_torch_bits(normed), want_n, "normed")
    assert np.array_equal(idx.cpu().numpy(), widx), (idx.cpu().numpy(), widx)
    assert_bits_equal(from_torch_bits(sc), wsc, "router scores")
    assert_f64(from_torch_bits(normed), ref.add_rms_norm64(a, b, nw, 1e-5)[1], "normed")
    idx64, sc64 = ref.router64(w, want_n, bias, k, renorm)
    assert np.array_equal(idx.cpu().numpy(), idx64)
    assert_f64(from_torch_bits(sc), sc64, "router scores")


@pytest.mark.parametrize("tokens,H", [(8, 2880), (3, 5120)])
def test_add_rms_norm_router_tokens(backend, device, tokens, H):
    """Several tokens in one call (above 4096 the per-token operators) equal the
    single-token calls, and the split launch equals the one-workgroup launch on two
    calls in a row (the arrival counters are left at zero)."""
    E, k = 32, 4
    g = rng(tokens + H)
    a, b = f16_normal(g, (tokens, H)), f16_normal(g, (tokens, H), 0.5)
    nw, w, bias = f16_normal(g, H, 0.1), f16_normal(g, (E, H), 0.05), f16_normal(g, E, 0.1)
    T = lambda x: to_torch(x, device)
    res = torch.empty((tokens, H), device=device, dtype=torch.float16)
    normed = torch.empty_like(res)
    idx = torch.empty((tokens, k), device=device, dtype=torch.int32)
    sc = torch.empty((tokens, k), device=device, dtype=torch.float16)
    backend.add_rms_norm_router_topk(T(a), T(b), res, T(nw), normed, 1e-5, T(w), idx, sc, bias=T(bias), renormalize=True)
    for t in range(tokens):
        r1, n1 = torch.empty(H, device=device, dtype=torch.float16), torch.empty(H, device=device, dtype=torch.float16)
        i1 = torch.empty(k, device=device, dtype=torch.int32)
        s1 = torch.empty(k, device=device, dtype=torch.float16)
        backend.add_rms_norm_router_topk(T(a[t]), T(b[t]), r1, T(nw), n1, 1e-5, T(w), i1, s1, bias=T(bias),
                                         renormalize=True)
        assert_bits_equal(from_torch_bits(res[t]), from_torch_bits(r1), f"residual {t}")
        assert_bits_equal(from_torch_bits(normed[t]), from_torch_bits(n1), f"normed {t}")
        assert torch.equal(idx[t], i1)
        assert_bits_equal(from_torch_bits(sc[t]), from_torch_bits(s1), f"scores {t}")
    for _ in range(2):
        r2, n2 = torch.empty_like(res), torch.empty_like(res)
        i2, s2 = torch.empty_like(idx), torch.empty_like(sc)
        backend.add_rms_norm_router_topk(T(a), T(b), r2, T(nw), n2, 1e-5, T(w), i2, s2, bias=T(bias), renormalize=True,
                                         split=False)
        assert torch.equal(res.view(torch.int16), r2.view(torch.int16))
        assert torch.equal(normed.view(torch.int16), n2.view(torch.int16))
        assert torch.equal(idx, i2) and torch.equal(sc.view(torch.int16), s2.view(torch.int16))
        backend.add_rms_norm_router_topk(T(a), T(b), res, T(nw), normed, 1e-5, T(w), idx, sc, bias=T(bias),
                                         renormalize=True)


def test_router_topk_on_logits_with_ties(backend, device):
    lg = np.array([1.0, 3.0, 3.0, -2.0, 3.0, 0.5, 2.0, 2.0], dtype=np.float16)
    idx = torch.empty(4, device=device, dtype=torch.int32)
    sc = torch.empty(4, device=device, dtype=torch.float16)
    backend.moe_router_topk(to_torch(lg, device), idx, sc, renormalize=True)
    assert idx.cpu().tolist() == [1, 2, 4, 6]  # equal logits: lowest index first
    widx = np.empty(4, dtype=np.int32)
    wsc = np.empty(4, dtype=np.float16)
    oracle.lib().tto_topk(P(lg), oracle.F16, 8, 4, 1, P(widx), P(wsc), oracle.F16)
    assert_bits_equal(from_torch_bits(sc), wsc, "topk scores")
    assert_f64(from_torch_bits(sc), ref.topk_softmax64(lg, 4, True)[1], "topk scores")


@pytest.mark.parametrize("E,k,renorm,special", [(128, 128, True, False), (128, 100, False, True), (65, 64, True, True),
                                                (100, 7, False, False), (32, 4, True, True), (3, 3, False, True)])
def test_router_topk_wave_selection(backend, device, E, k, renorm, special):
    """Many equal values (coarse quantisation), signed zeros, -inf and NaN logits:
    slot order, indices and scores equal the sequential oracle scan."""
    g = rng(E * 1000 + k)
    lg = (np.round(g.standard_normal(E) * 2) / 2).astype(np.float16)
    if special:
        lg[g.integers(0, E, size=max(1, E // 8))] = np.float16(0.0)
        lg[g.integers(0, E, size=max(1, E // 8))] = np.float16(-0.0)
        lg[g.integers(0, E, size=max(1, E // 16))] = np.float16(-np.inf)
        lg[g.integers(1, E, size=max(1, E // 16))] = np.float16(np.nan)
    idx = torch.empty(k, device=device, dtype=torch.int32)
    sc = torch.empty(k, device=device, dtype=torch.float16)
    backend.moe_router_topk(to_torch(lg, device), idx, sc, renormalize=renorm)
    widx = np.empty(k, dtype=np.int32)
    wsc = np.empty(k, dtype=np.float16)
    oracle.lib().tto_topk(P(lg), oracle.F16, E, k, int(renorm), P(widx), P(wsc), oracle.F16)
    assert np.array_equal(idx.cpu().numpy(), widx)
    assert_bits_equal(from_torch_bits(sc), wsc, "topk scores")
    if not special:  # NaN-free logits: stable-sort brute force and float64 softmax
        idx64, sc64 = ref.topk_softmax64(lg, k, renorm)
        assert np.array_equal(idx.cpu().numpy(), idx64)
        assert_f64(from_torch_bits(sc), sc64, "topk scores")


@pytest.mark.parametrize("rows,cols", [(128256, 2048), (201088, 2880), (4099, 5120)])
def test_lm_head_argmax(backend, device, rows, cols):
    g = rng(rows)
    w = f16_normal(g, (rows, cols), 0.02)
    x = f16_normal(g, cols)
    w_t = to_torch(w, device)
    tok = backend.matvec_argmax_tensor(w_t, to_torch(x, device))
    logits = from_torch_bits(backend.logits_buffer(rows, torch.float16))
    want_logits = oracle.gemv("f16w", "none", w.view(np.uint8).reshape(rows, -1), None, x, cols=cols, lpr=lanes(cols))
    assert_bits_equal(logits, want_logits, "lm_head logits")
    assert_f64(logits, ref.gemv64(w, x), "lm_head logits")
    want = int(np.argmax(want_logits.astype(np.float32)))
    assert int(tok.item()) == want == int(oracle.lib().tto_argmax(P(want_logits), oracle.F16, rows))


def test_argmax_ties_pick_lowest_index(backend, device):
    rows, cols = 5000, 64
    w = np.zeros((rows, cols), dtype=np.float16)
    w[[17, 3001, 4999], 0] = 1.0   # three identical maxima
    x = np.zeros(cols, dtype=np.float16)
    x[0] = 2.0
    tok = backend.matvec_argmax_tensor(to_torch(w, device), to_torch(x, device))
    assert int(tok.item()) == 17


def test_argmax_modes_rounded_vs_unrounded(device):
    """Rows 17 and 3001 tie after rounding to fp16 (1.0 and 1 + 2^-13) but not in
    binary32: the default mode picks the lower index of the rounded tie, the two-stage
    and persistent modes the larger binary32 value (triton_kernels.py:2245-2250,
    2524-2537), and argmax_mode="triton_two_stage" routes matvec_argmax_tensor there."""
    from thintensor_amd.backend import HipDecodeBackend

    rows, cols = 5000, 64
    w = np.zeros((rows, cols), dtype=np.float16)
    w[17, 0] = 1.0
    w[3001, 0] = 1.0
    w[3001, 1] = 1.0
    x = np.zeros(cols, dtype=np.float16)
    x[0], x[1] = 1.0, 2.0 ** -13
    be = HipDecodeBackend(device, torch.float16, cols, cols, cols, cols)
    wt, xt = to_torch(w, device), to_torch(x, device)
    assert int(be.matvec_argmax_tensor(wt, xt).item()) == 17
    assert int(be._matvec_argmax_tensor_triton_two_stage(wt, xt).item()) == 3001
    assert int(be.persistent_vocab_block_matvec_argmax_tensor(wt, xt).item()) == 3001
    be2 = HipDecodeBackend(device, torch.float16, cols, cols, cols, cols, argmax_mode="triton_two_stage")
    assert int(be2.matvec_argmax_tensor(wt, xt).item()) == 3001


@pytest.mark.parametrize("rows,cols", [(128256, 2048), (4099, 5120)])
def test_unrounded_argmax_matches_binary32_logits(backend, device, rows, cols):
    g = rng(rows + 5)
    w = f16_normal(g, (rows, cols), 0.02)
    x = f16_normal(g, cols)
    tok = backend.persistent_vocab_block_matvec_argmax_tensor(to_torch(w, device), to_torch(x, device))
    lg32 = oracle.gemv("f16w", "none", w.view(np.uint8).reshape(rows, -1), None, x, cols=cols, lpr=lanes(cols),
                       odtype=oracle.F32)
    assert int(tok.item()) == int(np.argmax(lg32))
    assert int(np.argmax(lg32)) == int(np.argmax(ref.gemv64(w, x)))


@pytest.mark.parametrize("heads,kv_heads,tokens,cap", [
    (32, 8, 577, 640),     # the 1B decode shape: ten active chunks, all from the first request
    (32, 8, 1500, 1536),   # 24 chunks: past the 16 requested with the weights
    (16, 16, 1, 64),       # one token, one query head per KV head
    (32, 4, 130, 1024),    # eight query heads per KV head, most of the capacity unused
    (8, 2, 200, 256),      # four heads of 64 (cols 512: 16 lanes per row)
    (32, 8, 8300, 8320),   # 130 chunks x 8 KV heads > 1024 workgroups: two chunks per workgroup, odd count on the 2nd call
])
def test_attention_then_int4_matvec(backend, device, heads, kv_heads, tokens, cap):
    """o_proj that combines the attention chunk partials itself: the combined activation
    equals single_token_gqa_attention's output bit for bit (and the oracle's), and the
    GEMV equals int4_scaled_matvec over it (and the oracle's) bit for bit.  Two calls in
    a row on one scratch, the second with fewer tokens."""
    from thintensor_amd import layouts

    D = 64
    cols, rows = heads * D, 2048
    g = rng(heads * 7 + tokens)
    q = f16_normal(g, cols)
    keys = f16_normal(g, (kv_heads, cap, D))
    vals = f16_normal(g, (kv_heads, cap, D))
    codes = g.integers(0, 16, size=(rows, cols), dtype=np.uint8)
    packed = layouts.pack_int4(codes)
    scales = (np.abs(g.standard_normal((rows, cols // 128))) * 0.02).astype(np.float16)
    qd, kd, vd = to_torch(q, device), to_torch(keys, device), to_torch(vals, device)
    pd, sd = to_torch(packed, device), to_torch(scales, device)
    attn = torch.empty(cols, device=device, dtype=torch.float16)
    attn_ref = torch.empty(cols, device=device, dtype=torch.float16)
    out = torch.empty(rows, device=device, dtype=torch.float16)
    out_ref = torch.empty(rows, device=device, dtype=torch.float16)
    for n in (tokens, max(1, tokens // 2 - 3)):
        pos = torch.tensor([n - 1], dtype=torch.int32, device=device)
        backend.attention_then_int4_matvec(qd, kd, vd, heads, kv_heads, D, pd, sd, out, active_tokens=(pos, 1),
                                           attn_out=attn)
        backend.single_token_gqa_attention(qd, kd, vd, attn_ref, heads, kv_heads, D, active_tokens=(pos, 1))
        backend.int4_scaled_matvec(pd, sd, attn_ref, out_ref, rows=rows, cols=cols, group_size=128)
        assert_bits_equal(from_torch_bits(attn), from_torch_bits(attn_ref), f"combined activation ({n} tokens)")
        assert_bits_equal(from_torch_bits(out), from_torch_bits(out_ref), f"o_proj ({n} tokens)")
        want_attn = np.empty(cols, dtype=np.float16)
        oracle.lib().tto_attention(P(q), P(keys), P(vals), oracle.F16, cap * D, D, cap * D, D, None, oracle.F16, n,
                                   heads, kv_heads, D, P(want_attn))
        assert_bits_equal(from_torch_bits(attn), want_attn, f"attention vs oracle ({n} tokens)")
        want = oracle.gemv("int4_sym", "group", packed, scales, want_attn, cols=cols, lpr=lanes(cols, 4), L=4,
                           s_row=cols // 128, s_grp=1)
        assert_bits_equal(from_torch_bits(out), want, f"o_proj vs oracle ({n} tokens)")


def test_attention_then_int4_matvec_rejects(backend, device):
    D, heads = 64, 48   # more than 32 query heads
    q = torch.zeros(heads * D, device=device, dtype=torch.float16)
    kv = torch.zeros((heads, 64, D), device=device, dtype=torch.float16)
    pk = torch.zeros((16, heads * D // 2), device=device, dtype=torch.uint8)
    sc = torch.zeros((16, heads * D // 128), device=device, dtype=torch.float16)
    out = torch.empty(16, device=device, dtype=torch.float16)
    with pytest.raises((ValueError, NotImplementedError, RuntimeError)):
        backend.attention_then_int4_matvec(q, kv, kv, heads, heads, D, pk, sc, out, active_tokens=10)
