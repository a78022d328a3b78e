"""GPU parity of the GEMV family against the CPU oracle.

Each case checks the HIP output (a) bit for bit against the binary32 restatement
in the kernels' reduction order and (b) against the float64 dequantise-then-matmul
closed form of the reference within the north-star tolerance (max relative error
1e-2, measured as max|diff| / max|ref|).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from oracle import ref
from tests.helpers import bf16_bits, bf16_to_f32, f16_normal, from_torch_bits, rng, to_torch
from thintensor_amd import _lib
from thintensor_amd import layouts

pytestmark = pytest.mark.gpu

TOL = 1e-2


def lanes(cols: int, group_chunks: int = 1) -> int:
    return _lib.load().tt_gemv_lanes_per_row(cols // 32, group_chunks)


def assert_bits_equal(got: np.ndarray, want: np.ndarray, what: str) -> None:
    g = got.view(np.uint16) if got.dtype != np.float32 else got.view(np.uint32)
    w = want.view(np.uint16) if want.dtype != np.float32 else want.view(np.uint32)
    bad = np.nonzero(g != w)[0]
    assert bad.size == 0, f"{what}: {bad.size} of {g.size} outputs differ; first at {bad[:5]}: got {got[bad[:5]]} want {want[bad[:5]]}"


def as_float(a: np.ndarray) -> np.ndarray:
    return bf16_to_f32(a) if a.dtype == np.uint16 else a.astype(np.float64)


INT4_CASES = [
    # rows, cols, group, scale dtype, x dtype, out dtype
    (8192, 2048, 128, np.float16, "f16", "f16"),   # BASELINE cfg0
    (2048, 8192, 128, np.float16, "f16", "f16"),   # cfg1 down_proj
    (512, 2048, 128, np.float16, "f16", "f16"),    # cfg1 k/v
    (1000, 5120, 128, np.float32, "f16", "f32"),   # cfg4a K, ragged rows, fp32 scales
    (384, 2048, 2048, np.float16, "f16", "f16"),   # one scale per row
    (300, 1024, 64, np.float16, "bf16", "bf16"),   # bf16 activations
    (257, 4096, 2048, np.float32, "f16", "f16"),   # group spanning many lanes
    (1, 32, 32, np.float16, "f16", "f16"),         # one row, one chunk
    (5, 2880, 32, np.float16, "f16", "f16"),       # 90 chunks: ragged last round of 32 lanes
    (7, 160, 32, np.float32, "f16", "f32"),        # 5 chunks on 16 lanes
    (96, 5632, 128, np.float16, "f16", "f16"),     # 16 lanes per row, 11 rounds: blocks of four and a tail
    (2048, 6144, 128, np.float16, "f16", "f16"),   # three rounds, requested together
    (16400, 5120, 128, np.float16, "f16", "f16"),  # four rows per wave of five rounds, ragged last batch
]


@pytest.mark.parametrize("rows,cols,group,sdt,xdt,odt", INT4_CASES)
def test_int4_scaled_matvec(backend, device, rows, cols, group, sdt, xdt, odt):
    g = rng(rows * 7 + cols)
    codes = g.integers(0, 16, size=(rows, cols), dtype=np.uint8)
    packed = layouts.pack_int4(codes)
    groups = max(cols // group, 1)
    scales = (np.abs(g.standard_normal((rows, groups))) * 0.02).astype(sdt)
    xf = g.standard_normal(cols).astype(np.float32)
    if xdt == "f16":
        x_np = xf.astype(np.float16)
        x_t = to_torch(x_np, device)
    else:
        x_np = bf16_bits(xf)
        x_t = to_torch(x_np, device, bf16=True)
    odtype = {"f16": torch.float16, "bf16": torch.bfloat16, "f32": torch.float32}[odt]
    out = torch.empty(rows, device=device, dtype=odtype)
    backend.int4_scaled_matvec(to_torch(packed, device), to_torch(scales, device), x_t, out, rows=rows, cols=cols,
                               group_size=group)
    got = from_torch_bits(out)
    L = 1 if group >= cols else group // 32
    smode = "row" if group >= cols else "group"
    want = oracle.gemv("int4_sym", smode, packed, scales, x_np, cols=cols, lpr=lanes(cols, L), L=L, s_row=groups,
                       s_grp=1, odtype={"f16": oracle.F16, "bf16": oracle.BF16, "f32": oracle.F32}[odt])
    assert_bits_equal(got, want, f"int4 {rows}x{cols} g{group}")
    w64 = ref.int4_dequant(packed, scales, group)
    y64 = ref.gemv64(w64, as_float(x_np))
    assert ref.max_rel_err(as_float(got), y64) < TOL


def test_int4_uint32_view_and_affine(backend, device):
    rows, cols, group = 640, 2048, 128
    g = rng(11)
    codes = g.integers(0, 16, size=(rows, cols), dtype=np.uint8)
    packed = layouts.pack_int4(codes)
    sm = np.stack([np.abs(g.standard_normal((rows, cols // group))) * 0.02,
                   g.standard_normal((rows, cols // group)) * 0.01], axis=-1).astype(np.float16)
    x = f16_normal(g, cols)
    out = torch.empty(rows, device=device, dtype=torch.float16)
    # the uint32 view of the same bytes (8 codes per word) is accepted unchanged
    packed_u32 = to_torch(layouts.int4_as_u32(packed).view(np.int32), device)
    backend.int4_scaled_matvec(packed_u32, to_torch(sm, device), to_torch(x, device), out, rows=rows, cols=cols,
                               group_size=group)
    want = oracle.gemv("int4_aff", "group_aff", packed, sm, x, cols=cols, lpr=lanes(cols, 4), L=4,
                       s_row=sm.shape[1] * 2, s_grp=2, s_pair=1)
    got = from_torch_bits(out)
    assert_bits_equal(got, want, "affine int4")
    assert ref.max_rel_err(got, ref.gemv64(ref.int4_dequant(packed, sm, group), x)) < TOL


def test_multi_int4_qkv(backend, device):
    cols, group = 2048, 128
    rows = (2048, 512, 512)
    g = rng(5)
    mats, scs, wants = [], [], []
    x = f16_normal(g, cols)
    for r in rows:
        p = layouts.pack_int4(g.integers(0, 16, size=(r, cols), dtype=np.uint8))
        s = (np.abs(g.standard_normal((r, cols // group))) * 0.02).astype(np.float16)
        mats.append(to_torch(p, device))
        scs.append(to_torch(s, device))
        wants.append(oracle.gemv("int4_sym", "group", p, s, x, cols=cols, lpr=lanes(cols, 4), L=4, s_row=s.shape[1], s_grp=1))
    out = torch.empty(sum(rows), device=device, dtype=torch.float16)
    backend.multi_int4_scaled_matvec(tuple(mats), tuple(scs), rows, cols, to_torch(x, device), out, group_size=group)
    assert_bits_equal(from_torch_bits(out), np.concatenate(wants), "multi int4")


@pytest.mark.parametrize("rows,cols", [(1000, 5120), (4096, 2048), (130, 2880)])
def test_fp8_scaled_matvec(backend, device, rows, cols):
    g = rng(rows + cols)
    w = g.standard_normal((rows, cols)).astype(np.float32) * 0.05
    w_t = torch.from_numpy(w).to(torch.float8_e4m3fn)
    bits = w_t.view(torch.uint8).numpy()
    s = (np.abs(g.standard_normal(rows)) * 0.1 + 0.01).astype(np.float32)
    x = f16_normal(g, cols)
    out = torch.empty(rows, device=device, dtype=torch.float16)
    backend.scaled_matvec(w_t.to(device), to_torch(s, device), to_torch(x, device), out)
    want = oracle.gemv("fp8", "row", bits, s, x, cols=cols, lpr=lanes(cols), s_row=1)
    got = from_torch_bits(out)
    assert_bits_equal(got, want, "fp8")
    y64 = ref.gemv64(ref.fp8_e4m3fn(bits) * s[:, None].astype(np.float64), x)
    assert ref.max_rel_err(got, y64) < TOL


@pytest.mark.parametrize("rows,cols,wdt", [(2000, 2048, "f16"), (4096 + 512 + 512, 2880, "f16"), (333, 4096, "bf16")])
def test_dense_matvec(backend, device, rows, cols, wdt):
    g = rng(rows)
    if wdt == "f16":
        w = f16_normal(g, (rows, cols), 0.02)
        w_t = to_torch(w, device)
        wf = w.astype(np.float64)
    else:
        wf32 = g.standard_normal((rows, cols)).astype(np.float32) * 0.02
        w = bf16_bits(wf32)
        w_t = to_torch(w, device, bf16=True)
        wf = bf16_to_f32(w).astype(np.float64)
    x = f16_normal(g, cols)
    out = torch.empty(rows, device=device, dtype=torch.float16)
    backend.matvec(w_t, to_torch(x, device), out)
    want = oracle.gemv("f16w" if wdt == "f16" else "bf16w", "none", w.view(np.uint8).reshape(rows, -1), None, x,
                       cols=cols, lpr=lanes(cols))
    got = from_torch_bits(out)
    assert_bits_equal(got, want, "dense matvec")
    assert ref.max_rel_err(got, ref.gemv64(wf, x)) < TOL


def test_multi_matvec_qkv(backend, device):
    cols = 2880
    rows = (4096, 512, 512)
    g = rng(17)
    ws = [f16_normal(g, (r, cols), 0.02) for r in rows]
    x = f16_normal(g, cols)
    out = torch.empty(sum(rows), device=device, dtype=torch.float16)
    backend.multi_matvec(tuple(to_torch(w, device) for w in ws), to_torch(x, device), out, block_m=64)
    want = np.concatenate([oracle.gemv("f16w", "none", w.view(np.uint8).reshape(w.shape[0], -1), None, x, cols=cols,
                                       lpr=lanes(cols)) for w in ws])
    assert_bits_equal(from_torch_bits(out), want, "multi matvec")


def _mxfp4_expert_weights(g, experts, rows, cols):
    codes = g.integers(0, 16, size=(experts, rows, cols), dtype=np.uint8)
    blocks = layouts.pack_mxfp4_blocks(codes)
    scales = g.integers(119, 124, size=(experts, rows, cols // 32), dtype=np.uint8)
    return blocks, scales


@pytest.mark.parametrize("per_slot_x", [False, True])
def test_mxfp4_selected_matvec(backend, device, per_slot_x):
    experts, rows, cols, top_k = 8, 5760, 2880, 4
    g = rng(21 + per_slot_x)
    blocks, scales = _mxfp4_expert_weights(g, experts, rows, cols)
    idx = np.array([5, 0, 7, 2], dtype=np.int32)
    x = f16_normal(g, (top_k, cols) if per_slot_x else cols)
    out = torch.empty((top_k, rows), device=device, dtype=torch.float16)
    backend.mxfp4_selected_matvec(to_torch(blocks, device), to_torch(scales, device), to_torch(x, device),
                                  to_torch(idx, device), out)
    got = from_torch_bits(out)
    lpr = lanes(cols)
    for s, e in enumerate(idx):
        xs = x[s] if per_slot_x else x
        want = oracle.gemv("mxfp4", "block_e8", blocks[e].reshape(rows, -1), scales[e], xs, cols=cols, lpr=lpr,
                           s_row=cols // 32)
        assert_bits_equal(got[s], want, f"mxfp4 slot {s}")
        y64 = ref.gemv64(ref.mxfp4_dequant(blocks[e], scales[e]), xs)
        assert ref.max_rel_err(got[s], y64) < TOL


@pytest.mark.parametrize("bits", [1, 2])
def test_lowbit_selected_matvec(backend, device, bits):
    experts, rows, cols = 6, 2880, 2880
    g = rng(31 + bits)
    codes = g.integers(0, 1 << bits, size=(experts, rows, cols), dtype=np.uint8)
    packed = layouts.pack_lowbit_blocks(codes, bits)
    scales = g.integers(118, 124, size=(experts, rows, cols // 32), dtype=np.uint8)
    idx = np.array([3, 1], dtype=np.int32)
    x = f16_normal(g, cols)
    out = torch.empty((2, rows), device=device, dtype=torch.float16)
    backend.mxfp_lowbit_selected_matvec(to_torch(packed, device), to_torch(scales, device), to_torch(x, device),
                                        to_torch(idx, device), out, bits=bits)
    got = from_torch_bits(out)
    for s, e in enumerate(idx):
        want = oracle.gemv("q2e8" if bits == 2 else "q1e8", "block_e8", packed[e].reshape(rows, -1), scales[e], x,
                           cols=cols, lpr=lanes(cols), s_row=cols // 32)
        assert_bits_equal(got[s], want, f"q{bits} slot {s}")
        assert ref.max_rel_err(got[s], ref.gemv64(ref.lowbit_e8_dequant(packed[e], scales[e], bits), x)) < TOL


@pytest.mark.parametrize("bits,with_bias", [(2, True), (1, False), (4, True)])
def test_fused_swiglu(backend, device, bits, with_bias):
    experts, inter, cols, top_k = 4, 2880, 2880, 4
    g = rng(41 + bits)
    if bits == 4:
        packed, scales = _mxfp4_expert_weights(g, experts, 2 * inter, cols)
        fmt = 5
        rt = oracle.F16
    else:
        codes = g.integers(0, 1 << bits, size=(experts, 2 * inter, cols), dtype=np.uint8)
        packed = layouts.pack_lowbit_blocks(codes, bits)
        scales = g.integers(118, 123, size=(experts, 2 * inter, cols // 32), dtype=np.uint8)
        fmt = 6 if bits == 2 else 7
        rt = oracle.BF16
    bias = f16_normal(g, (experts, 2 * inter), 0.5) if with_bias else None
    idx = np.array([2, 0, 3, 1], dtype=np.int32)
    x = f16_normal(g, cols)
    out = torch.empty((top_k, inter), device=device, dtype=torch.float16)
    backend.mxfp_lowbit_selected_swiglu(to_torch(packed, device), to_torch(scales, device), to_torch(x, device),
                                        to_torch(idx, device), out, bits=bits, alpha=1.702, limit=7.0,
                                        bias=to_torch(bias, device) if with_bias else None)
    want = np.empty((top_k, inter), dtype=np.float16)
    pw = np.ascontiguousarray(packed)
    sw = np.ascontiguousarray(scales)
    L = oracle.lib()
    rc = L.tto_swiglu(fmt, rt, pw.ctypes.data, pw.strides[0], pw.strides[1], sw.ctypes.data, sw.strides[0],
                      sw.strides[1], x.ctypes.data, oracle.F16, 0, idx.ctypes.data, top_k,
                      bias.ctypes.data if with_bias else None, oracle.F16, 2 * inter, 1.702, 7.0, want.ctypes.data,
                      oracle.F16, inter, inter, cols, lanes(cols))
    assert rc == 0
    assert_bits_equal(from_torch_bits(out).reshape(-1), want.reshape(-1), f"swiglu q{bits}")
    rnd = ref.f16_round64 if bits == 4 else ref.bf16_round64
    dq = ref.mxfp4_dequant(packed, scales) if bits == 4 else ref.lowbit_e8_dequant(packed, scales, bits)
    want64 = np.stack([ref.expert_swiglu64(dq[e], x, bias[e] if with_bias else None, 1.702, 7.0, rnd) for e in idx])
    assert ref.max_rel_err(from_torch_bits(out), want64) < TOL


@pytest.mark.parametrize("bits", [2, 4])
def test_fused_weighted_down(backend, device, bits):
    experts, rows, cols, top_k = 4, 2880, 2880, 4
    g = rng(51 + bits)
    if bits == 4:
        packed, scales = _mxfp4_expert_weights(g, experts, rows, cols)
        fmt, rt = 5, oracle.F16
    else:
        codes = g.integers(0, 4, size=(experts, rows, cols), dtype=np.uint8)
        packed = layouts.pack_lowbit_blocks(codes, 2)
        scales = g.integers(118, 123, size=(experts, rows, cols // 32), dtype=np.uint8)
        fmt, rt = 6, oracle.BF16
    bias = f16_normal(g, (experts, rows), 0.5)
    idx = np.array([1, 3, 0, 2], dtype=np.int32)
    scores = np.array([0.4, 0.3, 0.2, 0.1], dtype=np.float16)
    x = f16_normal(g, (top_k, cols))
    out = torch.empty(rows, device=device, dtype=torch.float16)
    backend.mxfp_lowbit_weighted_down(to_torch(packed, device), to_torch(scales, device), to_torch(x, device),
                                      to_torch(idx, device), to_torch(scores, device), out, bits=bits,
                                      bias=to_torch(bias, device))
    want = np.empty(rows, dtype=np.float16)
    pw, sw = np.ascontiguousarray(packed), np.ascontiguousarray(scales)
    rc = oracle.lib().tto_weighted_down(fmt, rt, pw.ctypes.data, pw.strides[0], pw.strides[1], sw.ctypes.data,
                                        sw.strides[0], sw.strides[1], x.ctypes.data, oracle.F16, cols, idx.ctypes.data,
                                        scores.ctypes.data, oracle.F16, top_k, bias.ctypes.data, oracle.F16, rows,
                                        want.ctypes.data, oracle.F16, rows, cols, lanes(cols))
    assert rc == 0
    assert_bits_equal(from_torch_bits(out), want, f"weighted down bits={bits}")
    rnd = ref.f16_round64 if bits == 4 else ref.bf16_round64
    dq = ref.mxfp4_dequant(packed, scales) if bits == 4 else ref.lowbit_e8_dequant(packed, scales, 2)
    want64 = ref.weighted_down64([dq[e] for e in idx], x, scores, [bias[e] for e in idx], rnd)
    assert ref.max_rel_err(from_torch_bits(out), want64) < TOL


@pytest.mark.parametrize("m,rows,cols,wdt", [(8, 2880, 4096, "f16"), (3, 1000, 2048, "bf16"), (5, 300, 5120, "f16"),
                                            (13, 2880, 4096, "f16"), (2, 77, 96, "f16")])
def test_matvec_bias_rows(backend, device, m, rows, cols, wdt):
    """M activation rows in one launch (or one per row past 4096 columns) equal the
    single-row GEMV with bias row by row."""
    g = rng(m + rows + cols)
    T = lambda a, bf=False: to_torch(a, device, bf16=bf)
    if wdt == "bf16":
        w = T(bf16_bits(g.standard_normal((rows, cols)).astype(np.float32) * 0.02), True)
        x = T(bf16_bits(g.standard_normal((m, cols)).astype(np.float32)), True)
        b = T(bf16_bits(g.standard_normal(rows).astype(np.float32) * 0.1), True)
        dt = torch.bfloat16
    else:
        w, x, b = T(f16_normal(g, (rows, cols), 0.02)), T(f16_normal(g, (m, cols))), T(f16_normal(g, rows, 0.1))
        dt = torch.float16
    out = torch.empty((m, rows), device=device, dtype=dt)
    backend.matvec_bias_rows(w, b, x, out)
    for t in range(m):
        o1 = torch.empty(rows, device=device, dtype=dt)
        backend.multi_matvec_bias((w,), (b,), x[t], o1)
        assert_bits_equal(from_torch_bits(out[t]), from_torch_bits(o1), f"row {t}")


@pytest.mark.parametrize("bits,tokens,same", [(4, 8, False), (2, 3, False), (4, 16, True), (1, 5, False),
                                              (4, 17, False)])
def test_expert_kernels_token_batched(backend, device, bits, tokens, same):
    """SwiGLU and weighted down over several tokens (each with its own activation
    vector, experts and scores) equal the single-token operators token by token.  Six
    experts, so slots share experts (`same`: every token picks the same experts)."""
    experts, inter, cols, top_k = 6, 2880, 2880, 4
    g = rng(71 + bits + tokens)
    if bits == 4:
        gu, gus = _mxfp4_expert_weights(g, experts, 2 * inter, cols)
        dw, dws = _mxfp4_expert_weights(g, experts, cols, inter)
    else:
        gu = layouts.pack_lowbit_blocks(g.integers(0, 4, size=(experts, 2 * inter, cols), dtype=np.uint8), 2)
        gus = g.integers(118, 123, size=(experts, 2 * inter, cols // 32), dtype=np.uint8)
        dw = layouts.pack_lowbit_blocks(g.integers(0, 4, size=(experts, cols, inter), dtype=np.uint8), 2)
        dws = g.integers(118, 123, size=(experts, cols, inter // 32), dtype=np.uint8)
    gub, db = f16_normal(g, (experts, 2 * inter), 0.5), f16_normal(g, (experts, cols), 0.5)
    if same:
        idx = np.tile(g.permutation(experts)[:top_k], (tokens, 1)).astype(np.int32)
    else:
        idx = np.stack([g.permutation(experts)[:top_k] for _ in range(tokens)]).astype(np.int32)
    sc = g.dirichlet(np.ones(top_k), size=tokens).astype(np.float16)
    x = f16_normal(g, (tokens, cols))
    T = lambda a: to_torch(a, device)
    gu_d, gus_d, dw_d, dws_d, gub_d, db_d = T(gu), T(gus), T(dw), T(dws), T(gub), T(db)
    act = torch.empty((tokens * top_k, inter), device=device, dtype=torch.float16)
    backend.mxfp_lowbit_selected_swiglu_tokens(gu_d, gus_d, T(x), T(idx), act, bits=bits, alpha=1.702, limit=7.0,
                                               bias=gub_d)
    out = torch.empty((tokens, cols), device=device, dtype=torch.float16)
    backend.mxfp_lowbit_weighted_down_tokens(dw_d, dws_d, act, T(idx), T(sc), out, bits=bits, bias=db_d)
    for t in range(tokens):
        a1 = torch.empty((top_k, inter), device=device, dtype=torch.float16)
        backend.mxfp_lowbit_selected_swiglu(gu_d, gus_d, T(x[t]), T(idx[t]), a1, bits=bits, alpha=1.702, limit=7.0,
                                            bias=gub_d)
        assert_bits_equal(from_torch_bits(act[t * top_k:(t + 1) * top_k]).reshape(-1),
                          from_torch_bits(a1).reshape(-1), f"swiglu token {t}")
        o1 = torch.empty(cols, device=device, dtype=torch.float16)
        backend.mxfp_lowbit_weighted_down(dw_d, dws_d, a1, T(idx[t]), T(sc[t]), o1, bits=bits, bias=db_d)
        assert_bits_equal(from_torch_bits(out[t]), from_torch_bits(o1), f"weighted down token {t}")


# cfg2 shapes (17920 x 5120 q2, 5120 x 5120 q1), every lanes-per-row choice, odd group
# counts (q1 falls back to the generic kernel), rows not a multiple of a wave's rows, bf16
@pytest.mark.parametrize("bits,rows,cols,bf16", [(2, 17920, 5120, False), (1, 5120, 5120, False),
                                                 (2, 1000, 2048, True), (1, 999, 2048, True),
                                                 (2, 77, 960, False), (1, 77, 960, False),
                                                 (1, 300, 4096, False), (2, 64, 192, True), (1, 130, 128, False)])
def test_lowbit_affine_matvec(backend, device, bits, rows, cols, bf16):
    group = 64
    g = rng(61 + bits + cols)
    codes = g.integers(0, 1 << bits, size=(rows, cols), dtype=np.uint8)
    packed = layouts.pack_bits(codes, bits)
    sz = np.stack([np.abs(g.standard_normal((rows, cols // group))) * 0.05,
                   g.uniform(0, (1 << bits) - 1, size=(rows, cols // group))], axis=-1).astype(np.float16)
    xf = g.standard_normal(cols).astype(np.float32)
    x = bf16_bits(xf) if bf16 else xf.astype(np.float16)
    odt = torch.bfloat16 if bf16 else torch.float16
    out = torch.empty(rows, device=device, dtype=odt)
    backend.lowbit_affine_matvec(to_torch(packed, device), to_torch(sz, device), to_torch(x, device, bf16=bf16), out,
                                 bits=bits, rows=rows, cols=cols, group_size=group)
    got = from_torch_bits(out)
    want = oracle.gemv("q2aff" if bits == 2 else "q1aff", "group_aff", packed, sz, x, cols=cols, lpr=lanes(cols, 2),
                       L=2, s_row=sz.shape[1] * 2, s_grp=2, s_pair=1, aff_zero=1,
                       odtype=oracle.BF16 if bf16 else oracle.F16)
    assert_bits_equal(got, want, f"affine q{bits} {rows}x{cols}")
    xd = bf16_to_f32(x) if bf16 else x
    y64 = ref.gemv64(ref.lowbit_affine_dequant(packed, sz, bits, group, cols), xd)
    gotf = bf16_to_f32(got) if bf16 else got
    assert ref.max_rel_err(gotf, y64) < TOL


@pytest.mark.parametrize("scale_dtype", [np.float16, np.float32])
def test_int4_selected_matvec(backend, device, scale_dtype):
    """The reference's int4 expert packs carry fp32 group scales (gpu_runtime.py:2613-2615)."""
    experts, rows, cols, group = 5, 1024, 2048, 128
    g = rng(71)
    codes = g.integers(0, 16, size=(experts, rows, cols), dtype=np.uint8)
    packed = layouts.pack_int4(codes)
    scales = (np.abs(g.standard_normal((experts, rows, cols // group))) * 0.02).astype(scale_dtype)
    idx = np.array([4, 1, 1], dtype=np.int32)
    x = f16_normal(g, (3, cols))
    out = torch.empty((3, rows), device=device, dtype=torch.float16)
    backend.int4_selected_matvec(to_torch(packed, device), to_torch(scales, device), to_torch(x, device),
                                 to_torch(idx, device), out, group_size=group)
    got = from_torch_bits(out)
    for s, e in enumerate(idx):
        want = oracle.gemv("int4_sym", "group", packed[e], scales[e], x[s], cols=cols, lpr=lanes(cols, 4), L=4,
                           s_row=cols // group, s_grp=1)
        assert_bits_equal(got[s], want, f"int4 selected slot {s}")
        assert ref.max_rel_err(got[s], ref.gemv64(ref.int4_dequant(packed[e], scales[e], group), x[s])) < TOL
