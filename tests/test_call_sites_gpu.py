"""The reference runtime's call sites, replayed against HipDecodeBackend.

Each test calls a backend method with the dtypes, shapes, views and strides that
`ThinGpuCausalLMRuntime` (thinruntime/gpu_runtime.py) passes at the cited line, and
checks the result bit for bit against the CPU oracle.  Selected-expert operators run
with the int32 router ids and with torch.long ids; both must give the same bits.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from oracle import ref
from oracle import ternary as T
from tests.helpers import f16_normal, from_torch_bits, rng, to_torch
from tests.test_gemv_gpu import assert_bits_equal, lanes
from thintensor_amd import layouts

pytestmark = pytest.mark.gpu

TOL = 1e-2
ID_DTYPES = [torch.int32, torch.long]


def P(a):
    return a.ctypes.data


def _mxfp4(g, experts, rows, cols):
    blocks = g.integers(0, 256, size=(experts, rows, cols // 32, 16), dtype=np.uint8)
    scales = g.integers(119, 124, size=(experts, rows, cols // 32), dtype=np.uint8)
    return blocks, scales


@pytest.mark.parametrize("bits", [1, 2])
def test_dense_lowbit_page_as_one_expert(backend, device, bits):
    """Dense q1/q2 page (gpu_runtime.py:12056-12079): the flat page viewed as
    [1, rows, groups, bytes_per_group], scales as [1, rows, groups], a torch.long
    zero expert id, x [cols] and the output viewed as [1, rows]."""
    rows, cols = 1536, 5120
    g = rng(900 + bits)
    codes = g.integers(0, 1 << bits, size=(1, rows, cols), dtype=np.uint8)
    packed = layouts.pack_lowbit_blocks(codes, bits)            # [1, rows, groups, bpg]
    scales = g.integers(118, 124, size=(1, rows, cols // 32), dtype=np.uint8)
    x = f16_normal(g, cols)
    bpg = 4 if bits == 1 else 8
    weight_page = to_torch(packed.reshape(-1), device)         # the stored page is flat bytes
    scale_page = to_torch(scales.reshape(-1), device)
    packed_view = weight_page.reshape(1, rows, cols // 32, bpg)
    scale_view = scale_page.reshape(1, rows, cols // 32)
    expert_index = torch.zeros(1, device=device, dtype=torch.long)
    out = torch.empty(rows, device=device, dtype=torch.float16)
    res = backend.mxfp_lowbit_selected_tensorcore_matvec(packed_view, scale_view, to_torch(x, device), expert_index,
                                                         out.reshape(1, rows), bits=bits)
    assert res.data_ptr() == out.data_ptr()
    want = oracle.gemv("q2e8" if bits == 2 else "q1e8", "block_e8", packed[0].reshape(rows, -1), scales[0], x,
                       cols=cols, lpr=lanes(cols), s_row=cols // 32)
    assert_bits_equal(from_torch_bits(out), want, f"dense q{bits} page")
    assert ref.max_rel_err(from_torch_bits(out), ref.gemv64(ref.lowbit_e8_dequant(packed[0], scales[0], bits), x)) < TOL


@pytest.mark.parametrize("experts", [129, 256, 512])
@pytest.mark.parametrize("act", ["f16", "bf16"])
def test_router_logits_topk_above_128_experts(backend, device, experts, act):
    """Router with more than 128 rows (gpu_runtime.py:9483-9496): logits =
    torch.mv(router_weight, hidden, out=logits_buffer), += bias, then moe_router_topk
    into the int32 index buffer [:top_k] and act-dtype score buffer [:top_k]."""
    hidden_size, top_k = 2880, 8
    dt = torch.float16 if act == "f16" else torch.bfloat16
    g = torch.Generator().manual_seed(experts)
    router_weight = (torch.randn(experts, hidden_size, generator=g) * 0.02).to(dt).to(device)
    router_bias = (torch.randn(experts, generator=g) * 0.1).to(dt).to(device)
    hidden = torch.randn(hidden_size, generator=g).to(dt).to(device)
    logits_buffer = torch.empty(experts, device=device, dtype=dt)
    indices_buffer = torch.empty(32, device=device, dtype=torch.int32)
    scores_buffer = torch.empty(32, device=device, dtype=dt)
    for renorm in (True, False):
        router_logits = torch.mv(router_weight, hidden, out=logits_buffer)
        router_logits.add_(router_bias)
        idx, sc = backend.moe_router_topk(router_logits, indices_buffer[:top_k], scores_buffer[:top_k],
                                          renormalize=renorm)
        assert idx.data_ptr() == indices_buffer.data_ptr()
        lg = router_logits.cpu()
        lg_np = lg.view(torch.int16).numpy().view(np.uint16) if act == "bf16" else lg.numpy()
        code = oracle.BF16 if act == "bf16" else oracle.F16
        widx = np.empty(top_k, dtype=np.int32)
        wsc = np.empty(top_k, dtype=np.uint16 if act == "bf16" else np.float16)
        oracle.lib().tto_topk(P(lg_np), code, experts, top_k, int(renorm), P(widx), P(wsc), code)
        assert np.array_equal(idx.cpu().numpy(), widx)
        assert_bits_equal(from_torch_bits(sc), wsc, "router scores")
        idx64, sc64 = ref.topk_softmax64(lg.float().numpy(), top_k, renorm)
        assert np.array_equal(idx.cpu().numpy(), idx64)
        got = from_torch_bits(sc)
        gotf = (got.astype(np.uint32) << 16).view(np.float32) if act == "bf16" else got
        assert ref.max_rel_err(gotf, sc64) < TOL


@pytest.mark.parametrize("E,k,renorm,special", [(129, 4, True, False), (256, 8, False, True), (512, 32, True, True),
                                                (512, 512, False, False), (2000, 300, True, True),
                                                (300, 129, False, False)])
def test_router_topk_block_selection(backend, device, E, k, renorm, special):
    """More than 128 experts (one workgroup): coarse values with many ties, signed zeros,
    -inf and NaN logits give the sequential oracle scan's slots, ids and scores; NaN-free
    logits also match the stable-sort brute force and the float64 softmax."""
    g = rng(E * 7 + k)
    lg = (np.round(g.standard_normal(E) * 2) / 2).astype(np.float16)
    if special:
        lg[g.integers(0, E, size=E // 8)] = np.float16(0.0)
        lg[g.integers(0, E, size=E // 8)] = np.float16(-0.0)
        lg[g.integers(0, E, size=E // 16)] = np.float16(-np.inf)
        lg[g.integers(1, E, size=E // 16)] = np.float16(np.nan)
    idx = torch.empty(k, device=device, dtype=torch.int32)
    sc = torch.empty(k, device=device, dtype=torch.float16)
    backend.moe_router_topk(to_torch(lg, device), idx, sc, renormalize=renorm)
    widx = np.empty(k, dtype=np.int32)
    wsc = np.empty(k, dtype=np.float16)
    oracle.lib().tto_topk(P(lg), oracle.F16, E, k, int(renorm), P(widx), P(wsc), oracle.F16)
    assert np.array_equal(idx.cpu().numpy(), widx)
    assert_bits_equal(from_torch_bits(sc), wsc, "topk scores")
    if not special:
        idx64, sc64 = ref.topk_softmax64(lg, k, renorm)
        assert np.array_equal(idx.cpu().numpy(), idx64)
        assert ref.max_rel_err(from_torch_bits(sc), sc64) < TOL


def test_router_topk_nan_first_untaken(backend, device):
    """A NaN at the first untaken position is taken for that slot (the sequential scan
    starts there and nothing compares greater); NaNs elsewhere are never taken."""
    E, k = 200, 3
    lg = np.full(E, -1.0, dtype=np.float16)
    lg[0] = np.float16(np.nan)
    lg[150] = np.float16(2.0)
    lg[199] = np.float16(np.nan)
    idx = torch.empty(k, device=device, dtype=torch.int32)
    sc = torch.empty(k, device=device, dtype=torch.float16)
    backend.moe_router_topk(to_torch(lg, device), idx, sc, renormalize=True)
    assert idx.cpu().tolist() == [0, 150, 1]
    widx = np.empty(k, dtype=np.int32)
    oracle.lib().tto_topk(P(lg), oracle.F16, E, k, 1, P(widx), P(np.empty(k, dtype=np.float16)), oracle.F16)
    assert widx.tolist() == [0, 150, 1]


@pytest.mark.parametrize("id_dtype", ID_DTYPES)
@pytest.mark.parametrize("top_k", [4, 1])
def test_mxfp4_expert_chain(backend, device, id_dtype, top_k):
    """MXFP4 gate/up into _moe_gate_up_buffer [top_k, 2I] (gpu_runtime.py:9648), then down
    on the activation buffer slice [:top_k] into _moe_down_buffer [top_k, H] (:9855);
    with top_k == 1 the activation is squeezed to [I] (:9699-9700)."""
    E, H, inter = 32, 2880, 2880
    g = rng(930 + top_k)
    gu_blocks, gu_scales = _mxfp4(g, E, 2 * inter, H)
    dn_blocks, dn_scales = _mxfp4(g, E, H, inter)
    router_ids = np.array([17, 3, 30, 8][:top_k], dtype=np.int32)
    hidden = f16_normal(g, H)
    act = f16_normal(g, (top_k, inter))
    indices_buffer = torch.zeros(4, device=device, dtype=id_dtype)
    indices_buffer[:top_k] = torch.from_numpy(router_ids).to(device=device, dtype=id_dtype)
    gate_up_buffer = torch.empty((top_k, 2 * inter), device=device, dtype=torch.float16)
    down_buffer = torch.empty((top_k, H), device=device, dtype=torch.float16)
    activation_buffer = to_torch(act, device)
    backend.mxfp4_selected_matvec(to_torch(gu_blocks, device), to_torch(gu_scales, device), to_torch(hidden, device),
                                  indices_buffer[:top_k], gate_up_buffer)
    activation = activation_buffer[:top_k]
    if top_k == 1:
        activation = activation.squeeze(0)
    backend.mxfp4_selected_tensorcore_matvec(to_torch(dn_blocks, device), to_torch(dn_scales, device), activation,
                                             indices_buffer[:top_k], down_buffer)
    gu = from_torch_bits(gate_up_buffer)
    dn = from_torch_bits(down_buffer)
    for s, e in enumerate(router_ids):
        want = oracle.gemv("mxfp4", "block_e8", gu_blocks[e].reshape(2 * inter, -1), gu_scales[e], hidden, cols=H,
                           lpr=lanes(H), s_row=H // 32)
        assert_bits_equal(gu[s], want, f"gate_up slot {s}")
        want = oracle.gemv("mxfp4", "block_e8", dn_blocks[e].reshape(H, -1), dn_scales[e], act[s], cols=inter,
                           lpr=lanes(inter), s_row=inter // 32)
        assert_bits_equal(dn[s], want, f"down slot {s}")


@pytest.mark.parametrize("id_dtype", ID_DTYPES)
@pytest.mark.parametrize("bits", [1, 2])
def test_lowbit_expert_chain(backend, device, id_dtype, bits):
    """Low-bit experts: fused SwiGLU into _moe_activation_buffer[:top_k] with the
    [E, 2I] bias (gpu_runtime.py:9612-9625), then the fused weighted down into
    _moe_combined_buffer [H] with act-dtype router scores (:9821-9833); the unfused
    q-bit selected GEMV on the same ids (:9631, :9838)."""
    E, H, inter, top_k = 32, 2880, 2880, 4
    g = rng(950 + bits)
    codes = g.integers(0, 1 << bits, size=(E, 2 * inter, H), dtype=np.uint8)
    gu = layouts.pack_lowbit_blocks(codes, bits)
    gu_s = g.integers(118, 123, size=(E, 2 * inter, H // 32), dtype=np.uint8)
    codes = g.integers(0, 1 << bits, size=(E, H, inter), dtype=np.uint8)
    dn = layouts.pack_lowbit_blocks(codes, bits)
    dn_s = g.integers(118, 123, size=(E, H, inter // 32), dtype=np.uint8)
    gu_bias = f16_normal(g, (E, 2 * inter), 0.5)
    dn_bias = f16_normal(g, (E, H), 0.5)
    router_ids = np.array([5, 31, 0, 12], dtype=np.int32)
    scores = np.array([0.4, 0.3, 0.2, 0.1], dtype=np.float16)
    hidden = f16_normal(g, H)
    ids = torch.from_numpy(router_ids).to(device=device, dtype=id_dtype)
    activation_buffer = torch.empty((top_k, inter), device=device, dtype=torch.float16)
    combined_buffer = torch.empty(H, device=device, dtype=torch.float16)
    gate_up_buffer = torch.empty((top_k, 2 * inter), device=device, dtype=torch.float16)
    t_gu, t_gus = to_torch(gu, device), to_torch(gu_s, device)
    act = backend.mxfp_lowbit_selected_swiglu(t_gu, t_gus, to_torch(hidden, device), ids, activation_buffer[:top_k],
                                              bits=bits, alpha=1.702, limit=7.0, bias=to_torch(gu_bias, device),
                                              block_m=8 if bits == 2 else 4, block_k=1024, num_warps=4)
    backend.mxfp_lowbit_weighted_down(to_torch(dn, device), to_torch(dn_s, device), act, ids, to_torch(scores, device),
                                      combined_buffer, bits=bits, bias=to_torch(dn_bias, device), block_m=8,
                                      block_k=1024 if bits == 2 else 512, num_warps=4)
    backend.mxfp_lowbit_selected_matvec(t_gu, t_gus, to_torch(hidden, device), ids, gate_up_buffer, bits=bits)
    fmt = 6 if bits == 2 else 7
    L = oracle.lib()
    want_act = np.empty((top_k, inter), dtype=np.float16)
    rc = L.tto_swiglu(fmt, oracle.BF16, gu.ctypes.data, gu.strides[0], gu.strides[1], gu_s.ctypes.data,
                      gu_s.strides[0], gu_s.strides[1], hidden.ctypes.data, oracle.F16, 0, router_ids.ctypes.data,
                      top_k, gu_bias.ctypes.data, oracle.F16, 2 * inter, 1.702, 7.0, want_act.ctypes.data, oracle.F16,
                      inter, inter, H, lanes(H))
    assert rc == 0
    assert_bits_equal(from_torch_bits(activation_buffer).reshape(-1), want_act.reshape(-1), "swiglu")
    want = np.empty(H, dtype=np.float16)
    rc = L.tto_weighted_down(fmt, oracle.BF16, dn.ctypes.data, dn.strides[0], dn.strides[1], dn_s.ctypes.data,
                             dn_s.strides[0], dn_s.strides[1], want_act.ctypes.data, oracle.F16, inter,
                             router_ids.ctypes.data, scores.ctypes.data, oracle.F16, top_k, dn_bias.ctypes.data,
                             oracle.F16, H, want.ctypes.data, oracle.F16, H, inter, lanes(inter))
    assert rc == 0
    assert_bits_equal(from_torch_bits(combined_buffer), want, "weighted down")
    gub = from_torch_bits(gate_up_buffer)
    for s, e in enumerate(router_ids):
        w = oracle.gemv("q2e8" if bits == 2 else "q1e8", "block_e8", gu[e].reshape(2 * inter, -1), gu_s[e], hidden,
                        cols=H, lpr=lanes(H), s_row=H // 32)
        assert_bits_equal(gub[s], w, f"q{bits} gate_up slot {s}")


@pytest.mark.parametrize("id_dtype", ID_DTYPES)
def test_int4_expert_pack_chain(backend, device, id_dtype):
    """int4 expert packs (gpu_runtime.py:9937-9956): gate/up into
    _moe_gate_up_buffer[:selected] with fp32 group scales, SiLU-mul on the two halves,
    then down into _moe_down_buffer[:selected]."""
    E, H, inter, group = 16, 2048, 1024, 128
    g = rng(970)
    gu_codes = g.integers(0, 16, size=(E, 2 * inter, H), dtype=np.uint8)
    gu_q = layouts.pack_int4(gu_codes)
    gu_s = (np.abs(g.standard_normal((E, 2 * inter, H // group))) * 0.02).astype(np.float32)
    dn_codes = g.integers(0, 16, size=(E, H, inter), dtype=np.uint8)
    dn_q = layouts.pack_int4(dn_codes)
    dn_s = (np.abs(g.standard_normal((E, H, inter // group))) * 0.02).astype(np.float32)
    router_ids = np.array([9, 2, 15, 4], dtype=np.int32)
    hidden = f16_normal(g, H)
    ids = torch.from_numpy(router_ids).to(device=device, dtype=id_dtype)
    gate_up_buffer = torch.empty((4, 2 * inter), device=device, dtype=torch.float16)
    down_buffer = torch.empty((4, H), device=device, dtype=torch.float16)
    gate_up = gate_up_buffer[: int(ids.numel())]
    backend.int4_selected_matvec(to_torch(gu_q, device), to_torch(gu_s, device), to_torch(hidden, device), ids, gate_up,
                                 group_size=group)
    gate, up = gate_up.chunk(2, dim=-1)
    activation = (torch.nn.functional.silu(gate) * up).contiguous()
    expert_output = down_buffer[: int(ids.numel())]
    backend.int4_selected_matvec(to_torch(dn_q, device), to_torch(dn_s, device), activation, ids, expert_output,
                                 group_size=group)
    gub = from_torch_bits(gate_up)
    act = from_torch_bits(activation)
    dnb = from_torch_bits(expert_output)
    for s, e in enumerate(router_ids):
        want = oracle.gemv("int4_sym", "group", gu_q[e], gu_s[e], hidden, cols=H, lpr=lanes(H, 4), L=4,
                           s_row=H // group, s_grp=1)
        assert_bits_equal(gub[s], want, f"int4 gate_up slot {s}")
        want = oracle.gemv("int4_sym", "group", dn_q[e], dn_s[e], act[s], cols=inter, lpr=lanes(inter, 4), L=4,
                           s_row=inter // group, s_grp=1)
        assert_bits_equal(dnb[s], want, f"int4 down slot {s}")


@pytest.mark.parametrize("id_dtype", ID_DTYPES)
def test_ternary_experts_long_ids(backend, device, id_dtype):
    """Ternary experts with int32 and torch.long ids give the oracle's bits; a long id
    whose low word is in range but whose high word is not stays out of range (NaN row)."""
    from tests.test_ternary_gpu import _random_packed

    E, rows, cols = 6, 640, 2880
    g = rng(990)
    packed, scales = _random_packed(g, E, rows, cols)
    router_ids = np.array([4, 0, 5], dtype=np.int64)
    if id_dtype == torch.long:
        router_ids = np.append(router_ids, np.int64(1 << 32))
    x = f16_normal(g, cols)
    out = torch.empty((len(router_ids), rows), device=device, dtype=torch.float32)
    ids = torch.from_numpy(router_ids).to(device=device, dtype=id_dtype)
    backend.mxfp_ternary_selected_tensorcore_matvec(to_torch(packed, device), to_torch(scales, device),
                                                    to_torch(x, device), ids, out)
    got = out.cpu().numpy()
    want = T.ternary_selected_gemv(packed, scales, x.astype(np.float32), router_ids[:3])
    assert np.array_equal(got[:3].view(np.uint32), want.view(np.uint32))
    if id_dtype == torch.long:
        assert np.all(np.isnan(got[3]))


def test_index_dtype_contract(backend, device):
    """int16 / uint8 ids and non-contiguous id views are refused before any launch."""
    E, rows, cols = 4, 64, 256
    blocks = torch.zeros((E, rows, cols // 32, 16), device=device, dtype=torch.uint8)
    scales = torch.full((E, rows, cols // 32), 127, device=device, dtype=torch.uint8)
    x = torch.zeros(cols, device=device, dtype=torch.float16)
    out = torch.empty((2, rows), device=device, dtype=torch.float16)
    for bad in (torch.zeros(2, device=device, dtype=torch.int16), torch.zeros(4, device=device, dtype=torch.int32)[::2]):
        with pytest.raises(ValueError):
            backend.mxfp4_selected_matvec(blocks, scales, x, bad, out)
