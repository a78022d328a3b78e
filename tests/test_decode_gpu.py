"""End-to-end greedy decode on the GPU against the oracle decode: token streams and
final logits must be identical (bit for bit), for graph replay and eager launches."""

from __future__ import annotations

import dataclasses

import numpy as np
import pytest
import torch

from oracle.decode_ref import DenseRef, MoERef
from thintensor_amd.backend import HipDecodeBackend
from thintensor_amd.decode import DenseDecoder, MoEBatchDecoder, MoEDecoder
from thintensor_amd.synth import GPT_OSS_20B, LLAMA_1B, DenseShape, MoEShape, make_dense, make_moe

pytestmark = pytest.mark.gpu

SMALL_DENSE = DenseShape(name="small-dense", layers=2, hidden=512, heads=8, kv_heads=2, head_dim=64, intermediate=1024,
                         vocab=4096, prior_tokens=100, max_new_tokens=64)
SMALL_MOE = MoEShape(name="small-moe", layers=2, hidden=512, heads=8, kv_heads=2, head_dim=64, experts=8, top_k=2,
                     intermediate=512, vocab=4096, prior_tokens=70, max_new_tokens=32)


def _backend(device, s):
    return HipDecodeBackend(device, torch.float16, s.hidden, s.q_dim, s.kv_dim, s.intermediate)


def _final_logits(dec) -> np.ndarray:
    return dec.be.logits_buffer(int(dec.w.lm_head.shape[0]), torch.float16).cpu().numpy()


@pytest.mark.parametrize("fused", [False, True])
@pytest.mark.parametrize("graph", [True, False])
def test_small_dense_64_tokens(device, graph, fused):
    s = SMALL_DENSE
    w = make_dense(s, device=device, seed=1)
    ref = DenseRef(w)
    dec = DenseDecoder(_backend(device, s), w, fused=fused)
    start, pos = 7, s.prior_tokens
    got = dec.generate(start, pos, s.max_new_tokens, use_graph=graph)
    want = ref.generate(start, pos, s.max_new_tokens)
    assert got == want
    # the last step's logits are bit-identical too
    _, logits = ref.step(want[-2], pos + s.max_new_tokens - 1)
    assert np.array_equal(_final_logits(dec).view(np.uint16), logits.view(np.uint16))


def _batch_caches(s, w, batch, device, seed):
    """Per-sequence KV caches [layers, batch * kv_heads, capacity, head_dim]: random prior
    tokens, zeros after them (as make_moe fills its own cache)."""
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    cap, P = int(w.k_cache.shape[2]), s.prior_tokens
    kc = torch.zeros((s.layers, batch * s.kv_heads, cap, s.head_dim), device=device, dtype=torch.float16)
    vc = torch.zeros_like(kc)
    shape = (s.layers, batch * s.kv_heads, P, s.head_dim)
    kc[:, :, :P] = torch.randn(shape, generator=g, device=device).half()
    vc[:, :, :P] = torch.randn(shape, generator=g, device=device).half()
    return kc, vc


def _sequence_weights(w, kc, vc, b, kv):
    return dataclasses.replace(w, k_cache=kc[:, b * kv:(b + 1) * kv].clone(), v_cache=vc[:, b * kv:(b + 1) * kv].clone())


@pytest.mark.parametrize("batch,against", [(3, "oracle"), (8, "bs1")])
def test_small_moe_batch(device, batch, against):
    """Lockstep decode of several sequences: every stream equals that sequence decoded
    alone (the oracle, or the fused bs=1 HIP decoder, which the oracle pins above)."""
    s = SMALL_MOE
    w = make_moe(s, device=device, seed=4)
    kc, vc = _batch_caches(s, w, batch, device, seed=9)
    starts = [(37 * b + 5) % s.vocab for b in range(batch)]
    steps, pos = 12, s.prior_tokens
    want = []
    for b in range(batch):
        wb = _sequence_weights(w, kc, vc, b, s.kv_heads)
        if against == "oracle":
            want.append(MoERef(wb).generate(starts[b], pos, steps))
        else:
            want.append(MoEDecoder(_backend(device, s), wb, fused=True).generate(starts[b], pos, steps))
    got = MoEBatchDecoder(_backend(device, s), w, batch, kc, vc).generate(starts, pos, steps)
    assert got == want


@pytest.mark.parametrize("fused", [False, True])
def test_small_moe_32_tokens(device, fused):
    s = SMALL_MOE
    w = make_moe(s, device=device, seed=2)
    ref = MoERef(w)
    dec = MoEDecoder(_backend(device, s), w, fused=fused)
    start, pos = 11, s.prior_tokens
    got = dec.generate(start, pos, s.max_new_tokens)
    want = ref.generate(start, pos, s.max_new_tokens)
    assert got == want
    _, logits = ref.step(want[-2], pos + s.max_new_tokens - 1)
    assert np.array_equal(_final_logits(dec).view(np.uint16), logits.view(np.uint16))


@pytest.mark.parametrize("fused", [False, True])
def test_llama_1b_shaped_tokens(device, fused):
    s = LLAMA_1B
    w = make_dense(s, device=device, seed=0)
    dec = DenseDecoder(_backend(device, s), w, fused=fused)
    ref = DenseRef(w)
    start, pos, n = 1, s.prior_tokens, 6
    got = dec.generate(start, pos, n)
    want = ref.generate(start, pos, n)
    assert got == want


@pytest.mark.parametrize("fused", [False, True])
def test_gpt_oss_20b_shaped_tokens(device, fused):
    s = GPT_OSS_20B
    w = make_moe(s, device=device, seed=0)
    dec = MoEDecoder(_backend(device, s), w, fused=fused)
    ref = MoERef(w)
    start, pos, n = 1, s.prior_tokens, 3
    got = dec.generate(start, pos, n)
    want = ref.generate(start, pos, n)
    assert got == want
