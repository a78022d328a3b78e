"""End-to-end greedy decode on the GPU against the oracle decode: token streams and
final logits must be identical (bit for bit), for graph replay and eager launches."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.decode_ref import DenseRef, MoERef
from thintensor_amd.backend import HipDecodeBackend
from thintensor_amd.decode import DenseDecoder, MoEDecoder
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
