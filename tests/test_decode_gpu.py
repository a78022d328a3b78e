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


@pytest.fixture(scope="module")
def llama_case(device):
    """Llama-3.2-1B-shaped model with centered int4 codes (q in [-7, 7]), 64 oracle
    tokens from start token 1 at position 512, the per-step top-2 logit margins and the
    final step's logits.  The oracle copies the weights and cache before any GPU run."""
    s = LLAMA_1B
    w = make_dense(s, device=device, seed=0, centered_codes=True)
    ref = DenseRef(w)
    margins: list[float] = []
    want = ref.generate(1, s.prior_tokens, 64, margins=margins)
    print(f"llama-1b oracle stream: {len(set(want))} distinct of 64, min top-2 margin {min(margins):.4g}: {want}",
          flush=True)
    return w, want, ref.last_logits, margins


def test_llama_1b_oracle_stream_fixture(llama_case):
    """The committed stream (tests/golden/llama1b_centered_tokens.json, which bench.py
    compares its timed tokens with) is this oracle's stream."""
    import json
    from pathlib import Path

    path = Path(__file__).with_name("golden") / "llama1b_centered_tokens.json"
    d = json.loads(path.read_text())
    assert d["seed"] == 0 and d["start_token"] == 1 and d["position"] == LLAMA_1B.prior_tokens
    assert d["tokens"] == llama_case[1]


@pytest.mark.parametrize("fused", [False, True])
def test_llama_1b_shaped_64_tokens(device, llama_case, fused):
    """64 graph-replayed tokens at the full 1B shape equal the oracle's, and the last
    step's 128256 logits are bit-identical."""
    w, want, logits, margins = llama_case
    s = LLAMA_1B
    dec = DenseDecoder(_backend(device, s), w, fused=fused)
    got = dec.generate(1, s.prior_tokens, 64)
    assert got == want
    assert len(set(want)) >= 8, f"degenerate stream {want}"
    assert np.array_equal(_final_logits(dec).view(np.uint16), logits.view(np.uint16))
    assert all(np.isfinite(margins))


def test_llama_1b_baseline_init_tokens(device):
    """The benchmark's own init (q in [-8, 7]): the fp16 residual overflows, so the
    stream is that of non-finite logits; it and the final logits still match the
    oracle bit for bit (NaN and inf propagate the same way)."""
    s = LLAMA_1B
    w = make_dense(s, device=device, seed=0)
    ref = DenseRef(w)
    want = ref.generate(1, s.prior_tokens, 16)
    dec = DenseDecoder(_backend(device, s), w, fused=True)
    assert dec.generate(1, s.prior_tokens, 16) == want
    assert np.array_equal(_final_logits(dec).view(np.uint16), ref.last_logits.view(np.uint16))


@pytest.mark.parametrize("graph", [True, False])
def test_small_dense_combined_o_proj(device, graph):
    """A capacity of whole 64-token chunks sends the fused step through the o_proj that
    combines the attention partials itself; 64 tokens from 100 prior ones cross two chunk
    boundaries.  Tokens and the last logits equal the oracle's bit for bit."""
    s = SMALL_DENSE
    w = make_dense(s, device=device, seed=3, capacity=192)
    ref = DenseRef(w)
    dec = DenseDecoder(_backend(device, s), w, fused=True)
    start, pos = 11, s.prior_tokens
    got = dec.generate(start, pos, s.max_new_tokens, use_graph=graph)
    want = ref.generate(start, pos, s.max_new_tokens)
    assert got == want
    _, logits = ref.step(want[-2], pos + s.max_new_tokens - 1)
    assert np.array_equal(_final_logits(dec).view(np.uint16), logits.view(np.uint16))


@pytest.fixture(scope="module")
def gptoss_case(device):
    s = GPT_OSS_20B
    w = make_moe(s, device=device, seed=0)
    ref = MoERef(w)
    margins: list[float] = []
    want = ref.generate(1, s.prior_tokens, 8, margins=margins)
    print(f"gpt-oss oracle stream: {want}, min top-2 margin {min(margins):.4g}", flush=True)
    return w, want, ref.last_logits, margins


@pytest.mark.parametrize("fused", [False, True])
def test_gpt_oss_20b_shaped_tokens(device, gptoss_case, fused):
    """8 graph-replayed tokens at the full gpt-oss-20B shape equal the oracle's, and the
    last step's 201088 logits are bit-identical."""
    w, want, logits, margins = gptoss_case
    s = GPT_OSS_20B
    dec = MoEDecoder(_backend(device, s), w, fused=fused)
    got = dec.generate(1, s.prior_tokens, 8)
    assert got == want
    assert len(set(want)) >= 4, f"degenerate stream {want}"
    assert np.array_equal(_final_logits(dec).view(np.uint16), logits.view(np.uint16))


def test_gpt_oss_20b_shaped_batch8(device, gptoss_case):
    """Eight sequences in lockstep at the full gpt-oss shape (one attention launch and
    one 8-row lm_head per step): every stream equals that sequence decoded alone by
    the bs=1 decoder (gpu_runtime.py:11130-11209 semantics, 8 independent routings)."""
    s = GPT_OSS_20B
    w = gptoss_case[0]
    batch, steps = 8, 4
    kc, vc = _batch_caches(s, w, batch, device, seed=11)
    starts = [(7919 * b + 3) % s.vocab for b in range(batch)]
    want = []
    for b in range(batch):
        wb = _sequence_weights(w, kc, vc, b, s.kv_heads)
        want.append(MoEDecoder(_backend(device, s), wb, fused=True).generate(starts[b], s.prior_tokens, steps))
        del wb
    got = MoEBatchDecoder(_backend(device, s), w, batch, kc, vc).generate(starts, s.prior_tokens, steps)
    assert got == want
    assert len({t for seq in want for t in seq}) >= 8
