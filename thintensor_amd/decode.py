"""Minimal bs=1 greedy decode harness on the HIP backend.

The step order and every rounding point mirror the reference runtime's Triton
paths, with the fused options the Triton backend provides:

* ``DenseDecoder`` follows ``_forward_token_triton`` (gpu_runtime.py:11429-11726)
  with fused residual+RMSNorm, fused RoPE, the fused Triton attention backend and
  Triton elementwise ops; the greedy token comes from ``next_token_tensor``
  (gpu_runtime.py:11130-11209) in its default lm_head mode;
* ``MoEDecoder`` follows ``_forward_token_moe`` and ``_packed_moe_forward``
  (gpu_runtime.py:8968-9908) for MXFP4 experts.

Differences from the reference, by design:

* a flat KV cache ``[layers, kv_heads, capacity, head_dim]`` replaces the paged
  cache (same values, same attention);
* the token id and the position live on the device, so one decode step is captured
  once in a HIP graph and replayed for every token (the reference disables its
  CUDA graph for causal KV because it hard-codes the position,
  gpu_runtime.py:12594-12601);
* QKV and gate/up projections are one multi-matrix launch each, the MoE experts
  run as two fused launches, and attention biases are fused into the GEMV
  epilogue -- each with the reference's rounding points, so outputs are unchanged;
* the post-attention add_rms_norm the MoE path issues twice per layer
  (gpu_runtime.py:9233-9252 and 9254-9275, idempotent) runs once.
"""

from __future__ import annotations

import torch

from . import _lib
from .backend import HipDecodeBackend
from .synth import DenseWeights, MoEWeights

_ACT = {torch.float16: _lib.F16, torch.bfloat16: _lib.BF16}


def _int4_segment(seg: _lib.FusedSegment, weight, out: torch.Tensor, rows: int, kind: int, weight2=None) -> None:
    packed, scales = weight
    seg.weight = packed.data_ptr()
    seg.w_row_bytes = packed.stride(0) * packed.element_size()
    seg.scales = scales.data_ptr()
    seg.s_row = scales.stride(0)
    if weight2 is not None:
        seg.weight2 = weight2[0].data_ptr()
        seg.scales2 = weight2[1].data_ptr()
    seg.out = out.data_ptr()
    seg.rows = rows
    seg.kind = kind


def _dense_segment(seg: _lib.FusedSegment, weight: torch.Tensor, bias: torch.Tensor | None, out: torch.Tensor | None,
                   kind: int) -> None:
    seg.weight = weight.data_ptr()
    seg.w_row_bytes = weight.stride(0) * weight.element_size()
    seg.bias = bias.data_ptr() if bias is not None else None
    seg.out = out.data_ptr() if out is not None else None
    seg.rows = int(weight.shape[0])
    seg.kind = kind


def _kv_context(d: _lib.FusedGemv, dec: "_GraphedDecoder", cos: torch.Tensor, sin: torch.Tensor, head_dim: int,
                cache: torch.Tensor) -> None:
    d.position = dec.position.data_ptr()
    d.capacity = dec.capacity
    d.cache_head = cache.stride(0)
    d.cos_table = cos.data_ptr()
    d.sin_table = sin.data_ptr()
    d.table_row = cos.stride(0)
    d.table_rows = int(cos.shape[0])
    d.head_dim = head_dim


class _GraphedDecoder:
    """Common state: device token / position, token history, graph capture."""

    def __init__(self, backend: HipDecodeBackend, device: torch.device, capacity: int, max_new: int,
                 fused: bool = False) -> None:
        self.be = backend
        self.fused = fused
        self.device = device
        self.capacity = capacity
        self.token = backend._argmax_out_idx               # int64 0-d, written by the lm_head argmax
        self.position = torch.zeros(1, device=device, dtype=torch.int32)
        self.history = torch.zeros(max_new, device=device, dtype=torch.int64)
        self.base = torch.zeros(1, device=device, dtype=torch.int32)   # position of the first generated step
        self.graph: torch.cuda.CUDAGraph | None = None
        self._graph_stream: torch.cuda.Stream | None = None

    def prime(self, token: int, position: int) -> None:
        """Set the next input token and its position (host -> device, outside graphs)."""
        if not 0 <= position < self.capacity:
            raise ValueError("position outside the KV cache")
        self.token.fill_(int(token))
        self.position.fill_(int(position))
        self.base.fill_(int(position))
        self.history.zero_()

    def step(self) -> None:  # pragma: no cover - implemented by subclasses
        raise NotImplementedError

    def _step_and_record(self) -> None:
        if self.fused:
            # the fused step logs the token and advances the position in its last kernel
            self.fused_step()
            return
        self.step()
        self.be.record_token(self.token, self.position, self.base, self.history)
        self.be.advance_position(self.position)

    def fused_step(self) -> None:  # pragma: no cover - implemented by subclasses
        raise NotImplementedError

    def _reserve_scratch(self) -> None:  # pragma: no cover - implemented by subclasses
        raise NotImplementedError

    def capture(self) -> None:
        """Record one decode step (including token logging and the position advance)
        into a HIP graph.  The graph reads token/position from device memory.  All
        scratch is reserved beforehand, so no step runs (and no state changes) here."""
        self._reserve_scratch()
        torch.cuda.synchronize(self.device)
        self._graph_stream = torch.cuda.Stream(self.device)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph, stream=self._graph_stream):
            self._step_and_record()

    def generate(self, start_token: int, position: int, steps: int, use_graph: bool = True) -> list[int]:
        """Greedy-decode `steps` tokens; returns the generated ids."""
        if position + steps > self.capacity:
            raise ValueError("not enough KV capacity for the requested steps")
        if steps > self.history.numel():
            raise ValueError("history buffer too small")
        if use_graph and self.graph is None:
            self.capture()
        self.prime(start_token, position)
        for _ in range(steps):
            if use_graph:
                self.graph.replay()
            else:
                self._step_and_record()
        torch.cuda.synchronize(self.device)
        return self.history[:steps].cpu().tolist()


class DenseDecoder(_GraphedDecoder):
    """Llama-3.2-1B-shaped int4 g128 decoder.

    ``fused=True`` runs the step as five launches per layer (QKV GEMV with the
    residual add + RMSNorm prologue and the RoPE / KV-append epilogue, attention
    partials and combine, o_proj, gate/up GEMV with the add + RMSNorm prologue and the
    SiLU epilogue, down_proj) and a final lm_head launch whose prologue is the last
    add + RMSNorm and whose finishing kernel also logs the token and advances the
    position.  Every rounding point is the unfused operator's, so both modes give
    the same bits."""

    def __init__(self, backend: HipDecodeBackend, weights: DenseWeights, fused: bool = False) -> None:
        s = weights.shape
        super().__init__(backend, weights.embed.device, int(weights.k_cache.shape[2]), s.max_new_tokens, fused)
        self.w = weights
        self.s = s
        dev, dt = weights.embed.device, torch.float16
        self.hidden_a = torch.empty(s.hidden, device=dev, dtype=dt)
        self.hidden_b = torch.empty(s.hidden, device=dev, dtype=dt)
        self.normed = torch.empty(s.hidden, device=dev, dtype=dt)
        self.qkv = torch.empty(s.q_dim + 2 * s.kv_dim, device=dev, dtype=dt)
        self.attn = torch.empty(s.q_dim, device=dev, dtype=dt)
        self.attn_out = torch.empty(s.hidden, device=dev, dtype=dt)
        self.gate_up = torch.empty(2 * s.intermediate, device=dev, dtype=dt)
        self.act = torch.empty(s.intermediate, device=dev, dtype=dt)
        self.mlp = torch.empty(s.hidden, device=dev, dtype=dt)
        self.final = torch.empty(s.hidden, device=dev, dtype=dt)

    def _reserve_scratch(self) -> None:
        s = self.s
        self.be._attention_scratch(s.heads, self.capacity, s.head_dim)
        self.be._argmax_scratch(int(self.w.lm_head.shape[0]), s.hidden)
        self.be.logits_buffer(int(self.w.lm_head.shape[0]), torch.float16)

    def step(self) -> None:
        be, w, s = self.be, self.w, self.s
        q, k, v = self.qkv[: s.q_dim], self.qkv[s.q_dim: s.q_dim + s.kv_dim], self.qkv[s.q_dim + s.kv_dim:]
        gate, up = self.gate_up[: s.intermediate], self.gate_up[s.intermediate:]
        be.embedding(w.embed, self.token, self.hidden_a)
        be.rms_norm(self.hidden_a, w.layers[0].ln1, self.normed, s.eps)
        for li, L in enumerate(w.layers):
            be.multi_int4_scaled_matvec((L.q[0], L.k[0], L.v[0]), (L.q[1], L.k[1], L.v[1]),
                                        (s.q_dim, s.kv_dim, s.kv_dim), s.hidden, self.normed, self.qkv,
                                        group_size=s.group)
            be.rope_qk_inplace(q, k, w.cos, w.sin, s.heads, s.kv_heads, s.head_dim, position=self.position)
            be.kv_append(k, v, w.k_cache[li], w.v_cache[li], self.position, s.kv_heads, s.head_dim)
            be.single_token_gqa_attention(q, w.k_cache[li], w.v_cache[li], self.attn, s.heads, s.kv_heads,
                                          s.head_dim, active_tokens=(self.position, 1))
            be.int4_scaled_matvec(L.o[0], L.o[1], self.attn, self.attn_out, rows=s.hidden, cols=s.q_dim,
                                  group_size=s.group)
            be.add_rms_norm(self.hidden_a, self.attn_out, self.hidden_b, L.ln2, self.normed, s.eps)
            be.multi_int4_scaled_matvec((L.gate[0], L.up[0]), (L.gate[1], L.up[1]), (s.intermediate, s.intermediate),
                                        s.hidden, self.normed, self.gate_up, group_size=s.group)
            be.silu_mul(gate, up, self.act)
            be.int4_scaled_matvec(L.down[0], L.down[1], self.act, self.mlp, rows=s.hidden, cols=s.intermediate,
                                  group_size=s.group)
            if li + 1 < len(w.layers):
                be.add_rms_norm(self.hidden_b, self.mlp, self.hidden_a, w.layers[li + 1].ln1, self.normed, s.eps)
            else:
                be.add_rms_norm(self.hidden_b, self.mlp, self.hidden_a, w.final_norm, self.final, s.eps)
        be.matvec_argmax_tensor(w.lm_head, self.final)

    def _build_fused(self) -> None:
        w, s = self.w, self.s
        act = _ACT[self.hidden_a.dtype]
        q = self.qkv[: s.q_dim]
        self._qkv_desc, self._gu_desc = [], []
        for li, L in enumerate(w.layers):
            d = _lib.FusedGemv()
            d.weight_format, d.group_size, d.act_dtype, d.cols = _lib.FMT_INT4_G, s.group, act, s.hidden
            if li == 0:
                d.prologue = _lib.PRO_EMBED_NORM
                d.embed, d.embed_row, d.vocab = w.embed.data_ptr(), w.embed.stride(0), int(w.embed.shape[0])
                d.token = self.token.data_ptr()
            else:
                d.prologue = _lib.PRO_ADD_NORM
                d.left, d.right = self.hidden_b.data_ptr(), self.mlp.data_ptr()
            d.norm_weight, d.eps, d.residual_out = L.ln1.data_ptr(), s.eps, self.hidden_a.data_ptr()
            d.count = 3
            _int4_segment(d.seg[0], L.q, q, s.q_dim, _lib.SEG_ROPE_OUT)
            _int4_segment(d.seg[1], L.k, w.k_cache[li], s.kv_dim, _lib.SEG_ROPE_CACHE)
            _int4_segment(d.seg[2], L.v, w.v_cache[li], s.kv_dim, _lib.SEG_CACHE)
            _kv_context(d, self, w.cos, w.sin, s.head_dim, w.k_cache[li])
            self._qkv_desc.append(d)
            g = _lib.FusedGemv()
            g.weight_format, g.group_size, g.act_dtype, g.cols = _lib.FMT_INT4_G, s.group, act, s.hidden
            g.prologue = _lib.PRO_ADD_NORM
            g.left, g.right = self.hidden_a.data_ptr(), self.attn_out.data_ptr()
            g.norm_weight, g.eps, g.residual_out = L.ln2.data_ptr(), s.eps, self.hidden_b.data_ptr()
            g.count = 1
            _int4_segment(g.seg[0], L.gate, self.act, s.intermediate, _lib.SEG_SILU, weight2=L.up)
            self._gu_desc.append(g)
        h = _lib.FusedGemv()
        h.weight_format, h.weight_dtype, h.act_dtype, h.cols = _lib.FMT_DENSE, _ACT[w.lm_head.dtype], act, s.hidden
        h.prologue = _lib.PRO_ADD_NORM
        h.left, h.right = self.hidden_b.data_ptr(), self.mlp.data_ptr()
        h.norm_weight, h.eps = w.final_norm.data_ptr(), s.eps
        h.count = 1
        _dense_segment(h.seg[0], w.lm_head, None, self.be.logits_buffer(int(w.lm_head.shape[0]), self.hidden_a.dtype),
                       _lib.SEG_PLAIN)
        self._head_desc = h

    def fused_step(self) -> None:
        be, w, s = self.be, self.w, self.s
        if not hasattr(self, "_head_desc"):
            self._build_fused()
        q = self.qkv[: s.q_dim]
        # the o_proj GEMV combines the attention chunk partials itself (head_dim-64 caches
        # of whole 64-token chunks, at most 32 query heads, 1/2/4/8 per KV head)
        combine = (s.head_dim == 64 and s.heads <= 32 and s.group == 128 and s.heads // s.kv_heads in (1, 2, 4, 8)
                   and int(w.k_cache[0].shape[1]) % 64 == 0 and w.k_cache[0].stride(1) == 64
                   and w.v_cache[0].stride(1) == 64)
        for li, L in enumerate(w.layers):
            be.fused_gemv(self._qkv_desc[li])
            if combine:
                be.attention_then_int4_matvec(q, w.k_cache[li], w.v_cache[li], s.heads, s.kv_heads, s.head_dim,
                                              L.o[0], L.o[1], self.attn_out, active_tokens=(self.position, 1))
            else:
                be.single_token_gqa_attention(q, w.k_cache[li], w.v_cache[li], self.attn, s.heads, s.kv_heads,
                                              s.head_dim, active_tokens=(self.position, 1))
                be.int4_scaled_matvec(L.o[0], L.o[1], self.attn, self.attn_out, rows=s.hidden, cols=s.q_dim,
                                      group_size=s.group)
            be.fused_gemv(self._gu_desc[li])
            be.int4_scaled_matvec(L.down[0], L.down[1], self.act, self.mlp, rows=s.hidden, cols=s.intermediate,
                                  group_size=s.group)
        be.fused_lm_head_argmax(self._head_desc, position=self.position, base=self.base, history=self.history)


class MoEDecoder(_GraphedDecoder):
    """gpt-oss-20B-shaped decoder with MXFP4 experts, fp16 attention with sinks.

    ``fused=True`` folds the embedding / residual add + RMSNorm into the QKV launch,
    RoPE and the KV append into its epilogue, the post-attention add + RMSNorm into the
    router launch, and the final add + RMSNorm, token log and position advance into the
    lm_head launches, with the unfused rounding points."""

    def __init__(self, backend: HipDecodeBackend, weights: MoEWeights, fused: bool = False) -> None:
        s = weights.shape
        super().__init__(backend, weights.embed.device, int(weights.k_cache.shape[2]), s.max_new_tokens, fused)
        self.w = weights
        self.s = s
        dev, dt = weights.embed.device, torch.float16
        self.hidden_a = torch.empty(s.hidden, device=dev, dtype=dt)
        self.hidden_b = torch.empty(s.hidden, device=dev, dtype=dt)
        self.normed = torch.empty(s.hidden, device=dev, dtype=dt)
        self.qkv = torch.empty(s.q_dim + 2 * s.kv_dim, device=dev, dtype=dt)
        self.attn = torch.empty(s.q_dim, device=dev, dtype=dt)
        self.attn_out = torch.empty(s.hidden, device=dev, dtype=dt)
        self.router_idx = torch.empty(s.top_k, device=dev, dtype=torch.int32)
        self.router_scores = torch.empty(s.top_k, device=dev, dtype=dt)
        self.router_logits = torch.empty((1, s.experts), device=dev, dtype=torch.float32)
        # the fused step hands the router logits to the SwiGLU launch, which takes the top-k
        # itself (False: the norm + router launch finishes the top-k)
        self.router_in_swiglu = True
        self.act = torch.empty((s.top_k, s.intermediate), device=dev, dtype=dt)
        self.moe = torch.empty(s.hidden, device=dev, dtype=dt)
        self.final = torch.empty(s.hidden, device=dev, dtype=dt)

    def _reserve_scratch(self) -> None:
        s = self.s
        self.be._attention_scratch(s.heads, self.capacity, s.head_dim)
        self.be._argmax_scratch(int(self.w.lm_head.shape[0]), s.hidden)
        self.be.logits_buffer(int(self.w.lm_head.shape[0]), torch.float16)
        self.be.reserve_batch_workspaces(1)

    def step(self) -> None:
        be, w, s = self.be, self.w, self.s
        q, k, v = self.qkv[: s.q_dim], self.qkv[s.q_dim: s.q_dim + s.kv_dim], self.qkv[s.q_dim + s.kv_dim:]
        be.embedding(w.embed, self.token, self.hidden_a)
        be.rms_norm(self.hidden_a, w.layers[0].ln1, self.normed, s.eps)
        for li, L in enumerate(w.layers):
            be.multi_matvec_bias((L.q, L.k, L.v), (L.q_bias, L.k_bias, L.v_bias), self.normed, self.qkv)
            be.rope_qk_inplace(q, k, w.cos, w.sin, s.heads, s.kv_heads, s.head_dim, position=self.position)
            be.kv_append(k, v, w.k_cache[li], w.v_cache[li], self.position, s.kv_heads, s.head_dim)
            be.single_token_gqa_attention(q, w.k_cache[li], w.v_cache[li], self.attn, s.heads, s.kv_heads,
                                          s.head_dim, sinks=L.sinks, active_tokens=(self.position, 1))
            be.multi_matvec_bias((L.o,), (L.o_bias,), self.attn, self.attn_out)
            be.add_rms_norm(self.hidden_a, self.attn_out, self.hidden_b, L.ln2, self.normed, s.eps)
            be.moe_router_matvec_topk(L.router, self.normed, self.router_idx, self.router_scores, bias=L.router_bias,
                                      renormalize=True)
            be.mxfp_lowbit_selected_swiglu(L.gate_up_blocks, L.gate_up_scales, self.normed, self.router_idx, self.act,
                                           bits=4, alpha=s.swiglu_alpha, limit=s.swiglu_limit, bias=L.gate_up_bias)
            be.mxfp_lowbit_weighted_down(L.down_blocks, L.down_scales, self.act, self.router_idx, self.router_scores,
                                         self.moe, bits=4, bias=L.down_bias)
            if li + 1 < len(w.layers):
                be.add_rms_norm(self.hidden_b, self.moe, self.hidden_a, w.layers[li + 1].ln1, self.normed, s.eps)
            else:
                be.add(self.hidden_b, self.moe, self.hidden_a)
                be.rms_norm(self.hidden_a, w.final_norm, self.final, s.eps)
        be.matvec_argmax_tensor(w.lm_head, self.final)

    def _build_fused(self) -> None:
        w, s = self.w, self.s
        act = _ACT[self.hidden_a.dtype]
        q = self.qkv[: s.q_dim]
        self._qkv_desc = []
        for li, L in enumerate(w.layers):
            d = _lib.FusedGemv()
            d.weight_format, d.weight_dtype, d.act_dtype, d.cols = _lib.FMT_DENSE, _ACT[L.q.dtype], act, s.hidden
            if li == 0:
                d.prologue = _lib.PRO_EMBED_NORM
                d.embed, d.embed_row, d.vocab = w.embed.data_ptr(), w.embed.stride(0), int(w.embed.shape[0])
                d.token = self.token.data_ptr()
            else:
                d.prologue = _lib.PRO_ADD_NORM
                d.left, d.right = self.hidden_b.data_ptr(), self.moe.data_ptr()
            d.norm_weight, d.eps, d.residual_out = L.ln1.data_ptr(), s.eps, self.hidden_a.data_ptr()
            d.count = 3
            _dense_segment(d.seg[0], L.q, L.q_bias, q, _lib.SEG_ROPE_OUT)
            _dense_segment(d.seg[1], L.k, L.k_bias, w.k_cache[li], _lib.SEG_ROPE_CACHE)
            _dense_segment(d.seg[2], L.v, L.v_bias, w.v_cache[li], _lib.SEG_CACHE)
            _kv_context(d, self, w.cos, w.sin, s.head_dim, w.k_cache[li])
            self._qkv_desc.append(d)
        h = _lib.FusedGemv()
        h.weight_format, h.weight_dtype, h.act_dtype, h.cols = _lib.FMT_DENSE, _ACT[w.lm_head.dtype], act, s.hidden
        h.prologue = _lib.PRO_ADD_RMS_NORM
        h.left, h.right = self.hidden_b.data_ptr(), self.moe.data_ptr()
        h.norm_weight, h.eps = w.final_norm.data_ptr(), s.eps
        h.count = 1
        _dense_segment(h.seg[0], w.lm_head, None, self.be.logits_buffer(int(w.lm_head.shape[0]), self.hidden_a.dtype),
                       _lib.SEG_PLAIN)
        self._head_desc = h

    def fused_step(self) -> None:
        be, w, s = self.be, self.w, self.s
        if not hasattr(self, "_head_desc"):
            self._build_fused()
        q = self.qkv[: s.q_dim]
        for li, L in enumerate(w.layers):
            be.fused_gemv(self._qkv_desc[li])
            be.single_token_gqa_attention(q, w.k_cache[li], w.v_cache[li], self.attn, s.heads, s.kv_heads,
                                          s.head_dim, sinks=L.sinks, active_tokens=(self.position, 1))
            be.multi_matvec_bias((L.o,), (L.o_bias,), self.attn, self.attn_out)
            if self.router_in_swiglu:
                be.add_rms_norm_router_logits(self.hidden_a, self.attn_out, self.hidden_b, L.ln2, self.normed, s.eps,
                                              L.router, self.router_logits, bias=L.router_bias)
                be.mxfp_lowbit_selected_swiglu_router(L.gate_up_blocks, L.gate_up_scales, self.normed,
                                                      self.router_logits, self.router_idx, self.router_scores,
                                                      self.act, bits=4, alpha=s.swiglu_alpha, limit=s.swiglu_limit,
                                                      renormalize=True, bias=L.gate_up_bias)
            else:
                be.add_rms_norm_router_topk(self.hidden_a, self.attn_out, self.hidden_b, L.ln2, self.normed, s.eps,
                                            L.router, self.router_idx, self.router_scores, bias=L.router_bias,
                                            renormalize=True)
                be.mxfp_lowbit_selected_swiglu(L.gate_up_blocks, L.gate_up_scales, self.normed, self.router_idx,
                                               self.act, bits=4, alpha=s.swiglu_alpha, limit=s.swiglu_limit,
                                               bias=L.gate_up_bias)
            be.mxfp_lowbit_weighted_down(L.down_blocks, L.down_scales, self.act, self.router_idx, self.router_scores,
                                         self.moe, bits=4, bias=L.down_bias)
        be.fused_lm_head_argmax(self._head_desc, position=self.position, base=self.base, history=self.history)


class MoEBatchDecoder:
    """``batch`` independent gpt-oss-shaped sequences decoded in lockstep, one token of each
    per step (eight independent bs=1 routings at batch 8; the reference decodes one token
    per step and has no batched path).

    Every sequence has its own KV cache (``k_cache``/``v_cache`` [layers, batch * kv_heads,
    capacity, head_dim]: sequence b owns KV heads b * kv_heads ...) and token; the position
    is shared.  Every launch covers the whole batch: the fused QKV (norm prologue, RoPE /
    cache epilogue) and o_proj with a token grid dimension, attention (the batch's query
    and KV heads are the heads of one call, so each head's arithmetic is the bs=1
    arithmetic), add+RMSNorm+router (one workgroup per token), the expert SwiGLU and
    weighted down (token-indexed slots) and the M-row lm_head argmax; only the final
    add + RMSNorm runs per sequence.  Each sequence's tokens equal
    MoEDecoder's stream for that sequence bit for bit."""

    def __init__(self, backend: HipDecodeBackend, weights: MoEWeights, batch: int, k_cache: torch.Tensor,
                 v_cache: torch.Tensor) -> None:
        s = weights.shape
        if batch < 1:
            raise ValueError("batch must be at least 1")
        want = (s.layers, batch * s.kv_heads)
        if tuple(k_cache.shape[:2]) != want or k_cache.shape != v_cache.shape or k_cache.shape[3] != s.head_dim:
            raise ValueError(f"KV caches must be [{s.layers}, {batch * s.kv_heads}, capacity, {s.head_dim}]")
        self.be, self.w, self.s, self.batch = backend, weights, s, batch
        dev = weights.embed.device
        self.device = dev
        self.k_cache, self.v_cache = k_cache, v_cache
        self.capacity = int(k_cache.shape[2])
        self.tokens = torch.zeros(batch, device=dev, dtype=torch.int64)
        self.position = torch.zeros(1, device=dev, dtype=torch.int32)
        self.base = torch.zeros(1, device=dev, dtype=torch.int32)
        self.history = torch.zeros((batch, s.max_new_tokens), device=dev, dtype=torch.int64)
        dt = torch.float16
        self.q_all = torch.empty((batch, s.q_dim), device=dev, dtype=dt)
        self.attn_all = torch.empty((batch, s.q_dim), device=dev, dtype=dt)
        self.final_all = torch.empty((batch, s.hidden), device=dev, dtype=dt)
        self.hidden_a = torch.empty((batch, s.hidden), device=dev, dtype=dt)
        self.hidden_b = torch.empty((batch, s.hidden), device=dev, dtype=dt)
        self.normed = torch.empty((batch, s.hidden), device=dev, dtype=dt)
        self.attn_out = torch.empty((batch, s.hidden), device=dev, dtype=dt)
        self.moe = torch.empty((batch, s.hidden), device=dev, dtype=dt)
        self.router_idx = torch.empty((batch, s.top_k), device=dev, dtype=torch.int32)
        self.router_scores = torch.empty((batch, s.top_k), device=dev, dtype=dt)
        self.router_logits = torch.empty((batch, s.experts), device=dev, dtype=torch.float32)
        # as MoEDecoder.router_in_swiglu; off here: the top-k of every wave in the batched
        # SwiGLU launch measured 2215 -> 2131 tok/s at eight sequences (bs=1: 711 -> 717)
        self.router_in_swiglu = False
        self.act = torch.empty((batch * s.top_k, s.intermediate), device=dev, dtype=dt)
        self.sinks = [L.sinks.repeat(batch).contiguous() for L in weights.layers]
        self._build_qkv()
        self.graph: torch.cuda.CUDAGraph | None = None
        self._graph_stream: torch.cuda.Stream | None = None

    def _build_qkv(self) -> None:
        """One multi-token fused QKV descriptor per layer: MoEDecoder's descriptor with the
        batch's buffers and per-token strides (sequence t's KV heads follow sequence t-1's)."""
        w, s, B = self.w, self.s, self.batch
        act = _ACT[torch.float16]
        self._qkv_desc = []
        for li, L in enumerate(w.layers):
            d = _lib.FusedGemv()
            d.weight_format, d.weight_dtype, d.act_dtype, d.cols = _lib.FMT_DENSE, _ACT[L.q.dtype], act, s.hidden
            if li == 0:
                d.prologue = _lib.PRO_EMBED_NORM
                d.embed, d.embed_row, d.vocab = w.embed.data_ptr(), w.embed.stride(0), int(w.embed.shape[0])
                d.token = self.tokens.data_ptr()
            else:
                d.prologue = _lib.PRO_ADD_NORM
                d.left, d.right = self.hidden_b.data_ptr(), self.moe.data_ptr()
            d.norm_weight, d.eps, d.residual_out = L.ln1.data_ptr(), s.eps, self.hidden_a.data_ptr()
            d.count = 3
            _dense_segment(d.seg[0], L.q, L.q_bias, self.q_all, _lib.SEG_ROPE_OUT)
            _dense_segment(d.seg[1], L.k, L.k_bias, self.k_cache[li], _lib.SEG_ROPE_CACHE)
            _dense_segment(d.seg[2], L.v, L.v_bias, self.v_cache[li], _lib.SEG_CACHE)
            _kv_context(d, self, w.cos, w.sin, s.head_dim, self.k_cache[li])
            d.tokens, d.token_x, d.token_out = B, s.hidden, s.q_dim
            d.token_cache = s.kv_heads * self.k_cache[li].stride(0)
            self._qkv_desc.append(d)

    def _reserve_scratch(self) -> None:
        s = self.s
        self.be._attention_scratch(self.batch * s.heads, self.capacity, s.head_dim)
        self.be._batched_argmax_scratch(self.batch, int(self.w.lm_head.shape[0]), s.hidden)
        self.be.reserve_batch_workspaces(self.batch)

    def step(self) -> None:
        """One token of every sequence, logged at history[:, position - base]; advances the position."""
        be, w, s, B = self.be, self.w, self.s, self.batch
        for li, L in enumerate(w.layers):
            be.fused_gemv(self._qkv_desc[li])
            be.single_token_gqa_attention(self.q_all.view(-1), self.k_cache[li], self.v_cache[li],
                                          self.attn_all.view(-1), B * s.heads, B * s.kv_heads, s.head_dim,
                                          sinks=self.sinks[li], active_tokens=(self.position, 1))
            be.matvec_bias_rows(L.o, L.o_bias, self.attn_all, self.attn_out)
            if self.router_in_swiglu:
                be.add_rms_norm_router_logits(self.hidden_a, self.attn_out, self.hidden_b, L.ln2, self.normed, s.eps,
                                              L.router, self.router_logits, bias=L.router_bias)
                be.mxfp_lowbit_selected_swiglu_router(L.gate_up_blocks, L.gate_up_scales, self.normed,
                                                      self.router_logits, self.router_idx, self.router_scores,
                                                      self.act, bits=4, alpha=s.swiglu_alpha, limit=s.swiglu_limit,
                                                      renormalize=True, bias=L.gate_up_bias)
            else:
                be.add_rms_norm_router_topk(self.hidden_a, self.attn_out, self.hidden_b, L.ln2, self.normed, s.eps,
                                            L.router, self.router_idx, self.router_scores, bias=L.router_bias,
                                            renormalize=True)
                be.mxfp_lowbit_selected_swiglu_tokens(L.gate_up_blocks, L.gate_up_scales, self.normed,
                                                      self.router_idx, self.act, bits=4, alpha=s.swiglu_alpha,
                                                      limit=s.swiglu_limit, bias=L.gate_up_bias)
            be.mxfp_lowbit_weighted_down_tokens(L.down_blocks, L.down_scales, self.act, self.router_idx,
                                                self.router_scores, self.moe, bits=4, bias=L.down_bias)
        be.add_then_rms_norm_rows(self.hidden_b, self.moe, self.hidden_a, w.final_norm, self.final_all, s.eps)
        be.matvec_argmax_batched(w.lm_head, self.final_all, out=self.tokens)
        be.record_tokens_advance(self.tokens, self.position, self.base, self.history)

    def capture(self) -> None:
        """Record one batched step into a HIP graph (scratch reserved first)."""
        self._reserve_scratch()
        torch.cuda.synchronize(self.device)
        self._graph_stream = torch.cuda.Stream(self.device)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph, stream=self._graph_stream):
            self.step()

    def prime(self, tokens: list[int], position: int) -> None:
        if len(tokens) != self.batch:
            raise ValueError("one start token per sequence")
        if not 0 <= position < self.capacity:
            raise ValueError("position outside the KV cache")
        self.tokens.copy_(torch.tensor(tokens, dtype=torch.int64))
        self.position.fill_(int(position))
        self.base.fill_(int(position))
        self.history.zero_()

    def generate(self, start_tokens: list[int], position: int, steps: int, use_graph: bool = True) -> list[list[int]]:
        """Greedy-decode `steps` tokens of every sequence; returns one id list per sequence."""
        if position + steps > self.capacity:
            raise ValueError("not enough KV capacity for the requested steps")
        if steps > self.history.shape[1]:
            raise ValueError("history buffer too small")
        if use_graph and self.graph is None:
            self.capture()
        self.prime(start_tokens, position)
        for _ in range(steps):
            if use_graph:
                self.graph.replay()
            else:
                self.step()
        torch.cuda.synchronize(self.device)
        return self.history[:, :steps].cpu().tolist()
