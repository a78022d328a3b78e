"""CPU baseline: the reference's own CPU dequant+matmul path, restated with the same
torch library ops -- TEST/BENCH INFRASTRUCTURE ONLY (bench.py's cpu_baseline leg).

The reference's CPU int4 path (ThinGpuPagePool.cpu_int4_matvec,
gpu_runtime.py:3107-3230) unpacks the nibbles to int32 [N, K], converts them with
torch.ops.aten._convert_weight_to_int4pack_for_cpu(codes, 1) and multiplies with
torch.ops.aten._weight_int4pack_mm_for_cpu(x_bf16[1, K], packed, group,
scale_zeros) where scale_zeros is bf16 [G, N, 2] = (s, 0) for symmetric codes
(w = (q - 8) * s).  The rest of a decode step (norms, RoPE, attention, SiLU,
lm_head) runs as plain torch CPU ops in float32, which is what the reference's
torch fallback does on a CPU device.  This is a port (kind "port"): the reference
itself is Python and needs a GPU runtime, so it is not run.
"""

from __future__ import annotations

import os
import time

import torch


def cpu_threads() -> int:
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:  # pragma: no cover
        return os.cpu_count() or 1


class Int4CPU:
    """One int4 matrix prepared for the reference's CPU op."""

    def __init__(self, packed_u8: torch.Tensor, scales: torch.Tensor, group: int) -> None:
        p = packed_u8.cpu()
        codes = torch.empty((p.shape[0], p.shape[1] * 2), dtype=torch.int32)
        codes[:, 0::2] = (p & 0x0F).to(torch.int32)
        codes[:, 1::2] = (p >> 4).to(torch.int32)
        self.packed = torch.ops.aten._convert_weight_to_int4pack_for_cpu(codes, 1)
        s = scales.cpu().to(torch.float32)
        sz = torch.zeros((s.shape[1], s.shape[0], 2), dtype=torch.bfloat16)
        sz[:, :, 0] = s.t().to(torch.bfloat16)
        self.scale_zeros = sz
        self.group = group
        self.rows = p.shape[0]

    def mv(self, x: torch.Tensor) -> torch.Tensor:
        xb = x.to(torch.bfloat16).reshape(1, -1)
        y = torch.ops.aten._weight_int4pack_mm_for_cpu(xb, self.packed, self.group, self.scale_zeros)
        return y.reshape(-1).to(torch.float16)


class DenseCPU:
    """Torch-CPU decode step of the dense model (same call order as the GPU decoder)."""

    def __init__(self, weights) -> None:
        s = self.s = weights.shape
        self.embed = weights.embed.cpu()
        self.lm_head = weights.lm_head.cpu().to(torch.float32)
        self.final_norm = weights.final_norm.cpu().float()
        self.layers = []
        for L in weights.layers:
            self.layers.append({k: Int4CPU(*getattr(L, k), s.group) for k in ("q", "k", "v", "o", "gate", "up", "down")}
                               | {"ln1": L.ln1.cpu().float(), "ln2": L.ln2.cpu().float()})
        self.kc = weights.k_cache.cpu().clone()
        self.vc = weights.v_cache.cpu().clone()
        self.cos = weights.cos.cpu().float()
        self.sin = weights.sin.cpu().float()

    @staticmethod
    def _rms(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
        xf = x.float()
        return (xf * torch.rsqrt(xf.pow(2).mean() + eps) * w).to(torch.float16)

    def _rope(self, t: torch.Tensor, heads: int, pos: int) -> torch.Tensor:
        d = self.s.head_dim
        x = t.float().reshape(heads, d)
        a, b = x[:, : d // 2], x[:, d // 2:]
        c, s_ = self.cos[pos], self.sin[pos]
        return torch.cat((a * c - b * s_, b * c + a * s_), dim=-1).reshape(-1).to(torch.float16)

    def step(self, token: int, pos: int) -> int:
        s = self.s
        h = self.embed[token].clone()
        normed = self._rms(h, self.layers[0]["ln1"], s.eps)
        for li, L in enumerate(self.layers):
            q = self._rope(L["q"].mv(normed), s.heads, pos)
            k = self._rope(L["k"].mv(normed), s.kv_heads, pos)
            v = L["v"].mv(normed)
            self.kc[li, :, pos] = k.reshape(s.kv_heads, s.head_dim)
            self.vc[li, :, pos] = v.reshape(s.kv_heads, s.head_dim)
            g = s.heads // s.kv_heads
            keys = self.kc[li, :, : pos + 1].float()
            vals = self.vc[li, :, : pos + 1].float()
            qh = q.float().reshape(s.kv_heads, g, s.head_dim)
            scores = torch.matmul(qh, keys.transpose(1, 2)) * (s.head_dim ** -0.5)
            attn = torch.matmul(torch.softmax(scores, dim=-1), vals).reshape(-1).to(torch.float16)
            o = L["o"].mv(attn)
            h = (h.float() + o.float()).to(torch.float16)
            normed = self._rms(h, L["ln2"], s.eps)
            gate = L["gate"].mv(normed).float()
            up = L["up"].mv(normed).float()
            act = (torch.nn.functional.silu(gate) * up).to(torch.float16)
            h = (h.float() + L["down"].mv(act).float()).to(torch.float16)
            nxt = self.layers[li + 1]["ln1"] if li + 1 < len(self.layers) else self.final_norm
            normed = self._rms(h, nxt, s.eps)
        logits = torch.mv(self.lm_head, normed.float()).to(torch.float16)
        return int(torch.argmax(logits))


def dense_decode_baseline(weights, start_token: int, budget_s: float = 12.0, max_tokens: int = 32) -> dict:
    """Time the CPU decode on a bounded sample: tokens until `budget_s` elapse."""
    threads = cpu_threads()
    torch.set_num_threads(threads)
    model = DenseCPU(weights)
    pos = weights.shape.prior_tokens
    tok = start_token
    model.step(tok, pos)  # warm-up (first-call overheads)
    n, t0 = 0, time.perf_counter()
    while n < max_tokens:
        tok = model.step(tok, pos + 1 + n)
        n += 1
        if time.perf_counter() - t0 > budget_s:
            break
    elapsed = time.perf_counter() - t0
    return {"value": n / elapsed, "unit": "tok/s", "cores": threads, "kind": "port",
            "sample": f"{n} greedy decode tokens of the same synthetic model after one warm-up token; int4 layers via "
                      f"torch.ops.aten._weight_int4pack_mm_for_cpu (the reference's CPU path), other ops torch CPU fp32"}
