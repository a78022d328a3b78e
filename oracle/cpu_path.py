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
    """Logical CPUs this process may run on."""
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:  # pragma: no cover
        return os.cpu_count() or 1


def host_info() -> dict:
    """CPU model, physical cores and logical threads available to this process
    (/proc/cpuinfo: a physical core is a distinct (physical id, core id) pair)."""
    try:
        allowed = os.sched_getaffinity(0)
    except AttributeError:  # pragma: no cover
        allowed = set(range(os.cpu_count() or 1))
    model, cores, cur = "unknown", set(), {}
    try:
        with open("/proc/cpuinfo") as f:
            for line in f.read().split("\n") + [""]:
                if not line.strip():
                    if cur.get("processor") is not None and int(cur["processor"]) in allowed:
                        cores.add((cur.get("physical id", "0"), cur.get("core id", cur["processor"])))
                        model = cur.get("model name", model)
                    cur = {}
                    continue
                k, _, v = line.partition(":")
                cur[k.strip()] = v.strip()
    except OSError:  # pragma: no cover
        pass
    physical = len(cores) or len(allowed)
    return {"cpu_model": model, "physical_cores": physical, "logical_threads": len(allowed)}


def physical_cores() -> int:
    return host_info()["physical_cores"]


def time_call(fn, min_s: float = 1.0, min_calls: int = 20, warmup: int = 2) -> float:
    """Median microseconds per call over at least `min_calls` calls and `min_s` seconds."""
    for _ in range(warmup):
        fn()
    ts = []
    t_end = time.perf_counter() + min_s
    while len(ts) < min_calls or time.perf_counter() < t_end:
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
        if len(ts) >= 2000:
            break
    ts.sort()
    return ts[len(ts) // 2] * 1e6


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
    threads = physical_cores()
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


# ---------------------------------------------------------------- dequantise-then-matmul rows (torch fallback form)

E2M1 = (0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0, -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0)


def dequant_mxfp4(blocks: torch.Tensor, scales: torch.Tensor, dtype=torch.float32) -> torch.Tensor:
    """[N, G, 16] e2m1 bytes + [N, G] E8M0 -> [N, G*32]: table lookup of both nibbles
    (element 2j = low nibble) then ldexp by e - 127, as gpu_runtime.py:12865-12915."""
    lut = torch.tensor(E2M1, dtype=dtype)
    low = lut[(blocks & 0x0F).long()]
    high = lut[(blocks >> 4).long()]
    vals = torch.stack((low, high), dim=-1).reshape(*blocks.shape[:-1], 32)
    vals = torch.ldexp(vals, (scales.to(torch.int32) - 127).unsqueeze(-1).to(dtype))
    return vals.reshape(blocks.shape[0], -1)


def dequant_int4(packed: torch.Tensor, scales: torch.Tensor, group: int) -> torch.Tensor:
    """(c - 8) * s with fp32 group scales (the torch fallback of an int4 page)."""
    c = torch.stack(((packed & 0x0F), (packed >> 4)), dim=-1).reshape(packed.shape[0], -1).float()
    return (c - 8.0) * scales.float().repeat_interleave(group, dim=1)


def dequant_lowbit_affine(packed: torch.Tensor, scale_zero: torch.Tensor, bits: int, group: int) -> torch.Tensor:
    """(c - z) * s for 2- or 1-bit codes packed LSB first, fp16 (s, z) pairs per group."""
    per = 8 // bits
    shifts = torch.arange(per, dtype=torch.uint8) * bits
    c = ((packed.unsqueeze(-1) >> shifts) & ((1 << bits) - 1)).reshape(packed.shape[0], -1).float()
    s = scale_zero[..., 0].float().repeat_interleave(group, dim=1)
    z = scale_zero[..., 1].float().repeat_interleave(group, dim=1)
    return (c - z) * s


def _slow(fn, budget_s):
    """time_call for calls of tens of milliseconds: five calls at least."""
    return time_call(fn, budget_s, min_calls=5, warmup=1)


def _row(name: str, nbytes: int, deq_us: float | None, mv_us: float, threads: int, op: str) -> dict:
    total = (deq_us or 0.0) + mv_us
    return {"row": name, "threads": threads, "dequant_us": deq_us, "matmul_us": mv_us, "us_per_call": total,
            "GB_s": nbytes / total / 1e3, "algorithmic_bytes": nbytes, "op": op}


def gemv_rows(seed: int, budget_s: float = 1.0) -> list[dict]:
    """BASELINE CPU rows C1-C3 on the GPU box's host (bounded: about one second each)."""
    g = torch.Generator().manual_seed(seed)
    n = physical_cores()
    rows = []
    # C1: the reference's CPU int4 path at 8192 x 2048, all physical cores and one thread
    R, K, G = 8192, 2048, 128
    pk = torch.randint(0, 256, (R, K // 2), generator=g, dtype=torch.uint8)
    sc = (torch.randn((R, K // G), generator=g).abs() * 0.02).to(torch.float16)
    x = torch.randn(K, generator=g).to(torch.float16)
    m = Int4CPU(pk, sc, G)
    nb = R * K // 2 + R * (K // G) * 2 + 2 * K + 2 * R
    for t in (n, 1):
        torch.set_num_threads(t)
        rows.append(_row("C1 int4 g128 8192x2048", nb, None, time_call(lambda: m.mv(x), budget_s), t,
                         "torch.ops.aten._weight_int4pack_mm_for_cpu"))
    torch.set_num_threads(n)
    # C2: dequantise then torch.mv in fp32 (gpu_runtime.py:12317-12324 form)
    xf = x.float()
    w = dequant_int4(pk, sc, G)
    rows.append(_row("C2 int4 g128 8192x2048 dequant+mv", nb, _slow(lambda: dequant_int4(pk, sc, G), budget_s),
                     _slow(lambda: torch.mv(w, xf), budget_s), n, "dequant (c-8)*s, torch.mv fp32"))
    R, K = 17920, 5120
    w8 = (torch.randn((R, K), generator=g) * 0.05).to(torch.float8_e4m3fn)
    s8 = torch.rand(R, generator=g) * 0.01
    x5 = torch.randn(K, generator=g).float()
    deq8 = lambda: w8.to(torch.float32) * s8[:, None]  # noqa: E731
    wf = deq8()
    rows.append(_row("C2 fp8-e4m3 17920x5120 dequant+mv", R * K + 4 * R + 2 * K + 2 * R, _slow(deq8, budget_s),
                     _slow(lambda: torch.mv(wf, x5), budget_s), n, "w.float() * s[:, None], torch.mv fp32"))
    del w8, wf
    for bits, R in ((2, 17920), (1, 5120)):
        pb = torch.randint(0, 256, (R, K * bits // 8), generator=g, dtype=torch.uint8)
        sz = torch.stack((torch.randn((R, K // 64), generator=g).abs() * 0.05,
                          torch.rand((R, K // 64), generator=g) * ((1 << bits) - 1)), dim=-1).to(torch.float16)
        deq = lambda pb=pb, sz=sz, bits=bits: dequant_lowbit_affine(pb, sz, bits, 64)  # noqa: E731
        wq = deq()
        rows.append(_row(f"C2 q{bits} g64 affine {R}x{K} dequant+mv", R * K * bits // 8 + R * (K // 64) * 4 + 2 * K + 2 * R,
                         _slow(deq, budget_s), _slow(lambda wq=wq: torch.mv(wq, x5), budget_s), n,
                         "(c-z)*s, torch.mv fp32"))
        del wq
    R, K = 5760, 2880
    blocks = torch.randint(0, 256, (R, K // 32, 16), generator=g, dtype=torch.uint8)
    exps = torch.randint(119, 124, (R, K // 32), generator=g, dtype=torch.uint8)
    xm = torch.randn(K, generator=g).float()
    wm = dequant_mxfp4(blocks, exps)
    rows.append(_row("C2 MXFP4 expert 5760x2880 dequant+mv", R * K // 2 + R * K // 32 + 2 * K + 2 * R,
                     _slow(lambda: dequant_mxfp4(blocks, exps), budget_s), _slow(lambda: torch.mv(wm, xm), budget_s),
                     n, "e2m1 LUT + ldexp (gpu_runtime.py:12865-12915), torch.mv fp32"))
    del wm
    # C3: lm_head fp32 GEMV, round to fp16, first-index argmax
    V, H = 128256, 2048
    head = (torch.randn((V, H), generator=g) * 0.02)
    xh = torch.randn(H, generator=g)
    us = time_call(lambda: torch.argmax(torch.mv(head, xh).to(torch.float16)), budget_s, min_calls=5)
    rows.append(_row("C3 lm_head 128256x2048 + argmax", 2 * V * H + 2 * H + 2 * V, None, us, n,
                     "torch.mv fp32 (weights held as fp32), fp16 round, torch.argmax"))
    return rows


# ---------------------------------------------------------------- gpt-oss-shaped decode on the CPU


class MoECPU:
    """Torch-CPU decode step of the gpt-oss-shaped MoE model, in the GPU decoder's call
    order, with each selected MXFP4 expert dequantised then multiplied by torch.mv
    (the reference's torch fallback, gpu_runtime.py:9663-9704)."""

    def __init__(self, weights) -> None:
        self.s = s = weights.shape
        self.embed = weights.embed.cpu()
        self.lm_head = weights.lm_head.cpu().float()
        self.final_norm = weights.final_norm.cpu().float()
        names = ("q", "k", "v", "o", "q_bias", "k_bias", "v_bias", "o_bias", "sinks", "ln1", "ln2", "router",
                 "router_bias", "gate_up_bias", "down_bias")
        self.layers = []
        for L in weights.layers:
            d = {n: getattr(L, n).cpu().float() for n in names}
            for n in ("gate_up_blocks", "gate_up_scales", "down_blocks", "down_scales"):
                d[n] = getattr(L, n).cpu()
            self.layers.append(d)
        self.kc = weights.k_cache.cpu().float()
        self.vc = weights.v_cache.cpu().float()
        self.cos = weights.cos.cpu().float()
        self.sin = weights.sin.cpu().float()

    @staticmethod
    def _rms(x, w, eps):
        return x * torch.rsqrt(x.pow(2).mean() + eps) * w

    def _rope(self, t, heads, pos):
        d = self.s.head_dim
        x = t.reshape(heads, d)
        a, b = x[:, : d // 2], x[:, d // 2:]
        c, s_ = self.cos[pos], self.sin[pos]
        return torch.cat((a * c - b * s_, b * c + a * s_), dim=-1).reshape(-1)

    def step(self, token: int, pos: int) -> int:
        s = self.s
        h = self.embed[token].float()
        for li, L in enumerate(self.layers):
            x = self._rms(h, L["ln1"], s.eps)
            q = self._rope(torch.mv(L["q"], x) + L["q_bias"], s.heads, pos)
            k = self._rope(torch.mv(L["k"], x) + L["k_bias"], s.kv_heads, pos)
            v = torch.mv(L["v"], x) + L["v_bias"]
            self.kc[li, :, pos] = k.reshape(s.kv_heads, s.head_dim)
            self.vc[li, :, pos] = v.reshape(s.kv_heads, s.head_dim)
            g = s.heads // s.kv_heads
            keys, vals = self.kc[li, :, : pos + 1], self.vc[li, :, : pos + 1]
            qh = q.reshape(s.kv_heads, g, s.head_dim)
            scores = torch.matmul(qh, keys.transpose(1, 2)) * (s.head_dim ** -0.5)
            sinks = L["sinks"].reshape(s.kv_heads, g, 1)
            full = torch.softmax(torch.cat((sinks, scores), dim=-1), dim=-1)[..., 1:]
            attn = torch.matmul(full, vals).reshape(-1)
            h = h + torch.mv(L["o"], attn) + L["o_bias"]
            x = self._rms(h, L["ln2"], s.eps)
            logits = torch.mv(L["router"], x) + L["router_bias"]
            top = torch.topk(logits, s.top_k)
            p = torch.softmax(top.values, dim=0)
            moe = torch.zeros_like(h)
            for slot in range(s.top_k):
                e = int(top.indices[slot])
                gu = torch.mv(dequant_mxfp4(L["gate_up_blocks"][e], L["gate_up_scales"][e]), x) + L["gate_up_bias"][e]
                gate = gu[0::2].clamp(max=s.swiglu_limit)
                up = gu[1::2].clamp(min=-s.swiglu_limit, max=s.swiglu_limit)
                act = (up + 1) * gate * torch.sigmoid(gate * s.swiglu_alpha)
                down = torch.mv(dequant_mxfp4(L["down_blocks"][e], L["down_scales"][e]), act) + L["down_bias"][e]
                moe = moe + p[slot] * down
            h = h + moe
        logits = torch.mv(self.lm_head, self._rms(h, self.final_norm, s.eps)).to(torch.float16)
        return int(torch.argmax(logits))


def moe_decode_baseline(weights, start_token: int, budget_s: float = 15.0, max_tokens: int = 8) -> dict:
    threads = physical_cores()
    torch.set_num_threads(threads)
    model = MoECPU(weights)
    pos = weights.shape.prior_tokens
    tok = model.step(start_token, pos)  # warm-up
    n, t0 = 0, time.perf_counter()
    while n < max_tokens:
        tok = model.step(tok, pos + 1 + n)
        n += 1
        if time.perf_counter() - t0 > budget_s:
            break
    elapsed = time.perf_counter() - t0
    return {"value": n / elapsed, "unit": "tok/s", "cores": threads, "kind": "port",
            "sample": f"{n} greedy decode tokens of the gpt-oss-20b-shaped model after one warm-up token; selected "
                      f"MXFP4 experts dequantised (e2m1 LUT + ldexp) then torch.mv, fp32 elsewhere"}
