"""CPU restatement of one greedy decode step -- TEST INFRASTRUCTURE ONLY.

Mirrors the reference runtime's dense Triton path (gpu_runtime.py:11429-11726) and
MoE path (gpu_runtime.py:8968-9908) operator by operator, using the binary32
restatements in tt_oracle.c, so a GPU decode can be compared token for token and
bit for bit.  Weights are numpy copies of the tensors the GPU decoder uses.
"""

from __future__ import annotations

import numpy as np

from . import F16, gemv, lib


def _np(t):
    """torch tensor -> numpy (fp16 stays float16, uint8 stays uint8)."""
    return t.detach().cpu().numpy()


def lanes(cols: int, group_chunks: int = 1) -> int:
    """The kernels' lanes-per-row rule (restated from tt_gemv_lanes_per_row)."""
    chunks = cols // 32
    best, best_util = 0, -1.0
    for c in (64, 32, 16):
        if group_chunks > 1 and c % group_chunks:
            continue
        r = -(-chunks // c)
        util = chunks / (r * c)
        if util > best_util + 1e-12:
            best, best_util = c, util
    return best


def int4_gemv(packed: np.ndarray, scales: np.ndarray, x: np.ndarray, group: int) -> np.ndarray:
    cols = packed.shape[1] * 2
    L = group // 32
    return gemv("int4_sym", "group", packed, scales, x, cols=cols, lpr=lanes(cols, L), L=L, s_row=scales.shape[1],
                s_grp=1)


def f16_gemv(w: np.ndarray, x: np.ndarray, bias: np.ndarray | None = None) -> np.ndarray:
    rows, cols = w.shape
    y = gemv("f16w", "none", w.view(np.uint8).reshape(rows, -1), None, x, cols=cols, lpr=lanes(cols))
    if bias is not None:
        y = (y.astype(np.float32) + bias.astype(np.float32)).astype(np.float16)
    return y


def _p(a: np.ndarray):
    return a.ctypes.data


def rms_norm(x, w, eps):
    out = np.empty_like(x)
    lib().tto_rms_norm(_p(x), F16, _p(w), F16, _p(out), F16, x.size, eps, 0.0)
    return out


def add_rms_norm(a, b, w, eps):
    res = np.empty_like(a)
    out = np.empty_like(a)
    lib().tto_add_rms_norm(_p(a), _p(b), _p(res), F16, _p(w), F16, _p(out), F16, a.size, eps)
    return res, out


def rope(q, k, cos_row, sin_row, heads, kv_heads, head_dim):
    q, k = q.copy(), k.copy()
    lib().tto_rope(_p(q), _p(k), F16, _p(np.ascontiguousarray(cos_row)), _p(np.ascontiguousarray(sin_row)), heads,
                   kv_heads, head_dim)
    return q, k


def attention(q, kc, vc, tokens, heads, kv_heads, D, sinks=None):
    cap = kc.shape[1]
    out = np.empty(heads * D, dtype=np.float16)
    lib().tto_attention(_p(q), _p(kc), _p(vc), F16, cap * D, D, cap * D, D, _p(sinks) if sinks is not None else None,
                        F16, tokens, heads, kv_heads, D, _p(out))
    return out


def lm_head_argmax(w, x) -> tuple[int, np.ndarray]:
    logits = f16_gemv(w, x)
    return int(lib().tto_argmax(_p(logits), F16, logits.size)), logits


class DenseRef:
    """Oracle twin of thintensor_amd.decode.DenseDecoder."""

    def __init__(self, weights) -> None:
        self.s = s = weights.shape
        self.embed = _np(weights.embed)
        self.lm_head = _np(weights.lm_head)
        self.final_norm = _np(weights.final_norm)
        self.layers = []
        for L in weights.layers:
            self.layers.append({k: (_np(getattr(L, k)[0]), _np(getattr(L, k)[1]))
                                for k in ("q", "k", "v", "o", "gate", "up", "down")}
                               | {"ln1": _np(L.ln1), "ln2": _np(L.ln2)})
        self.kc = _np(weights.k_cache).copy()
        self.vc = _np(weights.v_cache).copy()
        self.cos = _np(weights.cos)
        self.sin = _np(weights.sin)

    def step(self, token: int, pos: int) -> tuple[int, np.ndarray]:
        s = self.s
        g = s.group
        h = self.embed[token].copy()
        normed = rms_norm(h, self.layers[0]["ln1"], s.eps)
        final = None
        for li, L in enumerate(self.layers):
            q = int4_gemv(*L["q"], normed, g)
            k = int4_gemv(*L["k"], normed, g)
            v = int4_gemv(*L["v"], normed, g)
            q, k = rope(q, k, self.cos[pos], self.sin[pos], s.heads, s.kv_heads, s.head_dim)
            self.kc[li, :, pos, :] = k.reshape(s.kv_heads, s.head_dim)
            self.vc[li, :, pos, :] = v.reshape(s.kv_heads, s.head_dim)
            attn = attention(q, self.kc[li], self.vc[li], pos + 1, s.heads, s.kv_heads, s.head_dim)
            o = int4_gemv(*L["o"], attn, g)
            h2, normed = add_rms_norm(h, o, L["ln2"], s.eps)
            gate = int4_gemv(*L["gate"], normed, g)
            up = int4_gemv(*L["up"], normed, g)
            act = np.empty_like(gate)
            lib().tto_silu_mul(_p(gate), _p(up), _p(act), F16, gate.size)
            mlp = int4_gemv(*L["down"], act, g)
            nxt = self.layers[li + 1]["ln1"] if li + 1 < len(self.layers) else self.final_norm
            h, normed = add_rms_norm(h2, mlp, nxt, s.eps)
            final = normed
        return lm_head_argmax(self.lm_head, final)

    def generate(self, token: int, pos: int, steps: int, margins: list | None = None) -> list[int]:
        """Greedy tokens; ``margins`` (if given) receives each step's gap between the two
        largest logits, and ``self.last_logits`` holds the final step's logits."""
        out = []
        for i in range(steps):
            token, logits = self.step(token, pos + i)
            out.append(token)
            if margins is not None:
                top2 = np.partition(logits.astype(np.float32), -2)[-2:]
                margins.append(float(top2[1] - top2[0]))
        self.last_logits = logits if steps else None
        return out


class MoERef:
    """Oracle twin of thintensor_amd.decode.MoEDecoder."""

    def __init__(self, weights) -> None:
        self.s = weights.shape
        self.embed = _np(weights.embed)
        self.lm_head = _np(weights.lm_head)
        self.final_norm = _np(weights.final_norm)
        names = ("q", "k", "v", "o", "q_bias", "k_bias", "v_bias", "o_bias", "sinks", "ln1", "ln2", "router",
                 "router_bias", "gate_up_blocks", "gate_up_scales", "gate_up_bias", "down_blocks", "down_scales",
                 "down_bias")
        self.layers = [{n: np.ascontiguousarray(_np(getattr(L, n))) for n in names} for L in weights.layers]
        self.kc = _np(weights.k_cache).copy()
        self.vc = _np(weights.v_cache).copy()
        self.cos = _np(weights.cos)
        self.sin = _np(weights.sin)

    def step(self, token: int, pos: int) -> tuple[int, np.ndarray]:
        s = self.s
        h = self.embed[token].copy()
        normed = rms_norm(h, self.layers[0]["ln1"], s.eps)
        final = None
        for li, L in enumerate(self.layers):
            q = f16_gemv(L["q"], normed, L["q_bias"])
            k = f16_gemv(L["k"], normed, L["k_bias"])
            v = f16_gemv(L["v"], normed, L["v_bias"])
            q, k = rope(q, k, self.cos[pos], self.sin[pos], s.heads, s.kv_heads, s.head_dim)
            self.kc[li, :, pos, :] = k.reshape(s.kv_heads, s.head_dim)
            self.vc[li, :, pos, :] = v.reshape(s.kv_heads, s.head_dim)
            attn = attention(q, self.kc[li], self.vc[li], pos + 1, s.heads, s.kv_heads, s.head_dim, L["sinks"])
            o = f16_gemv(L["o"], attn, L["o_bias"])
            h2, normed = add_rms_norm(h, o, L["ln2"], s.eps)
            idx = np.empty(s.top_k, dtype=np.int32)
            scores = np.empty(s.top_k, dtype=np.float16)
            lib().tto_router(_p(L["router"]), F16, s.hidden, _p(normed), F16, s.hidden, _p(L["router_bias"]), F16,
                             s.experts, s.top_k, 1, _p(idx), _p(scores), F16)
            act = np.empty((s.top_k, s.intermediate), dtype=np.float16)
            gb, gs, gbias = L["gate_up_blocks"], L["gate_up_scales"], L["gate_up_bias"]
            lib().tto_swiglu(5, F16, _p(gb), gb.strides[0], gb.strides[1], _p(gs), gs.strides[0], gs.strides[1],
                             _p(normed), F16, 0, _p(idx), s.top_k, _p(gbias), F16, gbias.shape[1], s.swiglu_alpha,
                             s.swiglu_limit, _p(act), F16, s.intermediate, s.intermediate, s.hidden, lanes(s.hidden))
            moe = np.empty(s.hidden, dtype=np.float16)
            db, ds, dbias = L["down_blocks"], L["down_scales"], L["down_bias"]
            lib().tto_weighted_down(5, F16, _p(db), db.strides[0], db.strides[1], _p(ds), ds.strides[0], ds.strides[1],
                                    _p(act), F16, s.intermediate, _p(idx), _p(scores), F16, s.top_k, _p(dbias), F16,
                                    dbias.shape[1], _p(moe), F16, s.hidden, s.intermediate, lanes(s.intermediate))
            if li + 1 < len(self.layers):
                h, normed = add_rms_norm(h2, moe, self.layers[li + 1]["ln1"], s.eps)
            else:
                h = (h2.astype(np.float32) + moe.astype(np.float32)).astype(np.float16)
                final = rms_norm(h, self.final_norm, s.eps)
        return lm_head_argmax(self.lm_head, final)

    def generate(self, token: int, pos: int, steps: int, margins: list | None = None) -> list[int]:
        """Greedy tokens; ``margins`` (if given) receives each step's gap between the two
        largest logits, and ``self.last_logits`` holds the final step's logits."""
        out = []
        for i in range(steps):
            token, logits = self.step(token, pos + i)
            out.append(token)
            if margins is not None:
                top2 = np.partition(logits.astype(np.float32), -2)[-2:]
                margins.append(float(top2[1] - top2[0]))
        self.last_logits = logits if steps else None
        return out
