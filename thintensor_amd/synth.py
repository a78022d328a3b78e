"""Seeded synthetic model weights for the benchmark configurations.

No checkpoints are available offline, so weights are random with the shapes and
distributions the benchmark configurations name:

* Llama-3.2-1B-shaped dense model: int4 g128 linear layers (codes uniform over the
  16 values, fp16 scales |N(0,1)| * 0.02), fp16 embeddings and lm_head N(0, 0.02),
  RMSNorm weights 1, fp16 KV cache pre-filled with N(0,1) for the prior tokens.
* gpt-oss-20B-shaped MoE model: fp16 attention (with biases and per-head sinks),
  router fp16 N(0, 0.02) + bias, MXFP4 experts (e2m1 codes uniform over the 16
  values, E8M0 exponents uniform in [-8, -4]), expert biases, fp16 embeddings and
  lm_head N(0, 0.02).

Tensors are drawn with torch's generator on the target device from one seed, so a
run is reproducible and the same bytes can be copied to the host for the CPU check.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import torch


@dataclass(frozen=True)
class DenseShape:
    name: str = "llama-3.2-1b-shaped"
    layers: int = 16
    hidden: int = 2048
    heads: int = 32
    kv_heads: int = 8
    head_dim: int = 64
    intermediate: int = 8192
    vocab: int = 128256
    rope_theta: float = 500000.0
    eps: float = 1e-5
    group: int = 128
    prior_tokens: int = 512
    max_new_tokens: int = 64

    @property
    def q_dim(self) -> int:
        return self.heads * self.head_dim

    @property
    def kv_dim(self) -> int:
        return self.kv_heads * self.head_dim


@dataclass(frozen=True)
class MoEShape:
    name: str = "gpt-oss-20b-shaped"
    layers: int = 24
    hidden: int = 2880
    heads: int = 64
    kv_heads: int = 8
    head_dim: int = 64
    experts: int = 32
    top_k: int = 4
    intermediate: int = 2880
    vocab: int = 201088
    rope_theta: float = 150000.0
    eps: float = 1e-5
    prior_tokens: int = 1024
    max_new_tokens: int = 64
    swiglu_alpha: float = 1.702
    swiglu_limit: float = 7.0

    @property
    def q_dim(self) -> int:
        return self.heads * self.head_dim

    @property
    def kv_dim(self) -> int:
        return self.kv_heads * self.head_dim


LLAMA_1B = DenseShape()
GPT_OSS_20B = MoEShape()


def _normal(g: torch.Generator, shape, std: float, device) -> torch.Tensor:
    return (torch.randn(shape, generator=g, device=device, dtype=torch.float32) * std).to(torch.float16)


def _int4(g: torch.Generator, rows: int, cols: int, group: int, device,
          centered: bool = False) -> tuple[torch.Tensor, torch.Tensor]:
    """Packed int4 codes and fp16 group scales |N(0,1)| * 0.02.  Codes are uniform over
    q in [-8, 7] (the benchmark definition) or, when ``centered``, over q in [-7, 7]
    (the clamp of the reference's _quantize_int4_rows, gpu_runtime.py:6668), which has
    no mean and so no row bias common to every output."""
    if centered:
        lo = torch.randint(1, 16, (rows, cols // 2), generator=g, device=device, dtype=torch.uint8)
        hi = torch.randint(1, 16, (rows, cols // 2), generator=g, device=device, dtype=torch.uint8)
        packed = lo | (hi << 4)
    else:
        packed = torch.randint(0, 256, (rows, cols // 2), generator=g, device=device, dtype=torch.uint8)
    scales = (torch.randn((rows, cols // group), generator=g, device=device).abs() * 0.02).to(torch.float16)
    return packed, scales


@dataclass
class DenseLayer:
    q: tuple[torch.Tensor, torch.Tensor]
    k: tuple[torch.Tensor, torch.Tensor]
    v: tuple[torch.Tensor, torch.Tensor]
    o: tuple[torch.Tensor, torch.Tensor]
    gate: tuple[torch.Tensor, torch.Tensor]
    up: tuple[torch.Tensor, torch.Tensor]
    down: tuple[torch.Tensor, torch.Tensor]
    ln1: torch.Tensor
    ln2: torch.Tensor


@dataclass
class DenseWeights:
    shape: DenseShape
    embed: torch.Tensor
    lm_head: torch.Tensor
    final_norm: torch.Tensor
    layers: list[DenseLayer] = field(default_factory=list)
    k_cache: torch.Tensor | None = None   # [layers, kv_heads, capacity, head_dim]
    v_cache: torch.Tensor | None = None
    cos: torch.Tensor | None = None       # [capacity, head_dim/2]
    sin: torch.Tensor | None = None


def rope_tables(head_dim: int, theta: float, positions: int, device) -> tuple[torch.Tensor, torch.Tensor]:
    """cos/sin rows as the reference builds them (gpu_runtime.py:8754-8785): float32
    inv_freq = theta ** (-arange(0, d, 2) / d), angle = inv_freq * float(position),
    cos/sin in float32, then cast to fp16.  Evaluated on the host in float32."""
    freq_index = torch.arange(0, head_dim, 2, dtype=torch.float32)
    inv_freq = theta ** (-freq_index / head_dim)
    ang = torch.arange(positions, dtype=torch.float32)[:, None] * inv_freq[None, :]
    return ang.cos().to(torch.float16).to(device), ang.sin().to(torch.float16).to(device)


def make_dense(shape: DenseShape = LLAMA_1B, device="cuda", seed: int = 0, capacity: int | None = None,
               centered_codes: bool = False) -> DenseWeights:
    """Seeded random weights of a dense int4 model.  With the benchmark's codes
    (q in [-8, 7], mean -0.5) every row of a layer carries the same sign of bias, the
    MLP output grows about sixteenfold per layer at the Llama-1B shape and the fp16
    residual overflows after four layers, so the token stream is that of NaN logits;
    ``centered_codes`` draws q in [-7, 7] and keeps the activations finite."""
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    H, I, G = shape.hidden, shape.intermediate, shape.group
    w = DenseWeights(
        shape=shape,
        embed=_normal(g, (shape.vocab, H), 0.02, device),
        lm_head=_normal(g, (shape.vocab, H), 0.02, device),
        final_norm=torch.ones(H, device=device, dtype=torch.float16),
    )
    for _ in range(shape.layers):
        w.layers.append(DenseLayer(
            q=_int4(g, shape.q_dim, H, G, device, centered_codes), k=_int4(g, shape.kv_dim, H, G, device, centered_codes),
            v=_int4(g, shape.kv_dim, H, G, device, centered_codes), o=_int4(g, H, shape.q_dim, G, device, centered_codes),
            gate=_int4(g, I, H, G, device, centered_codes), up=_int4(g, I, H, G, device, centered_codes),
            down=_int4(g, H, I, G, device, centered_codes),
            ln1=torch.ones(H, device=device, dtype=torch.float16), ln2=torch.ones(H, device=device, dtype=torch.float16),
        ))
    cap = capacity or (shape.prior_tokens + shape.max_new_tokens)
    cap = (cap + 63) // 64 * 64
    kv = (shape.layers, shape.kv_heads, cap, shape.head_dim)
    w.k_cache = torch.zeros(kv, device=device, dtype=torch.float16)
    w.v_cache = torch.zeros(kv, device=device, dtype=torch.float16)
    P = shape.prior_tokens
    w.k_cache[:, :, :P] = _normal(g, (shape.layers, shape.kv_heads, P, shape.head_dim), 1.0, device)
    w.v_cache[:, :, :P] = _normal(g, (shape.layers, shape.kv_heads, P, shape.head_dim), 1.0, device)
    w.cos, w.sin = rope_tables(shape.head_dim, shape.rope_theta, cap, device)
    return w


@dataclass
class MoELayer:
    q: torch.Tensor
    k: torch.Tensor
    v: torch.Tensor
    o: torch.Tensor
    q_bias: torch.Tensor
    k_bias: torch.Tensor
    v_bias: torch.Tensor
    o_bias: torch.Tensor
    sinks: torch.Tensor
    ln1: torch.Tensor
    ln2: torch.Tensor
    router: torch.Tensor
    router_bias: torch.Tensor
    gate_up_blocks: torch.Tensor   # [E, 2I, H/32, 16], rows interleaved gate/up
    gate_up_scales: torch.Tensor   # [E, 2I, H/32]
    gate_up_bias: torch.Tensor     # [E, 2I]
    down_blocks: torch.Tensor      # [E, H, I/32, 16]
    down_scales: torch.Tensor      # [E, H, I/32]
    down_bias: torch.Tensor        # [E, H]


@dataclass
class MoEWeights:
    shape: MoEShape
    embed: torch.Tensor
    lm_head: torch.Tensor
    final_norm: torch.Tensor
    layers: list[MoELayer] = field(default_factory=list)
    k_cache: torch.Tensor | None = None
    v_cache: torch.Tensor | None = None
    cos: torch.Tensor | None = None
    sin: torch.Tensor | None = None


def _mxfp4(g: torch.Generator, experts: int, rows: int, cols: int, device) -> tuple[torch.Tensor, torch.Tensor]:
    blocks = torch.randint(0, 256, (experts, rows, cols // 32, 16), generator=g, device=device, dtype=torch.uint8)
    scales = torch.randint(119, 124, (experts, rows, cols // 32), generator=g, device=device, dtype=torch.uint8)
    return blocks, scales


def make_moe(shape: MoEShape = GPT_OSS_20B, device="cuda", seed: int = 0, capacity: int | None = None) -> MoEWeights:
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    H, I, E = shape.hidden, shape.intermediate, shape.experts
    w = MoEWeights(
        shape=shape,
        embed=_normal(g, (shape.vocab, H), 0.02, device),
        lm_head=_normal(g, (shape.vocab, H), 0.02, device),
        final_norm=torch.ones(H, device=device, dtype=torch.float16),
    )
    for _ in range(shape.layers):
        gub, gus = _mxfp4(g, E, 2 * I, H, device)
        db, ds = _mxfp4(g, E, H, I, device)
        w.layers.append(MoELayer(
            q=_normal(g, (shape.q_dim, H), 0.02, device), k=_normal(g, (shape.kv_dim, H), 0.02, device),
            v=_normal(g, (shape.kv_dim, H), 0.02, device), o=_normal(g, (H, shape.q_dim), 0.02, device),
            q_bias=_normal(g, shape.q_dim, 0.02, device), k_bias=_normal(g, shape.kv_dim, 0.02, device),
            v_bias=_normal(g, shape.kv_dim, 0.02, device), o_bias=_normal(g, H, 0.02, device),
            sinks=_normal(g, shape.heads, 1.0, device),
            ln1=torch.ones(H, device=device, dtype=torch.float16), ln2=torch.ones(H, device=device, dtype=torch.float16),
            router=_normal(g, (E, H), 0.02, device), router_bias=_normal(g, E, 0.02, device),
            gate_up_blocks=gub, gate_up_scales=gus, gate_up_bias=_normal(g, (E, 2 * I), 0.02, device),
            down_blocks=db, down_scales=ds, down_bias=_normal(g, (E, H), 0.02, device),
        ))
    cap = capacity or (shape.prior_tokens + shape.max_new_tokens)
    cap = (cap + 63) // 64 * 64
    kv = (shape.layers, shape.kv_heads, cap, shape.head_dim)
    w.k_cache = torch.zeros(kv, device=device, dtype=torch.float16)
    w.v_cache = torch.zeros(kv, device=device, dtype=torch.float16)
    P = shape.prior_tokens
    w.k_cache[:, :, :P] = _normal(g, (shape.layers, shape.kv_heads, P, shape.head_dim), 1.0, device)
    w.v_cache[:, :, :P] = _normal(g, (shape.layers, shape.kv_heads, P, shape.head_dim), 1.0, device)
    w.cos, w.sin = rope_tables(shape.head_dim, shape.rope_theta, cap, device)
    return w
