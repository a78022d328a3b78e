"""Seeded input generators shared by the tests."""

from __future__ import annotations

import numpy as np


def rng(seed: int) -> np.random.Generator:
    return np.random.default_rng(seed)


def f16_normal(g: np.random.Generator, shape, scale: float = 1.0) -> np.ndarray:
    return (g.standard_normal(shape) * scale).astype(np.float16)


def bf16_bits(values: np.ndarray) -> np.ndarray:
    """float32 -> raw bfloat16 bits (round to nearest even)."""
    u = np.asarray(values, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = u + 0x7FFF + ((u >> 16) & 1)
    return (u >> 16).astype(np.uint16)


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint32) << 16).view(np.float32)


def to_torch(a: np.ndarray, device, bf16: bool = False):
    import torch

    t = torch.from_numpy(np.ascontiguousarray(a))
    if bf16:
        t = t.view(torch.bfloat16)
    return t.to(device)


def from_torch_bits(t) -> np.ndarray:
    """Raw numpy view of a device tensor's bits (fp16 -> float16, bf16 -> uint16)."""
    import torch

    c = t.detach().cpu()
    if c.dtype == torch.bfloat16:
        return c.view(torch.int16).numpy().view(np.uint16)
    return c.numpy()
