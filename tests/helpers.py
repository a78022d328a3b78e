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


# ------------------------------------------------------------------ .thin archives
THIN_MAGIC = b"THINv0\0\0"


def page_spec(page_id: str, dtype: str, shape, size: int, kind: str = "weight", layer=None, op: str = "weight",
              **extra) -> dict:
    """A manifest page entry (fields of PageSpec, src/manifest.rs:160-184)."""
    spec = {"id": page_id, "kind": kind, "op": op, "dtype": dtype, "shape": list(shape),
            "backend_layout": "row_major", "size": int(size), "checksum": "0" * 64}
    if layer is not None:
        spec["layer"] = layer
    spec.update(extra)
    return spec


def write_thin_archive(path, manifest: dict, pages: dict) -> None:
    """Write a .thin v0 file laid out as the reference's writer does (src/archive.rs:
    457-520): 88-byte header, JSON manifest, page table (u16 id length, id, u64 offset,
    u64 stored size, u64 raw size, u32 flags, 32-byte checksum), then the payloads back
    to back.  Checksums are left zero (the readers do not check them)."""
    import json
    import struct

    manifest_bytes = json.dumps(manifest, indent=2).encode()
    ids = list(pages)
    table_len = sum(2 + len(i.encode()) + 60 for i in ids)
    manifest_off = 88
    page_table_off = manifest_off + len(manifest_bytes)
    data_off = page_table_off + table_len
    table = b""
    offset = data_off
    for pid in ids:
        data = bytes(pages[pid])
        b = pid.encode()
        table += struct.pack("<H", len(b)) + b + struct.pack("<QQQI", offset, len(data), len(data), 0) + bytes(32)
        offset += len(data)
    header = struct.pack("<8sIIQQQQQ32s", THIN_MAGIC, 88, 0, manifest_off, len(manifest_bytes), page_table_off,
                         len(ids), data_off, bytes(32))
    with open(path, "wb") as f:
        f.write(header)
        f.write(manifest_bytes)
        f.write(table)
        for pid in ids:
            f.write(bytes(pages[pid]))


def minimal_manifest(pages: list, layers: int = 1) -> dict:
    return {
        "format": "thintensor", "version": 0,
        "model": {"arch": "llama", "hidden_size": 64, "layers": layers, "heads": 1, "kv_heads": 1, "dtype": "bf16"},
        "execution_tape": [{"stage": "embed", "operator": "embedding", "page_refs": []}],
        "pages": pages,
        "memory_plan": {"scratch_bytes": 0, "min_vram_bytes": 0, "recommended_vram_bytes": 0,
                        "kv_cache": {"policy": "none", "recent_tokens_high_precision": 0, "old_tokens_codec": "none"}},
    }
