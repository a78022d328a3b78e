"""Decode weights from a ``.thin`` archive: pages are uploaded into HBM and the linear
layers are packed on the GPU into the grouped-INT4 layout the decode kernels read.

Follows the reference's page-pool ``--dense-int4`` load path (gpu_runtime.py:1786-1864,
page naming of ThinGpuWeights, :911-1127): every attention and MLP projection page is
quantized by quantize_to_int4_cpu (fp16 scales, codes in [-8, 7]), embeddings, norms
and the LM head stay in the activation dtype (fp16), and the LM head falls back to the
embedding table when the archive ties them.
"""

from __future__ import annotations

import os

import torch

from .archive import ThinArchive, upload_page
from .quantize import quantize_to_int4_cpu
from .synth import DenseLayer, DenseShape, DenseWeights, rope_tables

PROJECTIONS = {
    "q": "self_attn.q_proj.weight",
    "k": "self_attn.k_proj.weight",
    "v": "self_attn.v_proj.weight",
    "o": "self_attn.o_proj.weight",
    "gate": "mlp.gate_proj.weight",
    "up": "mlp.up_proj.weight",
    "down": "mlp.down_proj.weight",
}


def dense_shape_from_manifest(model: dict, group_size: int = 128, capacity: int = 1024) -> DenseShape:
    """DenseShape of a Llama-style manifest model block (src/manifest.rs:20-150)."""
    heads = int(model["heads"])
    hidden = int(model["hidden_size"])
    return DenseShape(
        name=str(model.get("arch", "archive")),
        layers=int(model["layers"]),
        hidden=hidden,
        heads=heads,
        kv_heads=int(model["kv_heads"]),
        head_dim=int(model.get("head_dim") or hidden // heads),
        intermediate=int(model["intermediate_size"]),
        vocab=int(model["vocab_size"]),
        rope_theta=float(model.get("rope_theta") or 10000.0),
        eps=float(model.get("rms_norm_eps") or model.get("norm_eps") or 1e-5),
        group=group_size,
        prior_tokens=0,
        max_new_tokens=capacity,
    )


def dense_weights_from_archive(archive: ThinArchive, device: torch.device | str = "cuda", *,
                               group_size: int = 128, capacity: int = 1024) -> DenseWeights:
    """DenseWeights (grouped INT4 projections, fp16 embeddings / norms / LM head, empty
    KV cache of ``capacity`` tokens) from a dense Llama-style archive."""
    if os.environ.get("THINTENSOR_AFFINE_INT4", "0") == "1":
        raise ValueError("the dense decode kernels read symmetric INT4; unset THINTENSOR_AFFINE_INT4")
    shape = dense_shape_from_manifest(archive.manifest["model"], group_size, capacity)
    dev = torch.device(device)

    def dense(page_id: str) -> torch.Tensor:
        return upload_page(archive, page_id, dev).to(torch.float16)

    embed = dense("model.embed_tokens.weight")
    lm_head = dense("lm_head.weight") if archive.has_page("lm_head.weight") else embed
    w = DenseWeights(shape=shape, embed=embed, lm_head=lm_head, final_norm=dense("model.norm.weight"))
    for layer in range(shape.layers):
        prefix = f"model.layers.{layer}."
        packed = {}
        for name, suffix in PROJECTIONS.items():
            source = upload_page(archive, prefix + suffix, dev)
            packed[name] = quantize_to_int4_cpu(source, group_size=group_size)
            del source
        w.layers.append(DenseLayer(
            **packed,
            ln1=dense(prefix + "input_layernorm.weight"),
            ln2=dense(prefix + "post_attention_layernorm.weight"),
        ))
    cap = (capacity + 63) // 64 * 64
    kv = (shape.layers, shape.kv_heads, cap, shape.head_dim)
    w.k_cache = torch.zeros(kv, device=dev, dtype=torch.float16)
    w.v_cache = torch.zeros(kv, device=dev, dtype=torch.float16)
    w.cos, w.sin = rope_tables(shape.head_dim, shape.rope_theta, cap, dev)
    return w
