"""Archive pages into HBM and through the decode path on the GPU.

* tt_archive_upload (pinned double-buffered staging) reproduces every page byte,
  including pages larger than one 32 MiB staging chunk and unaligned fused slices;
* a small dense Llama-style model stored as bf16 pages in a .thin archive is loaded by
  dense_weights_from_archive (GPU INT4 packing, as the reference's --dense-int4 page
  pool), its packed projections equal the oracle's quantize_to_int4_cpu restatement of
  the pages, and its greedy decode equals the oracle decode token for token with
  bit-identical final logits.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import quant as Q
from oracle.decode_ref import DenseRef
from tests.helpers import minimal_manifest, page_spec, write_thin_archive
from thintensor_amd.archive import ThinArchive, load_tensor_view, upload_page
from thintensor_amd.backend import HipDecodeBackend
from thintensor_amd.decode import DenseDecoder
from thintensor_amd.loader import PROJECTIONS, dense_weights_from_archive

pytestmark = pytest.mark.gpu


def test_upload_pages_round_trip(device, tmp_path):
    g = np.random.default_rng(5)
    small = g.integers(0, 256, 1000, dtype=np.uint8).tobytes()
    big = g.integers(0, 256, 70 * 2 ** 20 + 12, dtype=np.uint8).tobytes()
    specs = [
        page_spec("small", "U8", (1000,), 1000),
        page_spec("big", "U8", (len(big),), len(big), kind="fused_physical"),
        page_spec("slice", "U8", (5 * 2 ** 20 + 7,), 5 * 2 ** 20 + 7, fused_to="big", fused_offset=2 ** 20 + 3),
    ]
    path = tmp_path / "u.thin"
    write_thin_archive(path, minimal_manifest(specs), {"small": small, "big": big})
    a = ThinArchive(path)
    for _ in range(2):   # the second round reuses the staging buffers
        for pid, want in (("small", small), ("big", big), ("slice", big[2 ** 20 + 3: 2 ** 20 + 3 + 5 * 2 ** 20 + 7])):
            t = upload_page(a, pid, device)
            assert t.device.type == "cuda"
            assert t.cpu().numpy().tobytes() == want, pid
    view, _ = load_tensor_view(a, "slice")
    assert torch.equal(upload_page(a, "slice", device).cpu(), view)


def _bf16(g, shape, std, mean=0.0):
    return (torch.randn(shape, generator=g) * std + mean).to(torch.bfloat16)


def _write_dense_archive(path, s, seed=0):
    g = torch.Generator().manual_seed(seed)
    H, I, qd, kvd = s["hidden"], s["inter"], s["heads"] * 64, s["kv_heads"] * 64
    tensors = {"model.embed_tokens.weight": _bf16(g, (s["vocab"], H), 0.02),
               "lm_head.weight": _bf16(g, (s["vocab"], H), 0.02),
               "model.norm.weight": _bf16(g, (H,), 0.05, 1.0)}
    dims = {"q": (qd, H), "k": (kvd, H), "v": (kvd, H), "o": (H, qd), "gate": (I, H), "up": (I, H), "down": (H, I)}
    for layer in range(s["layers"]):
        for name, suffix in PROJECTIONS.items():
            tensors[f"model.layers.{layer}.{suffix}"] = _bf16(g, dims[name], 0.03)
        tensors[f"model.layers.{layer}.input_layernorm.weight"] = _bf16(g, (H,), 0.05, 1.0)
        tensors[f"model.layers.{layer}.post_attention_layernorm.weight"] = _bf16(g, (H,), 0.05, 1.0)
    specs = [page_spec(pid, "BF16", tuple(t.shape), t.numel() * 2) for pid, t in tensors.items()]
    manifest = minimal_manifest(specs, layers=s["layers"])
    manifest["model"].update(hidden_size=H, heads=s["heads"], kv_heads=s["kv_heads"], head_dim=64,
                             intermediate_size=I, vocab_size=s["vocab"], rms_norm_eps=1e-5, rope_theta=500000.0)
    write_thin_archive(path, manifest, {pid: t.view(torch.int16).numpy().tobytes() for pid, t in tensors.items()})
    return tensors


def test_dense_decode_from_archive(device, tmp_path, monkeypatch):
    monkeypatch.setenv("THINTENSOR_AFFINE_INT4", "0")
    s = dict(layers=2, hidden=512, heads=8, kv_heads=2, inter=1024, vocab=4096)
    path = tmp_path / "dense.thin"
    tensors = _write_dense_archive(path, s)
    a = ThinArchive(path)
    w = dense_weights_from_archive(a, device, group_size=128, capacity=128)
    assert w.shape.hidden == 512 and w.shape.layers == 2 and w.shape.kv_heads == 2
    # the packed projections are quantize_to_int4_cpu of the archive pages
    for layer in range(2):
        for name in ("q", "down"):
            src = tensors[f"model.layers.{layer}.{PROJECTIONS[name]}"].float().numpy()
            wp, ws = Q.int4_lsq(src, 128)
            packed, scales = getattr(w.layers[layer], name)
            assert np.array_equal(packed.cpu().numpy(), wp)
            assert np.array_equal(scales.cpu().view(torch.int16).numpy().view(np.uint16), ws.view(np.uint16))
    assert torch.equal(w.lm_head.cpu(), tensors["lm_head.weight"].to(torch.float16))
    be = HipDecodeBackend(device, torch.float16, 512, 512, 128, 1024)
    dec = DenseDecoder(be, w)
    ref = DenseRef(w)
    got = dec.generate(11, 0, 32)
    want = ref.generate(11, 0, 32)
    assert got == want
    assert len(set(want)) > 1
    _, logits = ref.step(want[-2], 31)
    final = be.logits_buffer(int(w.lm_head.shape[0]), torch.float16).cpu().numpy()
    assert np.array_equal(final.view(np.uint16), logits.view(np.uint16))
