"""The .thin reader (thintensor_amd.archive over csrc/archive.cpp) on the CPU: round
trips of archives laid out as the reference writes them, zero-copy views, fused
logical pages, and every structural check with the reference reader's message
(thinruntime/archive.py line numbers beside each case)."""

from __future__ import annotations

import struct

import numpy as np
import pytest
import torch

from tests.helpers import THIN_MAGIC, minimal_manifest, page_spec, write_thin_archive
from thintensor_amd import _lib
from thintensor_amd.archive import ThinArchive, load_tensor_view, map_dtype


@pytest.fixture(autouse=True)
def _need_lib():
    if not _lib.library_path().exists():
        pytest.skip("kernel library not built")


def sample(tmp_path, name="a.thin"):
    g = np.random.default_rng(3)
    w = g.standard_normal((4, 8)).astype(np.float32)
    bf16 = (w.view(np.uint32) >> 16).astype(np.uint16)
    f32 = g.standard_normal(3).astype(np.float32)
    fused = bytes(range(48))
    pages = {
        "model.layers.0.self_attn.q_proj.weight": bf16.tobytes(),
        "model.norm.weight": f32.tobytes(),
        "fused.qkv": fused,
    }
    specs = [
        page_spec("model.layers.0.self_attn.q_proj.weight", "BF16", (4, 8), 64, layer=0, op="q_proj"),
        page_spec("model.norm.weight", "F32", (3,), 12, op="norm"),
        page_spec("fused.qkv", "U8", (48,), 48, kind="fused_physical", op="qkv"),
        page_spec("fused.q", "U8", (16,), 16, op="q", fused_to="fused.qkv", fused_offset=0),
        page_spec("fused.kv", "I16", (16,), 32, op="kv", fused_to="fused.qkv", fused_offset=16),
    ]
    path = tmp_path / name
    write_thin_archive(path, minimal_manifest(specs), pages)
    return path, bf16, f32, fused


def test_round_trip_views_and_metadata(tmp_path):
    path, bf16, f32, fused = sample(tmp_path)
    with ThinArchive(path) as a:
        assert a.header["page_count"] == 3 and a.header["header_len"] == 88
        assert a.physical_page_ids() == ["model.layers.0.self_attn.q_proj.weight", "model.norm.weight", "fused.qkv"]
        assert a.tensor_page_ids()[-2:] == ["fused.q", "fused.kv"]
        assert a.fused_children == {"fused.qkv": ["fused.q", "fused.kv"]}
        assert a.has_page("fused.kv") and not a.has_page("nope")
        assert a.get_page_bytes("fused.kv") == fused[16:48]
        t, ok = load_tensor_view(a, "model.layers.0.self_attn.q_proj.weight")
        assert ok and t.dtype == torch.bfloat16 and tuple(t.shape) == (4, 8)
        assert np.array_equal(t.view(torch.int16).numpy().view(np.uint16), bf16)
        n, _ = load_tensor_view(a, "model.norm.weight")
        assert np.array_equal(n.numpy(), f32)
        kv, _ = load_tensor_view(a, "fused.kv")
        assert kv.dtype == torch.int16 and bytes(kv.numpy().tobytes()) == fused[16:48]
        meta = a.get_tensor_metadata("fused.kv")
        rec = a.get_page_record("fused.qkv")
        assert meta["offset"] == rec["offset"] + 16 and meta["size"] == 32 and meta["fused_to"] == "fused.qkv"
        assert meta is a.get_tensor_metadata("fused.kv")        # cached
        view = a.get_page_view("model.norm.weight")
        assert view.readonly
    # the view outlives close(): the mapping stays while tensors reference it
    assert np.array_equal(n.numpy(), f32)
    with pytest.raises(KeyError, match="Page nope not in manifest"):
        ThinArchive(path).get_manifest_page("nope")
    with pytest.raises(KeyError, match="Page fused.q not in page table"):
        ThinArchive(path).get_page_record("fused.q")


def test_map_dtype_table():
    assert map_dtype("bf16") is torch.bfloat16 and map_dtype("torch.float16") is torch.float16
    assert map_dtype(" float8_e4m3fn ") is torch.float8_e4m3fn and map_dtype("UINT8") is torch.uint8
    with pytest.raises(ValueError, match="Unsupported dtype string: 'q4'"):
        map_dtype("q4")


def test_load_tensor_view_checks(tmp_path):
    specs = [page_spec("p", "F32", (3,), 10), page_spec("q", "F32", (2, 2), 12)]
    path = tmp_path / "v.thin"
    write_thin_archive(path, minimal_manifest(specs), {"p": bytes(10), "q": bytes(12)})
    a = ThinArchive(path)
    with pytest.raises(ValueError, match="p: byte size 10 is not divisible by dtype size 4"):   # torch_loader.py:97-100
        load_tensor_view(a, "p")
    with pytest.raises(ValueError, match=r"q: metadata mismatch: shape \(2, 2\) expects 4 elements"):  # :105-108
        load_tensor_view(a, "q")


# ------------------------------------------------------------------ header checks
def corrupt(path, offset, data: bytes):
    b = bytearray(path.read_bytes())
    b[offset:offset + len(data)] = data
    path.write_bytes(bytes(b))


def u32(v):
    return struct.pack("<I", v)


def u64(v):
    return struct.pack("<Q", v)


@pytest.mark.parametrize("case,expect", [
    ("small", "File is too small to contain a ThinTensor header"),                    # archive.py:101
    ("magic", r"Invalid magic: b'XHINv0\\x00\\x00', expected b'THINv0\\x00\\x00'"),    # :116
    ("header_len", "Invalid header length: 89, expected 88"),                          # :118
    ("version", "Invalid format version: 1, expected 0"),                              # :120
    ("manifest_off", "Manifest offset 90 does not follow header length 88"),           # :122-124
    ("manifest_len", "Manifest range exceeds file size"),                              # :126
    ("page_table_off", "Page table does not immediately follow the manifest"),         # :128
])
def test_header_checks(tmp_path, case, expect):
    path, *_ = sample(tmp_path)
    size = path.stat().st_size
    if case == "small":
        path.write_bytes(path.read_bytes()[:87])
    elif case == "magic":
        corrupt(path, 0, b"X")
    elif case == "header_len":
        corrupt(path, 8, u32(89))
    elif case == "version":
        corrupt(path, 12, u32(1))
    elif case == "manifest_off":
        corrupt(path, 16, u64(90))
    elif case == "manifest_len":
        corrupt(path, 24, u64(size))
    elif case == "page_table_off":
        corrupt(path, 32, u64(5))
    with pytest.raises(ValueError, match=expect):
        ThinArchive(path)


def table_entry(path, index):
    """File offset of page-table record `index`'s tail (after its id)."""
    raw = path.read_bytes()
    pos = struct.unpack_from("<Q", raw, 32)[0]
    for _ in range(index):
        n = struct.unpack_from("<H", raw, pos)[0]
        pos += 2 + n + 60
    n = struct.unpack_from("<H", raw, pos)[0]
    return pos, pos + 2 + n


@pytest.mark.parametrize("case,expect", [
    ("flags", "Page model.norm.weight uses unsupported runtime flags 0x4"),                  # archive.py:180-183
    ("raw", "Uncompressed page model.norm.weight stored/raw sizes differ"),                  # :184-187
    ("before", "Page model.norm.weight offset starts before data_off"),                      # :174
    ("beyond", "Page model.norm.weight offset\\+size exceeds file size"),                    # :176
    ("wrap", "Page model.norm.weight offset\\+size exceeds file size"),                      # no 2^64 wrap-around
    ("zero", "Page model.norm.weight has zero stored_size but nonzero raw_size"),            # :178
    ("empty_id", "Empty page id at page index 1"),                                           # :162
    ("data_off", "Page table ends at"),                                                      # :148-151
    ("overlap", "Overlapping pages detected: model.layers.0.self_attn.q_proj.weight overlaps with model.norm.weight"),
])
def test_page_table_checks(tmp_path, case, expect):
    path, *_ = sample(tmp_path)
    head, tail = table_entry(path, 1)
    raw = path.read_bytes()
    off, stored = struct.unpack_from("<QQ", raw, tail)
    if case == "flags":
        corrupt(path, tail + 24, u32(4))
    elif case == "raw":
        corrupt(path, tail + 16, u64(stored + 1))
    elif case == "before":
        corrupt(path, tail, u64(10))
    elif case == "beyond":
        corrupt(path, tail, u64(path.stat().st_size - 4))
    elif case == "wrap":   # offset near 2^64 plus a small size: the sum would wrap in uint64
        corrupt(path, tail, u64(2**64 - 8) + u64(16) + u64(16))
    elif case == "zero":
        corrupt(path, tail + 8, u64(0))
    elif case == "empty_id":
        corrupt(path, head, struct.pack("<H", 0))
    elif case == "data_off":
        corrupt(path, 48, u64(struct.unpack_from("<Q", raw, 48)[0] - 1))
    elif case == "overlap":
        corrupt(path, tail, u64(off - 8))
    with pytest.raises(ValueError, match=expect):
        ThinArchive(path)


def test_duplicate_page_table_id(tmp_path):
    specs = [page_spec("a", "U8", (4,), 4), page_spec("b", "U8", (4,), 4)]
    path = tmp_path / "d.thin"
    write_thin_archive(path, minimal_manifest(specs), {"a": bytes(4), "b": bytes(4)})
    _, tail = table_entry(path, 1)
    corrupt(path, tail - 1, b"a")
    with pytest.raises(ValueError, match="Duplicate page id in page table: a"):   # archive.py:168
        ThinArchive(path)


@pytest.mark.parametrize("case,expect", [
    ("missing", "Manifest page extra missing from page table"),                              # archive.py:246
    ("orphan", "Page table entry b has no manifest page or fused-page reference"),           # :253-256
    ("dup", "Duplicate page id in manifest: a"),                                             # :218
    ("no_id", "Manifest page missing id"),                                                   # :215
    ("fused_missing", "Logical page c refers to missing fused page zz"),                     # :228
    ("fused_size", "Logical page c exceeds fused parent a"),                                 # :238-241
    ("fused_offset", "Logical page c has invalid fused_offset -1"),                          # :230-233
])
def test_manifest_checks(tmp_path, case, expect):
    specs = [page_spec("a", "U8", (4,), 4), page_spec("b", "U8", (4,), 4)]
    if case == "missing":
        specs.append(page_spec("extra", "U8", (4,), 4))
    elif case == "orphan":
        specs = specs[:1]
    elif case == "dup":
        specs.append(page_spec("a", "U8", (4,), 4))
    elif case == "no_id":
        specs.append({"kind": "weight"})
    elif case == "fused_missing":
        specs.append(page_spec("c", "U8", (2,), 2, fused_to="zz", fused_offset=0))
    elif case == "fused_size":
        specs.append(page_spec("c", "U8", (4,), 4, fused_to="a", fused_offset=2))
    elif case == "fused_offset":
        specs.append(page_spec("c", "U8", (2,), 2, fused_to="a", fused_offset=-1))
    path = tmp_path / "m.thin"
    write_thin_archive(path, minimal_manifest(specs), {"a": bytes(4), "b": bytes(4)})
    with pytest.raises(ValueError, match=expect):
        ThinArchive(path)


def test_verify_via_cli_is_not_available(tmp_path):
    path, *_ = sample(tmp_path)
    with pytest.raises(RuntimeError, match="CLI verify failed"):
        ThinArchive(path, run_verify=True)
