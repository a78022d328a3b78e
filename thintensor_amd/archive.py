"""ThinTensor ``.thin`` archives: the reference's reader interface over the native
memory-mapped parser (``csrc/archive.cpp``), zero-copy page views, and page upload
into device memory.

Mirrors ``ThinArchive`` (thinruntime/archive.py:16-369) and ``load_tensor_view`` /
``map_dtype`` (thinruntime/torch_loader.py:11-127): same attributes, methods, checks
and messages.  The binary checks (header, page table, overlaps) run natively; the
manifest JSON and its page index are handled here, between them, in the reference's
order.  ``upload_page`` is this build's addition: it moves a page into HBM through
pinned double-buffered staging instead of a pageable copy.
"""

from __future__ import annotations

import ctypes
import json
import math
import warnings
from functools import lru_cache
from pathlib import Path
from typing import Any, Dict, Optional

import torch

from . import _lib

MAGIC = b"THINv0\0\0"
HEADER_LEN = 88


_Info = _lib.ArchiveInfo
_Record = _lib.ArchiveRecord


def _native_error(lib) -> str:
    msg = lib.tt_last_error()
    return msg.decode("utf-8", "replace") if msg else "archive error"


class _Mapping:
    """Owns the native handle; every page view keeps a reference, so the mapping
    outlives the archive object as long as tensors view it."""

    def __init__(self, path: Path) -> None:
        self.lib = _lib.load()
        h = ctypes.c_void_p()
        if self.lib.tt_archive_open(str(path).encode(), ctypes.byref(h)) != 0:
            raise ValueError(_native_error(self.lib))
        self.handle = h

    def check(self, rc: int) -> None:
        if rc != 0:
            raise ValueError(_native_error(self.lib))

    def __del__(self) -> None:
        h = getattr(self, "handle", None)
        if h is not None and h.value:
            self.lib.tt_archive_close(h)
            self.handle = None


class ThinArchive:
    """Python interface of a ThinTensor ``.thin`` archive (thinruntime/archive.py:16-369):
    O(1) page metadata and manifest lookup, fused logical pages, zero-copy views."""

    def __init__(self, path: Path | str, run_verify: bool = False, bin_path: Optional[str] = None):
        self.path = Path(path)
        self.manifest: Dict[str, Any] = {}
        self.pages: Dict[str, Dict[str, Any]] = {}
        self.manifest_pages: Dict[str, Dict[str, Any]] = {}
        self.tensor_metadata_cache: Dict[str, Dict[str, Any]] = {}
        self.fused_children: Dict[str, list[str]] = {}
        self._map: _Mapping | None = None
        if run_verify:
            self.verify_via_cli(bin_path)
        self._open()
        self._parse()

    # ---------------------------------------------------------------- file access
    def _open(self) -> None:
        self._map = _Mapping(self.path)

    @property
    def file_size(self) -> int:
        return self.path.stat().st_size

    def verify_via_cli(self, bin_path: Optional[str] = None) -> None:
        """The reference shells out to its Rust ``thintensor verify`` (checksums); that
        tool is not part of this build."""
        raise RuntimeError("CLI verify failed: the thintensor archive CLI is not part of this build")

    def _slice(self, offset: int, length: int) -> memoryview:
        if offset < 0 or length < 0 or offset + length > self.file_size:
            raise ValueError(f"slice out of range: offset={offset}, length={length}")
        if self._map is None:
            raise ValueError("archive is closed")
        base = self._map.lib.tt_archive_data(self._map.handle)
        arr = (ctypes.c_uint8 * length).from_address(base + offset)
        arr._mapping = self._map            # keeps the mapping alive while the view lives
        return memoryview(arr).cast("B").toreadonly()

    def _read_bytes(self, offset: int, length: int) -> bytes:
        return self._slice(offset, length).tobytes()

    # --------------------------------------------------------------------- parse
    def _parse(self) -> None:
        info = _Info()
        self._map.check(self._map.lib.tt_archive_get_info(self._map.handle, ctypes.byref(info)))
        self.header = {
            "magic": MAGIC,
            "header_len": info.header_len,
            "version": info.version,
            "manifest_off": info.manifest_off,
            "manifest_len": info.manifest_len,
            "page_table_off": info.page_table_off,
            "page_count": info.page_count,
            "data_off": info.data_off,
            "archive_hash": bytes(info.archive_hash),
        }
        manifest_bytes = self._read_bytes(info.manifest_off, info.manifest_len)
        self.manifest = json.loads(manifest_bytes.decode("utf-8"))
        self._map.check(self._map.lib.tt_archive_parse_pages(self._map.handle))
        rec = _Record()
        for i in range(info.page_count):
            self._map.check(self._map.lib.tt_archive_get_record(self._map.handle, i, ctypes.byref(rec)))
            page_id = ctypes.string_at(rec.id, rec.id_len).decode("utf-8")
            self.pages[page_id] = {
                "offset": int(rec.offset),
                "size": int(rec.stored_size),
                "stored_size": int(rec.stored_size),
                "raw_size": int(rec.raw_size),
                "flags": int(rec.flags),
                "checksum": bytes(rec.checksum),
            }
        self._index_manifest_pages()
        self._validate_manifest_vs_table()
        self._map.check(self._map.lib.tt_archive_check_overlaps(self._map.handle))

    def _index_manifest_pages(self) -> None:
        for page in self.manifest.get("pages", []):
            page_id = page.get("id")
            if not page_id:
                raise ValueError("Manifest page missing id")
            if page_id in self.manifest_pages:
                raise ValueError(f"Duplicate page id in manifest: {page_id}")
            self.manifest_pages[page_id] = page
            fused_to = page.get("fused_to")
            if fused_to is not None:
                self.fused_children.setdefault(fused_to, []).append(page_id)

    def _validate_manifest_vs_table(self) -> None:
        for page_id, page in self.manifest_pages.items():
            fused_to = page.get("fused_to")
            if fused_to is not None:
                if fused_to not in self.pages:
                    raise ValueError(f"Logical page {page_id} refers to missing fused page {fused_to}")
                fused_offset = page.get("fused_offset")
                logical_size = page.get("size")
                if not isinstance(fused_offset, int) or fused_offset < 0:
                    raise ValueError(f"Logical page {page_id} has invalid fused_offset {fused_offset!r}")
                if not isinstance(logical_size, int) or logical_size <= 0:
                    raise ValueError(f"Logical page {page_id} has invalid size {logical_size!r}")
                if fused_offset + logical_size > self.pages[fused_to]["raw_size"]:
                    raise ValueError(f"Logical page {page_id} exceeds fused parent {fused_to}")
                continue
            if page.get("kind") == "fused_logical":
                continue
            if page_id not in self.pages:
                raise ValueError(f"Manifest page {page_id} missing from page table")
        fused_targets = {p.get("fused_to") for p in self.manifest_pages.values() if p.get("fused_to") is not None}
        for page_id in self.pages:
            if page_id not in self.manifest_pages and page_id not in fused_targets:
                raise ValueError(f"Page table entry {page_id} has no manifest page or fused-page reference")

    # ------------------------------------------------------------------- lookups
    def has_page(self, page_id: str) -> bool:
        return page_id in self.manifest_pages or page_id in self.pages

    def get_manifest_page(self, page_id: str) -> Dict[str, Any]:
        try:
            return self.manifest_pages[page_id]
        except KeyError as exc:
            raise KeyError(f"Page {page_id} not in manifest") from exc

    def get_page_record(self, page_id: str) -> Dict[str, Any]:
        try:
            return self.pages[page_id]
        except KeyError as exc:
            raise KeyError(f"Page {page_id} not in page table") from exc

    def _page_range(self, page_id: str) -> tuple[int, int]:
        """(file offset, size) of a physical or fused logical page."""
        manifest_page = self.get_manifest_page(page_id)
        fused_to = manifest_page.get("fused_to")
        if fused_to is not None:
            fused_record = self.get_page_record(fused_to)
            fused_offset = int(manifest_page.get("fused_offset", 0))
            size = int(manifest_page["size"])
            if fused_offset < 0 or fused_offset + size > fused_record["size"]:
                raise ValueError(f"Fused logical page {page_id} slice outside parent {fused_to}")
            return fused_record["offset"] + fused_offset, size
        record = self.get_page_record(page_id)
        return record["offset"], record["size"]

    def get_page_view(self, page_id: str) -> memoryview:
        """Zero-copy read-only view of physical or fused logical page bytes."""
        return self._slice(*self._page_range(page_id))

    def get_page_bytes(self, page_id: str) -> bytes:
        return self.get_page_view(page_id).tobytes()

    def get_tensor_metadata(self, page_id: str) -> Dict[str, Any]:
        cached = self.tensor_metadata_cache.get(page_id)
        if cached is not None:
            return cached
        manifest_page = self.get_manifest_page(page_id)
        offset, size = self._page_range(page_id)
        meta = {
            "id": page_id,
            "dtype": manifest_page["dtype"],
            "shape": manifest_page["shape"],
            "offset": offset,
            "size": size,
            "checksum": manifest_page.get("checksum"),
            "backend_layout": manifest_page.get("backend_layout", "unknown"),
            "kind": manifest_page.get("kind"),
            "layer": manifest_page.get("layer"),
            "op": manifest_page.get("op"),
            "fused_to": manifest_page.get("fused_to"),
            "fused_offset": manifest_page.get("fused_offset"),
        }
        self.tensor_metadata_cache[page_id] = meta
        return meta

    def physical_page_ids(self) -> list[str]:
        return list(self.pages.keys())

    def tensor_page_ids(self) -> list[str]:
        return list(self.manifest_pages.keys())

    # ------------------------------------------------------------------- device
    def upload(self, page_id: str, out: torch.Tensor) -> torch.Tensor:
        """Copy the page's bytes into the contiguous device tensor ``out`` (whose byte
        size must equal the page's) on the current stream."""
        offset, size = self._page_range(page_id)
        if out.device.type != "cuda" or not out.is_contiguous():
            raise ValueError("upload needs a contiguous device tensor")
        if out.numel() * out.element_size() != size:
            raise ValueError(f"{page_id}: page has {size} bytes, destination {out.numel() * out.element_size()}")
        if self._map is None:
            raise ValueError("archive is closed")
        stream = torch.cuda.current_stream(out.device).cuda_stream
        with torch.cuda.device(out.device):
            self._map.check(self._map.lib.tt_archive_upload(self._map.handle, offset, size, out.data_ptr(), stream))
        return out

    # -------------------------------------------------------------------- close
    def close(self) -> None:
        """Drops this object's reference to the mapping; views taken from it keep the
        mapping until they are gone."""
        self._map = None

    def __enter__(self) -> "ThinArchive":
        return self

    def __exit__(self, exc_type, exc_val, exc_tb) -> None:
        self.close()


# ------------------------------------------------------------ torch_loader mirror
_DTYPE_MAP: Dict[str, torch.dtype] = {
    "F16": torch.float16, "FP16": torch.float16, "FLOAT16": torch.float16, "HALF": torch.float16,
    "BF16": torch.bfloat16, "BFLOAT16": torch.bfloat16,
    "F32": torch.float32, "FP32": torch.float32, "FLOAT32": torch.float32, "FLOAT": torch.float32,
    "F64": torch.float64, "FP64": torch.float64, "FLOAT64": torch.float64, "DOUBLE": torch.float64,
    "I64": torch.int64, "INT64": torch.int64, "I32": torch.int32, "INT32": torch.int32,
    "I16": torch.int16, "INT16": torch.int16, "I8": torch.int8, "INT8": torch.int8,
    "U8": torch.uint8, "UINT8": torch.uint8, "BOOL": torch.bool, "BOOLEAN": torch.bool,
    "FLOAT8_E4M3FN": torch.float8_e4m3fn,
}


@lru_cache(maxsize=128)
def map_dtype(dtype_str: str) -> torch.dtype:
    """Manifest dtype string -> torch dtype (thinruntime/torch_loader.py:58-63)."""
    key = str(dtype_str).strip().replace("torch.", "").upper()
    try:
        return _DTYPE_MAP[key]
    except KeyError as exc:
        raise ValueError(f"Unsupported dtype string: {dtype_str!r}") from exc


def dtype_nbytes(dtype: torch.dtype) -> int:
    return torch.empty((), dtype=dtype).element_size()


def _shape_numel(shape: tuple[int, ...]) -> int:
    if not shape:
        return 1
    if any(dim < 0 for dim in shape):
        raise ValueError(f"invalid negative dimension in shape: {shape}")
    return math.prod(shape)


def _page_geometry(archive: ThinArchive, page_id: str) -> tuple[tuple[int, ...], torch.dtype, int]:
    metadata = archive.get_tensor_metadata(page_id)
    shape = tuple(int(x) for x in metadata["shape"])
    dtype = map_dtype(str(metadata["dtype"]))
    elem_size = dtype_nbytes(dtype)
    size_bytes = int(metadata["size"])
    if size_bytes < 0:
        raise ValueError(f"{page_id}: negative byte size {size_bytes}")
    if size_bytes % elem_size != 0:
        raise ValueError(f"{page_id}: byte size {size_bytes} is not divisible by dtype size {elem_size}")
    count = size_bytes // elem_size
    expected = _shape_numel(shape)
    if count != expected:
        raise ValueError(
            f"{page_id}: metadata mismatch: shape {shape} expects {expected} elements, "
            f"but page has {count} elements from {size_bytes} bytes of {dtype}"
        )
    return shape, dtype, count


def load_tensor_view(archive: ThinArchive, page_id: str) -> tuple[torch.Tensor, bool]:
    """Zero-copy CPU tensor over an archive page (thinruntime/torch_loader.py:82-127).
    The tensor keeps the mapping alive."""
    shape, dtype, count = _page_geometry(archive, page_id)
    view = archive.get_page_view(page_id)
    with warnings.catch_warnings():
        warnings.filterwarnings("ignore", message="The given buffer is not writable")
        tensor = torch.frombuffer(view, dtype=dtype, count=count)
    return tensor.reshape(shape), True


def upload_page(archive: ThinArchive, page_id: str, device: torch.device | str = "cuda") -> torch.Tensor:
    """The page as a new device tensor of its manifest shape and dtype, filled through
    the native pinned upload."""
    shape, dtype, _ = _page_geometry(archive, page_id)
    out = torch.empty(shape, dtype=dtype, device=device)
    return archive.upload(page_id, out)
