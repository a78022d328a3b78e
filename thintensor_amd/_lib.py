"""ctypes binding of ``libthintensor_hip.so`` (the C ABI in include/thintensor_hip.h).

The shared library is the product: every operator of :class:`HipDecodeBackend`
lands in one of these entry points.  Loading fails loudly when the library is
missing or was built without an entry point; there is no fallback path.
"""

from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

from . import build as _build

F16, BF16, F32 = 0, 1, 2
W_FP8 = 3   # weight format code of float8_e4m3fn (scaled GEMVs, tt_split_k_matvec)
W_INT8 = 4  # weight format code of int8 (the same entry points)
Q4_LSQ, Q4_LSQ_AFFINE, Q4_ROWS, Q4_ROWS_AFFINE = 0, 1, 2, 3   # tt_quantize_int4 modes

_P = ctypes.c_void_p
_I = ctypes.c_int
_L = ctypes.c_int64
_F = ctypes.c_float
_PP = ctypes.POINTER(ctypes.c_void_p)
_LP = ctypes.POINTER(ctypes.c_int64)

# Fused decode-step descriptors (mirror tt_fused_segment / tt_fused_gemv in
# include/thintensor_hip.h; tt_fused_struct_sizes checks the layout at load time).
FMT_INT4_G, FMT_DENSE = 0, 1
PRO_LOAD, PRO_ADD_NORM, PRO_EMBED_NORM, PRO_ADD_RMS_NORM = 0, 1, 2, 3
SEG_PLAIN, SEG_ROPE_OUT, SEG_ROPE_CACHE, SEG_CACHE, SEG_SILU = 0, 1, 2, 3, 4


class FusedSegment(ctypes.Structure):
    _fields_ = [
        ("weight", _P), ("weight2", _P), ("w_row_bytes", _L), ("scales", _P), ("scales2", _P), ("s_row", _L),
        ("out", _P), ("bias", _P), ("rows", _L), ("kind", ctypes.c_int32), ("reserved", ctypes.c_int32),
    ]


class FusedGemv(ctypes.Structure):
    _fields_ = [
        ("weight_format", ctypes.c_int32), ("weight_dtype", ctypes.c_int32), ("group_size", _L),
        ("act_dtype", ctypes.c_int32), ("prologue", ctypes.c_int32), ("cols", _L), ("x", _P), ("left", _P),
        ("right", _P), ("embed", _P), ("embed_row", _L), ("vocab", _L), ("token", _P), ("norm_weight", _P),
        ("eps", ctypes.c_float), ("count", ctypes.c_int32), ("residual_out", _P), ("seg", FusedSegment * 3),
        ("position", _P), ("capacity", _L), ("cache_head", _L), ("cos_table", _P), ("sin_table", _P),
        ("table_row", _L), ("table_rows", _L), ("head_dim", _L), ("tokens", _L), ("token_x", _L),
        ("token_out", _L), ("token_cache", _L),
    ]


_FGP = ctypes.POINTER(FusedGemv)


class ArchiveInfo(ctypes.Structure):
    """tt_archive_info: header fields of a .thin archive and its manifest bytes."""
    _fields_ = [
        ("header_len", ctypes.c_uint32), ("version", ctypes.c_uint32), ("manifest_off", ctypes.c_uint64),
        ("manifest_len", ctypes.c_uint64), ("page_table_off", ctypes.c_uint64), ("page_count", ctypes.c_uint64),
        ("data_off", ctypes.c_uint64), ("archive_hash", ctypes.c_uint8 * 32), ("file_size", ctypes.c_uint64),
        ("manifest", ctypes.c_void_p),
    ]


class ArchiveRecord(ctypes.Structure):
    """tt_archive_record: one page table record."""
    _fields_ = [
        ("id", ctypes.c_void_p), ("id_len", ctypes.c_int64), ("offset", ctypes.c_uint64),
        ("stored_size", ctypes.c_uint64), ("raw_size", ctypes.c_uint64), ("flags", ctypes.c_uint32),
        ("checksum", ctypes.c_uint8 * 32),
    ]

# name -> argtypes (restype is int unless listed in _RESTYPES)
SIGNATURES: dict[str, list] = {
    "tt_version": [],
    "tt_last_error": [],
    "tt_gemv_lanes_per_row": [_L, _L],
    "tt_int4_scaled_matvec": [_P, _L, _P, _I, _L, _L, _L, _I, _P, _I, _P, _I, _L, _L, _L, _P],
    "tt_multi_int4_scaled_matvec": [_I, _PP, _LP, _PP, _I, _LP, _LP, _L, _I, _LP, _P, _I, _P, _I, _L, _L, _P],
    "tt_scaled_matvec": [_P, _I, _L, _P, _I, _P, _I, _P, _I, _L, _L, _P],
    "tt_block_scaled_matvec": [_P, _I, _L, _P, _I, _L, _L, _L, _P, _I, _P, _I, _L, _L, _P],
    "tt_multi_scaled_matvec": [_I, _PP, _I, _LP, _PP, _I, _LP, _LP, _P, _I, _P, _I, _L, _P],
    "tt_split_k_matvec": [_P, _I, _L, _P, _I, _P, _I, _P, _I, _L, _L, _I, _P, _L, _P],
    "tt_scaled_gate_up_silu": [_P, _L, _P, _L, _P, _L, _P, _L, _I, _I, _P, _I, _P, _I, _L, _L, _P],
    "tt_head_rms_norm": [_P, _I, _P, _I, _P, _L, _L, _F, _P],
    "tt_qk_head_rmsnorm_rope_inplace": [_P, _P, _I, _P, _P, _I, _P, _P, _L, _L, _P, _L, _L, _L, _L, _F, _P],
    "tt_matvec": [_P, _I, _L, _P, _I, _P, _I, _L, _L, _P],
    "tt_multi_matvec": [_I, _PP, _I, _LP, _LP, _P, _I, _P, _I, _L, _P],
    "tt_mxfp4_selected_matvec": [_P, _L, _L, _P, _L, _L, _P, _I, _L, _P, _I, _L, _P, _I, _L, _L, _L, _P],
    "tt_mxfp_lowbit_selected_matvec": [_P, _L, _L, _P, _L, _L, _I, _P, _I, _L, _P, _I, _L, _P, _I, _L, _L, _L, _P],
    "tt_sparse_residual_matvec": [_P, _I, _L, _L, _P, _I, _L, _L, _P, _I, _P, _I, _L, _L, _L, _P],
    "tt_binary_residual_matvec": [_P, _L, _P, _I, _L, _P, _I, _P, _I, _L, _L, _P],
    "tt_mxfp_ternary_selected_matvec": [_P, _L, _L, _L, _P, _L, _L, _L, _L, _P, _I, _L, _P, _I, _L, _P, _I, _L, _L,
                                        _L, _P],
    "tt_mxfp_lowbit_selected_swiglu": [_P, _L, _L, _P, _L, _L, _I, _P, _I, _L, _P, _I, _L, _P, _I, _L, _F, _F, _P,
                                       _I, _L, _L, _L, _P],
    "tt_mxfp_lowbit_weighted_down": [_P, _L, _L, _P, _L, _L, _I, _P, _I, _L, _P, _I, _P, _I, _L, _P, _I, _L, _P, _I,
                                     _L, _L, _P],
    "tt_lowbit_affine_matvec": [_P, _L, _P, _L, _L, _I, _P, _I, _P, _I, _L, _L, _L, _P],
    "tt_int4_selected_matvec": [_P, _L, _L, _P, _I, _L, _L, _L, _P, _I, _L, _P, _I, _L, _P, _I, _L, _L, _L, _L, _P],
    "tt_multi_matvec_bias": [_I, _PP, _I, _LP, _LP, _PP, _P, _I, _P, _I, _L, _P],
    "tt_record_token": [_P, _P, _P, _P, ctypes.c_int32, _P],
    "tt_record_tokens_advance": [_P, ctypes.c_int32, _P, _P, _P, _L, ctypes.c_int32, ctypes.c_int32, _P],
    "tt_add_then_rms_norm_rows": [_P, _P, _P, _I, _L, _P, _I, _P, _I, _L, _L, _L, _F, _P],
    "tt_matvec_argmax_partials": [_L, _L],
    "tt_matvec_argmax": [_P, _I, _L, _P, _I, _P, _I, _L, _L, _P, _L, _P, _P, _P],
    "tt_matvec_argmax_noalloc": [_P, _I, _L, _P, _I, _P, _I, _L, _L, _P, _P, _P],
    "tt_rms_norm": [_P, _I, _P, _I, _P, _I, _L, _F, _F, _P],
    "tt_add_rms_norm": [_P, _P, _P, _I, _P, _I, _P, _I, _L, _F, _P],
    "tt_add": [_P, _P, _P, _I, _L, _P],
    "tt_silu_mul": [_P, _P, _P, _I, _L, _P],
    "tt_interleaved_swiglu": [_P, _L, _P, _L, _I, _L, _L, _F, _F, _P],
    "tt_weighted_expert_sum": [_P, _I, _L, _L, _P, _I, _P, _L, _P],
    "tt_rope_qk_inplace": [_P, _P, _I, _P, _P, _L, _L, _P, _L, _L, _L, _L, _P],
    "tt_embedding": [_P, _L, _L, _P, _L, _P, _L, _P],
    "tt_kv_append": [_P, _P, _P, _P, _L, _L, _P, _L, _L, _L, _L, _P],
    "tt_advance_position": [_P, ctypes.c_int32, _P],
    "tt_attention_scratch_floats": [_L, _L, _L],
    "tt_single_token_gqa_attention": [_P, _P, _P, _I, _L, _L, _L, _L, _P, _I, _P, _L, _L, _L, _L, _L, _P, _L, _P,
                                      _P],
    "tt_single_token_gqa_attention_partials": [_P, _P, _P, _I, _L, _L, _L, _L, _P, _L, _L, _L, _L, _L, _P, _L, _P],
    "tt_attention_combine_int4_matvec": [_P, _L, _P, _L, _L, _L, _L, _I, _P, _L, _P, _L, _L, _P, _P, _L, _P],
    "tt_moe_router_matvec_topk": [_P, _I, _L, _P, _I, _L, _P, _I, _L, _L, _I, _P, _P, _I, _P],
    "tt_moe_router_topk": [_P, _I, _L, _L, _I, _P, _P, _I, _P],
    "tt_add_rms_norm_router_topk": [_P, _P, _P, _I, _P, _I, _P, _I, _L, _F, _P, _I, _L, _P, _I, _L, _L, _I, _P, _P,
                                    _I, _L, _P, _L, _P],
    "tt_norm_router_workspace_bytes": [_L],
    "tt_add_rms_norm_router_logits": [_P, _P, _P, _I, _P, _I, _P, _I, _L, _F, _P, _I, _L, _P, _I, _L, _P, _L, _P],
    "tt_mxfp_lowbit_selected_swiglu_router": [_P, _L, _L, _P, _L, _L, _I, _P, _I, _L, _P, _L, _L, _I, _P, _P, _I,
                                              _P, _I, _L, _F, _F, _P, _I, _L, _L, _L, _L, _P],
    "tt_matvec_bias_rows": [_P, _I, _L, _P, _P, _I, _L, _P, _I, _L, _L, _L, _L, _P],
    "tt_mxfp_lowbit_selected_swiglu_tokens": [_P, _L, _L, _P, _L, _L, _I, _P, _I, _L, _P, _I, _L, _P, _I, _L, _F, _F,
                                              _P, _I, _L, _L, _L, _L, _P],
    "tt_mxfp_lowbit_weighted_down_tokens": [_P, _L, _L, _P, _L, _L, _I, _P, _I, _L, _P, _I, _P, _I, _L, _P, _I, _L,
                                            _P, _I, _L, _L, _L, _L, _P],
    "tt_batched_workspace_floats": [_L, _L, _L],
    "tt_int4_batched_matvec": [_P, _L, _P, _L, _P, _L, _P, _L, _L, _L, _L, _L, _P, _L, _P],
    "tt_scaled_batched_matvec": [_P, _L, _P, _P, _L, _P, _L, _L, _L, _L, _P, _L, _P],
    "tt_matvec_argmax_batched_partials": [_L, _L, _L],
    "tt_matvec_argmax_batched": [_P, _L, _P, _L, _L, _P, _L, _L, _L, _P, _L, _P, _P, _P],
    "tt_fused_struct_sizes": [_LP, _LP],
    "tt_fused_gemv_run": [_FGP, _P],
    "tt_fused_lm_head_argmax": [_FGP, _P, _L, _P, _P, _P, _P, _P, ctypes.c_int32, _P],
    "tt_stream_read_waves": [_L, _L],
    "tt_stream_read": [_P, _L, _L, _P, _L, _P],
    "tt_quantize_int4": [_P, _I, _L, _L, _L, _L, _I, _P, _P, _P, _P, _P],
    "tt_quantize_fp8_rows": [_P, _I, _L, _L, _L, _L, _I, _P, _P, _P],
    "tt_quantize_mxfp4_rows": [_P, _I, _L, _L, _L, _L, _P, _I, _P, _P, _P],
    "tt_requantize_mxfp4_lowbit": [_P, _P, _L, _I, _P, _P, _P],
    "tt_quantize_dense_lowbit": [_P, _I, _L, _L, _L, _I, _P, _P, _P],
    "tt_pack_mxfp4_ternary": [_P, _L, _L, _P, _P],
    "tt_archive_open": [ctypes.c_char_p, ctypes.POINTER(_P)],
    "tt_archive_parse_pages": [_P],
    "tt_archive_check_overlaps": [_P],
    "tt_archive_get_info": [_P, ctypes.POINTER(ArchiveInfo)],
    "tt_archive_get_record": [_P, _L, ctypes.POINTER(ArchiveRecord)],
    "tt_archive_find": [_P, ctypes.c_char_p, _L],
    "tt_archive_data": [_P],
    "tt_archive_upload": [_P, _L, _L, _P, _P],
    "tt_archive_close": [_P],
}
_RESTYPES = {"tt_last_error": ctypes.c_char_p, "tt_matvec_argmax_partials": ctypes.c_int64,
             "tt_batched_workspace_floats": ctypes.c_int64,
             "tt_norm_router_workspace_bytes": ctypes.c_int64,
             "tt_stream_read_waves": ctypes.c_int64,
             "tt_matvec_argmax_batched_partials": ctypes.c_int64, "tt_archive_find": ctypes.c_int64,
             "tt_archive_data": ctypes.c_void_p}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


class KernelLibraryError(RuntimeError):
    """The HIP kernel library is missing, stale or rejected a call."""


def library_path() -> Path:
    override = os.environ.get("THINTENSOR_HIP_LIB") or None
    return Path(override) if override else _build.LIB_PATH


def load(build_if_missing: bool = True) -> ctypes.CDLL:
    """Load the kernel library (building it with hipcc only if no build exists)."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        path = library_path()
        if not path.exists():
            if not build_if_missing:
                raise KernelLibraryError(f"HIP kernel library not built: {path}")
            _build.build()
        lib = ctypes.CDLL(str(path))
        missing = []
        for name, argtypes in SIGNATURES.items():
            try:
                fn = getattr(lib, name)
            except AttributeError:
                missing.append(name)
                continue
            fn.argtypes = argtypes
            fn.restype = _RESTYPES.get(name, ctypes.c_int)
        if missing:
            raise KernelLibraryError(f"{path} lacks entry points {missing}; rebuild with thintensor_amd.build")
        seg, desc = ctypes.c_int64(), ctypes.c_int64()
        lib.tt_fused_struct_sizes(ctypes.byref(seg), ctypes.byref(desc))
        if (seg.value, desc.value) != (ctypes.sizeof(FusedSegment), ctypes.sizeof(FusedGemv)):
            raise KernelLibraryError(f"fused descriptor layout mismatch: library {seg.value}/{desc.value} bytes, "
                                     f"binding {ctypes.sizeof(FusedSegment)}/{ctypes.sizeof(FusedGemv)}")
        _lib = lib
        return lib


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = load().tt_last_error().decode(errors="replace")
        if rc == -1:
            raise ValueError(f"{what}: {msg}")
        raise KernelLibraryError(f"{what} failed ({rc}): {msg}")


def ptr_array(values) -> ctypes.Array:
    arr = (ctypes.c_void_p * len(values))()
    for i, v in enumerate(values):
        arr[i] = v
    return arr


def i64_array(values) -> ctypes.Array:
    arr = (ctypes.c_int64 * len(values))()
    for i, v in enumerate(values):
        arr[i] = int(v)
    return arr
