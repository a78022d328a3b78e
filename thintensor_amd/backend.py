"""HipDecodeBackend: the MI355X drop-in for the reference's ``TritonDecodeBackend``.

Method names, positional/keyword arguments, return values, shape contracts and
their ``ValueError`` messages follow ``TritonDecodeBackend``
(thinruntime/triton_kernels.py:3553-5893) so the reference runtime can construct
this object where it constructs the Triton backend (gpu_runtime.py:5441-5457).
Every operator is destination-passing, launches on torch's current stream through
the C ABI of ``libthintensor_hip.so`` and never synchronises the host.

Launch-tuning keywords of the Triton backend (``block_m``, ``num_warps``,
``block_k``, ``config_name``) are accepted for signature compatibility and
ignored: the HIP kernels choose their own launch shape, and their reduction order
depends only on the tensor shapes.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Any

import torch

from . import _lib

_DTYPE_CODE = {torch.float16: _lib.F16, torch.bfloat16: _lib.BF16, torch.float32: _lib.F32}


def _code(t: torch.Tensor, what: str) -> int:
    try:
        return _DTYPE_CODE[t.dtype]
    except KeyError:
        raise ValueError(f"{what}: unsupported dtype {t.dtype}") from None


# one-byte weight formats of the scaled GEMVs (the reference kernels convert either to fp32)
_BYTE_WEIGHT_FORMATS = {torch.float8_e4m3fn: _lib.W_FP8, torch.int8: _lib.W_INT8}


def _byte_weight_format(weight: torch.Tensor, what: str) -> int:
    try:
        return _BYTE_WEIGHT_FORMATS[weight.dtype]
    except KeyError:
        raise ValueError(f"{what} supports float8_e4m3fn and int8 weights, got {weight.dtype}") from None


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _require_cuda(*tensors: torch.Tensor) -> None:
    for t in tensors:
        if t is not None and t.device.type != "cuda":
            raise ValueError("HipDecodeBackend operates on device tensors only")


@dataclass
class DecodeBuffers:
    """Persistent activation vectors, as ``TritonDecodeBuffers`` (triton_kernels.py:3516-3529)."""

    hidden_a: torch.Tensor
    hidden_b: torch.Tensor
    normed: torch.Tensor
    qkv: torch.Tensor
    q_norm: torch.Tensor
    k_norm: torch.Tensor
    attn: torch.Tensor
    attn_out: torch.Tensor
    gate_up: torch.Tensor
    mlp_act: torch.Tensor
    mlp: torch.Tensor
    final: torch.Tensor


class HipDecodeBackend:
    """HIP/gfx950 implementation of the decode operator set."""

    def __init__(
        self,
        device: torch.device,
        dtype: torch.dtype,
        hidden_size: int,
        q_dim: int,
        kv_dim: int,
        intermediate_size: int,
        argmax_mode: str = "torch",
    ) -> None:
        self.lib = _lib.load()
        self.device = torch.device(device)
        self.dtype = dtype
        self.hidden_size = hidden_size
        self.q_dim = q_dim
        self.kv_dim = kv_dim
        self.intermediate_size = intermediate_size
        self.argmax_mode = argmax_mode
        empty = lambda n: torch.empty(n, device=self.device, dtype=dtype)  # noqa: E731
        self.buffers = DecodeBuffers(
            hidden_a=empty(hidden_size),
            hidden_b=empty(hidden_size),
            normed=empty(hidden_size),
            qkv=empty(q_dim + 2 * kv_dim),
            q_norm=empty(q_dim),
            k_norm=empty(kv_dim),
            attn=empty(q_dim),
            attn_out=empty(hidden_size),
            gate_up=empty(2 * intermediate_size),
            mlp_act=empty(intermediate_size),
            mlp=empty(hidden_size),
            final=empty(hidden_size),
        )
        self._logits_buffer: torch.Tensor | None = None
        # The argmax result is a reused buffer: later calls overwrite it
        # (same ownership as triton_kernels.py:3595).
        self._argmax_out_idx = torch.empty((), device=self.device, dtype=torch.int64)
        self._argmax_out_val = torch.empty((), device=self.device, dtype=torch.float32)
        self._argmax_partials: torch.Tensor | None = None
        self._attention_partials: torch.Tensor | None = None
        self._batched_partials: torch.Tensor | None = None
        self._split_k_partials: torch.Tensor | None = None   # split-K scratch (triton_kernels.py:3797-3805)

    # ------------------------------------------------------------ helpers
    @staticmethod
    def _layout_key(tensor: torch.Tensor) -> tuple[Any, ...]:
        return (str(tensor.device), str(tensor.dtype), tuple(tensor.shape), tuple(tensor.stride()))

    def logits_buffer(self, rows: int, dtype: torch.dtype) -> torch.Tensor:
        if self._logits_buffer is None or self._logits_buffer.numel() != rows or self._logits_buffer.dtype != dtype:
            self._logits_buffer = torch.empty(rows, device=self.device, dtype=dtype)
        return self._logits_buffer

    # ------------------------------------------------------------ dense GEMV
    def matvec(
        self,
        weight: torch.Tensor,
        x: torch.Tensor,
        out: torch.Tensor,
        *,
        block_m: int | None = None,
        num_warps: int | None = None,
        config_name: str | None = None,
    ) -> torch.Tensor:
        """out = weight @ x for fp16/bf16 weight [rows, cols] (triton_kernels.py:3701-3771)."""
        _require_cuda(weight, x, out)
        rows, cols = int(weight.shape[0]), int(weight.shape[1])
        if weight.stride(1) != 1 or x.numel() != cols or out.numel() != rows or not out.is_contiguous():
            raise ValueError(f"matvec shape mismatch: weight {tuple(weight.shape)}, x {tuple(x.shape)}, out {tuple(out.shape)}")
        rc = self.lib.tt_matvec(
            weight.data_ptr(), _code(weight, "matvec"), weight.stride(0), x.data_ptr(), _code(x, "matvec"),
            out.data_ptr(), _code(out, "matvec"), rows, cols, _stream(out),
        )
        _lib.check(rc, "matvec")
        return out

    def multi_matvec(
        self,
        weights: tuple[torch.Tensor, ...],
        x: torch.Tensor,
        out: torch.Tensor,
        *,
        block_m: int = 8,
        num_warps: int = 8,
    ) -> torch.Tensor:
        """Two to four dense matrices sharing x, concatenated output (triton_kernels.py:4978-5064)."""
        if len(weights) == 4:
            first = sum(int(w.shape[0]) for w in weights[:2])
            self.multi_matvec(weights[:2], x, out[:first])
            self.multi_matvec(weights[2:], x, out[first:])
            return out
        if len(weights) not in {2, 3}:
            raise ValueError("multi_matvec supports two, three, or four matrices")
        cols = int(weights[0].shape[1])
        if any(int(w.shape[1]) != cols for w in weights):
            raise ValueError("multi_matvec matrices must have the same column count")
        _require_cuda(x, out, *weights)
        wdt = _code(weights[0], "multi_matvec")
        if any(_code(w, "multi_matvec") != wdt or w.stride(1) != 1 for w in weights):
            raise ValueError("multi_matvec matrices must share a dtype and be row-major")
        rows = [int(w.shape[0]) for w in weights]
        if out.numel() != sum(rows) or x.numel() != cols:
            raise ValueError("multi_matvec output/input size mismatch")
        rc = self.lib.tt_multi_matvec(
            len(weights), _lib.ptr_array([w.data_ptr() for w in weights]), wdt,
            _lib.i64_array([w.stride(0) for w in weights]), _lib.i64_array(rows), x.data_ptr(), _code(x, "multi_matvec"),
            out.data_ptr(), _code(out, "multi_matvec"), cols, _stream(out),
        )
        _lib.check(rc, "multi_matvec")
        return out

    # ------------------------------------------------------------ int4
    def int4_scaled_matvec(
        self,
        packed_weight: torch.Tensor,
        scales: torch.Tensor,
        x: torch.Tensor,
        out: torch.Tensor,
        *,
        rows: int,
        cols: int,
        group_size: int,
    ) -> torch.Tensor:
        """Group-scaled int4 GEMV (triton_kernels.py:4597-4743).

        packed_weight: uint8 [rows, cols/2] (or its int32/uint32 view [rows, cols/8]);
        scales: fp16/fp32 [rows, groups] (symmetric) or [rows, groups, 2] (affine s, m).
        """
        _require_cuda(packed_weight, scales, x, out)
        row_bytes = packed_weight.stride(0) * packed_weight.element_size()
        if int(packed_weight.shape[0]) != rows or packed_weight.shape[1] * packed_weight.element_size() * 2 != cols:
            raise ValueError(f"int4 packed weight {tuple(packed_weight.shape)} does not match rows={rows} cols={cols}")
        if x.numel() != cols or out.numel() != rows:
            raise ValueError("int4_scaled_matvec input/output size mismatch")
        affine = scales.ndim == 3
        s_row = scales.stride(0)
        s_group = scales.stride(1) if scales.ndim >= 2 else 0
        s_pair = scales.stride(2) if affine else 0
        rc = self.lib.tt_int4_scaled_matvec(
            packed_weight.data_ptr(), row_bytes, scales.data_ptr(), _code(scales, "int4 scales"), s_row, s_group,
            s_pair, int(affine), x.data_ptr(), _code(x, "int4_scaled_matvec"), out.data_ptr(),
            _code(out, "int4_scaled_matvec"), rows, cols, group_size, _stream(out),
        )
        _lib.check(rc, "int4_scaled_matvec")
        return out

    def multi_int4_scaled_matvec(
        self,
        weights: tuple[torch.Tensor, ...],
        scales: tuple[torch.Tensor, ...],
        rows: tuple[int, ...],
        cols: int,
        x: torch.Tensor,
        out: torch.Tensor,
        *,
        group_size: int | None = None,
    ) -> torch.Tensor:
        """Two or three int4 matrices in one launch (triton_kernels.py:5066-5117).

        The reference only uses this for one scale per row; here any group size the
        single-matrix op accepts works (``group_size`` defaults to one scale per row).
        """
        if len(weights) not in {2, 3} or len(scales) != len(weights):
            raise ValueError("multi INT4 matvec supports two or three matrices")
        _require_cuda(x, out, *weights, *scales)
        group = cols if group_size is None else group_size
        sdt = _code(scales[0], "int4 scales")
        affine = scales[0].ndim == 3
        if out.numel() != sum(rows) or x.numel() != cols:
            raise ValueError("multi INT4 matvec output/input size mismatch")
        rc = self.lib.tt_multi_int4_scaled_matvec(
            len(weights), _lib.ptr_array([w.data_ptr() for w in weights]),
            _lib.i64_array([w.stride(0) * w.element_size() for w in weights]),
            _lib.ptr_array([s.data_ptr() for s in scales]), sdt, _lib.i64_array([s.stride(0) for s in scales]),
            _lib.i64_array([s.stride(1) if s.ndim >= 2 else 0 for s in scales]),
            scales[0].stride(2) if affine else 0, int(affine), _lib.i64_array(rows), x.data_ptr(),
            _code(x, "multi_int4_scaled_matvec"), out.data_ptr(), _code(out, "multi_int4_scaled_matvec"), cols, group,
            _stream(out),
        )
        _lib.check(rc, "multi_int4_scaled_matvec")
        return out

    def int4_selected_matvec(
        self,
        packed_weight: torch.Tensor,
        scales: torch.Tensor,
        x: torch.Tensor,
        expert_indices: torch.Tensor,
        out: torch.Tensor,
        *,
        group_size: int,
        block_m: int = 8,
        num_warps: int = 8,
    ) -> torch.Tensor:
        """Selected-expert int4 GEMV (triton_kernels.py:4745-4805)."""
        if packed_weight.ndim != 3 or scales.ndim != 3:
            raise ValueError("selected INT4 expert weights/scales must both be rank 3")
        experts, rows, packed_cols = map(int, packed_weight.shape)
        if int(scales.shape[0]) != experts or int(scales.shape[1]) != rows:
            raise ValueError("selected INT4 expert scale shape mismatch")
        cols = packed_cols * 2
        selected = int(expert_indices.numel())
        stride_xe = self._selected_x_stride(x, selected, cols, "selected INT4")
        if tuple(out.shape) != (selected, rows):
            raise ValueError(f"selected INT4 output must be {(selected, rows)}, got {tuple(out.shape)}")
        index_bytes = self._check_indices(expert_indices)
        _require_cuda(packed_weight, scales, x, out)
        rc = self.lib.tt_int4_selected_matvec(
            packed_weight.data_ptr(), packed_weight.stride(0), packed_weight.stride(1), scales.data_ptr(),
            _code(scales, "int4 scales"), scales.stride(0), scales.stride(1), scales.stride(2), x.data_ptr(),
            _code(x, "int4_selected_matvec"), stride_xe, expert_indices.data_ptr(), index_bytes, selected, out.data_ptr(),
            _code(out, "int4_selected_matvec"), out.stride(0), rows, cols, group_size, _stream(out),
        )
        _lib.check(rc, "int4_selected_matvec")
        return out

    # ------------------------------------------------------------ fp8
    def scaled_matvec(
        self,
        weight: torch.Tensor,
        scales: torch.Tensor,
        x: torch.Tensor,
        out: torch.Tensor,
        config_name: str | None = None,
        *,
        block_m: int | None = None,
        num_warps: int | None = None,
    ) -> torch.Tensor:
        """y = (W @ x) * s_row for float8_e4m3fn or int8 W (triton_kernels.py:4452-4595,
        per-row or per-block scales; the kernels at :539-592 read either byte format)."""
        _require_cuda(weight, scales, x, out)
        wfmt = _byte_weight_format(weight, "scaled_matvec")
        rows, cols = int(weight.shape[0]), int(weight.shape[1])
        if scales.dim() == 2:
            # block-scaled branch (triton_kernels.py:4465-4497): blocks of
            # next_pow2(ceil(cols / blocks)) columns, scale [row, block]
            blocks = int(scales.shape[1])
            if int(scales.shape[0]) != rows or blocks < 1 or x.numel() != cols or out.numel() != rows or \
                    weight.stride(1) != 1:
                raise ValueError("scaled_matvec shape mismatch")
            block = 1 << max(0, (-(-cols // blocks) - 1).bit_length())
            _require_cuda(weight, scales, x, out)
            rc = self.lib.tt_block_scaled_matvec(
                weight.data_ptr(), wfmt, weight.stride(0), scales.data_ptr(), _code(scales, "fp8 scales"), scales.stride(0),
                scales.stride(1), block, x.data_ptr(), _code(x, "scaled_matvec"), out.data_ptr(),
                _code(out, "scaled_matvec"), rows, cols, _stream(out),
            )
            _lib.check(rc, "scaled_matvec")
            return out
        if scales.numel() != rows or x.numel() != cols or out.numel() != rows or weight.stride(1) != 1:
            raise ValueError("scaled_matvec shape mismatch")
        rc = self.lib.tt_scaled_matvec(
            weight.data_ptr(), wfmt, weight.stride(0), scales.data_ptr(), _code(scales, "fp8 scales"), x.data_ptr(),
            _code(x, "scaled_matvec"), out.data_ptr(), _code(out, "scaled_matvec"), rows, cols, _stream(out),
        )
        _lib.check(rc, "scaled_matvec")
        return out

    def multi_scaled_tensorcore_matvec(
        self,
        weights: tuple[torch.Tensor, ...],
        scales: tuple[torch.Tensor, ...],
        rows: tuple[int, ...],
        cols: int,
        x: torch.Tensor,
        out: torch.Tensor,
    ) -> torch.Tensor:
        """Two or three float8_e4m3fn or int8 matrices with per-row scales, outputs
        concatenated (triton_kernels.py:5119-5180, kernel :1958-2071)."""
        if len(weights) not in {2, 3} or len(scales) != len(weights):
            raise ValueError("multi scaled tensor-core matvec supports two or three matrices")
        if cols % 256:
            raise ValueError("tensor-core matvec columns must be divisible by 256")
        dtype = weights[0].dtype
        if dtype not in {torch.float8_e4m3fn, torch.int8}:
            raise ValueError("tensor-core matvec requires E4M3 or INT8 weights")
        if any(weight.dtype != dtype for weight in weights):
            raise ValueError("multi tensor-core weights must share one dtype")
        rows = tuple(int(r) for r in rows)[: len(weights)]
        if len(rows) != len(weights) or any(int(w.shape[0]) != r or int(w.shape[1]) != cols or w.stride(1) != 1
                                            for w, r in zip(weights, rows)):
            raise ValueError("multi scaled matvec shape mismatch")
        if any(sc.ndim != 1 or sc.numel() != r for sc, r in zip(scales, rows)):
            raise ValueError("multi scaled matvec requires one scale per output row")
        if len({sc.dtype for sc in scales}) != 1 or x.numel() != cols or out.numel() < sum(rows):
            raise ValueError("multi scaled matvec scale/input/output mismatch")
        _require_cuda(*weights, *scales, x, out)
        rc = self.lib.tt_multi_scaled_matvec(
            len(weights), _lib.ptr_array([w.data_ptr() for w in weights]),
            _lib.W_INT8 if dtype == torch.int8 else _lib.W_FP8, _lib.i64_array([w.stride(0) for w in weights]),
            _lib.ptr_array([sc.data_ptr() for sc in scales]), _code(scales[0], "fp8 scales"),
            _lib.i64_array([sc.stride(0) for sc in scales]), _lib.i64_array(rows), x.data_ptr(),
            _code(x, "multi_scaled_tensorcore_matvec"), out.data_ptr(), _code(out, "multi_scaled_tensorcore_matvec"),
            cols, _stream(out),
        )
        _lib.check(rc, "multi_scaled_tensorcore_matvec")
        return out

    def split_k_matvec(
        self,
        weight: torch.Tensor,
        x: torch.Tensor,
        out: torch.Tensor,
        *,
        scales: torch.Tensor | None = None,
        split_k: int = 4,
        block_m: int = 32,
        block_n: int = 256,
        num_warps: int = 4,
    ) -> torch.Tensor:
        """Split-K GEMV with binary32 partials and an in-order reduce
        (triton_kernels.py:3773-3845, kernels :3023-3100).  Slices are whole 32-column
        chunks; the tile arguments are accepted and ignored."""
        if split_k not in {2, 4, 8}:
            raise ValueError("split_k must be 2, 4, or 8")
        rows = int(weight.shape[0])
        cols = int(weight.shape[1])
        if scales is not None and (scales.ndim != 1 or scales.numel() != rows):
            raise ValueError("split-K scaled matvec requires one scale per output row")
        if weight.dtype == torch.float16:
            fmt = _lib.F16
        elif weight.dtype == torch.bfloat16:
            fmt = _lib.BF16
        elif weight.dtype in _BYTE_WEIGHT_FORMATS:
            fmt = _BYTE_WEIGHT_FORMATS[weight.dtype]
        else:
            raise ValueError(f"split_k_matvec supports fp16, bf16, float8_e4m3fn and int8 weights, got {weight.dtype}")
        if weight.stride(1) != 1 or x.numel() != cols or out.numel() != rows or not out.is_contiguous():
            raise ValueError("split_k_matvec shape mismatch")
        count = split_k * rows
        if self._split_k_partials is None or self._split_k_partials.numel() < count:
            self._split_k_partials = torch.empty(count, device=self.device, dtype=torch.float32)
        partials = self._split_k_partials
        _require_cuda(weight, x, out)
        rc = self.lib.tt_split_k_matvec(
            weight.data_ptr(), fmt, weight.stride(0) * weight.element_size(),
            scales.data_ptr() if scales is not None else None,
            _code(scales, "split-K scales") if scales is not None else _lib.F32, x.data_ptr(),
            _code(x, "split_k_matvec"), out.data_ptr(), _code(out, "split_k_matvec"), rows, cols, split_k,
            partials.data_ptr(), partials.numel(), _stream(out),
        )
        _lib.check(rc, "split_k_matvec")
        return out

    def fused_scaled_gate_up_silu(
        self,
        gate_weight: torch.Tensor,
        gate_scales: torch.Tensor,
        up_weight: torch.Tensor,
        up_scales: torch.Tensor,
        x: torch.Tensor,
        out: torch.Tensor,
        *,
        block_m: int | None = None,
        num_warps: int | None = None,
    ) -> torch.Tensor:
        """silu(bf16(W_g x * s_g)) * bf16(W_u x * s_u) in one launch
        (triton_kernels.py:4346-4436, kernels :3243-3350)."""
        if gate_scales.ndim != 1 or up_scales.ndim != 1:
            raise ValueError("fused scaled gate/up requires one scale per output row")
        rows = int(gate_weight.shape[0])
        cols = int(gate_weight.shape[1])
        if tuple(up_weight.shape) != tuple(gate_weight.shape):
            raise ValueError("fused scaled gate/up matrices must have equal shapes")
        if gate_scales.numel() != rows or up_scales.numel() != rows:
            raise ValueError("fused scaled gate/up scales must match matrix rows")
        wfmt = _byte_weight_format(gate_weight, "fused_scaled_gate_up_silu")
        if up_weight.dtype != gate_weight.dtype:
            raise ValueError("fused scaled gate/up matrices must share a dtype")
        if gate_scales.dtype != up_scales.dtype:
            raise ValueError("fused scaled gate/up scales must share a dtype")
        if gate_weight.stride(1) != 1 or up_weight.stride(1) != 1 or x.numel() != cols or out.numel() != rows:
            raise ValueError("fused_scaled_gate_up_silu shape mismatch")
        _require_cuda(gate_weight, gate_scales, up_weight, up_scales, x, out)
        rc = self.lib.tt_scaled_gate_up_silu(
            gate_weight.data_ptr(), gate_weight.stride(0), gate_scales.data_ptr(), gate_scales.stride(0),
            up_weight.data_ptr(), up_weight.stride(0), up_scales.data_ptr(), up_scales.stride(0), wfmt,
            _code(gate_scales, "gate/up scales"), x.data_ptr(), _code(x, "fused_scaled_gate_up_silu"), out.data_ptr(),
            _code(out, "fused_scaled_gate_up_silu"), rows, cols, _stream(out),
        )
        _lib.check(rc, "fused_scaled_gate_up_silu")
        return out

    # ------------------------------------------------------------ MoE experts
    @staticmethod
    def _selected_x_stride(x: torch.Tensor, selected: int, cols: int, what: str) -> int:
        if x.ndim == 1:
            if int(x.numel()) != cols:
                raise ValueError(f"{what} vector has {x.numel()} values, expected {cols}")
            return 0
        if x.ndim == 2 and tuple(x.shape) == (selected, cols) and x.stride(1) == 1:
            return int(x.stride(0))
        raise ValueError(f"{what} input must be {(cols,)} or {(selected, cols)}, got {tuple(x.shape)}")

    @staticmethod
    def _check_indices(expert_indices: torch.Tensor) -> int:
        """Byte width of a selected-expert index tensor.  The reference's kernels load
        the ids in whatever integer type they are given (triton_kernels.py:439, 886, 956,
        1157, 1240); the runtime passes int32 router output and, for dense low-bit
        pages, a torch.long id (gpu_runtime.py:12069-12072).  Both are read as is."""
        if expert_indices.dtype not in (torch.int32, torch.int64) or not expert_indices.is_contiguous():
            raise ValueError("expert_indices must be a contiguous int32 or int64 device tensor")
        return expert_indices.element_size()

    @staticmethod
    def _check_router_indices(indices_out: torch.Tensor) -> None:
        # the router writes int32 ids, the dtype of the runtime's router buffer
        # (gpu_runtime.py:5605-5607)
        if indices_out.dtype != torch.int32 or not indices_out.is_contiguous():
            raise ValueError("router indices_out must be a contiguous int32 device tensor")

    def mxfp4_selected_matvec(
        self,
        blocks: torch.Tensor,
        scales: torch.Tensor,
        x: torch.Tensor,
        expert_indices: torch.Tensor,
        out: torch.Tensor,
        *,
        block_m: int = 4,
        num_warps: int = 8,
    ) -> torch.Tensor:
        """MXFP4 selected-expert GEMV (triton_kernels.py:3847-3911)."""
        if blocks.ndim != 4 or scales.ndim != 3:
            raise ValueError("MXFP4 expert blocks/scales must be rank 4/rank 3")
        if blocks.shape[:-1] != scales.shape:
            raise ValueError(f"MXFP4 blocks/scales mismatch: {blocks.shape} vs {scales.shape}")
        rows = int(blocks.shape[1])
        cols = int(blocks.shape[2] * blocks.shape[3] * 2)
        selected = int(expert_indices.numel())
        stride_xe = self._selected_x_stride(x, selected, cols, "MXFP4")
        if tuple(out.shape) != (selected, rows):
            raise ValueError(f"MXFP4 output must be {(selected, rows)}, got {tuple(out.shape)}")
        if blocks.stride(3) != 1 or blocks.stride(2) != blocks.shape[3] or scales.stride(2) != 1:
            raise ValueError("MXFP4 blocks/scales must be contiguous within a row")
        index_bytes = self._check_indices(expert_indices)
        _require_cuda(blocks, scales, x, out)
        rc = self.lib.tt_mxfp4_selected_matvec(
            blocks.data_ptr(), blocks.stride(0), blocks.stride(1), scales.data_ptr(), scales.stride(0),
            scales.stride(1), x.data_ptr(), _code(x, "mxfp4_selected_matvec"), stride_xe, expert_indices.data_ptr(), index_bytes,
            selected, out.data_ptr(), _code(out, "mxfp4_selected_matvec"), out.stride(0), rows, cols, _stream(out),
        )
        _lib.check(rc, "mxfp4_selected_matvec")
        return out

    def mxfp4_selected_tensorcore_matvec(
        self,
        blocks: torch.Tensor,
        scales: torch.Tensor,
        x: torch.Tensor,
        expert_indices: torch.Tensor,
        out: torch.Tensor,
        *,
        block_m: int = 64,
        block_n: int = 8,
    ) -> torch.Tensor:
        """Same sum as ``mxfp4_selected_matvec`` (triton_kernels.py:3913-3976; the
        reference's Blackwell tensor-core twin of :416-481).  Tile arguments are
        accepted and ignored."""
        return self.mxfp4_selected_matvec(blocks, scales, x, expert_indices, out)

    # The reference's Blackwell tensor-core variant computes the same sum
    # (triton_kernels.py:865-930, 3913-3976); on gfx950 it is the same kernel.
    mxfp4_selected_tensorcore_matvec = mxfp4_selected_matvec

    def mxfp_lowbit_selected_matvec(
        self,
        packed_weight: torch.Tensor,
        scales: torch.Tensor,
        x: torch.Tensor,
        expert_indices: torch.Tensor,
        out: torch.Tensor,
        *,
        bits: int,
        block_m: int = 0,
        block_k: int = 0,
    ) -> torch.Tensor:
        """Q1/Q2 E8M0 selected-expert GEMV (triton_kernels.py:4132-4176)."""
        if bits not in {1, 2} or packed_weight.ndim != 4 or scales.ndim != 3:
            raise ValueError("low-bit expert weights must be packed Q1 or Q2")
        rows = int(packed_weight.shape[1])
        cols = int(scales.shape[2] * 32)
        selected = int(expert_indices.numel())
        stride_xe = self._selected_x_stride(x, selected, cols, "low-bit expert")
        if tuple(out.shape) != (selected, rows):
            raise ValueError(f"low-bit output must be {(selected, rows)}, got {tuple(out.shape)}")
        index_bytes = self._check_indices(expert_indices)
        _require_cuda(packed_weight, scales, x, out)
        rc = self.lib.tt_mxfp_lowbit_selected_matvec(
            packed_weight.data_ptr(), packed_weight.stride(0), packed_weight.stride(1), scales.data_ptr(),
            scales.stride(0), scales.stride(1), bits, x.data_ptr(), _code(x, "mxfp_lowbit_selected_matvec"), stride_xe,
            expert_indices.data_ptr(), index_bytes, selected, out.data_ptr(), _code(out, "mxfp_lowbit_selected_matvec"),
            out.stride(0), rows, cols, _stream(out),
        )
        _lib.check(rc, "mxfp_lowbit_selected_matvec")
        return out

    def mxfp_lowbit_selected_tensorcore_matvec(
        self,
        packed_weight: torch.Tensor,
        scales: torch.Tensor,
        x: torch.Tensor,
        expert_indices: torch.Tensor,
        out: torch.Tensor,
        *,
        bits: int,
        **_: Any,
    ) -> torch.Tensor:
        """Same sum as the scalar variant (triton_kernels.py:3978-4055)."""
        return self.mxfp_lowbit_selected_matvec(packed_weight, scales, x, expert_indices, out, bits=bits)

    def sparse_residual_matvec(
        self,
        residual_values: torch.Tensor,
        residual_indices: torch.Tensor,
        x: torch.Tensor,
        out: torch.Tensor,
    ) -> torch.Tensor:
        """out += sum_k values[:, k] * x[indices[:, k]] (triton_kernels.py:5429-5456)."""
        if residual_values.shape != residual_indices.shape:
            raise ValueError("sparse residual values/indices shape mismatch")
        rows = int(residual_values.shape[0])
        terms = int(residual_values.shape[1])
        if residual_indices.dtype not in (torch.int16, torch.int32, torch.int64):
            raise ValueError("sparse residual indices must be int16, int32 or int64")
        if out.numel() != rows or not out.is_contiguous() or not x.is_contiguous():
            raise ValueError("sparse residual output/input layout mismatch")
        _require_cuda(residual_values, residual_indices, x, out)
        rc = self.lib.tt_sparse_residual_matvec(
            residual_values.data_ptr(), _code(residual_values, "sparse residual values"), residual_values.stride(0),
            residual_values.stride(1), residual_indices.data_ptr(), residual_indices.element_size(),
            residual_indices.stride(0), residual_indices.stride(1), x.data_ptr(), _code(x, "sparse_residual_matvec"),
            out.data_ptr(), _code(out, "sparse_residual_matvec"), rows, terms, int(x.numel()), _stream(out),
        )
        _lib.check(rc, "sparse_residual_matvec")
        return out

    def binary_residual_matvec(
        self,
        packed_signs: torch.Tensor,
        scales: torch.Tensor,
        x: torch.Tensor,
        out: torch.Tensor,
    ) -> torch.Tensor:
        """out += sum_k sign_k * scale[:, k/32] * x[k] (triton_kernels.py:5458-5487)."""
        rows = int(packed_signs.shape[0])
        cols = int(x.numel())
        if tuple(packed_signs.shape) != (rows, cols // 8):
            raise ValueError("binary residual sign plane shape mismatch")
        if tuple(scales.shape) != (rows, cols // 32):
            raise ValueError("binary residual scale shape mismatch")
        if packed_signs.stride(1) != 1 or scales.stride(1) != 1 or out.numel() != rows or not out.is_contiguous():
            raise ValueError("binary residual sign plane, scales and output rows must be contiguous")
        if not x.is_contiguous():
            raise ValueError("binary residual input must be contiguous")
        _require_cuda(packed_signs, scales, x, out)
        rc = self.lib.tt_binary_residual_matvec(
            packed_signs.data_ptr(), packed_signs.stride(0), scales.data_ptr(), _code(scales, "binary residual scales"),
            scales.stride(0), x.data_ptr(), _code(x, "binary_residual_matvec"), out.data_ptr(),
            _code(out, "binary_residual_matvec"), rows, cols, _stream(out),
        )
        _lib.check(rc, "binary_residual_matvec")
        return out

    def mxfp_ternary_selected_tensorcore_matvec(
        self,
        packed_weight: torch.Tensor,
        scales: torch.Tensor,
        x: torch.Tensor,
        expert_indices: torch.Tensor,
        out: torch.Tensor,
        *,
        block_m: int = 0,
        block_n: int = 0,
    ) -> torch.Tensor:
        """Ternary selected-expert GEMV (triton_kernels.py:4057-4130, kernel :1022-1133).

        ``packed_weight`` uint8 [E, rows, ceil(cols/5) + ceil(3*cols/32/8)] (base-3 digits,
        then 3-bit magnitude selectors), ``scales`` E8M0 uint8 [E, rows, cols/32]; the
        tile arguments of the reference are accepted and ignored."""
        if packed_weight.ndim != 3 or scales.ndim != 3:
            raise ValueError("ternary expert weights/scales must be rank 3/rank 3")
        experts, rows, groups = map(int, scales.shape)
        cols = groups * 32
        ternary_bytes = (cols + 4) // 5
        magnitude_bytes = (groups * 3 + 7) // 8
        if tuple(packed_weight.shape) != (experts, rows, ternary_bytes + magnitude_bytes):
            raise ValueError(
                "ternary weight shape mismatch: "
                f"got {tuple(packed_weight.shape)}, expected {(experts, rows, ternary_bytes + magnitude_bytes)}"
            )
        selected = int(expert_indices.numel())
        if x.ndim == 1 and int(x.numel()) == cols and x.stride(0) == 1:
            stride_xe = 0
        elif x.ndim == 2 and tuple(x.shape) == (selected, cols) and x.stride(1) == 1:
            stride_xe = int(x.stride(0))
        else:
            raise ValueError(f"ternary input must be {(cols,)} or {(selected, cols)}, got {tuple(x.shape)}")
        if tuple(out.shape) != (selected, rows):
            raise ValueError(f"ternary output must be {(selected, rows)}, got {tuple(out.shape)}")
        if packed_weight.dtype != torch.uint8 or scales.dtype != torch.uint8:
            raise ValueError("ternary weights and scales must be uint8")
        if not packed_weight.is_contiguous() or not scales.is_contiguous() or out.stride(1) != 1:
            raise ValueError("ternary weights, scales and output rows must be contiguous")
        index_bytes = self._check_indices(expert_indices)
        _require_cuda(packed_weight, scales, x, out)
        rc = self.lib.tt_mxfp_ternary_selected_matvec(
            packed_weight.data_ptr(), packed_weight.stride(0), packed_weight.stride(1), packed_weight.numel(),
            scales.data_ptr(), scales.stride(0), scales.stride(1), scales.numel(), experts, x.data_ptr(),
            _code(x, "mxfp_ternary_selected_matvec"), stride_xe, expert_indices.data_ptr(), index_bytes, selected,
            out.data_ptr(), _code(out, "mxfp_ternary_selected_matvec"), out.stride(0), rows, cols, _stream(out),
        )
        _lib.check(rc, "mxfp_ternary_selected_matvec")
        return out

    def mxfp_lowbit_selected_swiglu(
        self,
        packed_weight: torch.Tensor,
        scales: torch.Tensor,
        x: torch.Tensor,
        expert_indices: torch.Tensor,
        out: torch.Tensor,
        *,
        bits: int,
        alpha: float,
        limit: float,
        bias: torch.Tensor | None = None,
        block_m: int = 4,
        block_k: int = 0,
        num_warps: int = 8,
    ) -> torch.Tensor:
        """Fused interleaved gate/up GEMV + gpt-oss SwiGLU (triton_kernels.py:4178-4235).

        ``bits`` 1/2 are the reference's E8M0 low-bit experts (bf16 rounding);
        ``bits=4`` runs MXFP4 ``blocks`` with rounding in the activation dtype, which
        reproduces the reference's unfused MXFP4 chain (gpu_runtime.py:9647-9704).
        """
        if bits not in {1, 2, 4} or packed_weight.ndim != 4 or scales.ndim != 3:
            raise ValueError("fused SwiGLU requires packed Q1 or Q2 experts")
        physical_rows = int(packed_weight.shape[1])
        if physical_rows % 2:
            raise ValueError("interleaved gate/up rows must be even")
        activation_rows = physical_rows // 2
        cols = int(scales.shape[2] * 32)
        selected = int(expert_indices.numel())
        if tuple(out.shape) != (selected, activation_rows):
            raise ValueError("fused SwiGLU output shape mismatch")
        stride_xe = self._selected_x_stride(x, selected, cols, "fused SwiGLU")
        index_bytes = self._check_indices(expert_indices)
        _require_cuda(packed_weight, scales, x, out)
        rc = self.lib.tt_mxfp_lowbit_selected_swiglu(
            packed_weight.data_ptr(), packed_weight.stride(0), packed_weight.stride(1), scales.data_ptr(),
            scales.stride(0), scales.stride(1), bits, x.data_ptr(), _code(x, "swiglu"), stride_xe,
            expert_indices.data_ptr(), index_bytes, selected, bias.data_ptr() if bias is not None else None,
            _code(bias, "bias") if bias is not None else _lib.F32, bias.stride(0) if bias is not None else 0,
            float(alpha), float(limit), out.data_ptr(), _code(out, "swiglu"), out.stride(0), activation_rows, cols,
            _stream(out),
        )
        _lib.check(rc, "mxfp_lowbit_selected_swiglu")
        return out

    def mxfp_lowbit_weighted_down(
        self,
        packed_weight: torch.Tensor,
        scales: torch.Tensor,
        x: torch.Tensor,
        expert_indices: torch.Tensor,
        router_scores: torch.Tensor,
        out: torch.Tensor,
        *,
        bits: int,
        bias: torch.Tensor | None = None,
        block_m: int = 4,
        block_k: int = 0,
        num_warps: int = 8,
    ) -> torch.Tensor:
        """Fused down GEMV + router-weighted expert sum (triton_kernels.py:4237-4285)."""
        if bits not in {1, 2, 4} or packed_weight.ndim != 4 or scales.ndim != 3:
            raise ValueError("fused down requires packed Q1 or Q2 experts")
        rows = int(packed_weight.shape[1])
        cols = int(scales.shape[2] * 32)
        selected = int(expert_indices.numel())
        if tuple(x.shape) != (selected, cols) or int(out.numel()) != rows:
            raise ValueError("fused weighted-down tensor shape mismatch")
        index_bytes = self._check_indices(expert_indices)
        _require_cuda(packed_weight, scales, x, out, router_scores)
        rc = self.lib.tt_mxfp_lowbit_weighted_down(
            packed_weight.data_ptr(), packed_weight.stride(0), packed_weight.stride(1), scales.data_ptr(),
            scales.stride(0), scales.stride(1), bits, x.data_ptr(), _code(x, "weighted_down"), x.stride(0),
            expert_indices.data_ptr(), index_bytes, router_scores.data_ptr(), _code(router_scores, "router scores"), selected,
            bias.data_ptr() if bias is not None else None, _code(bias, "bias") if bias is not None else _lib.F32,
            bias.stride(0) if bias is not None else 0, out.data_ptr(), _code(out, "weighted_down"), rows, cols,
            _stream(out),
        )
        _lib.check(rc, "mxfp_lowbit_weighted_down")
        return out

    def matvec_bias_rows(self, weight: torch.Tensor, bias: torch.Tensor | None, x: torch.Tensor,
                         out: torch.Tensor) -> torch.Tensor:
        """out[t] = W x[t] (+ bias) for x [M, cols], out [M, rows]; each row equals
        ``multi_matvec_bias((weight,), (bias,), x[t], out[t])``.  No reference
        counterpart (batched decode of independent sequences)."""
        rows, cols = map(int, weight.shape)
        if x.ndim != 2 or out.ndim != 2 or int(x.shape[1]) != cols or int(out.shape[1]) != rows or \
                x.shape[0] != out.shape[0] or x.stride(1) != 1 or out.stride(1) != 1 or weight.stride(1) != 1:
            raise ValueError("matvec_bias_rows takes W [rows, cols], x [M, cols] and out [M, rows]")
        if bias is not None and int(bias.numel()) != rows:
            raise ValueError("bias does not match the weight rows")
        _require_cuda(weight, x, out)
        rc = self.lib.tt_matvec_bias_rows(weight.data_ptr(), _code(weight, "matvec"), weight.stride(0),
                                          bias.data_ptr() if bias is not None else None, x.data_ptr(),
                                          _code(x, "matvec"), x.stride(0), out.data_ptr(), _code(out, "matvec"),
                                          out.stride(0), int(x.shape[0]), rows, cols, _stream(out))
        _lib.check(rc, "matvec_bias_rows")
        return out

    def mxfp_lowbit_selected_swiglu_tokens(self, packed_weight: torch.Tensor, scales: torch.Tensor, x: torch.Tensor,
                                           expert_indices: torch.Tensor, out: torch.Tensor, *, bits: int,
                                           alpha: float, limit: float,
                                           bias: torch.Tensor | None = None) -> torch.Tensor:
        """``mxfp_lowbit_selected_swiglu`` for T tokens at once: x [T, cols],
        expert_indices [T, k], out [T * k, I] (token t's slots are rows t*k ...).  No
        reference counterpart (batched decode of independent sequences); each token's
        rows equal the single-token operator's."""
        if bits not in {1, 2, 4} or packed_weight.ndim != 4 or scales.ndim != 3:
            raise ValueError("fused SwiGLU requires packed Q1, Q2 or MXFP4 experts")
        activation_rows = int(packed_weight.shape[1]) // 2
        cols = int(scales.shape[2] * 32)
        if x.ndim != 2 or expert_indices.ndim != 2 or int(x.shape[0]) != int(expert_indices.shape[0]):
            raise ValueError("batched SwiGLU takes x [T, cols] and expert_indices [T, k]")
        tokens, selected = map(int, expert_indices.shape)
        if int(x.shape[1]) != cols or x.stride(1) != 1 or tuple(out.shape) != (tokens * selected, activation_rows):
            raise ValueError("batched SwiGLU shape mismatch")
        index_bytes = self._check_indices(expert_indices)
        _require_cuda(packed_weight, scales, x, out)
        rc = self.lib.tt_mxfp_lowbit_selected_swiglu_tokens(
            packed_weight.data_ptr(), packed_weight.stride(0), packed_weight.stride(1), scales.data_ptr(),
            scales.stride(0), scales.stride(1), bits, x.data_ptr(), _code(x, "swiglu"), x.stride(0),
            expert_indices.data_ptr(), index_bytes, selected, bias.data_ptr() if bias is not None else None,
            _code(bias, "bias") if bias is not None else _lib.F32, bias.stride(0) if bias is not None else 0,
            float(alpha), float(limit), out.data_ptr(), _code(out, "swiglu"), out.stride(0), activation_rows, cols,
            tokens, _stream(out),
        )
        _lib.check(rc, "mxfp_lowbit_selected_swiglu_tokens")
        return out

    def _zeroed_workspace(self, name: str, need: int) -> torch.Tensor:
        """A byte workspace kept by the backend under `name`, zero-filled when it is
        (re)allocated: arrival counters at its head, which every call leaves at zero.
        Reserve it before graph capture so the capture records no allocation."""
        ws = getattr(self, name, None)
        if ws is None or ws.numel() < need:
            ws = torch.zeros(max(need, 1), device=self.device, dtype=torch.uint8)
            setattr(self, name, ws)
        return ws

    def reserve_batch_workspaces(self, tokens: int) -> None:
        """Allocate the router workspace of a `tokens`-row batched decode step ahead of
        graph capture."""
        need = int(self.lib.tt_norm_router_workspace_bytes(tokens))
        if need > 0:
            self._zeroed_workspace("_norm_router_ws", need)

    def mxfp_lowbit_weighted_down_tokens(self, packed_weight: torch.Tensor, scales: torch.Tensor, x: torch.Tensor,
                                         expert_indices: torch.Tensor, router_scores: torch.Tensor,
                                         out: torch.Tensor, *, bits: int,
                                         bias: torch.Tensor | None = None) -> torch.Tensor:
        """``mxfp_lowbit_weighted_down`` for T tokens at once: x [T * k, cols],
        expert_indices / router_scores [T, k], out [T, rows].  No reference counterpart;
        each token's output equals the single-token operator's."""
        if bits not in {1, 2, 4} or packed_weight.ndim != 4 or scales.ndim != 3:
            raise ValueError("fused down requires packed Q1, Q2 or MXFP4 experts")
        rows = int(packed_weight.shape[1])
        cols = int(scales.shape[2] * 32)
        if expert_indices.ndim != 2 or tuple(router_scores.shape) != tuple(expert_indices.shape):
            raise ValueError("batched weighted-down takes expert_indices and router_scores [T, k]")
        tokens, selected = map(int, expert_indices.shape)
        if tuple(x.shape) != (tokens * selected, cols) or out.ndim != 2 or tuple(out.shape) != (tokens, rows):
            raise ValueError("batched weighted-down shape mismatch")
        if not router_scores.is_contiguous() or out.stride(1) != 1:
            raise ValueError("batched weighted-down needs contiguous scores and output rows")
        index_bytes = self._check_indices(expert_indices)
        _require_cuda(packed_weight, scales, x, out, router_scores)
        rc = self.lib.tt_mxfp_lowbit_weighted_down_tokens(
            packed_weight.data_ptr(), packed_weight.stride(0), packed_weight.stride(1), scales.data_ptr(),
            scales.stride(0), scales.stride(1), bits, x.data_ptr(), _code(x, "weighted_down"), x.stride(0),
            expert_indices.data_ptr(), index_bytes, router_scores.data_ptr(), _code(router_scores, "router scores"), selected,
            bias.data_ptr() if bias is not None else None, _code(bias, "bias") if bias is not None else _lib.F32,
            bias.stride(0) if bias is not None else 0, out.data_ptr(), _code(out, "weighted_down"), out.stride(0),
            rows, cols, tokens, _stream(out),
        )
        _lib.check(rc, "mxfp_lowbit_weighted_down_tokens")
        return out

    # ------------------------------------------------------------ affine low-bit (no reference kernel)
    def lowbit_affine_matvec(
        self,
        packed_weight: torch.Tensor,
        scale_zero: torch.Tensor,
        x: torch.Tensor,
        out: torch.Tensor,
        *,
        bits: int,
        rows: int,
        cols: int,
        group_size: int,
    ) -> torch.Tensor:
        """w = (c - z) * s with fp16 (s, z) [rows, cols/group, 2]; q2 or q1 codes packed per row."""
        _require_cuda(packed_weight, scale_zero, x, out)
        if scale_zero.ndim != 3 or scale_zero.shape[-1] != 2 or scale_zero.dtype != torch.float16:
            raise ValueError("affine low-bit scale/zero must be fp16 [rows, groups, 2]")
        if x.numel() != cols or out.numel() != rows:
            raise ValueError("lowbit_affine_matvec input/output size mismatch")
        rc = self.lib.tt_lowbit_affine_matvec(
            packed_weight.data_ptr(), packed_weight.stride(0) * packed_weight.element_size(), scale_zero.data_ptr(),
            scale_zero.stride(0), scale_zero.stride(1), bits, x.data_ptr(), _code(x, "lowbit_affine_matvec"),
            out.data_ptr(), _code(out, "lowbit_affine_matvec"), rows, cols, group_size, _stream(out),
        )
        _lib.check(rc, "lowbit_affine_matvec")
        return out

    # ------------------------------------------------------------ lm_head + greedy argmax
    def _argmax_scratch(self, rows: int, cols: int) -> torch.Tensor:
        need = int(self.lib.tt_matvec_argmax_partials(rows, cols))
        if self._argmax_partials is None or self._argmax_partials.numel() < need:
            self._argmax_partials = torch.empty(need, device=self.device, dtype=torch.int64)
        return self._argmax_partials

    def _matvec_argmax(self, weight: torch.Tensor, x: torch.Tensor, logits: torch.Tensor | None,
                       unrounded: bool = False) -> torch.Tensor:
        """Shared lm_head launch.  The argmax key is taken from each logit rounded to the
        logits dtype (x's dtype without a logits buffer), or from the binary32 dot
        product itself when ``unrounded`` (the reference's two-stage and persistent
        modes, triton_kernels.py:2245-2250, 2524-2537)."""
        _require_cuda(weight, x)
        rows, cols = int(weight.shape[0]), int(weight.shape[1])
        if weight.stride(1) != 1 or x.numel() != cols:
            raise ValueError("matvec_argmax shape mismatch")
        partials = self._argmax_scratch(rows, cols)
        if unrounded:
            if logits is not None:
                raise ValueError("unrounded argmax writes no logits")
            key_code = _lib.F32
        else:
            key_code = _code(logits, "logits") if logits is not None else _code(x, "x")
        rc = self.lib.tt_matvec_argmax(
            weight.data_ptr(), _code(weight, "matvec_argmax"), weight.stride(0), x.data_ptr(), _code(x, "matvec_argmax"),
            logits.data_ptr() if logits is not None else None, key_code,
            rows, cols, partials.data_ptr(), partials.numel(), self._argmax_out_idx.data_ptr(),
            self._argmax_out_val.data_ptr(), _stream(x),
        )
        _lib.check(rc, "matvec_argmax")
        return self._argmax_out_idx

    def matvec_argmax_tensor(
        self,
        weight: torch.Tensor,
        x: torch.Tensor,
        *,
        block_m: int | None = None,
        num_warps: int | None = None,
        config_name: str | None = None,
    ) -> torch.Tensor:
        """Greedy lm_head: first index of the maximum logit rounded to x's dtype
        (triton_kernels.py:5365-5398).  Logits are also written to ``logits_buffer``.
        Returns a 0-d int64 device tensor that later calls overwrite.  With
        ``argmax_mode="triton_two_stage"`` it takes the two-stage path instead, as the
        reference does (:5381-5382)."""
        if self.argmax_mode == "triton_two_stage":
            return self._matvec_argmax_tensor_triton_two_stage(weight, x)
        logits = self.logits_buffer(int(weight.shape[0]), x.dtype)
        return self._matvec_argmax(weight, x, logits)

    def _matvec_argmax_tensor_triton_two_stage(self, weight: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
        """Two-stage greedy lm_head (triton_kernels.py:5564-5625, kernels :2222-2285 and
        :2456-2473): first index of the maximum of the *unrounded* binary32 logits; no
        logits are stored.  At a tie of rounded logits it can pick a different token
        than ``matvec_argmax_tensor``, exactly as the reference's modes differ."""
        return self._matvec_argmax(weight, x, None, unrounded=True)

    def persistent_vocab_block_matvec_argmax_tensor(self, weight: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
        """Persistent vocab-block mode (triton_kernels.py:5516-5562, kernel :2477-2558):
        the same unrounded binary32 argmax as the two-stage mode."""
        return self._matvec_argmax(weight, x, None, unrounded=True)

    def matvec_argmax(self, weight: torch.Tensor, x: torch.Tensor) -> int:
        raise RuntimeError("matvec_argmax() synchronizes CUDA; use matvec_argmax_tensor()")

    # ------------------------------------------------------------ norms / elementwise
    def rms_norm(self, x: torch.Tensor, weight: torch.Tensor, out: torch.Tensor, eps: float,
                 weight_offset: float = 0.0) -> torch.Tensor:
        """(triton_kernels.py:5632-5644)"""
        _require_cuda(x, weight, out)
        n = x.numel()
        if weight.numel() != n or out.numel() != n:
            raise ValueError("rms_norm size mismatch")
        rc = self.lib.tt_rms_norm(x.data_ptr(), _code(x, "rms_norm"), weight.data_ptr(), _code(weight, "rms_norm"),
                                  out.data_ptr(), _code(out, "rms_norm"), n, float(eps), float(weight_offset), _stream(x))
        _lib.check(rc, "rms_norm")
        return out

    def add_then_rms_norm_rows(self, left: torch.Tensor, right: torch.Tensor, sum_out: torch.Tensor,
                               weight: torch.Tensor, out: torch.Tensor, eps: float) -> torch.Tensor:
        """Rows [B, n]: sum_out = left + right, out = rms_norm(sum_out) * weight, each row
        bit-identical to add followed by rms_norm (triton_kernels.py:5862-5873, 5632-5644)."""
        _require_cuda(left, right, sum_out, weight, out)
        if left.ndim != 2 or any(t.shape != left.shape for t in (right, sum_out, out)):
            raise ValueError("add_then_rms_norm_rows: [B, n] tensors of one shape")
        if right.dtype != left.dtype or sum_out.dtype != left.dtype or weight.numel() != left.shape[1]:
            raise ValueError("add_then_rms_norm_rows: dtype or weight size mismatch")
        if any(t.stride(1) != 1 or t.stride(0) != left.stride(0) for t in (right, sum_out)) or out.stride(1) != 1:
            raise ValueError("add_then_rms_norm_rows: rows must be contiguous with one row stride")
        rows, n = int(left.shape[0]), int(left.shape[1])
        rc = self.lib.tt_add_then_rms_norm_rows(left.data_ptr(), right.data_ptr(), sum_out.data_ptr(),
                                                _code(left, "add_then_rms_norm_rows"), left.stride(0),
                                                weight.data_ptr(), _code(weight, "add_then_rms_norm_rows"),
                                                out.data_ptr(), _code(out, "add_then_rms_norm_rows"), out.stride(0),
                                                rows, n, float(eps), _stream(left))
        _lib.check(rc, "add_then_rms_norm_rows")
        return out

    def add_rms_norm(self, left: torch.Tensor, right: torch.Tensor, residual_out: torch.Tensor, weight: torch.Tensor,
                     norm_out: torch.Tensor, eps: float) -> tuple[torch.Tensor, torch.Tensor]:
        """(triton_kernels.py:5646-5667)"""
        _require_cuda(left, right, residual_out, weight, norm_out)
        n = left.numel()
        if any(t.numel() != n for t in (right, residual_out, weight, norm_out)):
            raise ValueError("add_rms_norm size mismatch")
        if right.dtype != left.dtype or residual_out.dtype != left.dtype:
            raise ValueError("add_rms_norm: left, right and residual_out must share a dtype")
        rc = self.lib.tt_add_rms_norm(left.data_ptr(), right.data_ptr(), residual_out.data_ptr(), _code(left, "add_rms_norm"),
                                      weight.data_ptr(), _code(weight, "add_rms_norm"), norm_out.data_ptr(),
                                      _code(norm_out, "add_rms_norm"), n, float(eps), _stream(left))
        _lib.check(rc, "add_rms_norm")
        return residual_out, norm_out

    def add(self, left: torch.Tensor, right: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
        _require_cuda(left, right, out)
        rc = self.lib.tt_add(left.data_ptr(), right.data_ptr(), out.data_ptr(), _code(out, "add"), left.numel(), _stream(out))
        _lib.check(rc, "add")
        return out

    def silu_mul(self, gate: torch.Tensor, up: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
        _require_cuda(gate, up, out)
        rc = self.lib.tt_silu_mul(gate.data_ptr(), up.data_ptr(), out.data_ptr(), _code(out, "silu_mul"), gate.numel(),
                                  _stream(out))
        _lib.check(rc, "silu_mul")
        return out

    def interleaved_swiglu(self, gate_up: torch.Tensor, out: torch.Tensor, *, alpha: float, limit: float) -> torch.Tensor:
        """gpt-oss SwiGLU on interleaved gate/up (triton_kernels.py:5764-5782)."""
        _require_cuda(gate_up, out)
        rows = int(gate_up.shape[0]) if gate_up.ndim == 2 else 1
        n = int(out.shape[-1])
        in_row = gate_up.stride(0) if gate_up.ndim == 2 else 0
        out_row = out.stride(0) if out.ndim == 2 else 0
        rc = self.lib.tt_interleaved_swiglu(gate_up.data_ptr(), in_row, out.data_ptr(), out_row, _code(out, "swiglu"),
                                            rows, n, float(alpha), float(limit), _stream(out))
        _lib.check(rc, "interleaved_swiglu")
        return out

    def weighted_expert_sum(self, experts: torch.Tensor, scores: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
        """(triton_kernels.py:5784-5801)"""
        _require_cuda(experts, scores, out)
        rc = self.lib.tt_weighted_expert_sum(experts.data_ptr(), _code(experts, "weighted_expert_sum"), experts.stride(0),
                                             int(experts.shape[0]), scores.data_ptr(), _code(scores, "scores"),
                                             out.data_ptr(), int(experts.shape[1]), _stream(out))
        _lib.check(rc, "weighted_expert_sum")
        return out

    def rope_qk_inplace(self, q: torch.Tensor, k: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, heads: int,
                        kv_heads: int, head_dim: int, *, position: torch.Tensor | int | None = None) -> tuple[torch.Tensor, torch.Tensor]:
        """RoPE in place (triton_kernels.py:5689-5714).  ``cos``/``sin`` are either the
        row for the current token ([head_dim/2]) or a full table [positions,
        head_dim/2] indexed by ``position`` (an int or a 0-d int32 device tensor)."""
        if head_dim % 2:
            raise ValueError(f"RoPE head_dim must be even, got {head_dim}")
        _require_cuda(q, k, cos, sin)
        if cos.ndim == 1:
            table_row, table_rows, pos_dev, pos = 0, 1, None, 0
        else:
            table_row, table_rows = cos.stride(0), int(cos.shape[0])
            if isinstance(position, torch.Tensor):
                if position.dtype != torch.int32:
                    raise ValueError("device position must be int32")
                pos_dev, pos = position.data_ptr(), 0
            else:
                pos_dev, pos = None, int(position or 0)
        rc = self.lib.tt_rope_qk_inplace(q.data_ptr(), k.data_ptr(), _code(q, "rope"), cos.data_ptr(), sin.data_ptr(),
                                         table_row, table_rows, pos_dev, pos, heads, kv_heads, head_dim, _stream(q))
        _lib.check(rc, "rope_qk_inplace")
        return q, k

    def head_rms_norm(self, x: torch.Tensor, weight: torch.Tensor, out: torch.Tensor, heads: int, head_dim: int,
                      eps: float) -> torch.Tensor:
        """Per-head RMSNorm (triton_kernels.py:5669-5687, kernel :2618-2634)."""
        _require_cuda(x, weight, out)
        if x.numel() < heads * head_dim or out.numel() < heads * head_dim or weight.numel() < head_dim:
            raise ValueError("head_rms_norm size mismatch")
        if not (x.is_contiguous() and out.is_contiguous() and weight.is_contiguous()):
            raise ValueError("head_rms_norm tensors must be contiguous")
        rc = self.lib.tt_head_rms_norm(x.data_ptr(), _code(x, "head_rms_norm"), weight.data_ptr(),
                                       _code(weight, "head_rms_norm"), out.data_ptr(), heads, head_dim, float(eps),
                                       _stream(x))
        _lib.check(rc, "head_rms_norm")
        return out

    def qk_head_rmsnorm_rope_inplace(self, q: torch.Tensor, k: torch.Tensor, q_weight: torch.Tensor,
                                     k_weight: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, heads: int,
                                     kv_heads: int, head_dim: int, eps: float, *,
                                     position: torch.Tensor | int | None = None) -> tuple[torch.Tensor, torch.Tensor]:
        """Per-head RMSNorm of q and k followed by RoPE, in place (triton_kernels.py:
        5716-5749, kernel :2691-2757).  ``cos``/``sin`` are the current row or a table
        indexed by ``position``, as in ``rope_qk_inplace``."""
        if head_dim % 2:
            raise ValueError(f"RoPE head_dim must be even, got {head_dim}")
        if q_weight.numel() != head_dim or k_weight.numel() != head_dim:
            raise ValueError("fused Q/K RMSNorm requires one weight per head channel")
        if q_weight.dtype != k_weight.dtype:
            raise ValueError("fused Q/K RMSNorm weights must share a dtype")
        _require_cuda(q, k, q_weight, k_weight, cos, sin)
        if cos.ndim == 1:
            table_row, table_rows, pos_dev, pos = 0, 1, None, 0
        else:
            table_row, table_rows = cos.stride(0), int(cos.shape[0])
            if isinstance(position, torch.Tensor):
                if position.dtype != torch.int32:
                    raise ValueError("device position must be int32")
                pos_dev, pos = position.data_ptr(), 0
            else:
                pos_dev, pos = None, int(position or 0)
        rc = self.lib.tt_qk_head_rmsnorm_rope_inplace(
            q.data_ptr(), k.data_ptr(), _code(q, "qk_head_rmsnorm_rope_inplace"), q_weight.data_ptr(),
            k_weight.data_ptr(), _code(q_weight, "qk norm weights"), cos.data_ptr(), sin.data_ptr(), table_row,
            table_rows, pos_dev, pos, heads, kv_heads, head_dim, float(eps), _stream(q),
        )
        _lib.check(rc, "qk_head_rmsnorm_rope_inplace")
        return q, k

    # ------------------------------------------------------------ attention
    def _attention_scratch(self, heads: int, max_tokens: int, head_dim: int) -> torch.Tensor:
        need = int(self.lib.tt_attention_scratch_floats(heads, max_tokens, head_dim))
        if self._attention_partials is None or self._attention_partials.numel() < need:
            # arrival counters at the head (zero-filled once; every call leaves them at zero)
            self._attention_partials = torch.zeros(need, device=self.device, dtype=torch.float32)
        return self._attention_partials

    @staticmethod
    def _check_attention_operands(query, keys, values, out, heads: int, kv_heads: int, head_dim: int,
                                  out_values: int) -> None:
        """Operand checks of the attention kernels, which read the query in the cache
        dtype and write their output in it: the reference leaves these to Triton's
        pointer arithmetic, here a short query or KV tensor would be read past its end,
        so the shapes are checked before anything is launched."""
        if keys.ndim != 3 or values.ndim != 3:
            raise ValueError("keys and values must be [kv_heads, capacity, head_dim]")
        if query.dtype != keys.dtype or values.dtype != keys.dtype or out.dtype != keys.dtype:
            raise ValueError("query, keys, values and out must share the cache dtype")
        if not query.is_contiguous() or int(query.numel()) != heads * head_dim:
            raise ValueError(f"query must be a contiguous tensor of heads * head_dim = {heads * head_dim} values")
        if int(keys.shape[0]) < kv_heads or int(values.shape[0]) < kv_heads:
            raise ValueError(f"keys and values must hold {kv_heads} KV heads")
        if int(values.shape[1]) != int(keys.shape[1]):
            raise ValueError("keys and values must have the same capacity")
        if int(keys.shape[2]) < head_dim or int(values.shape[2]) < head_dim:
            raise ValueError(f"keys and values must hold head_dim = {head_dim} values per token")
        if keys.stride(2) != 1 or values.stride(2) != 1:
            raise ValueError("keys and values must be contiguous along head_dim")
        if not out.is_contiguous() or int(out.numel()) < out_values:
            raise ValueError(f"out must be a contiguous tensor of at least {out_values} values")

    def single_token_gqa_attention(
        self,
        query: torch.Tensor,
        keys: torch.Tensor,
        values: torch.Tensor,
        out: torch.Tensor,
        heads: int,
        kv_heads: int,
        head_dim: int,
        sinks: torch.Tensor | None = None,
        active_tokens: torch.Tensor | int | None = None,
    ) -> torch.Tensor:
        """Decode attention over keys/values [kv_heads, tokens, head_dim]
        (triton_kernels.py:5228-5278).  ``active_tokens`` may be an int, an int32
        device scalar holding the count, or ``(position_tensor, 1)`` meaning
        position + 1 read on the device; the KV tensors give the capacity."""
        capacity = int(keys.shape[1])
        offset = 0
        tokens = capacity if active_tokens is None else active_tokens
        if isinstance(tokens, tuple):
            tokens, offset = tokens
        if isinstance(tokens, int) and tokens <= 0:
            raise ValueError("attention requires at least one KV token")
        if head_dim > 256:
            raise ValueError("fused single-token attention supports head_dim <= 256")
        _require_cuda(query, keys, values, out)
        self._check_attention_operands(query, keys, values, out, heads, kv_heads, head_dim, heads * head_dim)
        scratch = self._attention_scratch(heads, capacity, head_dim)
        if isinstance(tokens, torch.Tensor):
            if tokens.dtype != torch.int32:
                raise ValueError("active_tokens device tensor must be int32")
            tok_dev, tok = tokens.data_ptr(), int(offset)
        else:
            tok_dev, tok = None, int(tokens)
        rc = self.lib.tt_single_token_gqa_attention(
            query.data_ptr(), keys.data_ptr(), values.data_ptr(), _code(keys, "attention"), keys.stride(0), keys.stride(1),
            values.stride(0), values.stride(1), sinks.data_ptr() if sinks is not None else None,
            _code(sinks, "sinks") if sinks is not None else _lib.F16, tok_dev, tok, capacity, heads, kv_heads, head_dim,
            scratch.data_ptr(), scratch.numel(), out.data_ptr(), _stream(out),
        )
        _lib.check(rc, "single_token_gqa_attention")
        return out

    def attention_then_int4_matvec(
        self,
        query: torch.Tensor,
        keys: torch.Tensor,
        values: torch.Tensor,
        heads: int,
        kv_heads: int,
        head_dim: int,
        packed_weight: torch.Tensor,
        scales: torch.Tensor,
        out: torch.Tensor,
        active_tokens: torch.Tensor | int | tuple | None = None,
        attn_out: torch.Tensor | None = None,
    ) -> torch.Tensor:
        """Decode attention followed by the int4 (group 128, fp16 scales) o_proj GEMV
        (triton_kernels.py:5228-5278, then the o_proj matvec of gpu_runtime.py's layer
        loop) in two launches: the attention kernel stores its chunk partials only, and the
        GEMV combines them into its activation (the bits ``single_token_gqa_attention``
        writes) before the product.  ``attn_out``, when given, receives that activation.
        Head_dim-64 caches, at most 32 query heads, no sinks."""
        capacity = int(keys.shape[1])
        offset = 0
        tokens = capacity if active_tokens is None else active_tokens
        if isinstance(tokens, tuple):
            tokens, offset = tokens
        if isinstance(tokens, int) and tokens <= 0:
            raise ValueError("attention requires at least one KV token")
        _require_cuda(query, keys, values, packed_weight, scales, out)
        rows, cols = int(out.shape[-1]), heads * head_dim
        if int(packed_weight.shape[0]) != rows or packed_weight.shape[1] * packed_weight.element_size() * 2 != cols:
            raise ValueError(f"int4 packed weight {tuple(packed_weight.shape)} does not match rows={rows} cols={cols}")
        if scales.dtype != torch.float16 or tuple(scales.shape) != (rows, cols // 128):
            raise ValueError("o_proj scales must be fp16 [rows, cols / 128]")
        if packed_weight.stride(1) != 1 or not out.is_contiguous() or not query.is_contiguous():
            raise ValueError("o_proj weight rows, query and out must be contiguous")
        self._check_attention_operands(query, keys, values, out, heads, kv_heads, head_dim, rows)
        if attn_out is not None:
            _require_cuda(attn_out)
            if attn_out.dtype != keys.dtype or attn_out.numel() != cols or not attn_out.is_contiguous():
                raise ValueError("attn_out must hold heads * head_dim values of the cache dtype")
        scratch = self._attention_scratch(heads, capacity, head_dim)
        if isinstance(tokens, torch.Tensor):
            if tokens.dtype != torch.int32:
                raise ValueError("active_tokens device tensor must be int32")
            tok_dev, tok = tokens.data_ptr(), int(offset)
        else:
            tok_dev, tok = None, int(tokens)
        code = _code(keys, "attention")
        rc = self.lib.tt_single_token_gqa_attention_partials(
            query.data_ptr(), keys.data_ptr(), values.data_ptr(), code, keys.stride(0), keys.stride(1),
            values.stride(0), values.stride(1), tok_dev, tok, capacity, heads, kv_heads, head_dim,
            scratch.data_ptr(), scratch.numel(), _stream(out),
        )
        _lib.check(rc, "single_token_gqa_attention_partials")
        rc = self.lib.tt_attention_combine_int4_matvec(
            scratch.data_ptr(), scratch.numel(), tok_dev, tok, capacity, heads, head_dim, code,
            packed_weight.data_ptr(), packed_weight.stride(0) * packed_weight.element_size(), scales.data_ptr(),
            scales.stride(0), scales.stride(1), attn_out.data_ptr() if attn_out is not None else None,
            out.data_ptr(), rows, _stream(out),
        )
        _lib.check(rc, "attention_combine_int4_matvec")
        return out

    def split_single_token_gqa_attention(self, query, keys, values, out, heads, kv_heads, head_dim):
        """Split-KV attention (triton_kernels.py:5280-5363): the HIP kernel always splits
        the sequence into 64-token chunks."""
        return self.single_token_gqa_attention(query, keys, values, out, heads, kv_heads, head_dim)

    # ------------------------------------------------------------ router
    def moe_router_matvec_topk(
        self,
        weight: torch.Tensor,
        hidden: torch.Tensor,
        indices_out: torch.Tensor,
        scores_out: torch.Tensor,
        *,
        bias: torch.Tensor | None = None,
        renormalize: bool,
    ) -> tuple[torch.Tensor, torch.Tensor]:
        """(triton_kernels.py:5826-5860)"""
        experts, hidden_size = map(int, weight.shape)
        if hidden.ndim != 1 or int(hidden.numel()) != hidden_size:
            raise ValueError("router hidden vector does not match weight shape")
        if experts > 128:
            raise ValueError("fused router supports at most 128 experts")
        if bias is not None and int(bias.numel()) != experts:
            raise ValueError("router bias does not match expert count")
        self._check_router_indices(indices_out)
        _require_cuda(weight, hidden, indices_out, scores_out)
        rc = self.lib.tt_moe_router_matvec_topk(
            weight.data_ptr(), _code(weight, "router"), weight.stride(0), hidden.data_ptr(), _code(hidden, "router"),
            hidden_size, bias.data_ptr() if bias is not None else None, _code(bias, "bias") if bias is not None else _lib.F32,
            experts, int(indices_out.numel()), int(bool(renormalize)), indices_out.data_ptr(), scores_out.data_ptr(),
            _code(scores_out, "scores"), _stream(hidden),
        )
        _lib.check(rc, "moe_router_matvec_topk")
        return indices_out, scores_out

    def add_rms_norm_router_topk(
        self,
        left: torch.Tensor,
        right: torch.Tensor,
        residual_out: torch.Tensor,
        norm_weight: torch.Tensor,
        norm_out: torch.Tensor,
        eps: float,
        router_weight: torch.Tensor,
        indices_out: torch.Tensor,
        scores_out: torch.Tensor,
        *,
        bias: torch.Tensor | None = None,
        renormalize: bool,
        split: bool = True,
    ) -> tuple[torch.Tensor, torch.Tensor]:
        """``add_rms_norm`` then ``moe_router_matvec_topk`` on its output, as one launch
        where the shapes allow (<= 32 experts, hidden <= 4096, one activation dtype).

        No single reference operator: the reference's MoE layer calls add_rms_norm
        (triton_kernels.py:5646-5667) and moe_router_matvec_topk (:5826-5860) back to
        back (gpu_runtime.py:9465-9513).  Outputs and bits equal that pair's.  The vectors
        may hold several tokens ([tokens, hidden]; indices/scores [tokens, top_k]).
        ``split`` spreads each token's router rows over ceil(experts / 4) workgroups
        (a zeroed workspace kept by the backend); otherwise one workgroup per token."""
        experts, hidden_size = map(int, router_weight.shape)
        n = hidden_size
        tokens = int(left.numel()) // n if n else 0
        if tokens < 1 or any(t.numel() != tokens * n for t in (left, right, residual_out, norm_out)) or \
                int(norm_weight.numel()) != n:
            raise ValueError("add_rms_norm_router_topk: vectors must be [tokens, hidden] matching the router weight")
        if any(not t.is_contiguous() for t in (left, right, residual_out, norm_out, scores_out)):
            raise ValueError("add_rms_norm_router_topk: vectors must be contiguous")
        if right.dtype != left.dtype or residual_out.dtype != left.dtype:
            raise ValueError("add_rms_norm: left, right and residual_out must share a dtype")
        if int(indices_out.numel()) % tokens or int(scores_out.numel()) != int(indices_out.numel()):
            raise ValueError("add_rms_norm_router_topk: indices/scores must be [tokens, top_k]")
        if experts > 128:
            raise ValueError("fused router supports at most 128 experts")
        if bias is not None and int(bias.numel()) != experts:
            raise ValueError("router bias does not match expert count")
        self._check_router_indices(indices_out)
        _require_cuda(left, right, residual_out, norm_weight, norm_out, router_weight, indices_out, scores_out)
        ws = None
        if split:
            need = int(self.lib.tt_norm_router_workspace_bytes(tokens))
            ws = self._zeroed_workspace("_norm_router_ws", need)
        rc = self.lib.tt_add_rms_norm_router_topk(
            left.data_ptr(), right.data_ptr(), residual_out.data_ptr(), _code(left, "add_rms_norm"),
            norm_weight.data_ptr(), _code(norm_weight, "add_rms_norm"), norm_out.data_ptr(),
            _code(norm_out, "add_rms_norm"), n, float(eps), router_weight.data_ptr(), _code(router_weight, "router"),
            router_weight.stride(0), bias.data_ptr() if bias is not None else None,
            _code(bias, "bias") if bias is not None else _lib.F32, experts, int(indices_out.numel()) // tokens,
            int(bool(renormalize)), indices_out.data_ptr(), scores_out.data_ptr(), _code(scores_out, "scores"),
            tokens, ws.data_ptr() if ws is not None else None, ws.numel() if ws is not None else 0, _stream(left),
        )
        _lib.check(rc, "add_rms_norm_router_topk")
        return indices_out, scores_out

    def add_rms_norm_router_logits(self, left: torch.Tensor, right: torch.Tensor, residual_out: torch.Tensor,
                                   norm_weight: torch.Tensor, norm_out: torch.Tensor, eps: float,
                                   router_weight: torch.Tensor, logits_out: torch.Tensor, *,
                                   bias: torch.Tensor | None = None) -> torch.Tensor:
        """``add_rms_norm_router_topk`` without the top-k: the same residual and norm
        outputs, and logits_out [tokens, experts] fp32 holding the logits that operator
        ranks.  ``mxfp_lowbit_selected_swiglu_router`` takes the top-k from them.  No
        single reference operator (the pair at gpu_runtime.py:9465-9513)."""
        experts, n = map(int, router_weight.shape)
        tokens = int(left.numel()) // n if n else 0
        if tokens < 1 or any(t.numel() != tokens * n for t in (left, right, residual_out, norm_out)) or \
                int(norm_weight.numel()) != n:
            raise ValueError("add_rms_norm_router_logits: vectors must be [tokens, hidden] matching the router weight")
        if any(not t.is_contiguous() for t in (left, right, residual_out, norm_out, logits_out)):
            raise ValueError("add_rms_norm_router_logits: vectors must be contiguous")
        if right.dtype != left.dtype or residual_out.dtype != left.dtype:
            raise ValueError("add_rms_norm: left, right and residual_out must share a dtype")
        if logits_out.dtype != torch.float32 or int(logits_out.numel()) != tokens * experts:
            raise ValueError("add_rms_norm_router_logits: logits_out must be float32 [tokens, experts]")
        if bias is not None and int(bias.numel()) != experts:
            raise ValueError("router bias does not match expert count")
        _require_cuda(left, right, residual_out, norm_weight, norm_out, router_weight, logits_out)
        rc = self.lib.tt_add_rms_norm_router_logits(
            left.data_ptr(), right.data_ptr(), residual_out.data_ptr(), _code(left, "add_rms_norm"),
            norm_weight.data_ptr(), _code(norm_weight, "add_rms_norm"), norm_out.data_ptr(),
            _code(norm_out, "add_rms_norm"), n, float(eps), router_weight.data_ptr(), _code(router_weight, "router"),
            router_weight.stride(0), bias.data_ptr() if bias is not None else None,
            _code(bias, "bias") if bias is not None else _lib.F32, experts, logits_out.data_ptr(), tokens,
            _stream(left),
        )
        _lib.check(rc, "add_rms_norm_router_logits")
        return logits_out

    def mxfp_lowbit_selected_swiglu_router(self, packed_weight: torch.Tensor, scales: torch.Tensor, x: torch.Tensor,
                                           router_logits: torch.Tensor, indices_out: torch.Tensor,
                                           scores_out: torch.Tensor, out: torch.Tensor, *, bits: int, alpha: float,
                                           limit: float, renormalize: bool,
                                           bias: torch.Tensor | None = None) -> torch.Tensor:
        """``moe_router_topk`` + ``mxfp_lowbit_selected_swiglu`` in one launch: x [T, cols]
        (or [cols]), router_logits [T, experts] float32, indices_out / scores_out
        [T, k]; out [T * k, I].  Every wave takes its slot's expert from its own top-k
        over the token's logits (the router's selection and scores, bit for bit) and the
        slots' experts and scores are written for the weighted-down.  Replaces the pair
        at gpu_runtime.py:9465-9513 (triton_kernels.py:5826-5860, 4178-4235)."""
        if bits not in {1, 2, 4} or packed_weight.ndim != 4 or scales.ndim != 3:
            raise ValueError("fused SwiGLU requires packed Q1, Q2 or MXFP4 experts")
        activation_rows = int(packed_weight.shape[1]) // 2
        cols = int(scales.shape[2] * 32)
        lg = router_logits if router_logits.ndim == 2 else router_logits.reshape(1, -1)
        tokens, experts = map(int, lg.shape)
        if lg.dtype != torch.float32 or not lg.is_contiguous():
            raise ValueError("router logits must be contiguous float32 [tokens, experts]")
        if indices_out.dtype != torch.int32 or int(indices_out.numel()) % tokens or \
                int(scores_out.numel()) != int(indices_out.numel()) or not indices_out.is_contiguous() or \
                not scores_out.is_contiguous():
            raise ValueError("indices/scores must be contiguous [tokens, top_k] (int32 indices)")
        selected = int(indices_out.numel()) // tokens
        xv = x if x.ndim == 2 else x.reshape(1, -1)
        if int(xv.shape[0]) != tokens or int(xv.shape[1]) != cols or xv.stride(1) != 1:
            raise ValueError("router SwiGLU takes x [T, cols]")
        if tuple(out.shape) != (tokens * selected, activation_rows):
            raise ValueError("router SwiGLU output shape mismatch")
        _require_cuda(packed_weight, scales, x, lg, indices_out, scores_out, out)
        rc = self.lib.tt_mxfp_lowbit_selected_swiglu_router(
            packed_weight.data_ptr(), packed_weight.stride(0), packed_weight.stride(1), scales.data_ptr(),
            scales.stride(0), scales.stride(1), bits, xv.data_ptr(), _code(xv, "swiglu"), xv.stride(0),
            lg.data_ptr(), experts, selected, int(bool(renormalize)), indices_out.data_ptr(), scores_out.data_ptr(),
            _code(scores_out, "scores"), bias.data_ptr() if bias is not None else None,
            _code(bias, "bias") if bias is not None else _lib.F32, bias.stride(0) if bias is not None else 0,
            float(alpha), float(limit), out.data_ptr(), _code(out, "swiglu"), out.stride(0), activation_rows, cols,
            tokens, _stream(out),
        )
        _lib.check(rc, "mxfp_lowbit_selected_swiglu_router")
        return out

    def moe_router_topk(self, logits: torch.Tensor, indices_out: torch.Tensor, scores_out: torch.Tensor, *,
                        renormalize: bool) -> tuple[torch.Tensor, torch.Tensor]:
        """(triton_kernels.py:5803-5824)"""
        self._check_router_indices(indices_out)
        _require_cuda(logits, indices_out, scores_out)
        rc = self.lib.tt_moe_router_topk(logits.data_ptr(), _code(logits, "logits"), int(logits.numel()),
                                         int(indices_out.numel()), int(bool(renormalize)), indices_out.data_ptr(),
                                         scores_out.data_ptr(), _code(scores_out, "scores"), _stream(logits))
        _lib.check(rc, "moe_router_topk")
        return indices_out, scores_out

    # ------------------------------------------------------------ batched small-M GEMM (no reference counterpart)
    def int4_batched_matvec(self, packed_weight: torch.Tensor, scales: torch.Tensor, x: torch.Tensor,
                            out: torch.Tensor, *, group_size: int = 128) -> torch.Tensor:
        """out[m] = dequant(W) x[m] for x fp16 [M, cols], out fp16 [M, rows]; int4 group-128
        weights with fp16 scales.  M < 4 is bit-identical to int4_scaled_matvec per row;
        M >= 4 uses MFMA (tolerance parity)."""
        _require_cuda(packed_weight, scales, x, out)
        if x.ndim != 2 or out.ndim != 2 or x.shape[0] != out.shape[0]:
            raise ValueError("batched matvec takes x [M, cols] and out [M, rows]")
        if scales.dtype != torch.float16 or x.dtype != torch.float16 or out.dtype != torch.float16:
            raise ValueError("batched int4 matvec takes fp16 scales, activations and outputs")
        rows, cols = int(packed_weight.shape[0]), int(x.shape[1])
        if packed_weight.shape[1] * packed_weight.element_size() * 2 != cols or out.shape[1] != rows:
            raise ValueError("batched int4 matvec shape mismatch")
        ws = self._batched_workspace(int(x.shape[0]), rows, cols)
        rc = self.lib.tt_int4_batched_matvec(
            packed_weight.data_ptr(), packed_weight.stride(0) * packed_weight.element_size(), scales.data_ptr(),
            scales.stride(0), x.data_ptr(), x.stride(0), out.data_ptr(), out.stride(0), int(x.shape[0]), rows, cols,
            group_size, ws.data_ptr() if ws is not None else None, ws.numel() if ws is not None else 0, _stream(out))
        _lib.check(rc, "int4_batched_matvec")
        return out

    def scaled_batched_matvec(self, weight: torch.Tensor, scales: torch.Tensor, x: torch.Tensor,
                              out: torch.Tensor) -> torch.Tensor:
        """out[m] = (W x[m]) * s for fp8-e4m3 W [rows, cols] and fp32 s [rows]."""
        _require_cuda(weight, scales, x, out)
        if x.ndim != 2 or out.ndim != 2 or x.shape[0] != out.shape[0] or scales.dtype != torch.float32:
            raise ValueError("batched scaled matvec takes x [M, cols], out [M, rows] and fp32 scales")
        if x.dtype != torch.float16 or out.dtype != torch.float16:
            raise ValueError("batched scaled matvec takes fp16 activations and outputs")
        rows, cols = int(weight.shape[0]), int(weight.shape[1])
        ws = self._batched_workspace(int(x.shape[0]), rows, cols)
        rc = self.lib.tt_scaled_batched_matvec(
            weight.data_ptr(), weight.stride(0) * weight.element_size(), scales.data_ptr(), x.data_ptr(), x.stride(0),
            out.data_ptr(), out.stride(0), int(x.shape[0]), rows, cols, ws.data_ptr() if ws is not None else None,
            ws.numel() if ws is not None else 0, _stream(out))
        _lib.check(rc, "scaled_batched_matvec")
        return out

    def _batched_workspace(self, m: int, rows: int, cols: int) -> torch.Tensor | None:
        """Workspace of the MFMA path (fp32 partial tiles of row blocks shared
        between workgroups), reused between calls on this backend's stream."""
        need = int(self.lib.tt_batched_workspace_floats(m, rows, cols))
        if need == 0:
            return None
        ws = getattr(self, "_batched_ws", None)
        if ws is None or ws.numel() < need:
            ws = torch.empty(need, device=self.device, dtype=torch.float32)
            self._batched_ws = ws
        return ws

    def _batched_argmax_scratch(self, m: int, rows: int, cols: int) -> torch.Tensor:
        need = int(self.lib.tt_matvec_argmax_batched_partials(m, rows, cols))
        if self._batched_partials is None or self._batched_partials.numel() < need:
            self._batched_partials = torch.empty(need, device=self.device, dtype=torch.int64)
        return self._batched_partials

    def matvec_argmax_batched(self, weight: torch.Tensor, x: torch.Tensor,
                              logits: torch.Tensor | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
        """Greedy lm_head for x [M, cols]: int64 [M] tokens (first index of each row's
        maximum rounded logit), written to ``out`` when given (a new tensor otherwise).
        The partials scratch is reused between calls."""
        _require_cuda(weight, x)
        m, rows, cols = int(x.shape[0]), int(weight.shape[0]), int(weight.shape[1])
        if x.ndim != 2 or x.shape[1] != cols or weight.dtype != torch.float16 or x.dtype != torch.float16:
            raise ValueError("batched matvec_argmax takes fp16 W [rows, cols] and x [M, cols]")
        if out is not None and (out.dtype != torch.int64 or out.numel() != m or not out.is_contiguous()):
            raise ValueError("batched matvec_argmax: out must be a contiguous int64 tensor of M tokens")
        partials = self._batched_argmax_scratch(m, rows, cols)
        need = int(partials.numel())
        idx = out if out is not None else torch.empty(m, device=self.device, dtype=torch.int64)
        rc = self.lib.tt_matvec_argmax_batched(
            weight.data_ptr(), weight.stride(0), x.data_ptr(), x.stride(0), m,
            logits.data_ptr() if logits is not None else None, logits.stride(0) if logits is not None else 0, rows,
            cols, partials.data_ptr(), need, idx.data_ptr(), None, _stream(x))
        _lib.check(rc, "matvec_argmax_batched")
        return idx

    # ------------------------------------------------------------ fused decode-step GEMVs (no reference counterpart)
    def fused_gemv(self, desc: "_lib.FusedGemv") -> None:
        """One GEMV launch with its decode-step neighbours folded in (RMSNorm prologue,
        RoPE / KV-cache / SiLU epilogues); see tt_fused_gemv_run.  The outputs equal the
        unfused operator sequence bit for bit."""
        rc = self.lib.tt_fused_gemv_run(ctypes.byref(desc), torch.cuda.current_stream(self.device).cuda_stream)
        _lib.check(rc, "fused_gemv")

    def fused_lm_head_argmax(self, desc: "_lib.FusedGemv", *, position: torch.Tensor | None = None,
                             base: torch.Tensor | None = None, history: torch.Tensor | None = None) -> torch.Tensor:
        """Greedy lm_head with a fused prologue; with ``position`` the finishing kernel
        also logs the token at history[position - base] and advances the position.
        Returns the reused 0-d int64 token tensor."""
        rows = int(desc.seg[0].rows)
        partials = self._argmax_scratch(rows, int(desc.cols))
        rc = self.lib.tt_fused_lm_head_argmax(
            ctypes.byref(desc), partials.data_ptr(), partials.numel(), self._argmax_out_idx.data_ptr(),
            self._argmax_out_val.data_ptr(), position.data_ptr() if position is not None else None,
            base.data_ptr() if base is not None else None, history.data_ptr() if history is not None else None,
            int(history.numel()) if history is not None else 0, torch.cuda.current_stream(self.device).cuda_stream,
        )
        _lib.check(rc, "fused_lm_head_argmax")
        return self._argmax_out_idx

    # ------------------------------------------------------------ decode-step helpers (no reference counterpart)
    def embedding(self, embed: torch.Tensor, token: torch.Tensor | int, out: torch.Tensor) -> torch.Tensor:
        """out = embed[token]; a device token (0-d/1-element int64) is read on the GPU."""
        _require_cuda(embed, out)
        if isinstance(token, torch.Tensor):
            if token.dtype != torch.int64:
                raise ValueError("device token id must be int64")
            tok_dev, tok = token.data_ptr(), 0
        else:
            tok_dev, tok = None, int(token)
        rc = self.lib.tt_embedding(embed.data_ptr(), embed.stride(0), int(embed.shape[0]), tok_dev, tok, out.data_ptr(),
                                   out.numel(), _stream(out))
        _lib.check(rc, "embedding")
        return out

    def kv_append(self, k: torch.Tensor, v: torch.Tensor, keys: torch.Tensor, values: torch.Tensor,
                  position: torch.Tensor | int, kv_heads: int, head_dim: int) -> None:
        """keys/values [kv_heads, capacity, head_dim]: write token `position`."""
        _require_cuda(k, v, keys, values)
        if keys.stride() != values.stride():
            raise ValueError("keys and values must share a layout")
        if isinstance(position, torch.Tensor):
            pos_dev, pos = position.data_ptr(), 0
        else:
            pos_dev, pos = None, int(position)
        rc = self.lib.tt_kv_append(k.data_ptr(), v.data_ptr(), keys.data_ptr(), values.data_ptr(), keys.stride(0),
                                   keys.stride(1), pos_dev, pos, int(keys.shape[1]), kv_heads, head_dim, _stream(k))
        _lib.check(rc, "kv_append")

    def advance_position(self, position: torch.Tensor, step: int = 1) -> None:
        rc = self.lib.tt_advance_position(position.data_ptr(), int(step), _stream(position))
        _lib.check(rc, "advance_position")

    def record_token(self, token: torch.Tensor, position: torch.Tensor, base: torch.Tensor, history: torch.Tensor) -> None:
        """history[position - base] = token, all on the device (int64 / int32 / int32)."""
        rc = self.lib.tt_record_token(token.data_ptr(), position.data_ptr(), base.data_ptr(), history.data_ptr(),
                                      int(history.numel()), _stream(token))
        _lib.check(rc, "record_token")

    def record_tokens_advance(self, tokens: torch.Tensor, position: torch.Tensor, base: torch.Tensor,
                              history: torch.Tensor, step: int = 1) -> None:
        """history[r, position - base] = tokens[r] for every row, then position += step
        (record_token per row + advance_position in one launch)."""
        if tokens.dtype != torch.int64 or history.dtype != torch.int64 or history.ndim != 2:
            raise ValueError("record_tokens_advance: int64 tokens [B] and history [B, T]")
        if tokens.numel() != history.shape[0] or not tokens.is_contiguous() or history.stride(1) != 1:
            raise ValueError("record_tokens_advance: one token per history row, contiguous rows")
        rc = self.lib.tt_record_tokens_advance(tokens.data_ptr(), int(tokens.numel()), position.data_ptr(),
                                               base.data_ptr(), history.data_ptr(), history.stride(0),
                                               int(history.shape[1]), int(step), _stream(tokens))
        _lib.check(rc, "record_tokens_advance")

    def multi_matvec_bias(self, weights: tuple[torch.Tensor, ...], biases: tuple[torch.Tensor | None, ...],
                          x: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
        """multi_matvec followed by the per-matrix bias add, fused (same rounding as
        GEMV-then-add_ in the runtime, gpu_runtime.py:9100-9114)."""
        cols = int(weights[0].shape[1])
        rows = [int(w.shape[0]) for w in weights]
        _require_cuda(x, out, *weights)
        rc = self.lib.tt_multi_matvec_bias(
            len(weights), _lib.ptr_array([w.data_ptr() for w in weights]), _code(weights[0], "multi_matvec"),
            _lib.i64_array([w.stride(0) for w in weights]), _lib.i64_array(rows),
            _lib.ptr_array([b.data_ptr() if b is not None else None for b in biases]), x.data_ptr(),
            _code(x, "multi_matvec"), out.data_ptr(), _code(out, "multi_matvec"), cols, _stream(out),
        )
        _lib.check(rc, "multi_matvec_bias")
        return out
