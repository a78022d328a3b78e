"""Load-time quantizers on the GPU, under the reference's names and signatures.

Each function mirrors one reference quantizer (thinruntime/gpu_runtime.py, lines in
the docstrings): same arguments, same validation messages, same output layouts and
dtypes.  The work runs in the HIP kernels of ``csrc/quantize.hip`` (through the C ABI);
the ``*_cpu`` names keep the reference's contract of returning CPU tensors for CPU
inputs (device inputs give device outputs).  ``chunk_rows`` arguments are accepted
for signature compatibility: the kernels need no row chunking, every group is one
wave (or half-wave) with no temporaries.

Group sums are taken in binary64 in a fixed lane order and rounded once to binary32,
so codes and scales agree with the reference's binary32 torch sums except at
near-ties that the reference's own (CPU-vector-width dependent) order decides.
"""

from __future__ import annotations

import os

import torch

from . import _lib

_SRC_CODE = {torch.float16: _lib.F16, torch.bfloat16: _lib.BF16, torch.float32: _lib.F32}


def _device_of(t: torch.Tensor, device: torch.device | None = None) -> torch.device:
    if device is not None and torch.device(device).type == "cuda":
        return torch.device(device)
    if t.device.type == "cuda":
        return t.device
    if not torch.cuda.is_available():
        raise RuntimeError("the HIP quantizers need a GPU (torch.cuda.is_available() is False)")
    return torch.device("cuda", torch.cuda.current_device())


def _on_device(t: torch.Tensor, dev: torch.device, dtype: torch.dtype | None = None) -> torch.Tensor:
    """Contiguous device copy; float sources other than fp16/bf16/fp32 become fp32."""
    if dtype is None and t.dtype not in _SRC_CODE:
        dtype = torch.float32
    return t.to(device=dev, dtype=dtype or t.dtype).contiguous()


def _stream(dev: torch.device) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


def _back(t: torch.Tensor, like: torch.Tensor) -> torch.Tensor:
    return t if like.device.type == "cuda" else t.cpu()


# ----------------------------------------------------------------------------------- FP8
def quantize_to_fp8_via_gpu(
    source_cpu: torch.Tensor,
    device: torch.device = torch.device("cuda"),
    scale_block_size: int = 0,
) -> tuple[torch.Tensor, torch.Tensor]:
    """gpu_runtime.py:40-88: bfloat16 source, fp32 scales max(amax, 1e-12)/448 per row
    (or per block of columns), x/scale rounded to bfloat16 then to float8_e4m3fn.
    Returns CPU tensors."""
    dev = _device_of(source_cpu, device)
    src = source_cpu.to(device=dev, dtype=torch.bfloat16).contiguous()
    q, s = _fp8(src, int(scale_block_size), via_bf16=True)
    return q.cpu(), s.cpu()


def quantize_fp8_rows(
    source: torch.Tensor,
    chunk_rows: int = 256,
    scale_block_size: int = 0,
) -> tuple[torch.Tensor, torch.Tensor]:
    """ThinGpuCausalLMRuntime._quantize_fp8_rows (gpu_runtime.py:6551-6607): float8_e4m3fn
    rows and fp32 scales, on the source's device."""
    if source.dtype == torch.float8_e4m3fn:
        raise RuntimeError("FP8 head is already resident but its row scales are unavailable")
    dev = _device_of(source)
    q, s = _fp8(_on_device(source, dev), int(scale_block_size), via_bf16=False)
    return _back(q, source), _back(s, source)


def _fp8(src: torch.Tensor, block: int, via_bf16: bool) -> tuple[torch.Tensor, torch.Tensor]:
    rows, cols = int(src.shape[0]), int(src.shape[1])
    nb = (cols + block - 1) // block if block > 0 else 1
    q = torch.empty((rows, cols), device=src.device, dtype=torch.float8_e4m3fn)
    s = torch.empty((rows, nb) if block > 0 else (rows,), device=src.device, dtype=torch.float32)
    rc = _lib.load().tt_quantize_fp8_rows(src.data_ptr(), _SRC_CODE[src.dtype], rows, cols, cols, block,
                                          1 if via_bf16 else 0, q.data_ptr(), s.data_ptr(), _stream(src.device))
    _lib.check(rc, "quantize_fp8_rows")
    return q, s


# ---------------------------------------------------------------------------------- INT4
def quantize_to_int4_cpu(
    source: torch.Tensor,
    *,
    group_size: int = 128,
    chunk_rows: int = 256,
    input_rms: torch.Tensor | None = None,
    input_covariance32: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """gpu_runtime.py:91-304: grouped INT4 with fp16 scales.  Symmetric: amax/7, codes
    in [-8, 7], one least-squares refit of the scale.  With THINTENSOR_AFFINE_INT4=1
    (and rows < 65536): a min/max line refitted by (importance-weighted) least squares,
    codes in [0, 15], [scale, minimum] pairs; with ``input_covariance32`` (groups of 32)
    two GPTQ passes then requantize each group column by column (:217-262)."""
    rows, cols = int(source.shape[0]), int(source.shape[1])
    if cols % 2:
        raise ValueError("expert INT4 requires an even input width")
    if group_size <= 0 or group_size & (group_size - 1):
        raise ValueError("expert INT4 group size must be a positive power of two")
    groups = (cols + group_size - 1) // group_size
    affine = os.environ.get("THINTENSOR_AFFINE_INT4", "0") == "1" and rows < 65536
    dev = _device_of(source)
    importance = None
    if input_rms is not None:
        if tuple(input_rms.shape) != (cols,):
            raise ValueError(
                f"INT4 input RMS shape {tuple(input_rms.shape)} does not match the projection width {(cols,)}"
            )
        importance = input_rms.to(device=dev).float().square().clamp_min_(1e-8).contiguous()
    factors = None
    if input_covariance32 is not None:
        if group_size != 32:
            raise ValueError("GPTQ covariance blocks currently require INT4 group size 32")
        if tuple(input_covariance32.shape) != (groups, 32, 32):
            raise ValueError(
                f"INT4 covariance shape {tuple(input_covariance32.shape)} does not match {(groups, 32, 32)}"
            )
        factors = gptq_inverse_cholesky(input_covariance32).to(device=dev).contiguous()
    if affine and cols % group_size:
        raise ValueError("affine INT4 needs the input width to be a multiple of the group size")
    mode = _lib.Q4_LSQ_AFFINE if affine else _lib.Q4_LSQ
    # the reference computes the factors in both modes and uses them in the affine fit only
    packed, scales = _int4(_on_device(source, dev), group_size, groups, mode,
                           importance if affine else None, torch.float16, factors if affine else None)
    return _back(packed, source), _back(scales, source)


def gptq_inverse_cholesky(input_covariance32: torch.Tensor) -> torch.Tensor:
    """Per 32-column group the upper Cholesky factor of the inverse of the damped input
    covariance, in binary32 on the host as the reference computes it
    (gpu_runtime.py:130-150): H = cov + max(mean(diag H) * p, 1e-6) I with p =
    THINTENSOR_GPTQ_DAMP_PERCENT (default 0.01), U = cholesky(inv(H), upper=True).
    A [groups, 32, 32] set of 32 x 32 factorizations: set-up for the GPU passes, which
    read U."""
    hessian = input_covariance32.detach().to(device="cpu", dtype=torch.float32).clone()
    damp_percent = float(os.environ.get("THINTENSOR_GPTQ_DAMP_PERCENT", "0.01"))
    if damp_percent <= 0:
        raise ValueError("THINTENSOR_GPTQ_DAMP_PERCENT must be positive")
    damp = hessian.diagonal(dim1=1, dim2=2).mean(dim=1).mul(damp_percent).clamp_min_(1e-6)
    hessian.diagonal(dim1=1, dim2=2).add_(damp[:, None])
    return torch.linalg.cholesky(torch.linalg.inv(hessian), upper=True)


def quantize_int4_rows(
    source: torch.Tensor,
    *,
    group_size: int,
    chunk_rows: int = 256,
) -> tuple[torch.Tensor, torch.Tensor]:
    """ThinGpuCausalLMRuntime._quantize_int4_rows (gpu_runtime.py:6609-6700): codes
    round(x/scale) in [-7, 7] (+8) with fp32 scales amax/7, or with
    THINTENSOR_AFFINE_INT4=1 (rows < 65536) the min/max line with [scale, minimum]."""
    rows, cols = int(source.shape[0]), int(source.shape[1])
    if cols % 2:
        raise ValueError("body INT4 requires an even input width")
    groups = (cols + group_size - 1) // group_size
    affine = os.environ.get("THINTENSOR_AFFINE_INT4", "0") == "1" and rows < 65536
    dev = _device_of(source)
    mode = _lib.Q4_ROWS_AFFINE if affine else _lib.Q4_ROWS
    packed, scales = _int4(_on_device(source, dev), group_size, groups, mode, None, torch.float32)
    return _back(packed, source), _back(scales, source)


def _int4(src, group_size, groups, mode, importance, scale_dtype, factors=None):
    rows, cols = int(src.shape[0]), int(src.shape[1])
    if group_size not in (32, 64, 128, 256, 512):
        raise ValueError(f"INT4 group size {group_size} is not supported by the HIP quantizer (32..512, powers of two)")
    packed = torch.empty((rows, cols // 2), device=src.device, dtype=torch.uint8)
    pair = mode in (_lib.Q4_LSQ_AFFINE, _lib.Q4_ROWS_AFFINE)
    scales = torch.empty((rows, groups, 2) if pair else (rows, groups), device=src.device, dtype=scale_dtype)
    rc = _lib.load().tt_quantize_int4(src.data_ptr(), _SRC_CODE[src.dtype], rows, cols, cols, group_size, mode,
                                      importance.data_ptr() if importance is not None else None,
                                      factors.data_ptr() if factors is not None else None, packed.data_ptr(),
                                      scales.data_ptr(), _stream(src.device))
    _lib.check(rc, "quantize_int4")
    return packed, scales


# --------------------------------------------------------------------------------- MXFP4
def quantize_mxfp4_rows(
    source: torch.Tensor,
    *,
    chunk_rows: int = 256,
    hadamard: bool = False,
    hadamard_size: int = 0,
    signs: torch.Tensor | None = None,
    binary_residual: bool = False,
) -> tuple[torch.Tensor, torch.Tensor]:
    """ThinGpuCausalLMRuntime._quantize_mxfp4_rows (gpu_runtime.py:6702-6812): packed
    E2M1 nibbles [rows, cols/2] and E8M0 scales [rows, cols/32]; the exponent of each
    group is the better of ceil(log2(amax/6)) - 1 and ceil(log2(amax/6)) by squared
    error, optionally after a blockwise Walsh-Hadamard transform with sign flips."""
    rows, cols = int(source.shape[0]), int(source.shape[1])
    if cols % 32:
        raise ValueError("native MXFP4 requires a K dimension divisible by 32")
    transform = int(hadamard_size) or (32 if hadamard else 0)
    if transform and cols % transform:
        raise ValueError(f"Hadamard block size {transform} does not divide {cols}")
    dev = _device_of(source)
    src = _on_device(source, dev)
    sg = None
    if signs is not None and transform:
        sg = signs.to(device=dev, dtype=src.dtype).contiguous()
    packed = torch.empty((rows, cols // 2), device=dev, dtype=torch.uint8)
    scales = torch.empty((rows, cols // 32), device=dev, dtype=torch.uint8)
    rc = _lib.load().tt_quantize_mxfp4_rows(src.data_ptr(), _SRC_CODE[src.dtype], rows, cols, cols, transform,
                                            sg.data_ptr() if sg is not None else None, 1 if binary_residual else 0,
                                            packed.data_ptr(), scales.data_ptr(), _stream(dev))
    _lib.check(rc, "quantize_mxfp4_rows")
    return _back(packed, source), _back(scales, source)


def _check_mxfp4(blocks: torch.Tensor, scales: torch.Tensor) -> None:
    if blocks.ndim != 4 or scales.ndim != 3:
        raise ValueError("packed MXFP4 blocks/scales must be rank 4/rank 3")
    if tuple(blocks.shape[:3]) != tuple(scales.shape) or blocks.shape[3] != 16:
        raise ValueError(f"packed MXFP4 blocks/scales mismatch: {blocks.shape} vs {scales.shape}")


def quantize_mxfp4_to_lowbit_cpu(
    blocks: torch.Tensor,
    scales: torch.Tensor,
    *,
    bits: int,
    chunk_rows: int = 256,
) -> tuple[torch.Tensor, torch.Tensor]:
    """gpu_runtime.py:306-395: packed MXFP4 groups to Q2 ({+-0.5, +-1.5} * 2^d) or Q1
    (+-2^d) E8M0 groups, d in -2..3 chosen by mean squared error."""
    if bits not in {1, 2}:
        raise ValueError("packed MXFP4 expert precision must be Q1 or Q2")
    _check_mxfp4(blocks, scales)
    experts, rows, groups = map(int, scales.shape)
    bpg = 4 if bits == 1 else 8
    dev = _device_of(blocks)
    b = blocks.to(dev, torch.uint8).contiguous()
    s = scales.to(dev, torch.uint8).contiguous()
    out = torch.empty((experts, rows, groups, bpg), device=dev, dtype=torch.uint8)
    out_scales = torch.empty((experts, rows, groups), device=dev, dtype=torch.uint8)
    rc = _lib.load().tt_requantize_mxfp4_lowbit(b.data_ptr(), s.data_ptr(), experts * rows * groups, bits,
                                                out.data_ptr(), out_scales.data_ptr(), _stream(dev))
    _lib.check(rc, "quantize_mxfp4_to_lowbit")
    return _back(out, blocks), _back(out_scales, blocks)


def quantize_dense_to_mxfp_lowbit_cpu(
    source: torch.Tensor,
    *,
    bits: int,
    chunk_rows: int = 64,
    compute_device: torch.device | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """gpu_runtime.py:398-491: dense rank-2 weights to Q2/Q1 groups with E8M0 scales,
    the exponent floor(log2(amax/L)) + offset (offset -2..2) with the smallest mean
    squared error.  Returns CPU tensors, as the reference."""
    if bits not in {1, 2}:
        raise ValueError("dense low-bit precision must be Q1 or Q2")
    if source.ndim != 2:
        raise ValueError("dense low-bit source must be rank 2")
    rows, cols = map(int, source.shape)
    if cols % 32:
        raise ValueError("dense low-bit input width must be divisible by 32")
    if chunk_rows <= 0:
        raise ValueError("dense low-bit chunk_rows must be positive")
    dev = _device_of(source, compute_device)
    src = _on_device(source, dev)
    groups = cols // 32
    bpg = 4 if bits == 1 else 8
    out = torch.empty((rows, groups, bpg), device=dev, dtype=torch.uint8)
    out_scales = torch.empty((rows, groups), device=dev, dtype=torch.uint8)
    rc = _lib.load().tt_quantize_dense_lowbit(src.data_ptr(), _SRC_CODE[src.dtype], rows, cols, cols, bits,
                                              out.data_ptr(), out_scales.data_ptr(), _stream(dev))
    _lib.check(rc, "quantize_dense_to_mxfp_lowbit")
    return out.cpu(), out_scales.cpu()


def quantize_mxfp4_to_ternary_cpu(
    blocks: torch.Tensor,
    scales: torch.Tensor,
    *,
    chunk_rows: int = 256,
) -> tuple[torch.Tensor, torch.Tensor]:
    """gpu_runtime.py:494-583: MXFP4 to five base-3 digits per byte plus 3-bit magnitude
    selectors per 32-weight group (the selector of each group by mean squared error);
    the E8M0 scales are returned unchanged."""
    _check_mxfp4(blocks, scales)
    experts, rows, groups = map(int, scales.shape)
    cols = groups * 32
    width = (cols + 4) // 5 + (groups * 3 + 7) // 8
    dev = _device_of(blocks)
    b = blocks.to(dev, torch.uint8).contiguous()
    out = torch.empty((experts, rows, width), device=dev, dtype=torch.uint8)
    rc = _lib.load().tt_pack_mxfp4_ternary(b.data_ptr(), experts * rows, groups, out.data_ptr(), _stream(dev))
    _lib.check(rc, "quantize_mxfp4_to_ternary")
    return _back(out, blocks), scales
