"""Write the load-time quantizer golden vectors (tests/golden/quant_vectors.npz).

Runs in the build container only (the reference tree is not on the GPU box): it
imports the reference's pure-torch quantizers from /root/reference and records
small seeded inputs together with the reference outputs.  The committed .npz holds
data only; the GPU tests compare the HIP quantizers against it.

Functions recorded (reference thinruntime/gpu_runtime.py):
  quantize_to_fp8_via_gpu            :40-88     (called with device=cpu)
  quantize_to_int4_cpu               :91-304    (symmetric LSQ, affine refinement, importance,
                                                  GPTQ passes with a calibration covariance)
  quantize_mxfp4_to_lowbit_cpu       :306-395
  quantize_dense_to_mxfp_lowbit_cpu  :398-491
  quantize_mxfp4_to_ternary_cpu      :494-583
  ThinGpuCausalLMRuntime._quantize_fp8_rows   :6551-6607
  ThinGpuCausalLMRuntime._quantize_int4_rows  :6609-6700
  ThinGpuCausalLMRuntime._quantize_mxfp4_rows :6702-6812

Usage: python tests/golden/make_quant_vectors.py [/root/reference]
"""

from __future__ import annotations

import os
import zlib
import sys
from pathlib import Path

import numpy as np
import torch

OUT = Path(__file__).resolve().parent / "quant_vectors.npz"


def _source(seed: int, rows: int, cols: int, dtype=torch.bfloat16) -> torch.Tensor:
    """Seeded weights with the edge cases the quantizers branch on: an all-zero row,
    a row with one large outlier, signed zeros and a row of tiny values."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(rows, cols, generator=g) * 0.05
    x[0] = 0.0
    x[1, 7] = 3.0
    x[2, ::3] = -0.0
    x[3] = x[3] * 1e-6
    if rows > 5:
        x[5, : cols // 2] = 0.0
    return x.to(dtype)


def _mxfp4(seed: int, experts: int, rows: int, groups: int) -> tuple[torch.Tensor, torch.Tensor]:
    g = torch.Generator().manual_seed(seed)
    blocks = torch.randint(0, 256, (experts, rows, groups, 16), generator=g, dtype=torch.int64).to(torch.uint8)
    scales = torch.randint(110, 135, (experts, rows, groups), generator=g, dtype=torch.int64).to(torch.uint8)
    blocks[0, 0, 0] = 0          # all-zero group
    blocks[0, 0, 1] = 0x88       # all -0
    scales[0, 1, 0] = 0          # smallest exponent (clamps)
    scales[0, 1, 1] = 254
    return blocks, scales


def _bits(t: torch.Tensor) -> np.ndarray:
    if t.dtype in (torch.bfloat16, torch.float16):
        return t.view(torch.int16).numpy().astype(np.uint16)
    if t.dtype == torch.float8_e4m3fn:
        return t.view(torch.uint8).numpy()
    return t.numpy()


def main(ref_root: str) -> None:
    sys.path.insert(0, ref_root)
    import thinruntime.gpu_runtime as gr  # noqa: E402  (reference, read for vectors only)

    rt = gr.ThinGpuCausalLMRuntime
    vec: dict[str, np.ndarray] = {}

    def put(name: str, **arrays) -> None:
        for k, v in arrays.items():
            vec[f"{name}.{k}"] = _bits(v) if isinstance(v, torch.Tensor) else np.asarray(v)

    os.environ["THINTENSOR_AFFINE_INT4"] = "0"
    # grouped INT4, fp16 scales, one least-squares refinement (:237-253), clamp [-8, 7]
    for name, (rows, cols, gs) in {"int4_lsq": (16, 512, 128), "int4_lsq_ragged": (12, 320, 128),
                                   "int4_lsq_g32": (8, 256, 32)}.items():
        src = _source(zlib.crc32(name.encode()) & 0xFFFF, rows, cols)
        packed, scales = gr.quantize_to_int4_cpu(src, group_size=gs)
        put(name, source=src, packed=packed, scales=scales, group_size=gs)
    # body INT4 rows, fp32 scales, clamp [-7, 7] (:6680-6692)
    for name, (rows, cols, gs) in {"int4_rows": (16, 512, 128), "int4_rows_ragged": (12, 320, 128)}.items():
        src = _source(zlib.crc32(name.encode()) & 0xFFFF, rows, cols)
        packed, scales = rt._quantize_int4_rows(src, group_size=gs)
        put(name, source=src, packed=packed, scales=scales, group_size=gs)

    os.environ["THINTENSOR_AFFINE_INT4"] = "1"
    src = _source(11, 16, 512)
    packed, scales = gr.quantize_to_int4_cpu(src, group_size=128)
    put("int4_affine", source=src, packed=packed, scales=scales, group_size=128)
    g = torch.Generator().manual_seed(12)
    rms = (torch.rand(512, generator=g) * 2.0 + 0.05)
    packed, scales = gr.quantize_to_int4_cpu(src, group_size=128, input_rms=rms)
    put("int4_affine_rms", source=src, packed=packed, scales=scales, group_size=128, input_rms=rms)
    src = _source(13, 12, 384)
    packed, scales = rt._quantize_int4_rows(src, group_size=128)
    put("int4_rows_affine", source=src, packed=packed, scales=scales, group_size=128)
    # GPTQ passes (:130-150, :217-262): groups of 32, covariance of correlated calibration
    # activations (neighbouring columns mixed so the factors have large off-diagonals)
    src = _source(14, 12, 256)
    g = torch.Generator().manual_seed(15)
    calib = torch.randn(512, 256, generator=g)
    calib = (calib + 0.6 * torch.roll(calib, 1, dims=1)) * (torch.rand(256, generator=g) * 2.0 + 0.1)
    blocks = calib.reshape(512, 8, 32).permute(1, 2, 0)           # [groups, 32, samples]
    cov = (blocks @ blocks.transpose(1, 2)) / 512.0
    packed, scales = gr.quantize_to_int4_cpu(src, group_size=32, input_covariance32=cov)
    put("int4_affine_gptq", source=src, packed=packed, scales=scales, group_size=32, covariance=cov)
    rms = (torch.rand(256, generator=g) * 2.0 + 0.05)
    packed, scales = gr.quantize_to_int4_cpu(src, group_size=32, input_rms=rms, input_covariance32=cov)
    put("int4_affine_gptq_rms", source=src, packed=packed, scales=scales, group_size=32, covariance=cov,
        input_rms=rms)
    os.environ["THINTENSOR_AFFINE_INT4"] = "0"
    # the symmetric fit computes the factors but does not use them
    packed, scales = gr.quantize_to_int4_cpu(src, group_size=32, input_covariance32=cov)
    put("int4_lsq_gptq_unused", source=src, packed=packed, scales=scales, group_size=32, covariance=cov)

    # FP8 rows: per-row and per-block scales, direct fp32 -> e4m3 (:6551-6607)
    for name, (rows, cols, blk, dt) in {"fp8_rows": (16, 512, 0, torch.bfloat16),
                                        "fp8_rows_f16": (8, 256, 0, torch.float16),
                                        "fp8_block": (16, 512, 128, torch.bfloat16),
                                        "fp8_block_ragged": (8, 300, 128, torch.bfloat16)}.items():
        src = _source(zlib.crc32(name.encode()) & 0xFFFF, rows, cols, dt)
        q, s = rt._quantize_fp8_rows(src, scale_block_size=blk)
        put(name, source=src, quantized=q, scales=s, block=blk)
    # the via-GPU variant rounds through bf16 before e4m3 (:69-82); run on the CPU device
    for name, blk in {"fp8_via_bf16": 0, "fp8_via_bf16_block": 128}.items():
        src = _source(zlib.crc32(name.encode()) & 0xFFFF, 16, 512)
        q, s = gr.quantize_to_fp8_via_gpu(src, device=torch.device("cpu"), scale_block_size=blk)
        put(name, source=src, quantized=q, scales=s, block=blk)

    # native MXFP4 rows: plain, Hadamard-32, Hadamard-64 with signs, binary residual (:6702-6812)
    src = _source(21, 16, 256)
    g = torch.Generator().manual_seed(22)
    signs = torch.where(torch.rand(256, generator=g) < 0.5, -1.0, 1.0).to(torch.bfloat16)
    for name, kw in {"mxfp4_rows": {}, "mxfp4_rows_h32": {"hadamard": True},
                     "mxfp4_rows_h64s": {"hadamard_size": 64, "signs": signs},
                     "mxfp4_rows_resid": {"binary_residual": True}}.items():
        packed, scales = rt._quantize_mxfp4_rows(src, **kw)
        put(name, source=src, packed=packed, scales=scales, signs=signs)

    # MXFP4 -> Q2 / Q1 E8M0 groups (:306-395) and MXFP4 -> ternary (:494-583)
    blocks, scales = _mxfp4(31, 2, 8, 4)
    for bits in (2, 1):
        out, out_scales = gr.quantize_mxfp4_to_lowbit_cpu(blocks, scales, bits=bits)
        put(f"lowbit_q{bits}", blocks=blocks, scales=scales, packed=out, out_scales=out_scales)
    out, out_scales = gr.quantize_mxfp4_to_ternary_cpu(blocks, scales)
    put("ternary", blocks=blocks, scales=scales, packed=out, out_scales=out_scales)

    # dense -> Q2 / Q1 E8M0 groups with MSE exponent choice (:398-491)
    src = _source(41, 16, 256)
    for bits in (2, 1):
        out, out_scales = gr.quantize_dense_to_mxfp_lowbit_cpu(src, bits=bits)
        put(f"dense_q{bits}", source=src, packed=out, out_scales=out_scales)

    np.savez_compressed(OUT, **vec)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(vec)} arrays)")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
