// Load-time quantizers for gfx950: the packed weight layouts the decode kernels read,
// produced on the GPU from bf16/fp16/fp32 weights (or from packed MXFP4 experts).
//
// Semantics follow the reference's torch quantizers (thinruntime/gpu_runtime.py):
//   tt_quantize_int4             quantize_to_int4_cpu :91-304 (symmetric least-squares
//                                refinement; affine line fit with optional column
//                                importance and GPTQ passes) and _quantize_int4_rows
//                                :6609-6700
//   tt_quantize_fp8_rows         _quantize_fp8_rows :6551-6607, quantize_to_fp8_via_gpu :40-88
//   tt_quantize_mxfp4_rows       _quantize_mxfp4_rows :6702-6812 (Walsh-Hadamard blocks,
//                                sign flips, binary-residual error)
//   tt_requantize_mxfp4_lowbit   quantize_mxfp4_to_lowbit_cpu :306-395
//   tt_quantize_dense_lowbit     quantize_dense_to_mxfp_lowbit_cpu :398-491
//   tt_pack_mxfp4_ternary        quantize_mxfp4_to_ternary_cpu :494-583
//
// Arithmetic (restated in oracle/quant.py): every elementwise step is the reference's
// binary32 operation in its order (IEEE division, round-half-even rounding); every sum
// over a quantization group is taken in binary64 -- each lane adds its elements in
// index order from +0, then the lane partials are folded in halves (lane bit 32
// first for a 64-lane group, bit 16 first for a 32-lane MX group) -- and rounded once
// to binary32; ceil/floor of log2 come from the binary exponent.  One wave owns one
// quantization group (int4) or two 32-element MX groups (one per half-wave), so no
// group needs more than cross-lane moves.
#include <type_traits>

#include "tt_abi_internal.h"
#include "tt_common.h"

namespace tt {
namespace {

constexpr float kTiny = 1e-12f;

template <typename ST> __device__ __forceinline__ float src_at(const void* p, int64_t i) {
  return to_f32(reinterpret_cast<const ST*>(p)[i]);
}

template <int M> __device__ __forceinline__ double xor_partner_d(double v) {
  const uint64_t u = __builtin_bit_cast(uint64_t, v);
  const uint32_t lo = __builtin_bit_cast(uint32_t, xor_partner<M>(__builtin_bit_cast(float, (uint32_t)u)));
  const uint32_t hi = __builtin_bit_cast(uint32_t, xor_partner<M>(__builtin_bit_cast(float, (uint32_t)(u >> 32))));
  return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}

// Halving fold of the 64 lane partials (lanes l and l + 32 first), rounded once.
__device__ __forceinline__ float wave_sum64(double v) {
  v = v + xor_partner_d<32>(v);
  v = v + xor_partner_d<16>(v);
  v = v + xor_partner_d<8>(v);
  v = v + xor_partner_d<4>(v);
  v = v + xor_partner_d<2>(v);
  v = v + xor_partner_d<1>(v);
  return (float)v;
}

// The same fold inside each half-wave (lanes l and l + 16 of the half first).
__device__ __forceinline__ float half_sum32(double v) {
  v = v + xor_partner_d<16>(v);
  v = v + xor_partner_d<8>(v);
  v = v + xor_partner_d<4>(v);
  v = v + xor_partner_d<2>(v);
  v = v + xor_partner_d<1>(v);
  return (float)v;
}

__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, xor_partner<32>(v));
  v = fmaxf(v, xor_partner<16>(v));
  v = fmaxf(v, xor_partner<8>(v));
  v = fmaxf(v, xor_partner<4>(v));
  v = fmaxf(v, xor_partner<2>(v));
  return fmaxf(v, xor_partner<1>(v));
}
__device__ __forceinline__ float wave_min(float v) {
  v = fminf(v, xor_partner<32>(v));
  v = fminf(v, xor_partner<16>(v));
  v = fminf(v, xor_partner<8>(v));
  v = fminf(v, xor_partner<4>(v));
  v = fminf(v, xor_partner<2>(v));
  return fminf(v, xor_partner<1>(v));
}
__device__ __forceinline__ float half_max(float v) {
  v = fmaxf(v, xor_partner<16>(v));
  v = fmaxf(v, xor_partner<8>(v));
  v = fmaxf(v, xor_partner<4>(v));
  v = fmaxf(v, xor_partner<2>(v));
  return fmaxf(v, xor_partner<1>(v));
}

// floor(log2(v)) and ceil(log2(v)) of a positive finite binary32 value (normal or
// subnormal), exactly: from the binary64 exponent field.
__device__ __forceinline__ int floor_log2(float v) {
  const uint64_t u = __builtin_bit_cast(uint64_t, (double)v);
  return (int)((u >> 52) & 0x7ff) - 1023;
}
__device__ __forceinline__ int ceil_log2(float v) {
  const uint64_t u = __builtin_bit_cast(uint64_t, (double)v);
  const int e = (int)((u >> 52) & 0x7ff) - 1023;
  return (u & 0xfffffffffffffull) ? e + 1 : e;
}

__device__ __forceinline__ float clampf(float v, float lo, float hi) { return fminf(fmaxf(v, lo), hi); }

// E2M1 magnitude of code c in 0..7: 0, 0.5, 1, 1.5, 2, 3, 4, 6.
__device__ __forceinline__ float e2m1_mag(int c) {
  return c < 4 ? 0.5f * (float)c : (float)(1 << ((c >> 1) - 1)) * ((c & 1) ? 1.5f : 1.0f);
}

// binary32 -> float8_e4m3fn, round to nearest even on the e4m3 grid; magnitudes that
// round past 448, and NaN/inf, give the NaN pattern 0x7f.
__device__ __forceinline__ uint8_t f32_to_e4m3(float f) {
  const uint32_t bits = __builtin_bit_cast(uint32_t, f);
  const uint32_t sign = (bits >> 24) & 0x80u;
  const uint32_t u = bits & 0x7fffffffu;
  uint32_t code;
  if (u >= 0x43f00000u) {                 // >= 480, inf, NaN
    code = 0x7fu;
  } else if (u < 0x3c800000u) {           // below 2^-6: grid 2^-9 (f * 512 is exact here)
    code = (uint32_t)__builtin_rintf(__builtin_bit_cast(float, u) * 512.0f);
  } else {                                 // keep 3 mantissa bits, ties to even
    const uint32_t r = u + 0x7ffffu + ((u >> 20) & 1u);
    code = (r >> 20) - (120u << 3);        // exponent rebias 127 -> 7
  }
  return (uint8_t)(code | sign);
}

// ------------------------------------------------------------------------------ INT4
enum Q4Mode { kLsq = 0, kLsqAffine = 1, kRows = 2, kRowsAffine = 3 };

struct Q4Params {
  const void* src;
  int64_t src_row;       // elements between rows
  const float* importance;   // [cols] column weights (affine least squares) or null
  const float* gptq;     // [groups, 32, 32] upper Cholesky factors of the inverse Hessians, or null
  uint8_t* packed;       // [rows, cols / 2]
  void* scales;          // fp16 (LSQ modes) or fp32; [rows, groups] or [rows, groups, 2]
  int rows, cols, group, groups;
};

// One wave per (row, group).  Lane l holds elements [l * EPL, (l + 1) * EPL) of the
// group (EPL = G / 64), or element l for G = 32.
template <typename ST, int EPL, int MODE>
__global__ __launch_bounds__(256) void int4_quant_kernel(const Q4Params P) {
  const int lane = threadIdx.x & 63;
  const int64_t item = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (item >= (int64_t)P.rows * P.groups) return;
  const int row = (int)(item / P.groups);
  const int g = (int)(item % P.groups);
  const int in_group = lane * EPL;          // first element of this lane inside the group
  const int col0 = g * P.group + in_group;
  float x[EPL], w[EPL];
  bool pr[EPL];
#pragma unroll
  for (int k = 0; k < EPL; k++) {
    pr[k] = in_group + k < P.group && col0 + k < P.cols;
    x[k] = pr[k] ? src_at<ST>(P.src, (int64_t)row * P.src_row + col0 + k) : 0.0f;
    w[k] = (pr[k] && P.importance) ? P.importance[col0 + k] : 0.0f;
  }
  const bool weighted = P.importance != nullptr;
  float codes[EPL];
  float out_s = 0.0f, out_m = 0.0f;

  if constexpr (MODE == kLsq || MODE == kRows) {
    float amax = 0.0f;
#pragma unroll
    for (int k = 0; k < EPL; k++) amax = pr[k] ? fmaxf(amax, fabsf(x[k])) : amax;
    amax = wave_max(amax);
    const float s0 = fmaxf(amax, kTiny) / 7.0f;
    if constexpr (MODE == kRows) {
#pragma unroll
      for (int k = 0; k < EPL; k++) codes[k] = clampf(__builtin_rintf(x[k] / s0), -7.0f, 7.0f) + 8.0f;
      out_s = s0;
    } else {
      double pn = 0.0, pd = 0.0;
#pragma unroll
      for (int k = 0; k < EPL; k++) {
        const float q = clampf(__builtin_rintf(x[k] / s0), -8.0f, 7.0f);
        const float xq = x[k] * q, qq = q * q;
        if (pr[k]) {
          pn = pn + (double)xq;
          pd = pd + (double)qq;
        }
      }
      const float num = wave_sum64(pn);
      const float den = fmaxf(wave_sum64(pd), 1.0f);
      const float s = fmaxf(fabsf(num / den), kTiny);
#pragma unroll
      for (int k = 0; k < EPL; k++) codes[k] = clampf(__builtin_rintf(x[k] / s), -8.0f, 7.0f) + 8.0f;
      out_s = s;
    }
  } else {
    float mn = __builtin_inff(), mx = -__builtin_inff();
#pragma unroll
    for (int k = 0; k < EPL; k++) {
      mn = pr[k] ? fminf(mn, x[k]) : mn;
      mx = pr[k] ? fmaxf(mx, x[k]) : mx;
    }
    mn = wave_min(mn);
    mx = wave_max(mx);
    float s = fmaxf(mx - mn, kTiny) / 15.0f;
#pragma unroll
    for (int k = 0; k < EPL; k++) codes[k] = clampf(__builtin_rintf((x[k] - mn) / s), 0.0f, 15.0f);
    if constexpr (MODE == kLsqAffine) {
      // regression of the line on the assigned codes: two refits each followed by a
      // requantization, then a last refit of (scale, minimum)
      float wsum = 0.0f;
      if (weighted) {
        double pw = 0.0;
#pragma unroll
        for (int k = 0; k < EPL; k++) pw = pr[k] ? pw + (double)w[k] : pw;
        wsum = wave_sum64(pw);
      }
      // (scale, minimum) of the line regressed on the current codes
      auto fit = [&]() {
        double pq = 0.0, px = 0.0;
#pragma unroll
        for (int k = 0; k < EPL; k++) {
          const float tq = weighted ? codes[k] * w[k] : codes[k];
          const float tx = weighted ? x[k] * w[k] : x[k];
          if (pr[k]) {
            pq = pq + (double)tq;
            px = px + (double)tx;
          }
        }
        const float div = weighted ? wsum : (float)P.group;
        const float q_mean = wave_sum64(pq) / div;
        const float x_mean = wave_sum64(px) / div;
        double pn = 0.0, pd = 0.0;
#pragma unroll
        for (int k = 0; k < EPL; k++) {
          const float qc = codes[k] - q_mean;
          float t = (x[k] - x_mean) * qc;
          float d = qc * qc;
          if (weighted) {
            t = t * w[k];
            d = d * w[k];
          }
          if (pr[k]) {
            pn = pn + (double)t;
            pd = pd + (double)d;
          }
        }
        const float num = wave_sum64(pn);
        const float den = fmaxf(wave_sum64(pd), kTiny);
        s = fmaxf(num / den, kTiny);
        mn = x_mean - s * q_mean;
      };
      for (int it = 0; it < 3; it++) {
        fit();
        if (it < 2) {
#pragma unroll
          for (int k = 0; k < EPL; k++) codes[k] = clampf(__builtin_rintf((x[k] - mn) / s), 0.0f, 15.0f);
        }
      }
      if constexpr (EPL == 1) {
        if (P.gptq != nullptr) {
          // GPTQ passes over the 32 columns of the group (gpu_runtime.py:217-262): column
          // c is quantized on the current line, and its error divided by U[c][c] is taken
          // out of columns c.. through row c of U.  Lane j < 32 owns column j and keeps
          // column j of U; the line is refitted after the first pass only.
          const float* U = P.gptq + (int64_t)g * 1024;
          const int j = lane & 31;
          float ucol[32];
#pragma unroll
          for (int c = 0; c < 32; c++) ucol[c] = U[c * 32 + j];
          for (int pass = 0; pass < 2; pass++) {
            float adj = x[0];
            float code = 0.0f;
#pragma unroll
            for (int c = 0; c < 32; c++) {
              const float cur = __builtin_bit_cast(
                  float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, adj), c));
              const float cq = clampf(__builtin_rintf((cur - mn) / s), 0.0f, 15.0f);
              const float qv = cq * s + mn;   // product and sum rounded separately (no contraction)
              const float err = (cur - qv) / U[c * 33];
              code = lane == c ? cq : code;
              adj = lane > c ? adj - err * ucol[c] : adj;
            }
            codes[0] = code;
            if (pass == 0) fit();
          }
        }
      }
    }
    out_s = s;
    out_m = mn;
  }

  // codes -> nibbles (element 2j low, 2j + 1 high)
  uint8_t* prow = P.packed + (int64_t)row * (P.cols / 2);
  if constexpr (EPL >= 2) {
#pragma unroll
    for (int j = 0; j < EPL / 2; j++)
      if (pr[2 * j]) prow[(col0 >> 1) + j] = (uint8_t)((int)codes[2 * j] | ((int)codes[2 * j + 1] << 4));
  } else {
    const int c = (int)codes[0];
    const int partner = __builtin_amdgcn_mov_dpp(c, 0xB1, 0xF, 0xF, false);   // lane ^ 1
    if (pr[0] && (lane & 1) == 0) prow[col0 >> 1] = (uint8_t)(c | (partner << 4));
  }
  if (lane == 0) {
    const int64_t si = (int64_t)row * P.groups + g;
    if constexpr (MODE == kLsq) {
      reinterpret_cast<uint16_t*>(P.scales)[si] = f32_to_f16_bits(out_s);
    } else if constexpr (MODE == kLsqAffine) {
      reinterpret_cast<uint16_t*>(P.scales)[2 * si] = f32_to_f16_bits(out_s);
      reinterpret_cast<uint16_t*>(P.scales)[2 * si + 1] = f32_to_f16_bits(out_m);
    } else if constexpr (MODE == kRows) {
      reinterpret_cast<float*>(P.scales)[si] = out_s;
    } else {
      reinterpret_cast<float*>(P.scales)[2 * si] = out_s;
      reinterpret_cast<float*>(P.scales)[2 * si + 1] = out_m;
    }
  }
}

// ------------------------------------------------------------------------------- FP8
struct Fp8Params {
  const void* src;
  int64_t src_row;
  uint8_t* out;        // [rows, cols] e4m3fn
  float* scales;       // [rows, nblocks]
  int rows, cols, block, nblocks;
};

// One 256-thread workgroup per (row, column block).
template <typename ST, bool VIA_BF16>
__global__ __launch_bounds__(256) void fp8_quant_kernel(const Fp8Params P) {
  __shared__ float red[4];
  const int row = blockIdx.x / P.nblocks;
  const int b = blockIdx.x % P.nblocks;
  const int c0 = b * P.block;
  const int c1 = min(P.cols, c0 + P.block);
  const int64_t base = (int64_t)row * P.src_row;
  auto load = [&](int c) {
    const float v = src_at<ST>(P.src, base + c);
    return VIA_BF16 ? round_bf16(v) : v;
  };
  float amax = 0.0f;
  for (int c = c0 + (int)threadIdx.x; c < c1; c += 256) amax = fmaxf(amax, fabsf(load(c)));
  amax = wave_max(amax);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const float s = fmaxf(amax, kTiny) / 448.0f;
  uint8_t* orow = P.out + (int64_t)row * P.cols;
  for (int c = c0 + (int)threadIdx.x; c < c1; c += 256) {
    float y = load(c) / s;
    if (VIA_BF16) y = round_bf16(y);
    orow[c] = f32_to_e4m3(y);
  }
  if (threadIdx.x == 0) P.scales[(int64_t)row * P.nblocks + b] = s;
}

// ------------------------------------------------------------------------------ MXFP4
struct MxParams {
  const void* src;
  int64_t src_row;
  const void* signs;     // [cols] +-1 (source dtype) or null
  uint8_t* packed;       // [rows, cols / 2]
  uint8_t* scales;       // [rows, cols / 32] E8M0
  int rows, cols, transform;   // transform: Walsh-Hadamard block (0: none)
  int span;              // elements per wave: max(transform, 64)
  float transform_scale; // binary32 transform^-0.5
  int binary_residual;
};

// One wave per (row, span of max(T, 64) elements): the span is staged in LDS (and
// transformed there), then each half-wave quantizes one 32-element group at a time.
template <typename ST>
__global__ __launch_bounds__(64) void mxfp4_quant_kernel(const MxParams P) {
  __shared__ float buf[512];
  const int lane = threadIdx.x;
  const int spans = P.cols / P.span;
  const int row = blockIdx.x / spans;
  const int col0 = (blockIdx.x % spans) * P.span;
  const int64_t base = (int64_t)row * P.src_row + col0;
  for (int i = lane; i < P.span; i += 64) {
    float v = src_at<ST>(P.src, base + i);
    if (P.signs) v = v * src_at<ST>(P.signs, col0 + i);
    buf[i] = v;
  }
  __syncthreads();
  if (P.transform) {
    const int T = P.transform;
    for (int s = 1; s < T; s *= 2) {
      for (int pidx = lane; pidx < P.span / 2; pidx += 64) {
        const int i = (pidx / s) * (2 * s) + pidx % s;   // left element of pair pidx
        const float l = buf[i], r = buf[i + s];
        buf[i] = l + r;
        buf[i + s] = l - r;
      }
      __syncthreads();
    }
    for (int i = lane; i < P.span; i += 64) buf[i] = buf[i] * P.transform_scale;
    __syncthreads();
  }
  const int half = lane >> 5;
  const int hl = lane & 31;
  for (int off = 0; off < P.span; off += 64) {
    const int gcol = col0 + off + 32 * half;    // first column of this half's group
    const float v = buf[off + lane];
    const float amax = half_max(fabsf(v));
    const int e0 = min(max(ceil_log2(fmaxf(amax, 0x1p-126f) / 6.0f), -127), 127);
    int best_e = 0, best_code = 0;
    float best_err = 0.0f;
#pragma unroll
    for (int bias = -1; bias <= 0; bias++) {
      const int e = min(max(e0 + bias, -127), 127);
      const float f = pow2i(e);
      const float nrm = v / f;
      const float m = fabsf(nrm);
      int code = (m >= 0.25f) + (m >= 0.75f) + (m >= 1.25f) + (m >= 1.75f) + (m >= 2.5f) + (m >= 3.5f) + (m >= 5.0f);
      code |= __builtin_signbitf(nrm) ? 8 : 0;
      const float rec = (e2m1_mag(code & 7) * ((code & 8) ? -1.0f : 1.0f)) * f;
      float res = v - rec;
      if (P.binary_residual) {
        const float mean = fmaxf(half_sum32((double)fabsf(res)) / 32.0f, 0x1p-126f);
        const int re = (int)min(max(rint(log2((double)mean)), -127.0), 127.0);
        const float rs = pow2i(re);
        res = res - (res >= 0.0f ? rs : -rs);
      }
      const float err = half_sum32((double)(res * res));
      if (bias == -1 || err < best_err) {
        best_err = err;
        best_e = e;
        best_code = code;
      }
    }
    const int partner = __builtin_amdgcn_mov_dpp(best_code, 0xB1, 0xF, 0xF, false);
    if ((hl & 1) == 0) P.packed[(int64_t)row * (P.cols / 2) + ((gcol + hl) >> 1)] = (uint8_t)(best_code | (partner << 4));
    if (hl == 0) P.scales[(int64_t)row * (P.cols / 32) + gcol / 32] = (uint8_t)(best_e + 127);
  }
}

// ------------------------------------------------------------- MXFP4 -> Q2/Q1 E8M0
// Signed E2M1 value of nibble l of a 16-byte MXFP4 group (code 8 is -0).
__device__ __forceinline__ float mx_value(const uint8_t* grp, int l, int* nib_out) {
  const uint8_t byte = grp[l >> 1];
  const int nib = (l & 1) ? (byte >> 4) : (byte & 15);
  *nib_out = nib;
  const float mag = e2m1_mag(nib & 7);
  return (nib & 8) ? -mag : mag;
}

// Write the 32 codes of each half-wave's group: Q2 four per byte (2 bits, element 4j
// lowest), Q1 eight per byte (bit b = element 8j + b).
// Every lane of the wave takes part in the cross-lane moves; only lanes with `write`
// store (dst is the half-wave group's first output byte).
__device__ __forceinline__ void store_lowbit(int code, int bits, uint8_t* dst, int hl, bool write) {
  if (bits == 2) {
    const int lane = (int)(threadIdx.x & 63);
    const int c1 = __builtin_amdgcn_ds_bpermute(4 * min(lane + 1, 63), code);
    const int c2 = __builtin_amdgcn_ds_bpermute(4 * min(lane + 2, 63), code);
    const int c3 = __builtin_amdgcn_ds_bpermute(4 * min(lane + 3, 63), code);
    if (write && (hl & 3) == 0) dst[hl >> 2] = (uint8_t)(code | (c1 << 2) | (c2 << 4) | (c3 << 6));
  } else {
    const uint64_t mask = __builtin_amdgcn_ballot_w64(code != 0);
    const uint32_t mine = (uint32_t)(mask >> (threadIdx.x & 32));
    if (write && hl < 4) dst[hl] = (uint8_t)(mine >> (8 * hl));
  }
}

// One half-wave per MXFP4 group (blocks [n, 16] bytes, scales [n]).
__global__ __launch_bounds__(256) void lowbit_requant_kernel(const uint8_t* __restrict__ blocks,
                                                             const uint8_t* __restrict__ scales, int64_t n, int bits,
                                                             uint8_t* __restrict__ out, uint8_t* __restrict__ out_scales) {
  const int64_t gid = ((int64_t)blockIdx.x * 256 + threadIdx.x) >> 5;
  const int hl = threadIdx.x & 31;
  const bool live = gid < n;
  const int64_t gc = live ? gid : n - 1;
  int nib;
  const float v = mx_value(blocks + gc * 16, hl, &nib);
  const bool neg = (nib & 8) != 0;
  int best_code = 0, best_d = -2;
  float best_err = 0.0f;
#pragma unroll
  for (int d = -2; d <= 3; d++) {
    const float f = pow2i(d);
    int code;
    float rec;
    if (bits == 2) {
      const bool outer = fabsf(v) >= f;
      code = neg ? (outer ? 0 : 1) : (outer ? 3 : 2);
      const float lv = code == 0 ? -1.5f : code == 1 ? -0.5f : code == 2 ? 0.5f : 1.5f;
      rec = lv * f;
    } else {
      code = neg ? 0 : 1;
      rec = neg ? -f : f;
    }
    const float dv = v - rec;
    const float err = half_sum32((double)(dv * dv)) / 32.0f;
    if (d == -2 || err < best_err) {
      best_err = err;
      best_code = code;
      best_d = d;
    }
  }
  const int bpg = bits == 2 ? 8 : 4;
  store_lowbit(best_code, bits, out + gc * bpg, hl, live);
  if (live && hl == 0) out_scales[gc] = (uint8_t)(min(max((int)scales[gc] - 127 + best_d, -127), 127) + 127);
}

// --------------------------------------------------------------- dense -> Q2/Q1 E8M0
template <typename ST>
__global__ __launch_bounds__(256) void dense_lowbit_kernel(const void* src, int64_t src_row, int rows, int cols,
                                                           int bits, uint8_t* __restrict__ out,
                                                           uint8_t* __restrict__ out_scales) {
  const int groups = cols / 32;
  const int64_t gid = ((int64_t)blockIdx.x * 256 + threadIdx.x) >> 5;
  const int hl = threadIdx.x & 31;
  const bool live = gid < (int64_t)rows * groups;
  const int64_t gc = live ? gid : (int64_t)rows * groups - 1;
  const int row = (int)(gc / groups), g = (int)(gc % groups);
  const float v = src_at<ST>(src, (int64_t)row * src_row + g * 32 + hl);
  const float amax = fmaxf(half_max(fabsf(v)), 0x1p-126f);
  const float level = bits == 2 ? 1.5f : 1.0f;
  const int base = floor_log2(amax / level);
  int best_code = 0, best_e = 0;
  float best_err = 0.0f;
#pragma unroll
  for (int off = -2; off <= 2; off++) {
    const int e = min(max(base + off, -127), 127);
    const float f = pow2i(e);
    const float nrm = v / f;
    int code;
    float rec;
    if (bits == 2) {
      const bool outer = fabsf(nrm) >= 1.0f;
      const bool neg = nrm < 0.0f;
      code = neg ? (outer ? 0 : 1) : (outer ? 3 : 2);
      rec = __builtin_copysignf(outer ? 1.5f : 0.5f, nrm) * f;
    } else {
      code = nrm >= 0.0f ? 1 : 0;
      rec = code ? f : -f;
    }
    const float dv = v - rec;
    const float err = half_sum32((double)(dv * dv)) / 32.0f;
    if (off == -2 || err < best_err) {
      best_err = err;
      best_code = code;
      best_e = e;
    }
  }
  const int bpg = bits == 2 ? 8 : 4;
  store_lowbit(best_code, bits, out + gc * bpg, hl, live);
  if (live && hl == 0) out_scales[gc] = (uint8_t)min(max(best_e + 127, 0), 254);
}

// ------------------------------------------------------------------ MXFP4 -> ternary
// One 256-thread workgroup per row of groups: digits (0: -a, 1: 0, 2: +a) and the
// magnitude index of each group go to LDS, then five digits per byte (3^k weights)
// and the 3-bit magnitude selectors, bit-packed, are written.
constexpr int kTernaryMaxCols = 16384;
__global__ __launch_bounds__(256) void ternary_pack_kernel(const uint8_t* __restrict__ blocks, int groups,
                                                           uint8_t* __restrict__ out) {
  __shared__ uint8_t digits[kTernaryMaxCols];
  __shared__ uint8_t mags[kTernaryMaxCols / 32];
  const int64_t row = blockIdx.x;
  const int cols = groups * 32;
  const int tb = (cols + 4) / 5;
  const int mb = (groups * 3 + 7) / 8;
  const int hl = threadIdx.x & 31;
  for (int g0 = 0; g0 < groups; g0 += 8) {
    const int g = g0 + (int)(threadIdx.x >> 5);
    const int gc = g < groups ? g : groups - 1;
    int nib;
    const float v = mx_value(blocks + (row * groups + gc) * 16, hl, &nib);
    int best_digit = 1, best_idx = 0;
    float best_err = 0.0f;
#pragma unroll
    for (int idx = 0; idx < 7; idx++) {
      const float mag = e2m1_mag(idx + 1);
      const int digit = fabsf(v) > mag * 0.5f ? (v < 0.0f ? 0 : 2) : 1;
      const float rec = digit == 1 ? 0.0f : (digit == 0 ? -mag : mag);
      const float dv = v - rec;
      const float err = half_sum32((double)(dv * dv)) / 32.0f;
      if (idx == 0 || err < best_err) {
        best_err = err;
        best_digit = digit;
        best_idx = idx;
      }
    }
    if (g < groups) {
      digits[g * 32 + hl] = (uint8_t)best_digit;
      if (hl == 0) mags[g] = (uint8_t)best_idx;
    }
  }
  __syncthreads();
  uint8_t* orow = out + row * (tb + mb);
  for (int b = threadIdx.x; b < tb; b += 256) {
    int val = 0, pw = 1;
    for (int k = 0; k < 5; k++) {
      const int c = 5 * b + k;
      if (c < cols) val += digits[c] * pw;
      pw *= 3;
    }
    orow[b] = (uint8_t)val;
  }
  for (int m = threadIdx.x; m < mb; m += 256) {
    int val = 0;
    for (int g = (8 * m) / 3; g < groups && 3 * g < 8 * m + 8; g++) {
      const int shift = 3 * g - 8 * m;
      val |= shift >= 0 ? (mags[g] << shift) : (mags[g] >> -shift);
    }
    orow[tb + m] = (uint8_t)val;
  }
}

template <typename F>
int by_src_dtype(int dtype, const char* what, F&& f) {
  switch (dtype) {
    case TT_F16: return f(f16_t{});
    case TT_BF16: return f(bf16_t{});
    case TT_F32: return f(float{});
  }
  set_error("%s: source dtype must be fp16, bf16 or fp32", what);
  return TT_ERR_INVALID;
}

}  // namespace
}  // namespace tt

using namespace tt;

extern "C" int tt_quantize_int4(const void* src, int src_dtype, int64_t rows, int64_t cols, int64_t src_row,
                                int64_t group_size, int mode, const float* importance, const float* gptq_factors,
                                uint8_t* packed, void* scales, void* stream) {
  const char* what = "quantize_int4";
  TT_REQUIRE(src && packed && scales, "%s: null pointer", what);
  TT_REQUIRE(mode >= TT_Q4_LSQ && mode <= TT_Q4_ROWS_AFFINE, "%s: unknown mode %d", what, mode);
  TT_REQUIRE(rows > 0 && cols > 0 && rows < (1 << 30) && cols < (1 << 30), "%s: bad shape", what);
  TT_REQUIRE(cols % 2 == 0, "%s: INT4 requires an even input width", what);
  TT_REQUIRE(group_size == 32 || group_size == 64 || group_size == 128 || group_size == 256 || group_size == 512,
             "%s: group size must be a power of two in [32, 512] (got %lld)", what, (long long)group_size);
  TT_REQUIRE(src_row >= cols, "%s: source row stride below the width", what);
  TT_REQUIRE(mode != TT_Q4_LSQ_AFFINE || cols % group_size == 0,
             "%s: affine least-squares INT4 needs the width to be a multiple of the group", what);
  TT_REQUIRE(importance == nullptr || mode == TT_Q4_LSQ_AFFINE, "%s: column importance applies to the affine fit only",
             what);
  TT_REQUIRE(gptq_factors == nullptr || (mode == TT_Q4_LSQ_AFFINE && group_size == 32),
             "%s: GPTQ factors apply to the affine fit with groups of 32 only", what);
  const int groups = (int)((cols + group_size - 1) / group_size);
  Q4Params P{src, src_row, importance, gptq_factors, packed, scales, (int)rows, (int)cols, (int)group_size, groups};
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t waves = rows * groups;
  TT_REQUIRE((waves + 3) / 4 < (1ll << 31), "%s: too many groups", what);
  const dim3 grid((unsigned)((waves + 3) / 4));
  return by_src_dtype(src_dtype, what, [&](auto t) -> int {
    using ST = decltype(t);
    auto go = [&](auto epl_c) -> int {
      constexpr int EPL = decltype(epl_c)::value;
      switch (mode) {
        case TT_Q4_LSQ: hipLaunchKernelGGL((int4_quant_kernel<ST, EPL, kLsq>), grid, dim3(256), 0, st, P); break;
        case TT_Q4_LSQ_AFFINE: hipLaunchKernelGGL((int4_quant_kernel<ST, EPL, kLsqAffine>), grid, dim3(256), 0, st, P); break;
        case TT_Q4_ROWS: hipLaunchKernelGGL((int4_quant_kernel<ST, EPL, kRows>), grid, dim3(256), 0, st, P); break;
        default: hipLaunchKernelGGL((int4_quant_kernel<ST, EPL, kRowsAffine>), grid, dim3(256), 0, st, P); break;
      }
      return check_launch(what);
    };
    switch (group_size) {
      case 32:
      case 64: return go(std::integral_constant<int, 1>{});
      case 128: return go(std::integral_constant<int, 2>{});
      case 256: return go(std::integral_constant<int, 4>{});
      default: return go(std::integral_constant<int, 8>{});
    }
  });
}

extern "C" int tt_quantize_fp8_rows(const void* src, int src_dtype, int64_t rows, int64_t cols, int64_t src_row,
                                    int64_t block, int via_bf16, uint8_t* out, float* scales, void* stream) {
  const char* what = "quantize_fp8_rows";
  TT_REQUIRE(src && out && scales, "%s: null pointer", what);
  TT_REQUIRE(rows > 0 && cols > 0 && cols < (1 << 30) && src_row >= cols, "%s: bad shape", what);
  TT_REQUIRE(block >= 0, "%s: negative scale block", what);
  const int nb = block > 0 ? (int)((cols + block - 1) / block) : 1;
  TT_REQUIRE(rows * nb < (1ll << 31), "%s: too many blocks", what);
  TT_REQUIRE(block < (1ll << 30), "%s: scale block too large", what);
  Fp8Params P{src, src_row, out, scales, (int)rows, (int)cols, block > 0 ? (int)block : (int)cols, nb};
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)(rows * nb));
  return by_src_dtype(src_dtype, what, [&](auto t) -> int {
    using ST = decltype(t);
    if (via_bf16) hipLaunchKernelGGL((fp8_quant_kernel<ST, true>), grid, dim3(256), 0, st, P);
    else hipLaunchKernelGGL((fp8_quant_kernel<ST, false>), grid, dim3(256), 0, st, P);
    return check_launch(what);
  });
}

extern "C" int tt_quantize_mxfp4_rows(const void* src, int src_dtype, int64_t rows, int64_t cols, int64_t src_row,
                                      int64_t transform, const void* signs, int binary_residual, uint8_t* packed,
                                      uint8_t* scales, void* stream) {
  const char* what = "quantize_mxfp4_rows";
  TT_REQUIRE(src && packed && scales, "%s: null pointer", what);
  TT_REQUIRE(rows > 0 && cols > 0 && cols < (1 << 30) && src_row >= cols, "%s: bad shape", what);
  TT_REQUIRE(cols % 32 == 0, "%s: native MXFP4 requires a K dimension divisible by 32", what);
  TT_REQUIRE(transform == 0 || transform == 32 || transform == 64 || transform == 128 || transform == 256 ||
                 transform == 512,
             "%s: Hadamard block must be 0 or a power of two in [32, 512] (got %lld)", what, (long long)transform);
  TT_REQUIRE(transform == 0 || cols % transform == 0, "%s: Hadamard block size %lld does not divide %lld", what,
             (long long)transform, (long long)cols);
  TT_REQUIRE(signs == nullptr || transform != 0, "%s: sign flips apply to the Hadamard transform only", what);
  const int span = transform > 64 ? (int)transform : 64;
  TT_REQUIRE(cols % span == 0, "%s: width must be a multiple of %d", what, span);
  MxParams P{src, src_row, signs, packed, scales, (int)rows, (int)cols, (int)transform, span,
             transform ? (float)(1.0 / __builtin_sqrt((double)transform)) : 1.0f, binary_residual ? 1 : 0};
  TT_REQUIRE(rows * (cols / span) < (1ll << 31), "%s: too many spans", what);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)(rows * (cols / span)));
  return by_src_dtype(src_dtype, what, [&](auto t) -> int {
    using ST = decltype(t);
    hipLaunchKernelGGL((mxfp4_quant_kernel<ST>), grid, dim3(64), 0, st, P);
    return check_launch(what);
  });
}

extern "C" int tt_requantize_mxfp4_lowbit(const uint8_t* blocks, const uint8_t* scales, int64_t n_groups, int bits,
                                          uint8_t* out, uint8_t* out_scales, void* stream) {
  const char* what = "quantize_mxfp4_to_lowbit";
  TT_REQUIRE(blocks && scales && out && out_scales, "%s: null pointer", what);
  TT_REQUIRE(bits == 1 || bits == 2, "%s: packed MXFP4 expert precision must be Q1 or Q2", what);
  TT_REQUIRE(n_groups > 0, "%s: bad group count", what);
  // eight groups per 256-thread workgroup: 32 work-items per group, and a launch
  // holds fewer than 2^32 work-items
  TT_UNSUPPORTED(n_groups < (1ll << 27), "%s: at most 2^27 groups per call", what);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)((n_groups + 7) / 8));
  hipLaunchKernelGGL(lowbit_requant_kernel, grid, dim3(256), 0, st, blocks, scales, n_groups, bits, out, out_scales);
  return check_launch(what);
}

extern "C" int tt_quantize_dense_lowbit(const void* src, int src_dtype, int64_t rows, int64_t cols, int64_t src_row,
                                        int bits, uint8_t* out, uint8_t* out_scales, void* stream) {
  const char* what = "quantize_dense_to_mxfp_lowbit";
  TT_REQUIRE(src && out && out_scales, "%s: null pointer", what);
  TT_REQUIRE(bits == 1 || bits == 2, "%s: dense low-bit precision must be Q1 or Q2", what);
  TT_REQUIRE(rows > 0 && cols > 0 && cols < (1 << 30) && src_row >= cols, "%s: bad shape", what);
  TT_REQUIRE(cols % 32 == 0, "%s: dense low-bit input width must be divisible by 32", what);
  const int64_t n = rows * (cols / 32);
  TT_UNSUPPORTED(n < (1ll << 27), "%s: at most 2^27 groups per call (32 work-items each)", what);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)((n + 7) / 8));
  return by_src_dtype(src_dtype, what, [&](auto t) -> int {
    using ST = decltype(t);
    hipLaunchKernelGGL((dense_lowbit_kernel<ST>), grid, dim3(256), 0, st, src, src_row, (int)rows, (int)cols, bits,
                       out, out_scales);
    return check_launch(what);
  });
}

extern "C" int tt_pack_mxfp4_ternary(const uint8_t* blocks, int64_t rows, int64_t groups, uint8_t* out, void* stream) {
  const char* what = "quantize_mxfp4_to_ternary";
  TT_REQUIRE(blocks && out, "%s: null pointer", what);
  TT_REQUIRE(rows > 0 && rows < (1ll << 31) && groups > 0, "%s: bad shape", what);
  TT_REQUIRE(groups * 32 <= kTernaryMaxCols, "%s: rows wider than %d columns", what, kTernaryMaxCols);
  hipStream_t st = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(ternary_pack_kernel, dim3((unsigned)rows), dim3(256), 0, st, blocks, (int)groups, out);
  return check_launch(what);
}
