// Dequant-fused GEMV machinery shared by the dense, selected-expert and fused MoE
// kernels.
//
// Reduction order (the contract the CPU restatement in oracle/ follows):
//   * the K axis is cut into chunks of 32 consecutive elements; chunk j is handled
//     by lane (j mod LPR) of the row's lane group in round (j div LPR);
//   * chunk partial  p_j = fma-chain over its 32 elements in ascending k, from +0;
//   * group formats: chunks of one quantisation group sit in L = group/32 adjacent
//     lanes; S_g = xor-butterfly over those L lanes; t_g = S_g * scale_g (affine:
//     fmaf(X_g, m_g, S_g * s_g) with X_g the same tree over sequential x-sums);
//     every lane keeps A = ((+0 + t_round0) + t_round1) + ...; the row value is the
//     xor-butterfly of A over the lane bits [L, LPR);
//   * row formats (per-row scale or none): A = ((+0 + p_round0) + p_round1) + ...;
//     row value = xor-butterfly over all LPR lanes, then * scale_row;
//   * chunks past the end of K contribute +0 at the same positions.
#pragma once

#include "tt_common.h"

namespace tt {

enum class Fmt : int {
  kInt4Sym = 0,   // code c in [0,15], w = (c - 8) * s_group
  kInt4Aff = 1,   // w = c * s_group + m_group
  kFp8 = 2,       // float8_e4m3fn, y = (sum w*x) * s_row
  kF16W = 3,      // plain fp16 weights
  kBF16W = 4,     // plain bf16 weights
  kMxfp4 = 5,     // e2m1 codes, E8M0 scale per 32-element block
  kQ2E8 = 6,      // 2-bit codebook {-1.5,-0.5,0.5,1.5}, E8M0 scale per 32-element block
  kQ1E8 = 7,      // 1-bit codebook {-1,+1}, E8M0 scale per 32-element block
  kQ2Aff = 8,     // 2-bit code c in [0,3], w = (c - z) * s per group
  kQ1Aff = 9,     // 1-bit code c in {0,1}, w = (c - z) * s per group
  kInt8 = 10,     // int8 rows, y = (sum w*x) * s_row (or per block)
};

template <Fmt F> struct FmtInfo;
template <> struct FmtInfo<Fmt::kInt4Sym> { static constexpr int kBytes = 16; };
template <> struct FmtInfo<Fmt::kInt4Aff> { static constexpr int kBytes = 16; };
template <> struct FmtInfo<Fmt::kFp8> { static constexpr int kBytes = 32; };
template <> struct FmtInfo<Fmt::kF16W> { static constexpr int kBytes = 64; };
template <> struct FmtInfo<Fmt::kBF16W> { static constexpr int kBytes = 64; };
template <> struct FmtInfo<Fmt::kMxfp4> { static constexpr int kBytes = 16; };
template <> struct FmtInfo<Fmt::kQ2E8> { static constexpr int kBytes = 8; };
template <> struct FmtInfo<Fmt::kQ1E8> { static constexpr int kBytes = 4; };
template <> struct FmtInfo<Fmt::kQ2Aff> { static constexpr int kBytes = 8; };
template <> struct FmtInfo<Fmt::kQ1Aff> { static constexpr int kBytes = 4; };
template <> struct FmtInfo<Fmt::kInt8> { static constexpr int kBytes = 32; };

template <int B> struct Raw { uint32_t w[B / 4]; };

template <int B>
__device__ __forceinline__ Raw<B> load_raw(const uint8_t* p) {
  Raw<B> r;
  if constexpr (B == 4) {
    r.w[0] = *reinterpret_cast<const uint32_t*>(__builtin_assume_aligned(p, 4));
  } else if constexpr (B == 8) {
    uint2 v = *reinterpret_cast<const uint2*>(__builtin_assume_aligned(p, 8));
    r.w[0] = v.x; r.w[1] = v.y;
  } else {
    const uint4* q = reinterpret_cast<const uint4*>(__builtin_assume_aligned(p, 16));
#pragma unroll
    for (int i = 0; i < B / 16; i++) {
      uint4 v = q[i];
      r.w[4 * i + 0] = v.x; r.w[4 * i + 1] = v.y; r.w[4 * i + 2] = v.z; r.w[4 * i + 3] = v.w;
    }
  }
  return r;
}

template <typename XT>
__device__ __forceinline__ float xv(const uint32_t* xw, int e) {
  return (e & 1) ? hi_f32<XT>(xw[e >> 1]) : lo_f32<XT>(xw[e >> 1]);
}

__device__ __forceinline__ h2 as_h2(uint32_t v) { return __builtin_bit_cast(h2, v); }

// (a & mask) | bits in one VALU op (v_and_or_b32).  The compiler splits this into
// v_and + v_or when both constants are literals, so it is spelled out here.
__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t mask, uint32_t bits) {
  uint32_t r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "s"(mask), "v"(bits));
  return r;
}
__device__ __forceinline__ h2 hfma(h2 a, float b, float c) {
  return __builtin_elementwise_fma(a, (h2){(_Float16)b, (_Float16)b}, (h2){(_Float16)c, (_Float16)c});
}

// Exact fp16 value pairs of 4-bit fields (f, f+4 of the word) minus `off`.
// (w & 0x000F000F) | 0x6400 6400 encodes 1024 + c; (w & 0x00F000F0) encodes 1024 + 16c.
__device__ __forceinline__ void nib_pairs(uint32_t w, float off, h2& a, h2& b, h2& c, h2& d) {
  uint32_t w8 = w >> 8;
  a = hfma(as_h2(and_or(w, 0x000F000Fu, 0x64006400u)), 1.0f, -(1024.0f + off));
  b = hfma(as_h2(and_or(w, 0x00F000F0u, 0x64006400u)), 0.0625f, -(64.0f + off));
  c = hfma(as_h2(and_or(w8, 0x000F000Fu, 0x64006400u)), 1.0f, -(1024.0f + off));
  d = hfma(as_h2(and_or(w8, 0x00F000F0u, 0x64006400u)), 0.0625f, -(64.0f + off));
}

// Decoded weights of one chunk, element e of the chunk in wv[e] (exact values).
// Formats whose values fit binary16 exactly decode to _Float16 so the fma consumes
// them through v_fma_mix without a conversion.
template <Fmt F> struct WVal { using T = _Float16; };
template <> struct WVal<Fmt::kFp8> { using T = float; };
template <> struct WVal<Fmt::kInt8> { using T = float; };
template <> struct WVal<Fmt::kBF16W> { using T = float; };

template <Fmt F>
__device__ __forceinline__ void decode_chunk(const Raw<FmtInfo<F>::kBytes>& r, typename WVal<F>::T* wv) {
  if constexpr (F == Fmt::kInt4Sym || F == Fmt::kInt4Aff) {
    // byte b holds k = 2b (low nibble) and k = 2b + 1 (high nibble); word i holds
    // k = 8i .. 8i+7 with nibble n at bits 4n.
    const float off = (F == Fmt::kInt4Sym) ? 8.0f : 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      h2 a, b, c, d;
      nib_pairs(r.w[i], off, a, b, c, d);
      wv[8 * i + 0] = a[0]; wv[8 * i + 1] = b[0]; wv[8 * i + 2] = c[0]; wv[8 * i + 3] = d[0];
      wv[8 * i + 4] = a[1]; wv[8 * i + 5] = b[1]; wv[8 * i + 6] = c[1]; wv[8 * i + 7] = d[1];
    }
  } else if constexpr (F == Fmt::kMxfp4) {
    // e2m1 pairs: byte b of word i holds k = 8i + 2b (low nibble) and 8i + 2b + 1
    // (high nibble); v_cvt_scalef32_pk_f16_fp4 with scale 1 turns one byte into the
    // two exact binary16 values (low nibble in the low half).
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const h2 p0 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(r.w[i], 1.0f, 0);
      const h2 p1 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(r.w[i], 1.0f, 1);
      const h2 p2 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(r.w[i], 1.0f, 2);
      const h2 p3 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(r.w[i], 1.0f, 3);
      wv[8 * i + 0] = p0[0]; wv[8 * i + 1] = p0[1]; wv[8 * i + 2] = p1[0]; wv[8 * i + 3] = p1[1];
      wv[8 * i + 4] = p2[0]; wv[8 * i + 5] = p2[1]; wv[8 * i + 6] = p3[0]; wv[8 * i + 7] = p3[1];
    }
  } else if constexpr (F == Fmt::kFp8) {
    // 32 bytes, byte e = element e; e4m3fn -> f32 is exact.
#pragma unroll
    for (int i = 0; i < 8; i++) {
      auto lo = __builtin_amdgcn_cvt_pk_f32_fp8(r.w[i], false);
      auto hi = __builtin_amdgcn_cvt_pk_f32_fp8(r.w[i], true);
      wv[4 * i + 0] = lo[0]; wv[4 * i + 1] = lo[1]; wv[4 * i + 2] = hi[0]; wv[4 * i + 3] = hi[1];
    }
  } else if constexpr (F == Fmt::kInt8) {
    // 32 bytes, byte e = element e as a two's-complement integer; int8 -> f32 is exact.
#pragma unroll
    for (int i = 0; i < 8; i++) {
#pragma unroll
      for (int b = 0; b < 4; b++) wv[4 * i + b] = (float)(int8_t)(r.w[i] >> (8 * b));
    }
  } else if constexpr (F == Fmt::kF16W) {
#pragma unroll
    for (int i = 0; i < 16; i++) {
      h2 v = as_h2(r.w[i]);
      wv[2 * i] = v[0]; wv[2 * i + 1] = v[1];
    }
  } else if constexpr (F == Fmt::kBF16W) {
#pragma unroll
    for (int i = 0; i < 16; i++) {
      wv[2 * i] = lo_f32<bf16_t>(r.w[i]);
      wv[2 * i + 1] = hi_f32<bf16_t>(r.w[i]);
    }
  } else if constexpr (F == Fmt::kQ2E8 || F == Fmt::kQ2Aff) {
    // 8 bytes; element i at byte i/4, bits 2*(i%4), so word q holds elements
    // 16q..16q+15 with element n at bits 2n.  Fields are moved to bits 2..9 (and
    // 18..25) first so that every fp16 constant below is exactly representable:
    // field f' (1..4) encodes 1024 + 4^f' c, scaled back by 4^-f'.
    const float off = (F == Fmt::kQ2E8) ? 1.5f : 0.0f;
#pragma unroll
    for (int q = 0; q < 2; q++) {
      const uint32_t u0 = r.w[q] << 2;   // elements 0..3 | 8..11 of this word
      const uint32_t u1 = r.w[q] >> 6;   // elements 4..7 | 12..15
      const uint32_t m[4] = {0x000C000Cu, 0x00300030u, 0x00C000C0u, 0x03000300u};
      const float k[4] = {0.25f, 0.0625f, 0.015625f, 0.00390625f};
      const float c[4] = {256.0f, 64.0f, 16.0f, 4.0f};
#pragma unroll
      for (int f = 0; f < 4; f++) {
        h2 a = hfma(as_h2(and_or(u0, m[f], 0x64006400u)), k[f], -(c[f] + off));
        h2 b = hfma(as_h2(and_or(u1, m[f], 0x64006400u)), k[f], -(c[f] + off));
        wv[16 * q + f] = a[0];
        wv[16 * q + 4 + f] = b[0];
        wv[16 * q + 8 + f] = a[1];
        wv[16 * q + 12 + f] = b[1];
      }
    }
  } else if constexpr (F == Fmt::kQ1E8 || F == Fmt::kQ1Aff) {
    // 4 bytes; element i at byte i/8, bit i%8, i.e. bit i of the word.  Bits move
    // to positions 1..8 (17..24) so the fp16 constants stay exact: bit n' encodes
    // 1024 + 2^n' b.  E8M0 q1 maps b to 2b - 1, the affine form keeps b.
    const uint32_t w = r.w[0];
#pragma unroll
    for (int half = 0; half < 2; half++) {
      const uint32_t u = half ? (w >> 7) : (w << 1);   // elements 8*half + n | 16 + 8*half + n
#pragma unroll
      for (int n = 1; n <= 8; n++) {
        h2 t = as_h2(and_or(u, 0x00010001u << n, 0x64006400u));
        h2 v;
        if constexpr (F == Fmt::kQ1E8)
          v = hfma(t, 2.0f / (float)(1 << n), -(2048.0f / (float)(1 << n) + 1.0f));
        else
          v = hfma(t, 1.0f / (float)(1 << n), -(1024.0f / (float)(1 << n)));
        wv[8 * half + n - 1] = v[0];
        wv[16 + 8 * half + n - 1] = v[1];
      }
    }
  }
}

// Decoded values of word q (elements 8q .. 8q+7) of a 16-byte int4 / MXFP4 chunk.
template <Fmt F>
__device__ __forceinline__ void decode_word8(uint32_t w, _Float16* v) {
  if constexpr (F == Fmt::kInt4Sym || F == Fmt::kInt4Aff) {
    const float off = (F == Fmt::kInt4Sym) ? 8.0f : 0.0f;
    h2 a, b, c, d;
    nib_pairs(w, off, a, b, c, d);
    v[0] = a[0]; v[1] = b[0]; v[2] = c[0]; v[3] = d[0];
    v[4] = a[1]; v[5] = b[1]; v[6] = c[1]; v[7] = d[1];
  } else {
    const h2 p0 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 1.0f, 0);
    const h2 p1 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 1.0f, 1);
    const h2 p2 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 1.0f, 2);
    const h2 p3 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 1.0f, 3);
    v[0] = p0[0]; v[1] = p0[1]; v[2] = p1[0]; v[3] = p1[1];
    v[4] = p2[0]; v[5] = p2[1]; v[6] = p3[0]; v[7] = p3[1];
  }
}

// MXFP4 word q (elements 8q .. 8q+7) decoded straight to binary32: the exact values the
// binary16 decode gives, so the fma chains below run as plain fp32 fmas (full issue
// rate) instead of mixed-precision ones, with the same bits.
__device__ __forceinline__ void decode_word8_mxfp4_f32(uint32_t w, float* v) {
  typedef float f2 __attribute__((ext_vector_type(2)));
  const f2 p0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 0);
  const f2 p1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 1);
  const f2 p2 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 2);
  const f2 p3 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 3);
  v[0] = p0[0]; v[1] = p0[1]; v[2] = p1[0]; v[3] = p1[1];
  v[4] = p2[0]; v[5] = p2[1]; v[6] = p3[0]; v[7] = p3[1];
}

// Chunk partials of NR rows: for each row an fma chain over the chunk's 32 elements
// in ascending k, starting from +0.  The rows' chains are interleaved element by
// element so no fma waits on the one issued just before it.  The 4-bit formats are
// decoded one 32-bit word (8 elements) at a time so only 8 values per row are live.
template <Fmt F, typename XT, int NR>
__device__ __forceinline__ void chunk_dot_rows(const Raw<FmtInfo<F>::kBytes>* r, const uint32_t* xw, float* p) {
#pragma unroll
  for (int i = 0; i < NR; i++) p[i] = 0.0f;
  if constexpr (F == Fmt::kMxfp4) {
#pragma unroll
    for (int q = 0; q < 4; q++) {
      float wv[NR][8];
#pragma unroll
      for (int i = 0; i < NR; i++) decode_word8_mxfp4_f32(r[i].w[q], wv[i]);
#pragma unroll
      for (int e = 0; e < 8; e++) {
        const float xe = xv<XT>(xw, 8 * q + e);
#pragma unroll
        for (int i = 0; i < NR; i++) p[i] = __builtin_fmaf(wv[i][e], xe, p[i]);
      }
    }
  } else if constexpr (F == Fmt::kInt4Sym || F == Fmt::kInt4Aff) {
#pragma unroll
    for (int q = 0; q < 4; q++) {
      _Float16 wv[NR][8];
#pragma unroll
      for (int i = 0; i < NR; i++) decode_word8<F>(r[i].w[q], wv[i]);
#pragma unroll
      for (int e = 0; e < 8; e++) {
        const float xe = xv<XT>(xw, 8 * q + e);
#pragma unroll
        for (int i = 0; i < NR; i++) p[i] = __builtin_fmaf((float)wv[i][e], xe, p[i]);
      }
    }
  } else {
    typename WVal<F>::T wv[NR][32];
#pragma unroll
    for (int i = 0; i < NR; i++) decode_chunk<F>(r[i], wv[i]);
#pragma unroll
    for (int e = 0; e < 32; e++) {
      const float xe = xv<XT>(xw, e);
#pragma unroll
      for (int i = 0; i < NR; i++) p[i] = __builtin_fmaf((float)wv[i][e], xe, p[i]);
    }
  }
}

// chunk_dot_rows for MR activation rows at once: every weight word is decoded once
// and feeds the fma chains of all MR activation rows (each chain in the single-row
// order, so row m's partials equal chunk_dot_rows on activation row m).
template <Fmt F, typename XT, int NR, int MR>
__device__ __forceinline__ void chunk_dot_rows_multi(const Raw<FmtInfo<F>::kBytes>* r, const uint32_t (*xw)[16],
                                                     float (*p)[NR]) {
  if constexpr (MR == 1) {
    chunk_dot_rows<F, XT, NR>(r, xw[0], p[0]);
  } else {
#pragma unroll
    for (int m = 0; m < MR; m++)
#pragma unroll
      for (int i = 0; i < NR; i++) p[m][i] = 0.0f;
    if constexpr (F == Fmt::kMxfp4) {
#pragma unroll
      for (int q = 0; q < 4; q++) {
        float wv[NR][8];
#pragma unroll
        for (int i = 0; i < NR; i++) decode_word8_mxfp4_f32(r[i].w[q], wv[i]);
#pragma unroll
        for (int e = 0; e < 8; e++) {
#pragma unroll
          for (int m = 0; m < MR; m++) {
            const float xe = xv<XT>(xw[m], 8 * q + e);
#pragma unroll
            for (int i = 0; i < NR; i++) p[m][i] = __builtin_fmaf(wv[i][e], xe, p[m][i]);
          }
        }
      }
    } else if constexpr (F == Fmt::kInt4Sym || F == Fmt::kInt4Aff) {
#pragma unroll
      for (int q = 0; q < 4; q++) {
        _Float16 wv[NR][8];
#pragma unroll
        for (int i = 0; i < NR; i++) decode_word8<F>(r[i].w[q], wv[i]);
#pragma unroll
        for (int e = 0; e < 8; e++) {
#pragma unroll
          for (int m = 0; m < MR; m++) {
            const float xe = xv<XT>(xw[m], 8 * q + e);
#pragma unroll
            for (int i = 0; i < NR; i++) p[m][i] = __builtin_fmaf((float)wv[i][e], xe, p[m][i]);
          }
        }
      }
    } else {
      typename WVal<F>::T wv[NR][32];
#pragma unroll
      for (int i = 0; i < NR; i++) decode_chunk<F>(r[i], wv[i]);
#pragma unroll
      for (int e = 0; e < 32; e++) {
#pragma unroll
        for (int m = 0; m < MR; m++) {
          const float xe = xv<XT>(xw[m], e);
#pragma unroll
          for (int i = 0; i < NR; i++) p[m][i] = __builtin_fmaf((float)wv[i][e], xe, p[m][i]);
        }
      }
    }
  }
}

template <Fmt F, typename XT>
__device__ __forceinline__ float chunk_dot(const Raw<FmtInfo<F>::kBytes>& r, const uint32_t* xw) {
  float p;
  chunk_dot_rows<F, XT, 1>(&r, xw, &p);
  return p;
}

// Row values of NR rows in the E8M0 block-scale order (one 32-element block per
// chunk): t_j = p_j * 2^(e_j - 127), A = ((+0 + t_round0) + ...),
// value = xor-butterfly over the LPR lanes.  `xs` is the activation vector in LDS.
// Weights and exponents of round r+1 are loaded while round r is computed.
template <Fmt F, int NR>
struct E8Round {
  Raw<FmtInfo<F>::kBytes> w[NR];
  int e[NR];
};

template <Fmt F, int LPR, int NR>
__device__ __forceinline__ void e8_fetch(E8Round<F, NR>& d, int r, int l, int nchunks, const uint8_t* const* wrow,
                                         const uint8_t* const* srow, const bool* rv) {
  constexpr int B = FmtInfo<F>::kBytes;
  const int j = r * LPR + l;
  const bool cv = j < nchunks;
#pragma unroll
  for (int i = 0; i < NR; i++) {
    if (cv && rv[i]) {
      d.w[i] = load_raw<B>(wrow[i] + (int64_t)j * B);
      d.e[i] = srow[i][j];
    } else {
#pragma unroll
      for (int q = 0; q < B / 4; q++) d.w[i].w[q] = 0u;
      d.e[i] = 127;
    }
  }
}

template <Fmt F, typename XT, int LPR, int NR>
__device__ __forceinline__ void e8_rows_dot(E8Round<F, NR>& cur, const uint8_t* const* wrow, const uint8_t* const* srow,
                                            const bool* rv, const uint32_t* xs, int nchunks, int l,
                                            float* out) {
  const int rounds = (nchunks + LPR - 1) / LPR;
  float acc[NR];
#pragma unroll
  for (int i = 0; i < NR; i++) acc[i] = 0.0f;
  for (int r = 0; r < rounds; r++) {
    E8Round<F, NR> nxt;
    if (r + 1 < rounds) e8_fetch<F, LPR, NR>(nxt, r + 1, l, nchunks, wrow, srow, rv);
    const int j = r * LPR + l;
    const bool cv = j < nchunks;
    uint32_t xw[16];
    {
      const uint4* xp = reinterpret_cast<const uint4*>(xs + (cv ? j : 0) * 16);
#pragma unroll
      for (int q = 0; q < 4; q++) {
        uint4 v = xp[q];
        xw[4 * q] = v.x; xw[4 * q + 1] = v.y; xw[4 * q + 2] = v.z; xw[4 * q + 3] = v.w;
      }
    }
    float pr[NR];
    chunk_dot_rows<F, XT, NR>(cur.w, xw, pr);
#pragma unroll
    for (int i = 0; i < NR; i++) {
      const float t = pr[i] * pow2i(cur.e[i] - 127);
      acc[i] = acc[i] + ((cv && rv[i]) ? t : 0.0f);
    }
    if (r + 1 < rounds) cur = nxt;
  }
#pragma unroll
  for (int i = 0; i < NR; i++) out[i] = xor_sum(acc[i], 1, LPR);
}

}  // namespace tt
