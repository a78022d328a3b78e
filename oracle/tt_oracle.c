/*
 * tt_oracle.c -- CPU restatement of ThinTensor's decode-path operators.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker for the HIP kernels: only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.  The
 * product never links or calls it.
 *
 * Each operator restates the reference semantics (file:line cited per function)
 * and evaluates it in binary32 in the documented reduction order of the kernels,
 * so every output can be compared bit for bit.  Compile with -ffp-contract=off:
 * every fused multiply-add below is an explicit fmaf().
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define TTO_F16 0
#define TTO_BF16 1
#define TTO_F32 2

/* ------------------------------------------------------------ conversions */

static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

float tto_f16_to_f32(uint16_t h) {
  uint32_t s = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 31u, m = h & 1023u;
  if (e == 0) {
    float v = ldexpf((float)m, -24);
    return s ? -v : v;
  }
  if (e == 31) return u2f(s | 0x7f800000u | (m << 13));
  return u2f(s | ((e + 112u) << 23) | (m << 13));
}

/* round to nearest even, IEEE binary16 (subnormals, overflow to inf, NaN kept quiet) */
uint16_t tto_f32_to_f16(float f) {
  uint32_t x = f2u(f);
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t ax = x & 0x7fffffffu;
  if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu));
  if (ax >= 0x47800000u) {           /* >= 65536: inf (values in [65520, 65536) handled below) */
    return (uint16_t)(sign | 0x7c00u);
  }
  int e = (int)(ax >> 23) - 127;
  uint32_t m = (ax & 0x7fffffu) | 0x800000u;
  if (ax < 0x38800000u) {            /* below 2^-14: subnormal half or zero */
    if (ax == 0) return (uint16_t)sign;
    int sh = -14 - e + 13;             /* shift of the 24-bit significand */
    if (sh > 24) return (uint16_t)sign;
    uint32_t q = m >> sh, r = m & ((1u << sh) - 1u), half = 1u << (sh - 1);
    if (r > half || (r == half && (q & 1u))) q++;
    return (uint16_t)(sign | q);
  }
  uint32_t q = m >> 13, r = m & 0x1fffu;
  if (r > 0x1000u || (r == 0x1000u && (q & 1u))) q++;
  uint32_t h = ((uint32_t)(e + 15) << 10) + (q - 1024u);   /* carry into exponent is fine */
  if (h >= 0x7c00u) return (uint16_t)(sign | 0x7c00u);
  return (uint16_t)(sign | h);
}

float tto_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

uint16_t tto_f32_to_bf16(float f) {
  uint32_t u = f2u(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

float tto_round_bf16(float f) { return tto_bf16_to_f32(tto_f32_to_bf16(f)); }
float tto_round_f16(float f) { return tto_f16_to_f32(tto_f32_to_f16(f)); }

static float act_get(const void* p, int dtype, int64_t i) {
  if (dtype == TTO_F16) return tto_f16_to_f32(((const uint16_t*)p)[i]);
  if (dtype == TTO_BF16) return tto_bf16_to_f32(((const uint16_t*)p)[i]);
  return ((const float*)p)[i];
}

static void act_put(void* p, int dtype, int64_t i, float v) {
  if (dtype == TTO_F16) ((uint16_t*)p)[i] = tto_f32_to_f16(v);
  else if (dtype == TTO_BF16) ((uint16_t*)p)[i] = tto_f32_to_bf16(v);
  else ((float*)p)[i] = v;
}

static float round_to(int dtype, float v) {
  if (dtype == TTO_F16) return tto_round_f16(v);
  if (dtype == TTO_BF16) return tto_round_bf16(v);
  return v;
}

/* 2^e as binary32 for e in [-149, 128] */
static float pow2i(int e) {
  if (e >= -126) return u2f((uint32_t)(e + 127) << 23);
  return u2f(1u << (e + 149));
}

/* Device exp_f32 (tt_common.h): Cody-Waite reduction + degree-7 Taylor/Horner. */
float tto_exp_f32(float x) {
  if (x != x) return x;
  if (x < -0x1.5d589ep+6f) return 0.0f;
  if (x > 0x1.62e42ep+6f) return u2f(0x7f800000u);
  const float log2e = 0x1.715476p+0f;
  float n = rintf(x * log2e);
  float r = fmaf(n, -0x1.62e4p-1f, x);
  r = fmaf(n, -0x1.7f7d1cp-20f, r);
  float p = 0x1.a01a02p-13f;
  p = fmaf(p, r, 0x1.6c16c2p-10f);
  p = fmaf(p, r, 0x1.111112p-7f);
  p = fmaf(p, r, 0x1.555556p-5f);
  p = fmaf(p, r, 0x1.555556p-3f);
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  int ni = (int)n;
  int n1 = ni / 2, n2 = ni - n1;
  p = p * u2f((uint32_t)(n1 + 127) << 23);
  p = p * u2f((uint32_t)(n2 + 127) << 23);
  return p;
}

/* ------------------------------------------------------------ weight formats */

enum {
  FMT_INT4_SYM = 0, FMT_INT4_AFF = 1, FMT_FP8 = 2, FMT_F16W = 3, FMT_BF16W = 4,
  FMT_MXFP4 = 5, FMT_Q2E8 = 6, FMT_Q1E8 = 7, FMT_Q2AFF = 8, FMT_Q1AFF = 9, FMT_INT8 = 10
};
enum { SM_NONE = 0, SM_ROW = 1, SM_GROUP = 2, SM_GROUP_AFF = 3, SM_BLOCK_E8 = 4 };

static int fmt_bytes(int fmt) {
  switch (fmt) {
    case FMT_INT4_SYM: case FMT_INT4_AFF: case FMT_MXFP4: return 16;
    case FMT_FP8: case FMT_INT8: return 32;
    case FMT_F16W: case FMT_BF16W: return 64;
    case FMT_Q2E8: case FMT_Q2AFF: return 8;
    default: return 4;
  }
}

/* float8_e4m3fn -> binary32, exact (reference weights are torch.float8_e4m3fn). */
float tto_fp8e4m3_to_f32(uint8_t b) {
  int s = b >> 7, e = (b >> 3) & 15, m = b & 7;
  float v;
  if (e == 15 && m == 7) return NAN;
  if (e == 0) v = ldexpf((float)m, -9);
  else v = ldexpf((float)(8 + m), e - 10);
  return s ? -v : v;
}

/* e2m1 code -> value (triton_kernels.py:249-276, gpu_runtime.py:12876-12897). */
float tto_e2m1(int code) {
  static const float mag[8] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f};
  float v = mag[code & 7];
  return (code & 8) ? -v : v;
}

/* Value of element e (0..31) of one chunk as the kernel feeds it to the fma.
 */
static float chunk_weight(int fmt, const uint8_t* c, int e) {
  switch (fmt) {
    case FMT_INT4_SYM: return (float)(((c[e >> 1] >> ((e & 1) * 4)) & 15) - 8);
    case FMT_INT4_AFF: return (float)((c[e >> 1] >> ((e & 1) * 4)) & 15);
    case FMT_FP8: return tto_fp8e4m3_to_f32(c[e]);
    case FMT_F16W: return tto_f16_to_f32(((const uint16_t*)c)[e]);
    case FMT_BF16W: return tto_bf16_to_f32(((const uint16_t*)c)[e]);
    case FMT_MXFP4: return tto_e2m1((c[e >> 1] >> ((e & 1) * 4)) & 15);
    case FMT_Q2E8: return (float)((c[e >> 2] >> ((e & 3) * 2)) & 3) - 1.5f;
    case FMT_Q1E8: return ((c[e >> 3] >> (e & 7)) & 1) ? 1.0f : -1.0f;
    case FMT_Q2AFF: return (float)((c[e >> 2] >> ((e & 3) * 2)) & 3);
    case FMT_Q1AFF: return (float)((c[e >> 3] >> (e & 7)) & 1);
    case FMT_INT8: return (float)(int8_t)c[e];   /* triton_kernels.py:554-560: int8 rows .to(fp32) */
  }
  return 0.0f;
}

/* Butterfly over lane bits [m0, m1): v[i] <- v[i] + v[i ^ m] for m = m0, 2*m0, ... */
static void xor_sum(float* v, int lanes, int m0, int m1) {
  float t[64];
  for (int m = m0; m < m1; m <<= 1) {
    for (int i = 0; i < lanes; i++) t[i] = v[i] + v[i ^ m];
    memcpy(v, t, sizeof(float) * (size_t)lanes);
  }
}

static float scale_get(const void* s, int sdtype, int64_t i) {
  if (sdtype == TTO_F16) return tto_f16_to_f32(((const uint16_t*)s)[i]);
  if (sdtype == TTO_BF16) return tto_bf16_to_f32(((const uint16_t*)s)[i]);
  return ((const float*)s)[i];
}

/* Decode the 32 weights of one chunk (values as fed to the fma). */
static void chunk_weights(int fmt, const uint8_t* c, float* wv) {
  for (int e = 0; e < 32; e++) wv[e] = chunk_weight(fmt, c, e);
}

/*
 * One output row in the kernels' reduction order (thintensor_amd/csrc/tt_gemv.h):
 * chunks of 32, chunk j -> lane j % lpr, round j / lpr; fma chain per chunk; group
 * butterfly and scale; sequential accumulation over rounds; final butterfly.
 * xf: the activation vector already converted to binary32.
 */
static float gemv_row_f(int fmt, int smode, const uint8_t* wrow, const void* srow, int sdtype, int64_t s_grp,
                        int64_t s_pair, int aff_zero, const float* xf, int cols, int L, int lpr) {
  const int B = fmt_bytes(fmt);
  const int nchunks = cols / 32;
  const int rounds = (nchunks + lpr - 1) / lpr;
  float A[64], p[64], xs[64], wv[32];
  for (int l = 0; l < lpr; l++) A[l] = 0.0f;
  for (int r = 0; r < rounds; r++) {
    for (int l = 0; l < lpr; l++) {
      const int j = r * lpr + l;
      p[l] = 0.0f;
      xs[l] = 0.0f;
      if (j < nchunks) {
        chunk_weights(fmt, wrow + (int64_t)j * B, wv);
        const float* xc = xf + 32 * (int64_t)j;
        float acc = 0.0f;
        for (int e = 0; e < 32; e++) acc = fmaf(wv[e], xc[e], acc);
        p[l] = acc;
        if (smode == SM_GROUP_AFF) {
          float sx = 0.0f;
          for (int e = 0; e < 32; e++) sx = sx + xc[e];
          xs[l] = sx;
        }
      }
    }
    if (smode == SM_NONE || smode == SM_ROW) {
      for (int l = 0; l < lpr; l++) A[l] = A[l] + p[l];
    } else if (smode == SM_BLOCK_E8) {
      for (int l = 0; l < lpr; l++) {
        const int j = r * lpr + l;
        float t = 0.0f;
        if (j < nchunks) {
          const int e = ((const uint8_t*)srow)[j];
          t = p[l] * pow2i(e - 127);
        }
        A[l] = A[l] + t;
      }
    } else {
      xor_sum(p, lpr, 1, L);
      if (smode == SM_GROUP_AFF) xor_sum(xs, lpr, 1, L);
      for (int l = 0; l < lpr; l++) {
        const int j = r * lpr + l;
        float t = 0.0f;
        if (j < nchunks) {
          const int g = j / L;
          const float s = scale_get(srow, sdtype, (int64_t)g * s_grp);
          if (smode == SM_GROUP_AFF) {
            float m = scale_get(srow, sdtype, (int64_t)g * s_grp + s_pair);
            if (aff_zero) m = -(m * s);
            t = fmaf(xs[l], m, p[l] * s);
          } else {
            t = p[l] * s;
          }
        }
        A[l] = A[l] + t;
      }
    }
  }
  if (smode == SM_GROUP || smode == SM_GROUP_AFF) xor_sum(A, lpr, L, lpr);
  else xor_sum(A, lpr, 1, lpr);
  float v = A[0];
  if (smode == SM_ROW) v = v * scale_get(srow, sdtype, 0);
  return v;
}

static float* to_f32_vec(const void* x, int xdtype, int n) {
  float* xf = (float*)malloc(sizeof(float) * (size_t)n);
  for (int i = 0; i < n; i++) xf[i] = act_get(x, xdtype, i);
  return xf;
}

float tto_gemv_row(int fmt, int smode, const uint8_t* wrow, const void* srow, int sdtype, int64_t s_grp,
                   int64_t s_pair, int aff_zero, const void* x, int xdtype, int cols, int L,
                   int lpr) {
  float* xf = to_f32_vec(x, xdtype, cols);
  const float v = gemv_row_f(fmt, smode, wrow, srow, sdtype, s_grp, s_pair, aff_zero, xf, cols, L, lpr);
  free(xf);
  return v;
}

/*
 * Generic GEMV over `rows` rows (optionally a selected expert and a per-slot
 * activation row).  w points at the first row of the chosen matrix/expert.
 */
int tto_gemv(int fmt, int smode, const uint8_t* w, int64_t w_row_bytes, const void* s, int sdtype, int64_t s_row,
             int64_t s_grp, int64_t s_pair, int aff_zero, const void* x, int xdtype, void* out,
             int odtype, int64_t rows, int cols, int L, int lpr) {
  if (cols % 32 || lpr < 1 || lpr > 64) return -1;
  float* xf = to_f32_vec(x, xdtype, cols);
  const size_t es = smode == SM_BLOCK_E8 ? 1 : (sdtype == TTO_F32 ? 4 : 2);
#pragma omp parallel for schedule(static)
  for (int64_t n = 0; n < rows; n++) {
    const void* srow = s ? (const void*)((const uint8_t*)s + (size_t)(n * s_row) * es) : NULL;
    const float v = gemv_row_f(fmt, smode, w + n * w_row_bytes, srow, sdtype, s_grp, s_pair, aff_zero, xf,
                               cols, L, lpr);
    act_put(out, odtype, n, v);
  }
  free(xf);
  return 0;
}

/* ------------------------------------------------------------ fused MoE experts */

static float round_rt(int rt, float v) { return round_to(rt, v); }

/*
 * Fused interleaved gate/up GEMV + gpt-oss SwiGLU for one launch
 * (triton_kernels.py:1214-1343; MXFP4 chain gpu_runtime.py:9647-9704 + :2778-2793).
 * fmt: FMT_Q2E8 / FMT_Q1E8 / FMT_MXFP4; rt: rounding dtype of dot results and
 * bias sums (bf16 for q1/q2, activation dtype for MXFP4).
 */
int tto_swiglu(int fmt, int rt, const uint8_t* w, int64_t w_expert, int64_t w_row, const uint8_t* s,
               int64_t s_expert, int64_t s_row, const void* x, int xdtype, int64_t x_slot, const int32_t* experts,
               int selected, const void* bias, int bdtype, int64_t bias_expert, float alpha, float limit, void* out,
               int odtype, int64_t out_slot, int act_rows, int cols, int lpr) {
  const size_t xes = xdtype == TTO_F32 ? 4 : 2;
  for (int slot = 0; slot < selected; slot++) {
    const int64_t e = experts[slot];
    const void* xs = (const uint8_t*)x + (size_t)(slot * x_slot) * xes;
    float* xf = to_f32_vec(xs, xdtype, cols);
#pragma omp parallel for schedule(static)
    for (int a = 0; a < act_rows; a++) {
      float g = gemv_row_f(fmt, SM_BLOCK_E8, w + e * w_expert + (2 * (int64_t)a) * w_row,
                           s + e * s_expert + (2 * (int64_t)a) * s_row, TTO_F32, 1, 0, 0, xf, cols, 1, lpr);
      float u = gemv_row_f(fmt, SM_BLOCK_E8, w + e * w_expert + (2 * (int64_t)a + 1) * w_row,
                           s + e * s_expert + (2 * (int64_t)a + 1) * s_row, TTO_F32, 1, 0, 0, xf, cols, 1, lpr);
      g = round_rt(rt, g);
      u = round_rt(rt, u);
      if (bias) {
        g = round_rt(rt, g + act_get(bias, bdtype, e * bias_expert + 2 * (int64_t)a));
        u = round_rt(rt, u + act_get(bias, bdtype, e * bias_expert + 2 * (int64_t)a + 1));
      }
      g = fminf(g, limit);
      u = fmaxf(fminf(u, limit), -limit);
      const float num = (u + 1.0f) * g;
      const float den = 1.0f + tto_exp_f32(-g * alpha);
      act_put(out, odtype, slot * out_slot + a, num / den);
    }
    free(xf);
  }
  return 0;
}

/* Fused down GEMV + router-weighted sum in slot order (triton_kernels.py:1347-1435). */
int tto_weighted_down(int fmt, int rt, const uint8_t* w, int64_t w_expert, int64_t w_row, const uint8_t* s,
                      int64_t s_expert, int64_t s_row, const void* x, int xdtype, int64_t x_slot,
                      const int32_t* experts, const void* scores, int sdtype, int selected, const void* bias,
                      int bdtype, int64_t bias_expert, void* out, int odtype, int rows, int cols, int lpr) {
  const size_t xes = xdtype == TTO_F32 ? 4 : 2;
  float* xf[64];
  for (int slot = 0; slot < selected && slot < 64; slot++)
    xf[slot] = to_f32_vec((const uint8_t*)x + (size_t)(slot * x_slot) * xes, xdtype, cols);
#pragma omp parallel for schedule(static)
  for (int n = 0; n < rows; n++) {
    float combined = 0.0f;
    for (int slot = 0; slot < selected; slot++) {
      const int64_t e = experts[slot];
      float v = gemv_row_f(fmt, SM_BLOCK_E8, w + e * w_expert + (int64_t)n * w_row, s + e * s_expert + (int64_t)n * s_row,
                           TTO_F32, 1, 0, 0, xf[slot], cols, 1, lpr);
      v = round_rt(rt, v);
      if (bias) v = round_rt(rt, v + act_get(bias, bdtype, e * bias_expert + n));
      combined = fmaf(v, act_get(scores, sdtype, slot), combined);
    }
    act_put(out, odtype, n, combined);
  }
  for (int slot = 0; slot < selected && slot < 64; slot++) free(xf[slot]);
  return 0;
}

/* ------------------------------------------------------------ norms / elementwise */

/* 256-thread block sum: per-wave butterfly over 64 lanes, then (w0 + w1) + (w2 + w3). */
static float block_sum256(const float* part) {
  float w[4];
  for (int wv = 0; wv < 4; wv++) {
    float v[64];
    memcpy(v, part + 64 * wv, sizeof v);
    xor_sum(v, 64, 1, 64);
    w[wv] = v[0];
  }
  return (w[0] + w[1]) + (w[2] + w[3]);
}

/* The kernels' RMSNorm partition: pieces of 8 elements, piece p to thread p % 256; a
 * thread's sum of squares is an fma chain over its elements in increasing index order. */
#define TTO_PIECE_OWNER(i) ((int)(((i) / 8) % 256))

/* RMSNorm (triton_kernels.py:2562-2577): out = (x * inv) * (w + offset). */
int tto_rms_norm(const void* x, int xdt, const void* w, int wdt, void* out, int odt, int n, float eps, float offset) {
  float part[256];
  for (int t = 0; t < 256; t++) part[t] = 0.0f;
  for (int i = 0; i < n; i++) {
    const float v = act_get(x, xdt, i);
    part[TTO_PIECE_OWNER(i)] = fmaf(v, v, part[TTO_PIECE_OWNER(i)]);
  }
  const float total = block_sum256(part);
  const float inv = 1.0f / sqrtf(total / (float)n + eps);
  for (int i = 0; i < n; i++) act_put(out, odt, i, (act_get(x, xdt, i) * inv) * (act_get(w, wdt, i) + offset));
  return 0;
}

/* add + RMSNorm with the residual rounded through bf16 (triton_kernels.py:2581-2614). */
int tto_add_rms_norm(const void* l, const void* r, void* res_out, int xdt, const void* w, int wdt, void* out, int odt,
                     int n, float eps) {
  float part[256];
  for (int t = 0; t < 256; t++) part[t] = 0.0f;
  for (int i = 0; i < n; i++) {
    const float v = tto_round_bf16(act_get(l, xdt, i) + act_get(r, xdt, i));
    part[TTO_PIECE_OWNER(i)] = fmaf(v, v, part[TTO_PIECE_OWNER(i)]);
  }
  const float total = block_sum256(part);
  const float inv = 1.0f / sqrtf(total / (float)n + eps);
  for (int i = 0; i < n; i++) {
    const float v = tto_round_bf16(act_get(l, xdt, i) + act_get(r, xdt, i));
    act_put(res_out, xdt, i, v);
    act_put(out, odt, i, (v * inv) * act_get(w, wdt, i));
  }
  return 0;
}

/* silu(g) * u = (g / (1 + exp(-g))) * u (triton_kernels.py:2761-2774) */
int tto_silu_mul(const void* g, const void* u, void* out, int dt, int n) {
  for (int i = 0; i < n; i++) {
    const float gv = act_get(g, dt, i);
    act_put(out, dt, i, (gv / (1.0f + tto_exp_f32(-gv))) * act_get(u, dt, i));
  }
  return 0;
}

/* gpt-oss SwiGLU on interleaved gate/up (triton_kernels.py:2778-2793) */
int tto_interleaved_swiglu(const void* gu, void* out, int dt, int rows, int n, float alpha, float limit) {
  for (int r = 0; r < rows; r++)
    for (int i = 0; i < n; i++) {
      float g = act_get(gu, dt, (int64_t)r * 2 * n + 2 * i), u = act_get(gu, dt, (int64_t)r * 2 * n + 2 * i + 1);
      g = fminf(g, limit);
      u = fmaxf(fminf(u, limit), -limit);
      act_put(out, dt, (int64_t)r * n + i, ((u + 1.0f) * g) / (1.0f + tto_exp_f32(-g * alpha)));
    }
  return 0;
}

/* sum_e experts[e] * scores[e] in expert order (triton_kernels.py:2797-2817) */
int tto_weighted_expert_sum(const void* ex, int dt, const void* sc, int sdt, void* out, int width, int count) {
  for (int i = 0; i < width; i++) {
    float acc = 0.0f;
    for (int e = 0; e < count; e++) acc = fmaf(act_get(ex, dt, (int64_t)e * width + i), act_get(sc, sdt, e), acc);
    act_put(out, dt, i, acc);
  }
  return 0;
}

/* RoPE with per-op rounding to the activation dtype (gpu_runtime.py:8696-8705). */
int tto_rope(void* q, void* k, int dt, const void* cos_row, const void* sin_row, int heads, int kv_heads, int head_dim) {
  const int half = head_dim / 2;
  for (int h = 0; h < heads + kv_heads; h++) {
    void* base = h < heads ? q : k;
    const int64_t off = (int64_t)(h < heads ? h : h - heads) * head_dim;
    for (int i = 0; i < half; i++) {
      const float c = act_get(cos_row, dt, i), s = act_get(sin_row, dt, i);
      const float a = act_get(base, dt, off + i), b = act_get(base, dt, off + i + half);
      const float ac = round_to(dt, a * c), bs = round_to(dt, b * s), bc = round_to(dt, b * c), as = round_to(dt, a * s);
      act_put(base, dt, off + i, ac - bs);
      act_put(base, dt, off + i + half, bc + as);
    }
  }
  return 0;
}

/* Per-head RMSNorm (triton_kernels.py:2618-2634) in the kernel's order: lane l sums the
 * squares of elements l, l + 64, ... as an fma chain, then the 64-lane butterfly. */
int tto_head_rms_norm(const void* x, int dt, const void* w, int wdt, void* out, int heads, int D, float eps) {
  for (int h = 0; h < heads; h++) {
    float s[64];
    for (int l = 0; l < 64; l++) {
      float a = 0.0f;
      for (int i = l; i < D; i += 64) {
        const float v = act_get(x, dt, (int64_t)h * D + i);
        a = fmaf(v, v, a);
      }
      s[l] = a;
    }
    xor_sum(s, 64, 1, 64);
    const float inv = 1.0f / sqrtf(s[0] / (float)D + eps);
    for (int i = 0; i < D; i++)
      act_put(out, dt, (int64_t)h * D + i, (act_get(x, dt, (int64_t)h * D + i) * inv) * act_get(w, wdt, i));
  }
  return 0;
}

/* Per-head RMSNorm + RoPE in place (triton_kernels.py:2691-2757) in the kernel's order:
 * lane l takes pairs (i, i + half), i = l, l + 64, ...: s = fma(a, a, s), s = fma(b, b, s);
 * 64-lane butterfly; a' = a * (inv * w[i]), b' = b * (inv * w[i + half]); binary32
 * rotation with cos/sin from the activation-dtype table row, rounded once. */
int tto_qk_head_rope(void* q, void* k, int dt, const void* qw, const void* kw, int wdt, const void* cos_row,
                     const void* sin_row, int heads, int kv_heads, int D, float eps) {
  const int half = D / 2;
  for (int hh = 0; hh < heads + kv_heads; hh++) {
    void* base = hh < heads ? q : k;
    const void* w = hh < heads ? qw : kw;
    const int64_t off = (int64_t)(hh < heads ? hh : hh - heads) * D;
    float s[64];
    for (int l = 0; l < 64; l++) {
      float a = 0.0f;
      for (int i = l; i < half; i += 64) {
        const float x1 = act_get(base, dt, off + i), x2 = act_get(base, dt, off + i + half);
        a = fmaf(x1, x1, a);
        a = fmaf(x2, x2, a);
      }
      s[l] = a;
    }
    xor_sum(s, 64, 1, 64);
    const float inv = 1.0f / sqrtf(s[0] / (float)D + eps);
    for (int i = 0; i < half; i++) {
      const float an = act_get(base, dt, off + i) * (inv * act_get(w, wdt, i));
      const float bn = act_get(base, dt, off + i + half) * (inv * act_get(w, wdt, i + half));
      const float c = act_get(cos_row, dt, i), sn = act_get(sin_row, dt, i);
      act_put(base, dt, off + i, an * c - bn * sn);
      act_put(base, dt, off + i + half, bn * c + an * sn);
    }
  }
  return 0;
}

/* ------------------------------------------------------------ attention */

/*
 * Single-token GQA attention (triton_kernels.py:15-109) in the kernel's split-KV
 * order (thintensor_amd/csrc/attention.hip): 64-token chunks, score = fma chain over
 * d times scale, chunk max, p = exp(s - m), l = 64-lane butterfly, o = fma over the
 * chunk's tokens; chunks combined in order with an optional sink.
 * keys/values: [kv_heads][...] with strides (elements).
 */
int tto_attention(const void* q, const void* keys, const void* values, int dt, int64_t k_head, int64_t k_tok,
                  int64_t v_head, int64_t v_tok, const void* sinks, int sdt, int tokens, int heads, int kv_heads,
                  int D, void* out) {
  const int G = heads / kv_heads;
  const int nc = (tokens + 63) / 64;
  const float scale = (float)(1.0 / sqrt((double)D));
#pragma omp parallel for schedule(static)
  for (int h = 0; h < heads; h++) {
    float* pm = (float*)malloc(sizeof(float) * (size_t)nc);
    float* pl = (float*)malloc(sizeof(float) * (size_t)nc);
    float* po = (float*)malloc(sizeof(float) * (size_t)nc * (size_t)D);
    const int kvh = h / G;
    for (int c = 0; c < nc; c++) {
      float s[64], p[64];
      float m = -INFINITY;
      for (int lane = 0; lane < 64; lane++) {
        const int t = c * 64 + lane;
        if (t < tokens) {
          float acc = 0.0f;
          for (int d = 0; d < D; d++)
            acc = fmaf(act_get(q, dt, (int64_t)h * D + d), act_get(keys, dt, kvh * k_head + (int64_t)t * k_tok + d), acc);
          s[lane] = acc * scale;
        } else {
          s[lane] = -INFINITY;
        }
        m = fmaxf(m, s[lane]);
      }
      for (int lane = 0; lane < 64; lane++) p[lane] = (c * 64 + lane < tokens) ? tto_exp_f32(s[lane] - m) : 0.0f;
      float l[64];
      memcpy(l, p, sizeof l);
      xor_sum(l, 64, 1, 64);
      pm[c] = m;
      pl[c] = l[0];
      const int nt = tokens - c * 64 < 64 ? tokens - c * 64 : 64;
      for (int d = 0; d < D; d++) {
        float o = 0.0f;
        for (int tt = 0; tt < nt; tt++) o = fmaf(p[tt], act_get(values, dt, kvh * v_head + (int64_t)(c * 64 + tt) * v_tok + d), o);
        po[(size_t)c * D + d] = o;
      }
    }
    float M = -INFINITY, sink = 0.0f;
    if (sinks) {
      sink = act_get(sinks, sdt, h);
      M = sink;
    }
    for (int c = 0; c < nc; c++) M = fmaxf(M, pm[c]);
    float den = sinks ? tto_exp_f32(sink - M) : 0.0f;
    for (int c = 0; c < nc; c++) den = fmaf(pl[c], tto_exp_f32(pm[c] - M), den);
    for (int d = 0; d < D; d++) {
      float acc = 0.0f;
      for (int c = 0; c < nc; c++) acc = fmaf(po[(size_t)c * D + d], tto_exp_f32(pm[c] - M), acc);
      act_put(out, dt, (int64_t)h * D + d, acc / den);
    }
    free(pm);
    free(pl);
    free(po);
  }
  return 0;
}

/* ------------------------------------------------------------ router / argmax */

/* Top-k by iterated argmax (lowest index on ties) + softmax (triton_kernels.py:2821-2851). */
static void topk_softmax(const float* lg, int E, int k, int renorm, int32_t* idx, float* score) {
  float maximum = -INFINITY;
  for (int e = 0; e < E; e++) maximum = fmaxf(maximum, lg[e]);
  char* taken = (char*)calloc((size_t)E, 1);
  for (int s = 0; s < k; s++) {
    int bi = -1;
    float bv = 0.0f;
    for (int e = 0; e < E; e++) {
      if (taken[e]) continue;
      if (bi < 0 || lg[e] > bv) { bi = e; bv = lg[e]; }
    }
    taken[bi] = 1;
    idx[s] = bi;
    score[s] = bv;
  }
  free(taken);
  float den = 0.0f;
  if (renorm) for (int s = 0; s < k; s++) den = den + tto_exp_f32(score[s] - maximum);
  else for (int e = 0; e < E; e++) den = den + tto_exp_f32(lg[e] - maximum);
  for (int s = 0; s < k; s++) score[s] = tto_exp_f32(score[s] - maximum) / den;
}

/* Router GEMV (64 lanes per row) + bf16 logits + bias + top-k + softmax
 * (triton_kernels.py:2855-2921). */
int tto_router(const void* w, int wdt, int64_t w_row, const void* x, int xdt, int H, const void* bias, int bdt, int E,
               int k, int renorm, int32_t* idx, void* scores, int odt) {
  float lg[1024], sc[1024];
  const int fmt = wdt == TTO_BF16 ? FMT_BF16W : FMT_F16W;
  for (int e = 0; e < E; e++) {
    float v = tto_gemv_row(fmt, SM_NONE, (const uint8_t*)w + (size_t)(e * w_row) * 2, NULL, TTO_F32, 0, 0, 0, x, xdt,
                           H, 1, 64);
    v = tto_round_bf16(v);
    if (bias) v = tto_round_bf16(v + act_get(bias, bdt, e));
    lg[e] = v;
  }
  topk_softmax(lg, E, k, renorm, idx, sc);
  for (int s = 0; s < k; s++) act_put(scores, odt, s, sc[s]);
  return 0;
}

int tto_topk(const void* logits, int ldt, int E, int k, int renorm, int32_t* idx, void* scores, int odt) {
  float* lg = (float*)malloc(sizeof(float) * (size_t)E);
  float* sc = (float*)malloc(sizeof(float) * (size_t)k);
  for (int e = 0; e < E; e++) lg[e] = act_get(logits, ldt, e);
  topk_softmax(lg, E, k, renorm, idx, sc);
  for (int s = 0; s < k; s++) act_put(scores, odt, s, sc[s]);
  free(lg);
  free(sc);
  return 0;
}

/* torch.argmax over rounded logits: first index of the maximum, NaN wins. */
int64_t tto_argmax(const void* logits, int dt, int64_t n) {
  int64_t bi = 0;
  float bv = act_get(logits, dt, 0);
  for (int64_t i = 1; i < n; i++) {
    const float v = act_get(logits, dt, i);
    if (bv != bv) break;
    if (v != v || v > bv) { bi = i; bv = v; }
  }
  return bi;
}
