// Batched small-M dequant GEMM: y[m] = W x[m] for M activation rows.
//
//   * M < 16: the GEMV engine with up to four activation rows per wave (every
//     weight word decoded once, one fma chain per activation row), so row m equals
//     the single-row GEMV bit for bit;
//   * M >= 16: MFMA.  Each wave owns 16 output rows and all M (<= 64, in tiles of
//     16) activation rows; per quantisation group of 128 columns it issues four
//     v_mfma_f32_16x16x32_f16 with the dequantised weights as the A operand and the
//     activations (staged in LDS per 256-column slice) as the B operand, then scales
//     the group's fp32 tile (int4) or accumulates it (fp8, row scale at the end).
//     MFMA sums products in a hardware-defined order, so this path matches the
//     dequantise-then-matmul reference to the stated tolerance, not bit for bit.
//   * the M-row lm_head argmax runs the GEMV engine with four activation rows per
//     launch and one argmax key per (wave, row); a finishing kernel picks each row's
//     token, as tt_matvec_argmax does for one row.
#include "gemv_impl.h"

#include <type_traits>

using namespace tt;

namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int kSlice = 256;   // columns of x staged in LDS per step (two int4 groups)

enum class WFmt : int { kInt4G128 = 0, kFp8Row = 1 };

struct MfmaParams {
  const uint8_t* w;
  int64_t w_row;        // bytes between weight rows
  const void* s;        // int4: fp16 [N, K/128] (s_row elements between rows); fp8: fp32 [N]
  int64_t s_row;
  const uint16_t* x;    // fp16 [M, x_row]
  int64_t x_row;
  uint16_t* out;        // fp16 [M, out_row]
  int64_t out_row;
  int m, n, k;
};

// Weights of one 128-column group for this lane: row n0 + lane % 16, columns
// 128 g + 32 (lane / 16) + [0, 32).
// int4 chunks carry the group scales of the four output rows the lane accumulates
// (rows n0 + 4 (lane / 16) + i), requested together with the weights.
template <WFmt W>
struct WChunk {
  uint32_t w[W == WFmt::kInt4G128 ? 4 : 8];
  f16_t sc[W == WFmt::kInt4G128 ? 4 : 1];
};

template <WFmt W>
__device__ __forceinline__ WChunk<W> load_chunk(const MfmaParams& P, int row, int grp, int lane, int n0) {
  WChunk<W> c;
  if constexpr (W == WFmt::kInt4G128) {
    const uint4 v = *reinterpret_cast<const uint4*>(P.w + (int64_t)row * P.w_row + (int64_t)grp * 64 + 16 * (lane >> 4));
    c.w[0] = v.x; c.w[1] = v.y; c.w[2] = v.z; c.w[3] = v.w;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int r = n0 + 4 * (lane >> 4) + i;
      c.sc[i] = reinterpret_cast<const f16_t*>(P.s)[(int64_t)(r < P.n ? r : P.n - 1) * P.s_row + grp];
    }
  } else {
    const uint4* p = reinterpret_cast<const uint4*>(P.w + (int64_t)row * P.w_row + (int64_t)grp * 128 + 32 * (lane >> 4));
    const uint4 a = p[0], b = p[1];
    c.w[0] = a.x; c.w[1] = a.y; c.w[2] = a.z; c.w[3] = a.w;
    c.w[4] = b.x; c.w[5] = b.y; c.w[6] = b.z; c.w[7] = b.w;
  }
  return c;
}

// A operand of step q (8 consecutive columns of this lane's 32) as exact fp16 values.
template <WFmt W>
__device__ __forceinline__ h8 a_operand(const WChunk<W>& c, int q) {
  h8 a;
  if constexpr (W == WFmt::kInt4G128) {
    _Float16 v[8];
    decode_word8<Fmt::kInt4Sym>(c.w[q], v);
#pragma unroll
    for (int e = 0; e < 8; e++) a[e] = v[e];
  } else {
#pragma unroll
    for (int h = 0; h < 2; h++) {
      const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8(c.w[2 * q + h], false);
      const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8(c.w[2 * q + h], true);
      a[4 * h + 0] = (_Float16)lo[0];
      a[4 * h + 1] = (_Float16)lo[1];
      a[4 * h + 2] = (_Float16)hi[0];
      a[4 * h + 3] = (_Float16)hi[1];
    }
  }
  return a;
}

template <WFmt W, int MT>
__global__ __launch_bounds__(256) void mfma_gemm_kernel(MfmaParams P) {
  // Two LDS buffers of activation slices: slice s + 1 is loaded into registers while
  // slice s computes, then written to the other buffer (one barrier per slice).  The
  // weights of a slice are requested kAhead slices before they are used.
  constexpr int kAhead = 4;
  constexpr int XS = MT * 16 * kSlice;                 // halves per buffer
  constexpr int XV = XS / 8 / 256;                     // 16-byte pieces per thread per slice
  __shared__ __attribute__((aligned(16))) uint16_t xs[2 * XS];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n0 = (blockIdx.x * 4 + wave) * 16;
  const int arow = n0 + (lane & 15);                 // weight row this lane loads (A operand)
  const int lrow = arow < P.n ? arow : P.n - 1;
  const int g = lane >> 4;
  const int slices = P.k / kSlice;
  auto load_x = [&](int sl, uint4* regs) {
#pragma unroll
    for (int v = 0; v < XV; v++) {
      const int i = threadIdx.x + 256 * v;
      const int r = i / (kSlice / 8), c8 = i - r * (kSlice / 8);
      regs[v] = r < P.m ? *reinterpret_cast<const uint4*>(P.x + (int64_t)r * P.x_row + (int64_t)sl * kSlice + 8 * c8)
                        : (uint4){0u, 0u, 0u, 0u};
    }
  };
  auto store_x = [&](int buf, const uint4* regs) {
#pragma unroll
    for (int v = 0; v < XV; v++) {
      const int i = threadIdx.x + 256 * v;
      const int r = i / (kSlice / 8), c8 = i - r * (kSlice / 8);
      *reinterpret_cast<uint4*>(xs + buf * XS + r * kSlice + 8 * c8) = regs[v];
    }
  };
  f4 acc[MT];
#pragma unroll
  for (int t = 0; t < MT; t++) acc[t] = (f4){0.0f, 0.0f, 0.0f, 0.0f};
  WChunk<W> ring[kAhead][kSlice / 128];
#pragma unroll
  for (int u = 0; u < kAhead; u++)
    if (u < slices)
#pragma unroll
      for (int gs = 0; gs < kSlice / 128; gs++) ring[u][gs] = load_chunk<W>(P, lrow, u * (kSlice / 128) + gs, lane, n0);
  uint4 xr[XV];
  load_x(0, xr);
  store_x(0, xr);
  __syncthreads();
  for (int s0 = 0; s0 < slices; s0 += kAhead) {
#pragma unroll
    for (int u = 0; u < kAhead; u++) {
      const int sl = s0 + u;
      if (sl < slices) {
        if (sl + 1 < slices) load_x(sl + 1, xr);
        const uint16_t* xb = xs + (sl & 1) * XS;
#pragma unroll
        for (int gs = 0; gs < kSlice / 128; gs++) {
          f4 part[MT];
#pragma unroll
          for (int t = 0; t < MT; t++) part[t] = (f4){0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
          for (int q = 0; q < 4; q++) {
            const h8 a = a_operand<W>(ring[u][gs], q);
#pragma unroll
            for (int t = 0; t < MT; t++) {
              const h8 b = *reinterpret_cast<const h8*>(xb + (16 * t + (lane & 15)) * kSlice + 128 * gs + 32 * g + 8 * q);
              if constexpr (W == WFmt::kInt4G128) part[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, part[t], 0, 0, 0);
              else acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, acc[t], 0, 0, 0);
            }
          }
          if constexpr (W == WFmt::kInt4G128) {
            // group scale of the four output rows this lane holds (rows n0 + 4g + i)
#pragma unroll
            for (int t = 0; t < MT; t++)
#pragma unroll
              for (int i = 0; i < 4; i++) acc[t][i] = __builtin_fmaf(part[t][i], to_f32(ring[u][gs].sc[i]), acc[t][i]);
          }
        }
        if (sl + kAhead < slices) {
#pragma unroll
          for (int gs = 0; gs < kSlice / 128; gs++)
            ring[u][gs] = load_chunk<W>(P, lrow, (sl + kAhead) * (kSlice / 128) + gs, lane, n0);
        }
        if (sl + 1 < slices) store_x((sl + 1) & 1, xr);
        __syncthreads();
      }
    }
  }
  // out[m][n]: lane holds rows n0 + 4g + i of activation row 16t + lane % 16
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int r = n0 + 4 * g + i;
    if (r >= P.n) continue;
    float rs = 1.0f;
    if constexpr (W == WFmt::kFp8Row) rs = reinterpret_cast<const float*>(P.s)[r];
#pragma unroll
    for (int t = 0; t < MT; t++) {
      const int m = 16 * t + (lane & 15);
      if (m < P.m) {
        const float v = W == WFmt::kFp8Row ? acc[t][i] * rs : acc[t][i];
        P.out[(int64_t)m * P.out_row + r] = f32_to_f16_bits(v);
      }
    }
  }
}

template <WFmt W>
int launch_mfma(const MfmaParams& P, hipStream_t st, const char* what) {
  const int blocks = (P.n + 63) / 64;
  const int mt = (P.m + 15) / 16;
  switch (mt) {
    case 1: hipLaunchKernelGGL((mfma_gemm_kernel<W, 1>), dim3(blocks), dim3(256), 0, st, P); break;
    case 2: hipLaunchKernelGGL((mfma_gemm_kernel<W, 2>), dim3(blocks), dim3(256), 0, st, P); break;
    case 3: hipLaunchKernelGGL((mfma_gemm_kernel<W, 3>), dim3(blocks), dim3(256), 0, st, P); break;
    default: hipLaunchKernelGGL((mfma_gemm_kernel<W, 4>), dim3(blocks), dim3(256), 0, st, P); break;
  }
  return check_launch(what);
}

// Up to four activation rows per GEMV launch (VALU, bit-exact per row).
template <Fmt F, SMode SM, typename ST, int ROWS, int L, bool AM>
int launch_rows(GemvParams P, int64_t m_total, int64_t x_row, int64_t out_row, int lpr, hipStream_t st,
                const char* what, int64_t partial_stride) {
  P.x_slot = x_row;
  P.out_slot = out_row;
  const uint16_t* x0 = static_cast<const uint16_t*>(P.x);
  uint8_t* out0 = static_cast<uint8_t*>(P.seg[0].out);
  uint64_t* part0 = P.am_partials;
  for (int64_t m0 = 0; m0 < m_total;) {
    const int64_t left = m_total - m0;
    const int mr = left >= 4 ? 4 : (left >= 2 ? 2 : 1);
    GemvParams Q = P;
    Q.x = x0 + m0 * x_row;
    if (out0) Q.seg[0].out = out0 + m0 * out_row * 2;
    if (AM) Q.am_partials = part0 + m0 * partial_stride;
    int rc;
    switch (mr) {
      case 4: rc = launch_lpr<F, SM, f16_t, f16_t, ST, ROWS, L, Pro::kLoad, false, 1, 4>(lpr, Q, 1, st, what); break;
      case 2: rc = launch_lpr<F, SM, f16_t, f16_t, ST, ROWS, L, Pro::kLoad, false, 1, 2>(lpr, Q, 1, st, what); break;
      default: rc = launch_lpr<F, SM, f16_t, f16_t, ST, ROWS, L, Pro::kLoad, false, 1, 1>(lpr, Q, 1, st, what); break;
    }
    if (rc) return rc;
    m0 += mr;
  }
  return TT_OK;
}

// Token of each activation row.  Rows go to GEMV launches of four (then two, then
// one for the tail); the launch holding rows m0 .. m0 + mr - 1 writes the key of
// (wave w, row r) at partials[m0 * per + w * mr + r].
__global__ __launch_bounds__(256) void argmax_rows_kernel(const uint64_t* partials, int64_t per, int64_t m_total,
                                                          int64_t* out_idx, float* out_val) {
  const int64_t m = blockIdx.x;
  const int64_t full = m_total / 4 * 4;
  int64_t m0, mr;
  if (m < full) {
    m0 = m / 4 * 4;
    mr = 4;
  } else if (m_total - full >= 2 && m < full + 2) {
    m0 = full;
    mr = 2;
  } else {
    m0 = m;
    mr = 1;
  }
  const uint64_t* base = partials + m0 * per + (m - m0);
  __shared__ uint64_t red[256];
  uint64_t best = 0;
  for (int64_t i = threadIdx.x; i < per; i += 256) {
    const uint64_t k = base[i * mr];
    best = k > best ? k : best;
  }
  red[threadIdx.x] = best;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if (threadIdx.x < s) red[threadIdx.x] = red[threadIdx.x + s] > red[threadIdx.x] ? red[threadIdx.x + s] : red[threadIdx.x];
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    const uint64_t k = red[0];
    const uint32_t o = (uint32_t)(k >> 32);
    const uint32_t bits = o == 0xffffffffu ? 0x7fc00000u : ((o & 0x80000000u) ? (o & 0x7fffffffu) : ~o);
    out_idx[m] = (int64_t)(0xffffffffu - (uint32_t)k);
    if (out_val) out_val[m] = __builtin_bit_cast(float, bits);
  }
}

}  // namespace

extern "C" int tt_int4_batched_matvec(const void* packed, int64_t w_row_bytes, const void* scales, int64_t s_row,
                                      const void* x, int64_t x_row, void* out, int64_t out_row, int64_t m,
                                      int64_t rows, int64_t cols, int64_t group_size, void* stream) {
  const char* what = "int4_batched_matvec";
  TT_UNSUPPORTED(group_size == 128, "%s: batched int4 uses group size 128", what);
  TT_REQUIRE(cols > 0 && cols % 256 == 0 && cols <= 8192, "%s: cols must be a multiple of 256 up to 8192", what);
  TT_REQUIRE(m >= 1 && m <= 64, "%s: 1 to 64 activation rows", what);
  TT_REQUIRE(rows > 0 && rows < (1 << 28), "%s: bad rows", what);
  TT_REQUIRE(packed && aligned(packed, 16) && w_row_bytes % 16 == 0 && w_row_bytes >= cols / 2,
             "%s: packed weights must be 16-byte aligned rows", what);
  TT_REQUIRE(scales && x && out && aligned(x, 16) && x_row % 8 == 0 && x_row >= cols && out_row >= rows,
             "%s: null or misaligned pointer / bad row strides", what);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (m >= 16) {
    MfmaParams P{static_cast<const uint8_t*>(packed), w_row_bytes, scales, s_row, static_cast<const uint16_t*>(x),
                 x_row, static_cast<uint16_t*>(out), out_row, (int)m, (int)rows, (int)cols};
    return launch_mfma<WFmt::kInt4G128>(P, st, what);
  }
  GemvParams P{};
  P.nseg = 1;
  P.seg[0] = Seg{static_cast<const uint8_t*>(packed), w_row_bytes, scales, s_row, 1, out, (int)rows};
  P.x = x;
  P.cols = (int)cols;
  const int lpr = tt_gemv_lanes_per_row(cols / 32, 4);
  return launch_rows<Fmt::kInt4Sym, SMode::kGroup, f16_t, 2, 4, false>(P, m, x_row, out_row, lpr, st, what, 0);
}

extern "C" int tt_scaled_batched_matvec(const void* weight, int64_t w_row_bytes, const float* scales, const void* x,
                                        int64_t x_row, void* out, int64_t out_row, int64_t m, int64_t rows,
                                        int64_t cols, void* stream) {
  const char* what = "scaled_batched_matvec";
  TT_REQUIRE(cols > 0 && cols % 256 == 0 && cols <= 8192, "%s: cols must be a multiple of 256 up to 8192", what);
  TT_REQUIRE(m >= 1 && m <= 64, "%s: 1 to 64 activation rows", what);
  TT_REQUIRE(rows > 0 && rows < (1 << 28), "%s: bad rows", what);
  TT_REQUIRE(weight && aligned(weight, 16) && w_row_bytes % 16 == 0 && w_row_bytes >= cols,
             "%s: fp8 weights must be 16-byte aligned rows", what);
  TT_REQUIRE(scales && x && out && aligned(x, 16) && x_row % 8 == 0 && x_row >= cols && out_row >= rows,
             "%s: null or misaligned pointer / bad row strides", what);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (m >= 16) {
    MfmaParams P{static_cast<const uint8_t*>(weight), w_row_bytes, scales, 1, static_cast<const uint16_t*>(x), x_row,
                 static_cast<uint16_t*>(out), out_row, (int)m, (int)rows, (int)cols};
    return launch_mfma<WFmt::kFp8Row>(P, st, what);
  }
  GemvParams P{};
  P.nseg = 1;
  P.seg[0] = Seg{static_cast<const uint8_t*>(weight), w_row_bytes, scales, 1, 0, out, (int)rows};
  P.x = x;
  P.cols = (int)cols;
  const int lpr = tt_gemv_lanes_per_row(cols / 32, 1);
  return launch_rows<Fmt::kFp8, SMode::kRow, float, 2, 1, false>(P, m, x_row, out_row, lpr, st, what, 0);
}

extern "C" int64_t tt_matvec_argmax_batched_partials(int64_t m, int64_t rows, int64_t cols) {
  return m * tt_matvec_argmax_partials(rows, cols);
}

extern "C" int tt_matvec_argmax_batched(const void* weight, int64_t w_row, const void* x, int64_t x_row, int64_t m,
                                        void* logits, int64_t logits_row, int64_t rows, int64_t cols,
                                        uint64_t* partials, int64_t partials_capacity, int64_t* out_idx,
                                        float* out_val, void* stream) {
  const char* what = "matvec_argmax_batched";
  TT_REQUIRE(m >= 1 && m <= 1024, "%s: 1 to 1024 activation rows", what);
  TT_REQUIRE(weight && aligned(weight, 16) && (w_row * 2) % 16 == 0 && w_row >= cols, "%s: bad weight layout", what);
  TT_REQUIRE(x && aligned(x, 16) && x_row % 8 == 0 && x_row >= cols && partials && out_idx,
             "%s: null or misaligned pointer", what);
  TT_REQUIRE(rows > 0 && rows < (1LL << 31) && cols > 0 && cols % 32 == 0 && cols <= 8192, "%s: bad shape", what);
  TT_REQUIRE(logits == nullptr || logits_row >= rows, "%s: bad logits stride", what);
  const int64_t per = tt_matvec_argmax_partials(rows, cols);
  TT_REQUIRE(partials_capacity >= m * per, "%s: partials buffer needs %lld entries", what, (long long)(m * per));
  GemvParams P{};
  P.nseg = 1;
  P.seg[0] = Seg{static_cast<const uint8_t*>(weight), w_row * 2, nullptr, 0, 0, logits, (int)rows};
  P.x = x;
  P.cols = (int)cols;
  P.am_partials = partials;
  const int lpr = tt_gemv_lanes_per_row(cols / 32, 1);
  hipStream_t st = static_cast<hipStream_t>(stream);
  int rc = launch_rows<Fmt::kF16W, SMode::kNone, float, 2, 1, true>(P, m, x_row, logits ? logits_row : 0, lpr, st,
                                                                    what, per);
  if (rc) return rc;
  hipLaunchKernelGGL(argmax_rows_kernel, dim3((unsigned)m), dim3(256), 0, st, partials, per, m, out_idx, out_val);
  return check_launch(what);
}
