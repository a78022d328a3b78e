// Dequant-fused GEMV kernels (dense, multi-matrix and selected-expert) for gfx950.
//
// Design (memory-bound regime):
//   * packed weights stream from HBM with 128-bit (or 64/32-bit for q2/q1 chunks)
//     coalesced loads: a wave reads LPR consecutive chunks of one row per round;
//   * the activation vector is staged once per workgroup in LDS and each lane keeps
//     its 32-element slice in registers for ROWS rows at a time;
//   * unpacking happens in registers (magic-number fp16 construction, exact), the
//     multiply-accumulate is an IEEE fp32 fma chain (v_fma_mix_f32 for fp16 inputs);
//   * rows are reduced with wave-level butterflies; per-group scales are applied to
//     the group sums, as the reference does (triton_kernels.py:1628-1651).
// The reduction order is documented in tt_gemv.h and restated in oracle/.
#include "tt_abi_internal.h"
#include "tt_gemv.h"

namespace tt {

enum class SMode : int { kNone = 0, kRow = 1, kGroup = 2, kGroupAff = 3, kBlockE8 = 4 };

struct Seg {
  const uint8_t* w;     // weight bytes of expert 0 / the matrix
  int64_t w_row;        // bytes between rows
  const void* s;        // scales
  int64_t s_row, s_grp; // scale element strides
  void* out;            // output (slot 0)
  int rows;
};

struct GemvParams {
  Seg seg[3];
  int nseg;
  int seg_end[3];          // cumulative row ends
  const void* x;
  int64_t x_slot;          // activation elements between slots (0: shared vector)
  const int32_t* experts;  // expert id per slot (nullptr: dense)
  int64_t w_expert;        // bytes between experts
  int64_t s_expert;        // scale elements between experts
  int64_t out_slot;        // output elements between slots
  int64_t s_pair;          // affine: element offset of the second scale value
  int aff_zero;            // affine pair holds (s, z) instead of (s, m)
  int cols;
  int L;                   // chunks per quantisation group (group modes)
  int e8_extra;            // extra power of two folded into E8M0 block scales
};

template <Fmt F, SMode SM, typename XT, typename OT, typename ST, int LPR, int ROWS>
__global__ __launch_bounds__(256) void gemv_kernel(GemvParams P) {
  extern __shared__ uint32_t xs_lds[];
  constexpr int B = FmtInfo<F>::kBytes;
  constexpr int SUBS = 64 / LPR;
  const int slot = blockIdx.y;
  const int nwords = P.cols >> 1;
  {
    const uint32_t* xg = reinterpret_cast<const uint32_t*>(reinterpret_cast<const uint16_t*>(P.x) + (int64_t)slot * P.x_slot);
    for (int i = threadIdx.x; i < nwords; i += blockDim.x) xs_lds[i] = xg[i];
  }
  __syncthreads();

  int64_t woff = 0, soff = 0;
  if (P.experts != nullptr) {
    const int64_t e = P.experts[slot];
    woff = e * P.w_expert;
    soff = e * P.s_expert;
  }
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int sub = lane / LPR;
  const int l = lane % LPR;
  const int nchunks = P.cols >> 5;
  const int rounds = (nchunks + LPR - 1) / LPR;
  const int total = P.seg_end[P.nseg - 1];
  const int per_iter = ROWS * SUBS;
  const int waves_total = gridDim.x * (blockDim.x >> 6);

  for (int base = (blockIdx.x * (blockDim.x >> 6) + wave) * per_iter; base < total; base += waves_total * per_iter) {
    const uint8_t* wrow[ROWS];
    const ST* sptr[ROWS];
    int64_t sgrp[ROWS];
    OT* optr[ROWS];
    bool rv[ROWS];
#pragma unroll
    for (int i = 0; i < ROWS; i++) {
      const int row = base + i * SUBS + sub;
      rv[i] = row < total;
      int s = 0;
      if (P.nseg > 1 && row >= P.seg_end[0]) s = 1;
      if (P.nseg > 2 && row >= P.seg_end[1]) s = 2;
      const Seg& sgm = s == 0 ? P.seg[0] : (s == 1 ? P.seg[1] : P.seg[2]);
      const int lrow = row - (s ? P.seg_end[s - 1] : 0);
      wrow[i] = sgm.w + woff + (int64_t)lrow * sgm.w_row;
      sptr[i] = reinterpret_cast<const ST*>(sgm.s) + soff + (int64_t)lrow * sgm.s_row;
      sgrp[i] = sgm.s_grp;
      optr[i] = reinterpret_cast<OT*>(sgm.out) + (int64_t)slot * P.out_slot + lrow;
    }
    float acc[ROWS];
#pragma unroll
    for (int i = 0; i < ROWS; i++) acc[i] = 0.0f;

    for (int r = 0; r < rounds; r++) {
      const int j = r * LPR + l;
      const bool cv = j < nchunks;
      uint32_t xw[16];
      if (cv) {
        const uint4* xp = reinterpret_cast<const uint4*>(xs_lds + j * 16);
#pragma unroll
        for (int q = 0; q < 4; q++) {
          uint4 v = xp[q];
          xw[4 * q] = v.x; xw[4 * q + 1] = v.y; xw[4 * q + 2] = v.z; xw[4 * q + 3] = v.w;
        }
      } else {
#pragma unroll
        for (int q = 0; q < 16; q++) xw[q] = 0u;
      }
      Raw<B> raw[ROWS];
#pragma unroll
      for (int i = 0; i < ROWS; i++) {
        if (cv && rv[i]) raw[i] = load_raw<B>(wrow[i] + (int64_t)j * B);
        else {
#pragma unroll
          for (int q = 0; q < B / 4; q++) raw[i].w[q] = 0u;
        }
      }
      float xsum = 0.0f;
      if constexpr (SM == SMode::kGroupAff) {
        if (cv) {
#pragma unroll
          for (int e = 0; e < 32; e++) xsum = xsum + xv<XT>(xw, e);
        }
        xsum = xor_sum(xsum, 1, P.L);
      }
#pragma unroll
      for (int i = 0; i < ROWS; i++) {
        float p = cv ? chunk_dot<F, XT>(raw[i], xw) : 0.0f;
        if constexpr (SM == SMode::kNone || SM == SMode::kRow) {
          acc[i] = acc[i] + p;
        } else if constexpr (SM == SMode::kBlockE8) {
          float t = 0.0f;
          if (cv && rv[i]) {
            const int e = (int)reinterpret_cast<const uint8_t*>(sptr[i])[j];
            float q = p;
            if (P.e8_extra) q = q * pow2i(P.e8_extra);
            t = q * pow2i(e - 127);
          }
          acc[i] = acc[i] + t;
        } else {
          p = xor_sum(p, 1, P.L);
          float t = 0.0f;
          if (cv && rv[i]) {
            const int g = j / P.L;
            const float s = to_f32(sptr[i][(int64_t)g * sgrp[i]]);
            if constexpr (SM == SMode::kGroupAff) {
              float m = to_f32(sptr[i][(int64_t)g * sgrp[i] + P.s_pair]);
              if (P.aff_zero) m = -(m * s);
              t = __builtin_fmaf(xsum, m, p * s);
            } else {
              t = p * s;
            }
          }
          acc[i] = acc[i] + t;
        }
      }
    }
#pragma unroll
    for (int i = 0; i < ROWS; i++) {
      float v;
      if constexpr (SM == SMode::kNone || SM == SMode::kRow) {
        v = xor_sum(acc[i], 1, LPR);
        if constexpr (SM == SMode::kRow) {
          if (rv[i]) v = v * to_f32(sptr[i][0]);
        }
      } else if constexpr (SM == SMode::kBlockE8) {
        v = xor_sum(acc[i], 1, LPR);
      } else {
        v = xor_sum(acc[i], P.L, LPR);
      }
      if (rv[i] && l == i) store<OT>(optr[i], v);
    }
  }
}

// ------------------------------------------------------------------ dispatch

template <Fmt F, SMode SM, typename XT, typename OT, typename ST, int LPR, int ROWS>
static int launch_one(const GemvParams& P, int slots, hipStream_t stream, const char* what) {
  constexpr int SUBS = 64 / LPR;
  const int total = P.seg_end[P.nseg - 1];
  const int rows_per_block = 4 * ROWS * SUBS;
  int blocks = (total + rows_per_block - 1) / rows_per_block;
  if (blocks < 1) blocks = 1;
  const size_t lds = (size_t)P.cols * 2;
  hipLaunchKernelGGL((gemv_kernel<F, SM, XT, OT, ST, LPR, ROWS>), dim3(blocks, slots), dim3(256), lds, stream, P);
  return check_launch(what);
}

template <Fmt F, SMode SM, typename XT, typename OT, typename ST, int ROWS>
static int launch_lpr(int lpr, const GemvParams& P, int slots, hipStream_t stream, const char* what) {
  switch (lpr) {
    case 64: return launch_one<F, SM, XT, OT, ST, 64, ROWS>(P, slots, stream, what);
    case 32: return launch_one<F, SM, XT, OT, ST, 32, ROWS>(P, slots, stream, what);
    case 16: return launch_one<F, SM, XT, OT, ST, 16, ROWS>(P, slots, stream, what);
    default: set_error("%s: invalid lanes per row %d", what, lpr); return TT_ERR_INVALID;
  }
}

template <Fmt F, SMode SM, typename ST, int ROWS>
static int launch_types(int x_dtype, int out_dtype, int lpr, const GemvParams& P, int slots, hipStream_t stream, const char* what) {
  if (x_dtype == TT_F16) {
    if (out_dtype == TT_F16) return launch_lpr<F, SM, f16_t, f16_t, ST, ROWS>(lpr, P, slots, stream, what);
    if (out_dtype == TT_F32) return launch_lpr<F, SM, f16_t, float, ST, ROWS>(lpr, P, slots, stream, what);
  } else if (x_dtype == TT_BF16) {
    if (out_dtype == TT_BF16) return launch_lpr<F, SM, bf16_t, bf16_t, ST, ROWS>(lpr, P, slots, stream, what);
    if (out_dtype == TT_F32) return launch_lpr<F, SM, bf16_t, float, ST, ROWS>(lpr, P, slots, stream, what);
  }
  set_error("%s: unsupported activation/output dtype pair (%d, %d); output must match the activation dtype or be fp32",
            what, x_dtype, out_dtype);
  return TT_ERR_UNSUPPORTED;
}

}  // namespace tt

using namespace tt;

extern "C" int tt_gemv_lanes_per_row(int64_t chunks, int64_t group_chunks) {
  if (chunks <= 0) return 0;
  int best = 0;
  double best_util = -1.0;
  const int cand[3] = {64, 32, 16};
  for (int c : cand) {
    if (group_chunks > 1 && (c % group_chunks) != 0) continue;
    const int64_t r = (chunks + c - 1) / c;
    const double util = (double)chunks / (double)(r * c);
    if (util > best_util + 1e-12) { best = c; best_util = util; }
  }
  return best;
}

namespace {

// Validates the common GEMV contract and fills group information.
int plan_groups(const char* what, int64_t cols, int64_t group_size, int* L, bool* row_mode) {
  TT_REQUIRE(cols > 0 && cols % 32 == 0, "%s: cols must be a positive multiple of 32 (got %lld)", what, (long long)cols);
  TT_REQUIRE(cols <= 32768, "%s: cols %lld exceeds the staged-activation limit 32768", what, (long long)cols);
  if (group_size >= cols) { *row_mode = true; *L = 1; return TT_OK; }
  *row_mode = false;
  TT_REQUIRE(group_size >= 32 && group_size % 32 == 0 && cols % group_size == 0,
             "%s: group_size %lld must be a multiple of 32 dividing cols %lld", what, (long long)group_size, (long long)cols);
  const int64_t Lg = group_size / 32;
  TT_UNSUPPORTED(Lg <= 64 && (Lg & (Lg - 1)) == 0, "%s: group_size %lld must be 32 * 2^k <= 2048", what, (long long)group_size);
  *L = (int)Lg;
  return TT_OK;
}

}  // namespace

extern "C" int tt_int4_scaled_matvec(const void* packed, int64_t w_row_bytes, const void* scales, int scale_dtype,
                                     int64_t s_row, int64_t s_group, int64_t s_pair, int affine, const void* x,
                                     int x_dtype, void* out, int out_dtype, int64_t rows, int64_t cols,
                                     int64_t group_size, void* stream) {
  const int64_t rows_arr[1] = {rows};
  const void* p_arr[1] = {packed};
  const int64_t wr_arr[1] = {w_row_bytes};
  const void* s_arr[1] = {scales};
  const int64_t sr_arr[1] = {s_row};
  const int64_t sg_arr[1] = {s_group};
  return tt_multi_int4_scaled_matvec(1, p_arr, wr_arr, s_arr, scale_dtype, sr_arr, sg_arr, s_pair, affine, rows_arr, x,
                                     x_dtype, out, out_dtype, cols, group_size, stream);
}

extern "C" int tt_multi_int4_scaled_matvec(int count, const void* const* packed, const int64_t* w_row_bytes,
                                           const void* const* scales, int scale_dtype, const int64_t* s_row,
                                           const int64_t* s_group, int64_t s_pair, int affine, const int64_t* rows,
                                           const void* x, int x_dtype, void* out, int out_dtype, int64_t cols,
                                           int64_t group_size, void* stream) {
  const char* what = "int4_scaled_matvec";
  TT_REQUIRE(count >= 1 && count <= 3, "%s: supports one to three matrices (got %d)", what, count);
  TT_REQUIRE(valid_act_dtype(x_dtype) && valid_out_dtype(out_dtype), "%s: bad dtype codes", what);
  TT_REQUIRE(scale_dtype == TT_F16 || scale_dtype == TT_F32, "%s: scales must be fp16 or fp32", what);
  TT_REQUIRE(x != nullptr && out != nullptr && aligned(x, 4), "%s: x must be a 4-byte aligned device pointer", what);
  int L = 1;
  bool row_mode = false;
  int rc = plan_groups(what, cols, group_size, &L, &row_mode);
  if (rc) return rc;
  GemvParams P{};
  P.nseg = count;
  int64_t acc_rows = 0;
  const size_t osz = out_dtype == TT_F32 ? 4 : 2;
  for (int i = 0; i < count; i++) {
    TT_REQUIRE(rows[i] > 0, "%s: rows must be positive", what);
    TT_REQUIRE(packed[i] != nullptr && aligned(packed[i], 16) && w_row_bytes[i] % 16 == 0 && w_row_bytes[i] >= cols / 2,
               "%s: packed weights must be 16-byte aligned with a row stride >= cols/2 that is a multiple of 16", what);
    TT_REQUIRE(scales[i] != nullptr, "%s: scales missing", what);
    P.seg[i].w = static_cast<const uint8_t*>(packed[i]);
    P.seg[i].w_row = w_row_bytes[i];
    P.seg[i].s = scales[i];
    P.seg[i].s_row = s_row[i];
    P.seg[i].s_grp = s_group[i];
    P.seg[i].out = static_cast<char*>(out) + acc_rows * osz;
    P.seg[i].rows = (int)rows[i];
    acc_rows += rows[i];
    P.seg_end[i] = (int)acc_rows;
  }
  TT_REQUIRE(acc_rows < (1LL << 30), "%s: too many rows", what);
  P.x = x;
  P.cols = (int)cols;
  P.L = L;
  P.s_pair = s_pair;
  const int lpr = tt_gemv_lanes_per_row(cols / 32, row_mode ? 1 : L);
  TT_UNSUPPORTED(lpr > 0, "%s: no lane mapping for cols %lld / group %lld", what, (long long)cols, (long long)group_size);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (affine) {
    TT_UNSUPPORTED(!row_mode, "%s: affine int4 needs group_size < cols", what);
    if (scale_dtype == TT_F16) return launch_types<Fmt::kInt4Aff, SMode::kGroupAff, f16_t, 4>(x_dtype, out_dtype, lpr, P, 1, st, what);
    return launch_types<Fmt::kInt4Aff, SMode::kGroupAff, float, 4>(x_dtype, out_dtype, lpr, P, 1, st, what);
  }
  if (row_mode) {
    if (scale_dtype == TT_F16) return launch_types<Fmt::kInt4Sym, SMode::kRow, f16_t, 4>(x_dtype, out_dtype, lpr, P, 1, st, what);
    return launch_types<Fmt::kInt4Sym, SMode::kRow, float, 4>(x_dtype, out_dtype, lpr, P, 1, st, what);
  }
  if (scale_dtype == TT_F16) return launch_types<Fmt::kInt4Sym, SMode::kGroup, f16_t, 4>(x_dtype, out_dtype, lpr, P, 1, st, what);
  return launch_types<Fmt::kInt4Sym, SMode::kGroup, float, 4>(x_dtype, out_dtype, lpr, P, 1, st, what);
}

extern "C" int tt_int4_selected_matvec(const void* packed, int64_t w_expert_bytes, int64_t w_row_bytes,
                                       const void* scales, int scale_dtype, int64_t s_expert, int64_t s_row,
                                       int64_t s_group, const void* x, int x_dtype, int64_t x_slot,
                                       const int32_t* expert_indices, int64_t selected, void* out, int out_dtype,
                                       int64_t out_slot, int64_t rows, int64_t cols, int64_t group_size,
                                       void* stream) {
  const char* what = "int4_selected_matvec";
  TT_REQUIRE(valid_act_dtype(x_dtype) && valid_out_dtype(out_dtype), "%s: bad dtype codes", what);
  TT_REQUIRE(scale_dtype == TT_F16 || scale_dtype == TT_F32, "%s: scales must be fp16 or fp32", what);
  TT_REQUIRE(selected >= 1 && selected <= 65535 && expert_indices != nullptr, "%s: need 1..65535 selected experts", what);
  TT_REQUIRE(packed && aligned(packed, 16) && w_row_bytes % 16 == 0 && w_expert_bytes % 16 == 0,
             "%s: packed weights must be 16-byte aligned", what);
  TT_REQUIRE(x && aligned(x, 4) && (x_slot % 2) == 0, "%s: x must be 4-byte aligned (even slot stride)", what);
  TT_REQUIRE(rows > 0 && rows < (1 << 30), "%s: bad rows", what);
  int L = 1;
  bool row_mode = false;
  int rc = plan_groups(what, cols, group_size, &L, &row_mode);
  if (rc) return rc;
  GemvParams P{};
  P.nseg = 1;
  P.seg[0] = Seg{static_cast<const uint8_t*>(packed), w_row_bytes, scales, s_row, s_group, out, (int)rows};
  P.seg_end[0] = (int)rows;
  P.x = x;
  P.x_slot = x_slot;
  P.experts = expert_indices;
  P.w_expert = w_expert_bytes;
  P.s_expert = s_expert;
  P.out_slot = out_slot;
  P.cols = (int)cols;
  P.L = L;
  const int lpr = tt_gemv_lanes_per_row(cols / 32, row_mode ? 1 : L);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (row_mode) {
    if (scale_dtype == TT_F16) return launch_types<Fmt::kInt4Sym, SMode::kRow, f16_t, 4>(x_dtype, out_dtype, lpr, P, (int)selected, st, what);
    return launch_types<Fmt::kInt4Sym, SMode::kRow, float, 4>(x_dtype, out_dtype, lpr, P, (int)selected, st, what);
  }
  if (scale_dtype == TT_F16) return launch_types<Fmt::kInt4Sym, SMode::kGroup, f16_t, 4>(x_dtype, out_dtype, lpr, P, (int)selected, st, what);
  return launch_types<Fmt::kInt4Sym, SMode::kGroup, float, 4>(x_dtype, out_dtype, lpr, P, (int)selected, st, what);
}

extern "C" int tt_scaled_matvec(const void* weight, int64_t w_row_bytes, const void* scales, int scale_dtype,
                                const void* x, int x_dtype, void* out, int out_dtype, int64_t rows, int64_t cols,
                                void* stream) {
  const char* what = "scaled_matvec";
  TT_REQUIRE(valid_act_dtype(x_dtype) && valid_out_dtype(out_dtype), "%s: bad dtype codes", what);
  TT_REQUIRE(scale_dtype == TT_F16 || scale_dtype == TT_F32, "%s: scales must be fp16 or fp32", what);
  TT_REQUIRE(weight && aligned(weight, 16) && w_row_bytes % 16 == 0 && w_row_bytes >= cols, "%s: fp8 weights must be 16-byte aligned rows", what);
  TT_REQUIRE(x && aligned(x, 4) && scales && out, "%s: null or misaligned pointer", what);
  TT_REQUIRE(rows > 0 && rows < (1 << 30), "%s: bad rows", what);
  int L;
  bool row_mode;
  int rc = plan_groups(what, cols, cols, &L, &row_mode);
  if (rc) return rc;
  GemvParams P{};
  P.nseg = 1;
  P.seg[0] = Seg{static_cast<const uint8_t*>(weight), w_row_bytes, scales, 1, 0, out, (int)rows};
  P.seg_end[0] = (int)rows;
  P.x = x;
  P.cols = (int)cols;
  P.L = 1;
  const int lpr = tt_gemv_lanes_per_row(cols / 32, 1);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (scale_dtype == TT_F16) return launch_types<Fmt::kFp8, SMode::kRow, f16_t, 4>(x_dtype, out_dtype, lpr, P, 1, st, what);
  return launch_types<Fmt::kFp8, SMode::kRow, float, 4>(x_dtype, out_dtype, lpr, P, 1, st, what);
}

extern "C" int tt_multi_matvec(int count, const void* const* weights, int w_dtype, const int64_t* w_row,
                               const int64_t* rows, const void* x, int x_dtype, void* out, int out_dtype,
                               int64_t cols, void* stream) {
  const char* what = "matvec";
  TT_REQUIRE(count >= 1 && count <= 3, "%s: supports one to three matrices", what);
  TT_REQUIRE(w_dtype == TT_F16 || w_dtype == TT_BF16, "%s: weights must be fp16 or bf16", what);
  TT_REQUIRE(valid_act_dtype(x_dtype) && valid_out_dtype(out_dtype), "%s: bad dtype codes", what);
  TT_REQUIRE(x && aligned(x, 4) && out, "%s: null or misaligned pointer", what);
  int L;
  bool row_mode;
  int rc = plan_groups(what, cols, cols, &L, &row_mode);
  if (rc) return rc;
  GemvParams P{};
  P.nseg = count;
  int64_t acc_rows = 0;
  const size_t osz = out_dtype == TT_F32 ? 4 : 2;
  for (int i = 0; i < count; i++) {
    TT_REQUIRE(rows[i] > 0, "%s: rows must be positive", what);
    TT_REQUIRE(weights[i] && aligned(weights[i], 16) && (w_row[i] * 2) % 16 == 0 && w_row[i] >= cols,
               "%s: weights must be 16-byte aligned with a row stride that is a multiple of 8 elements", what);
    P.seg[i] = Seg{static_cast<const uint8_t*>(weights[i]), w_row[i] * 2, nullptr, 0, 0,
                   static_cast<char*>(out) + acc_rows * osz, (int)rows[i]};
    acc_rows += rows[i];
    P.seg_end[i] = (int)acc_rows;
  }
  TT_REQUIRE(acc_rows < (1LL << 30), "%s: too many rows", what);
  P.x = x;
  P.cols = (int)cols;
  P.L = 1;
  const int lpr = tt_gemv_lanes_per_row(cols / 32, 1);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (w_dtype == TT_F16) return launch_types<Fmt::kF16W, SMode::kNone, float, 2>(x_dtype, out_dtype, lpr, P, 1, st, what);
  return launch_types<Fmt::kBF16W, SMode::kNone, float, 2>(x_dtype, out_dtype, lpr, P, 1, st, what);
}

extern "C" int tt_matvec(const void* weight, int w_dtype, int64_t w_row, const void* x, int x_dtype, void* out,
                         int out_dtype, int64_t rows, int64_t cols, void* stream) {
  const void* w_arr[1] = {weight};
  const int64_t wr[1] = {w_row};
  const int64_t r[1] = {rows};
  return tt_multi_matvec(1, w_arr, w_dtype, wr, r, x, x_dtype, out, out_dtype, cols, stream);
}

namespace {

int selected_e8(const char* what, Fmt fmt, const void* packed, int64_t w_expert_bytes, int64_t w_row_bytes,
                const void* scales, int64_t s_expert, int64_t s_row, const void* x, int x_dtype, int64_t x_slot,
                const int32_t* experts, int64_t selected, void* out, int out_dtype, int64_t out_slot, int64_t rows,
                int64_t cols, void* stream) {
  TT_REQUIRE(valid_act_dtype(x_dtype) && valid_out_dtype(out_dtype), "%s: bad dtype codes", what);
  TT_REQUIRE(selected >= 1 && selected <= 65535 && experts != nullptr, "%s: need 1..65535 selected experts", what);
  const int align = fmt == Fmt::kMxfp4 ? 16 : (fmt == Fmt::kQ2E8 ? 8 : 4);
  TT_REQUIRE(packed && aligned(packed, align) && w_row_bytes % align == 0 && w_expert_bytes % align == 0,
             "%s: packed weights must be %d-byte aligned", what, align);
  TT_REQUIRE(scales && x && aligned(x, 4) && (x_slot % 2) == 0 && out, "%s: null or misaligned pointer", what);
  TT_REQUIRE(rows > 0 && rows < (1 << 30), "%s: bad rows", what);
  int L;
  bool row_mode;
  int rc = plan_groups(what, cols, cols, &L, &row_mode);
  if (rc) return rc;
  GemvParams P{};
  P.nseg = 1;
  P.seg[0] = Seg{static_cast<const uint8_t*>(packed), w_row_bytes, scales, s_row, 1, out, (int)rows};
  P.seg_end[0] = (int)rows;
  P.x = x;
  P.x_slot = x_slot;
  P.experts = experts;
  P.w_expert = w_expert_bytes;
  P.s_expert = s_expert;
  P.out_slot = out_slot;
  P.cols = (int)cols;
  P.L = 1;
  P.e8_extra = fmt == Fmt::kMxfp4 ? 14 : 0;
  const int lpr = tt_gemv_lanes_per_row(cols / 32, 1);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int slots = (int)selected;
  switch (fmt) {
    case Fmt::kMxfp4: return launch_types<Fmt::kMxfp4, SMode::kBlockE8, uint8_t, 4>(x_dtype, out_dtype, lpr, P, slots, st, what);
    case Fmt::kQ2E8: return launch_types<Fmt::kQ2E8, SMode::kBlockE8, uint8_t, 4>(x_dtype, out_dtype, lpr, P, slots, st, what);
    case Fmt::kQ1E8: return launch_types<Fmt::kQ1E8, SMode::kBlockE8, uint8_t, 4>(x_dtype, out_dtype, lpr, P, slots, st, what);
    default: break;
  }
  set_error("%s: bad format", what);
  return TT_ERR_INVALID;
}

}  // namespace

extern "C" int tt_mxfp4_selected_matvec(const void* blocks, int64_t b_expert_bytes, int64_t b_row_bytes,
                                        const void* scales, int64_t s_expert, int64_t s_row, const void* x,
                                        int x_dtype, int64_t x_slot, const int32_t* expert_indices, int64_t selected,
                                        void* out, int out_dtype, int64_t out_slot, int64_t rows, int64_t cols,
                                        void* stream) {
  return selected_e8("mxfp4_selected_matvec", Fmt::kMxfp4, blocks, b_expert_bytes, b_row_bytes, scales, s_expert,
                     s_row, x, x_dtype, x_slot, expert_indices, selected, out, out_dtype, out_slot, rows, cols, stream);
}

extern "C" int tt_mxfp_lowbit_selected_matvec(const void* packed, int64_t w_expert_bytes, int64_t w_row_bytes,
                                              const void* scales, int64_t s_expert, int64_t s_row, int bits,
                                              const void* x, int x_dtype, int64_t x_slot,
                                              const int32_t* expert_indices, int64_t selected, void* out,
                                              int out_dtype, int64_t out_slot, int64_t rows, int64_t cols,
                                              void* stream) {
  if (bits != 1 && bits != 2) {
    set_error("mxfp_lowbit_selected_matvec: low-bit expert weights must be packed Q1 or Q2");
    return TT_ERR_INVALID;
  }
  return selected_e8("mxfp_lowbit_selected_matvec", bits == 2 ? Fmt::kQ2E8 : Fmt::kQ1E8, packed, w_expert_bytes,
                     w_row_bytes, scales, s_expert, s_row, x, x_dtype, x_slot, expert_indices, selected, out,
                     out_dtype, out_slot, rows, cols, stream);
}

extern "C" int tt_lowbit_affine_matvec(const void* packed, int64_t w_row_bytes, const void* scale_zero, int64_t s_row,
                                       int64_t s_group, int bits, const void* x, int x_dtype, void* out,
                                       int out_dtype, int64_t rows, int64_t cols, int64_t group_size, void* stream) {
  const char* what = "lowbit_affine_matvec";
  TT_REQUIRE(bits == 1 || bits == 2, "%s: bits must be 1 or 2", what);
  TT_REQUIRE(valid_act_dtype(x_dtype) && valid_out_dtype(out_dtype), "%s: bad dtype codes", what);
  const int align = bits == 2 ? 8 : 4;
  TT_REQUIRE(packed && aligned(packed, align) && w_row_bytes % align == 0 && w_row_bytes * 8 >= cols * bits,
             "%s: packed rows must be %d-byte aligned", what, align);
  TT_REQUIRE(scale_zero && x && aligned(x, 4) && out, "%s: null or misaligned pointer", what);
  TT_REQUIRE(rows > 0 && rows < (1 << 30), "%s: bad rows", what);
  int L;
  bool row_mode;
  int rc = plan_groups(what, cols, group_size, &L, &row_mode);
  if (rc) return rc;
  TT_UNSUPPORTED(!row_mode, "%s: group_size must be smaller than cols", what);
  GemvParams P{};
  P.nseg = 1;
  P.seg[0] = Seg{static_cast<const uint8_t*>(packed), w_row_bytes, scale_zero, s_row, s_group, out, (int)rows};
  P.seg_end[0] = (int)rows;
  P.x = x;
  P.cols = (int)cols;
  P.L = L;
  P.s_pair = 1;
  P.aff_zero = 1;
  const int lpr = tt_gemv_lanes_per_row(cols / 32, L);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (bits == 2) return launch_types<Fmt::kQ2Aff, SMode::kGroupAff, f16_t, 4>(x_dtype, out_dtype, lpr, P, 1, st, what);
  return launch_types<Fmt::kQ1Aff, SMode::kGroupAff, f16_t, 4>(x_dtype, out_dtype, lpr, P, 1, st, what);
}
