// int4 GEMV entry points (dense, multi-matrix, selected expert).
#include "gemv_impl.h"

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
  TT_REQUIRE(x != nullptr && out != nullptr && aligned(x, 16), "%s: x must be a 16-byte aligned device pointer", what);
  int L = 1;
  bool row_mode = false;
  int rc = tt::plan_groups(what, cols, group_size, &L, &row_mode);
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
  }
  TT_REQUIRE(acc_rows < (1LL << 30), "%s: too many rows", what);
  P.x = x;
  P.cols = (int)cols;
  const int Lg = L;
  P.s_pair = s_pair;
  const int lpr = tt_gemv_lanes_per_row(cols / 32, row_mode ? 1 : L);
  TT_UNSUPPORTED(lpr > 0, "%s: no lane mapping for cols %lld / group %lld", what, (long long)cols, (long long)group_size);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (affine) {
    TT_UNSUPPORTED(!row_mode, "%s: affine int4 needs group_size < cols", what);
    if (scale_dtype == TT_F16) return launch_types<Fmt::kInt4Aff, SMode::kGroupAff, f16_t, 4>(x_dtype, out_dtype, Lg, lpr, P, 1, st, what);
    return launch_types<Fmt::kInt4Aff, SMode::kGroupAff, float, 4>(x_dtype, out_dtype, Lg, lpr, P, 1, st, what);
  }
  if (row_mode) {
    if (scale_dtype == TT_F16) return launch_types<Fmt::kInt4Sym, SMode::kRow, f16_t, 4>(x_dtype, out_dtype, Lg, lpr, P, 1, st, what);
    return launch_types<Fmt::kInt4Sym, SMode::kRow, float, 4>(x_dtype, out_dtype, Lg, lpr, P, 1, st, what);
  }
  if (scale_dtype == TT_F16 && Lg == 4 && x_dtype == out_dtype) {
    // the decode hot path (group 128, fp16 scales): launch shape chosen from the matrix
    int rpw, pf;
    int4_shape(acc_rows, (int)((cols / 32 + lpr - 1) / lpr), false, &rpw, &pf);
    if (x_dtype == TT_F16) return launch_int4_g128<f16_t, f16_t, Pro::kLoad, false>(lpr, rpw, pf, P, st, what);
    return launch_int4_g128<bf16_t, bf16_t, Pro::kLoad, false>(lpr, rpw, pf, P, st, what);
  }
  if (scale_dtype == TT_F16) return launch_types<Fmt::kInt4Sym, SMode::kGroup, f16_t, 4>(x_dtype, out_dtype, Lg, lpr, P, 1, st, what);
  return launch_types<Fmt::kInt4Sym, SMode::kGroup, float, 4>(x_dtype, out_dtype, Lg, lpr, P, 1, st, what);
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
  TT_REQUIRE(x && aligned(x, 16) && (x_slot % 8) == 0, "%s: x must be 16-byte aligned (slot stride a multiple of 8)", what);
  TT_REQUIRE(rows > 0 && rows < (1 << 30), "%s: bad rows", what);
  int L = 1;
  bool row_mode = false;
  int rc = tt::plan_groups(what, cols, group_size, &L, &row_mode);
  if (rc) return rc;
  GemvParams P{};
  P.nseg = 1;
  P.seg[0] = Seg{static_cast<const uint8_t*>(packed), w_row_bytes, scales, s_row, s_group, out, (int)rows};
  P.x = x;
  P.x_slot = x_slot;
  P.experts = expert_indices;
  P.w_expert = w_expert_bytes;
  P.s_expert = s_expert;
  P.out_slot = out_slot;
  P.cols = (int)cols;
  const int Lg = L;
  const int lpr = tt_gemv_lanes_per_row(cols / 32, row_mode ? 1 : L);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (row_mode) {
    if (scale_dtype == TT_F16) return launch_types<Fmt::kInt4Sym, SMode::kRow, f16_t, 4>(x_dtype, out_dtype, Lg, lpr, P, (int)selected, st, what);
    return launch_types<Fmt::kInt4Sym, SMode::kRow, float, 4>(x_dtype, out_dtype, Lg, lpr, P, (int)selected, st, what);
  }
  if (scale_dtype == TT_F16) return launch_types<Fmt::kInt4Sym, SMode::kGroup, f16_t, 4>(x_dtype, out_dtype, Lg, lpr, P, (int)selected, st, what);
  return launch_types<Fmt::kInt4Sym, SMode::kGroup, float, 4>(x_dtype, out_dtype, Lg, lpr, P, (int)selected, st, what);
}

