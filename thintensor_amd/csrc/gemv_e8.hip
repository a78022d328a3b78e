// E8M0 block-scaled (MXFP4, q1, q2) and affine low-bit GEMV entry points.
#include "gemv_lean.h"

using namespace tt;

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
  TT_REQUIRE(scales && x && aligned(x, 16) && (x_slot % 8) == 0 && out, "%s: null or misaligned pointer", what);
  TT_REQUIRE(rows > 0 && rows < (1 << 30), "%s: bad rows", what);
  int L;
  bool row_mode;
  int rc = tt::plan_groups(what, cols, cols, &L, &row_mode);
  if (rc) return rc;
  GemvParams P{};
  P.nseg = 1;
  P.seg[0] = Seg{static_cast<const uint8_t*>(packed), w_row_bytes, scales, s_row, 1, out, (int)rows};
  P.x = x;
  P.x_slot = x_slot;
  P.experts = experts;
  P.w_expert = w_expert_bytes;
  P.s_expert = s_expert;
  P.out_slot = out_slot;
  P.cols = (int)cols;
  const int Lg = 1;
  const int lpr = tt_gemv_lanes_per_row(cols / 32, 1);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int slots = (int)selected;
  if (x_dtype == out_dtype && lean_fits(rows, w_row_bytes, s_row, cols)) {
    LeanParams L{};
    L.w = static_cast<const uint8_t*>(packed);
    L.s = scales;
    L.x = x;
    L.out = out;
    L.experts = experts;
    L.w_expert = w_expert_bytes;
    L.s_expert = s_expert;
    L.x_slot = x_slot;
    L.out_slot = out_slot;
    L.w_row = (uint32_t)w_row_bytes;
    L.s_row = (uint32_t)s_row;
    L.rows = (int)rows;
    L.cols = (int)cols;
    switch (fmt) {
      case Fmt::kMxfp4: return lean_launch<Fmt::kMxfp4, SMode::kBlockE8, uint8_t, 1>(x_dtype, lpr, L, slots, st, what);
      case Fmt::kQ2E8: return lean_launch<Fmt::kQ2E8, SMode::kBlockE8, uint8_t, 1>(x_dtype, lpr, L, slots, st, what);
      case Fmt::kQ1E8: return lean_launch<Fmt::kQ1E8, SMode::kBlockE8, uint8_t, 1>(x_dtype, lpr, L, slots, st, what);
      default: break;
    }
  }
  switch (fmt) {
    case Fmt::kMxfp4: return launch_types<Fmt::kMxfp4, SMode::kBlockE8, uint8_t, 4>(x_dtype, out_dtype, Lg, lpr, P, slots, st, what);
    case Fmt::kQ2E8: return launch_types<Fmt::kQ2E8, SMode::kBlockE8, uint8_t, 4>(x_dtype, out_dtype, Lg, lpr, P, slots, st, what);
    case Fmt::kQ1E8: return launch_types<Fmt::kQ1E8, SMode::kBlockE8, uint8_t, 4>(x_dtype, out_dtype, Lg, lpr, P, slots, st, what);
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
  TT_REQUIRE(scale_zero && x && aligned(x, 16) && out, "%s: null or misaligned pointer", what);
  TT_REQUIRE(rows > 0 && rows < (1 << 30), "%s: bad rows", what);
  int L;
  bool row_mode;
  int rc = tt::plan_groups(what, cols, group_size, &L, &row_mode);
  if (rc) return rc;
  TT_UNSUPPORTED(!row_mode, "%s: group_size must be smaller than cols", what);
  GemvParams P{};
  P.nseg = 1;
  P.seg[0] = Seg{static_cast<const uint8_t*>(packed), w_row_bytes, scale_zero, s_row, s_group, out, (int)rows};
  P.x = x;
  P.cols = (int)cols;
  const int Lg = L;
  P.s_pair = 1;
  P.aff_zero = 1;
  const int lpr = tt_gemv_lanes_per_row(cols / 32, L);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (x_dtype == out_dtype && lean_group_ok(Lg) && lean_fits(rows, w_row_bytes, 2 * s_row, cols) && s_group >= 0 &&
      s_group * (cols / group_size) < (1LL << 30)) {
    LeanParams Q{};
    Q.w = static_cast<const uint8_t*>(packed);
    Q.s = scale_zero;
    Q.x = x;
    Q.out = out;
    Q.s_pair = 1;
    Q.aff_zero = 1;
    Q.w_row = (uint32_t)w_row_bytes;
    Q.s_row = (uint32_t)s_row;
    Q.s_grp = (uint32_t)s_group;
    Q.rows = (int)rows;
    Q.cols = (int)cols;
    if (bits == 2) return lean_launch_group<Fmt::kQ2Aff, SMode::kGroupAff, f16_t>(Lg, x_dtype, lpr, Q, 1, st, what);
    return lean_launch_group<Fmt::kQ1Aff, SMode::kGroupAff, f16_t>(Lg, x_dtype, lpr, Q, 1, st, what);
  }
  if (bits == 2) return launch_types<Fmt::kQ2Aff, SMode::kGroupAff, f16_t, 4>(x_dtype, out_dtype, Lg, lpr, P, 1, st, what);
  return launch_types<Fmt::kQ1Aff, SMode::kGroupAff, f16_t, 4>(x_dtype, out_dtype, Lg, lpr, P, 1, st, what);
}
