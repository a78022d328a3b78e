// Fused decode-step GEMVs: the GEMV engine of gemv_impl.h instantiated with the
// RMSNorm prologues and the RoPE / KV-cache / SiLU epilogues, plus the greedy lm_head
// with the step's token bookkeeping in its finishing kernel.
#include "gemv_impl.h"

#include <type_traits>

using namespace tt;

namespace {

constexpr const char* kWhat = "fused_gemv";

// Highest key among n partials (256 threads), then token / value / bookkeeping.
__global__ __launch_bounds__(256) void argmax_step_kernel(const uint64_t* partials, int n, int64_t* out_idx,
                                                          float* out_val, int32_t* pos, const int32_t* base,
                                                          int64_t* history, int32_t history_len) {
  __shared__ uint64_t red[256];
  uint64_t best = 0;
  for (int i = threadIdx.x; i < n; i += 256) best = partials[i] > best ? partials[i] : best;
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
    const int64_t token = (int64_t)(0xffffffffu - (uint32_t)k);
    out_idx[0] = token;
    if (out_val) out_val[0] = __builtin_bit_cast(float, bits);
    if (pos) {
      const int32_t i = pos[0] - (base ? base[0] : 0);
      if (history && i >= 0 && i < history_len) history[i] = token;
      pos[0] += 1;
    }
  }
}

int validate(const tt_fused_gemv* d, bool lm_head) {
  TT_REQUIRE(d != nullptr, "%s: null descriptor", kWhat);
  TT_REQUIRE(d->act_dtype == TT_F16 || d->act_dtype == TT_BF16, "%s: activations must be fp16 or bf16", kWhat);
  TT_REQUIRE(d->cols > 0 && d->cols % 32 == 0 && d->cols <= 32768, "%s: cols must be a multiple of 32 up to 32768",
             kWhat);
  TT_REQUIRE(d->count >= 1 && d->count <= 3, "%s: one to three segments", kWhat);
  TT_REQUIRE(!lm_head || d->count == 1, "%s: the lm_head takes one segment", kWhat);
  TT_REQUIRE(d->weight_format == TT_FMT_INT4_G || d->weight_format == TT_FMT_DENSE, "%s: unknown weight format",
             kWhat);
  TT_REQUIRE(!lm_head || d->weight_format == TT_FMT_DENSE, "%s: the lm_head is a dense matrix", kWhat);
  if (d->weight_format == TT_FMT_INT4_G)
    TT_UNSUPPORTED(d->group_size == 128 && d->cols % 128 == 0, "%s: fused int4 GEMVs use group size 128", kWhat);
  else
    TT_REQUIRE(d->weight_dtype == TT_F16 || d->weight_dtype == TT_BF16, "%s: dense weights must be fp16 or bf16",
               kWhat);
  switch (d->prologue) {
    case TT_PRO_LOAD:
      TT_REQUIRE(d->x && aligned(d->x, 16), "%s: x must be a 16-byte aligned pointer", kWhat);
      break;
    case TT_PRO_ADD_NORM:
    case TT_PRO_ADD_RMS_NORM:
      TT_REQUIRE(d->left && d->right && d->norm_weight, "%s: add+norm prologue needs left, right and the weight",
                 kWhat);
      break;
    case TT_PRO_EMBED_NORM:
      TT_REQUIRE(d->embed && d->token && d->norm_weight && d->vocab > 0 && d->embed_row >= d->cols,
                 "%s: embedding prologue needs the table, the device token and the weight", kWhat);
      break;
    default:
      TT_REQUIRE(false, "%s: unknown prologue %d", kWhat, d->prologue);
  }
  bool needs_pos = false, needs_rope = false;
  for (int i = 0; i < d->count; i++) {
    const tt_fused_segment& g = d->seg[i];
    TT_REQUIRE(g.weight && aligned(g.weight, 16) && g.w_row_bytes % 16 == 0, "%s: segment %d weights misaligned",
               kWhat, i);
    TT_REQUIRE(g.out != nullptr && g.rows > 0 && g.rows < (1 << 28), "%s: segment %d needs an output and rows", kWhat,
               i);
    if (d->weight_format == TT_FMT_INT4_G) {
      TT_REQUIRE(g.w_row_bytes >= d->cols / 2 && g.scales, "%s: segment %d int4 layout", kWhat, i);
      TT_UNSUPPORTED(g.bias == nullptr, "%s: int4 segments take no bias", kWhat);
    } else {
      TT_REQUIRE(g.w_row_bytes >= d->cols * 2, "%s: segment %d dense layout", kWhat, i);
    }
    switch (g.kind) {
      case TT_SEG_PLAIN: break;
      case TT_SEG_ROPE_OUT:
      case TT_SEG_ROPE_CACHE:
        needs_rope = true;
        needs_pos = true;
        TT_REQUIRE(d->head_dim >= 2 && d->head_dim % 2 == 0 && g.rows % d->head_dim == 0 && g.rows % 8 == 0,
                   "%s: RoPE rows must be whole heads of an even head_dim", kWhat);
        break;
      case TT_SEG_CACHE:
        needs_pos = true;
        TT_REQUIRE(d->head_dim >= 1 && g.rows % d->head_dim == 0, "%s: cache rows must be whole heads", kWhat);
        break;
      case TT_SEG_SILU:
        TT_REQUIRE(g.weight2 && aligned(g.weight2, 16) && g.rows % 8 == 0, "%s: SiLU pairs need the up rows and "
                   "a multiple of 8 activation rows", kWhat);
        TT_REQUIRE(d->weight_format == TT_FMT_DENSE || g.scales2, "%s: SiLU pairs need the up scales", kWhat);
        TT_UNSUPPORTED(g.bias == nullptr, "%s: SiLU pairs take no bias", kWhat);
        break;
      default: TT_REQUIRE(false, "%s: unknown segment kind %d", kWhat, g.kind);
    }
    TT_UNSUPPORTED(!lm_head || g.kind == TT_SEG_PLAIN, "%s: the lm_head segment is plain", kWhat);
  }
  if (needs_pos) {
    TT_REQUIRE(d->position && d->capacity > 0 && d->cache_head >= d->capacity * d->head_dim,
               "%s: cache segments need the device position and the cache geometry", kWhat);
  }
  if (needs_rope) {
    TT_REQUIRE(d->cos_table && d->sin_table && d->table_rows > 0 && d->table_row >= d->head_dim / 2,
               "%s: RoPE segments need the cos / sin tables", kWhat);
  }
  return TT_OK;
}

GemvParams params(const tt_fused_gemv* d) {
  GemvParams P{};
  P.nseg = d->count;
  for (int i = 0; i < d->count; i++) {
    const tt_fused_segment& g = d->seg[i];
    Seg& S = P.seg[i];
    S.w = static_cast<const uint8_t*>(g.weight);
    S.w_row = g.w_row_bytes;
    S.s = g.scales;
    S.s_row = g.s_row;
    S.s_grp = 1;
    S.out = g.out;
    S.rows = (int)(g.kind == TT_SEG_SILU ? 2 * g.rows : g.rows);
    S.bias = g.bias;
    S.kind = g.kind;
    S.w2 = static_cast<const uint8_t*>(g.weight2);
    S.s2 = g.scales2;
  }
  P.x = d->x;
  P.cols = (int)d->cols;
  FuseParams& f = P.f;
  f.left = d->left;
  f.right = d->right;
  f.embed = d->embed;
  f.embed_row = d->embed_row;
  f.vocab = d->vocab;
  f.token = d->token;
  f.norm_w = d->norm_weight;
  f.eps = d->eps;
  f.residual_out = d->residual_out;
  f.pos = d->position;
  f.capacity = d->capacity;
  f.cache_head = d->cache_head;
  f.cos = d->cos_table;
  f.sin = d->sin_table;
  f.table_row = d->table_row;
  f.table_rows = d->table_rows;
  f.head_dim = (int)d->head_dim;
  return P;
}

template <typename AT, Pro PRO>
int launch(const tt_fused_gemv* d, GemvParams& P, int lpr, bool argmax, hipStream_t st) {
  if (d->weight_format == TT_FMT_INT4_G) {
    int64_t rows = 0;
    for (int i = 0; i < d->count; i++) rows += d->seg[i].kind == TT_SEG_SILU ? 2 * d->seg[i].rows : d->seg[i].rows;
    int rpw, pf;
    int4_shape(rows, (int)((d->cols / 32 + lpr - 1) / lpr), true, &rpw, &pf);
    return launch_int4_g128<AT, AT, PRO, true>(lpr, rpw, pf, P, st, kWhat);
  }
  if (argmax) {
    if (d->weight_dtype == TT_F16)
      return launch_lpr<Fmt::kF16W, SMode::kNone, AT, AT, float, 2, 1, PRO, false>(lpr, P, 1, st, kWhat);
    return launch_lpr<Fmt::kBF16W, SMode::kNone, AT, AT, float, 2, 1, PRO, false>(lpr, P, 1, st, kWhat);
  }
  if (d->weight_dtype == TT_F16)
    return launch_lpr<Fmt::kF16W, SMode::kNone, AT, AT, float, 2, 1, PRO, true>(lpr, P, 1, st, kWhat);
  return launch_lpr<Fmt::kBF16W, SMode::kNone, AT, AT, float, 2, 1, PRO, true>(lpr, P, 1, st, kWhat);
}

template <typename AT>
int launch_pro(const tt_fused_gemv* d, GemvParams& P, int lpr, bool argmax, hipStream_t st) {
  switch (d->prologue) {
    case TT_PRO_ADD_NORM: return launch<AT, Pro::kAddNorm>(d, P, lpr, argmax, st);
    case TT_PRO_EMBED_NORM: return launch<AT, Pro::kEmbedNorm>(d, P, lpr, argmax, st);
    case TT_PRO_ADD_RMS_NORM: return launch<AT, Pro::kAddRmsNorm>(d, P, lpr, argmax, st);
    default: return launch<AT, Pro::kLoad>(d, P, lpr, argmax, st);
  }
}

int run(const tt_fused_gemv* d, GemvParams& P, bool argmax, hipStream_t st) {
  const int64_t chunks = d->cols / 32;
  const int lpr = tt_gemv_lanes_per_row(chunks, d->weight_format == TT_FMT_INT4_G ? d->group_size / 32 : 1);
  TT_UNSUPPORTED(lpr > 0, "%s: no lane mapping for %lld columns", kWhat, (long long)d->cols);
  if (d->act_dtype == TT_F16) return launch_pro<f16_t>(d, P, lpr, argmax, st);
  return launch_pro<bf16_t>(d, P, lpr, argmax, st);
}

}  // namespace

extern "C" int tt_fused_struct_sizes(int64_t* segment_size, int64_t* desc_size) {
  TT_REQUIRE(segment_size && desc_size, "fused_struct_sizes: null pointer");
  *segment_size = (int64_t)sizeof(tt_fused_segment);
  *desc_size = (int64_t)sizeof(tt_fused_gemv);
  return TT_OK;
}

extern "C" int tt_fused_gemv_run(const tt_fused_gemv* desc, void* stream) {
  int rc = validate(desc, false);
  if (rc) return rc;
  GemvParams P = params(desc);
  return run(desc, P, false, static_cast<hipStream_t>(stream));
}

extern "C" int tt_fused_lm_head_argmax(const tt_fused_gemv* desc, uint64_t* partials, int64_t partials_capacity,
                                       int64_t* out_idx, float* out_val, int32_t* position, const int32_t* base,
                                       int64_t* history, int32_t history_len, void* stream) {
  int rc = validate(desc, true);
  if (rc) return rc;
  TT_REQUIRE(partials && out_idx, "%s: lm_head needs partials and the token output", kWhat);
  const int64_t need = tt_matvec_argmax_partials(desc->seg[0].rows, desc->cols);
  TT_REQUIRE(partials_capacity >= need, "%s: partials buffer needs %lld entries", kWhat, (long long)need);
  TT_REQUIRE(history_len >= 0, "%s: bad history length", kWhat);
  GemvParams P = params(desc);
  P.am_partials = partials;
  hipStream_t st = static_cast<hipStream_t>(stream);
  rc = run(desc, P, true, st);
  if (rc) return rc;
  hipLaunchKernelGGL(argmax_step_kernel, dim3(1), dim3(256), 0, st, partials, (int)need, out_idx, out_val, position,
                     base, history, history_len);
  return check_launch(kWhat);
}
