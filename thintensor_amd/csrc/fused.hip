// Fused decode-step GEMVs: the GEMV engine of gemv_impl.h instantiated with the
// RMSNorm prologues and the RoPE / KV-cache / SiLU epilogues, plus the greedy lm_head
// with the step's token bookkeeping in its finishing kernel.
#include "gemv_impl.h"

#include <type_traits>

using namespace tt;

namespace {

constexpr const char* kWhat = "fused_gemv";

// ----------------------------------------------------------------------------
// Lean fused GEMV of the decode step (int4 g128 or dense fp16/bf16 weights): one batch of ROWS * (64 / LPR) virtual
// rows per wave (segments padded to whole batches, as in gemv_kernel), the RMSNorm
// prologue and the RoPE / KV-cache / SiLU epilogues of gemv_kernel with the same
// row pairing, rounding points and reduction order, without its persistent loop.
// The prologue's inputs (and the token position of the epilogues) are requested first,
// then round 0's weights and scales, so the prologue's memory wait overlaps the weight
// stream without waiting behind it.
struct LeanSeg {
  const uint8_t* w;     // weights (kSegSilu: gate rows)
  const uint8_t* w2;    // kSegSilu: up rows
  const f16_t* s;
  const f16_t* s2;
  void* out;
  const void* bias;     // dense segments: optional per-row bias (activation dtype)
  uint32_t w_row, s_row;
  int rows;             // virtual rows (kSegSilu: 2 x activation rows)
  int vbegin;
  int kind;
};

struct LeanFused {
  LeanSeg seg[3];
  int nseg, vtotal, cols, head_dim;
  const void* x;
  const void* left;
  const void* right;
  const void* embed;
  int64_t embed_row, vocab;
  const int64_t* token;
  const void* norm_w;
  float eps;
  void* residual_out;
  const int32_t* pos;
  int64_t capacity, cache_head;
  const void* cos;
  const void* sin;
  int64_t table_row, table_rows;
  int64_t token_x, token_out, token_cache;   // strides of token blockIdx.y
};

__device__ __forceinline__ LeanSeg pick_seg(const LeanSeg a, const LeanSeg b, const LeanSeg c, int si) {
  LeanSeg r;
  r.w = si == 0 ? a.w : (si == 1 ? b.w : c.w);
  r.w2 = si == 0 ? a.w2 : (si == 1 ? b.w2 : c.w2);
  r.s = si == 0 ? a.s : (si == 1 ? b.s : c.s);
  r.s2 = si == 0 ? a.s2 : (si == 1 ? b.s2 : c.s2);
  r.out = si == 0 ? a.out : (si == 1 ? b.out : c.out);
  r.bias = si == 0 ? a.bias : (si == 1 ? b.bias : c.bias);
  r.w_row = si == 0 ? a.w_row : (si == 1 ? b.w_row : c.w_row);
  r.s_row = si == 0 ? a.s_row : (si == 1 ? b.s_row : c.s_row);
  r.rows = si == 0 ? a.rows : (si == 1 ? b.rows : c.rows);
  r.vbegin = si == 0 ? a.vbegin : (si == 1 ? b.vbegin : c.vbegin);
  r.kind = si == 0 ? a.kind : (si == 1 ? b.kind : c.kind);
  return r;
}

template <Fmt F, typename XT, int LPR, int ROWS, Pro PRO, bool MULTI>
__global__ __launch_bounds__(256) void fused_lean_kernel(const LeanFused P) {
  constexpr bool kInt4 = F == Fmt::kInt4Sym;
  constexpr int B = FmtInfo<F>::kBytes;
  constexpr int L = kInt4 ? 4 : 1;
  constexpr int SUBS = 64 / LPR;
  constexpr int NVG = kInt4 ? (ROWS / L > 0 ? ROWS / L : 1) : ROWS;
  constexpr int NS = kInt4 ? NVG : 1;
  constexpr int GLEV = kInt4 ? (log2c(L) < log2c(ROWS) ? log2c(L) : log2c(ROWS)) : 0;
  static_assert(ROWS >= 2, "paired segments need two rows per wave");
  extern __shared__ uint32_t xs_lds[];
  const int lane = threadIdx.x & 63;
  const int sub = lane / LPR;
  const int l = lane % LPR;
  const int cols = P.cols;
  const int nchunks = cols >> 5;
  const int rounds = (nchunks + LPR - 1) / LPR;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int v0 = (int)(blockIdx.x * 4 + wave) * (ROWS * SUBS);   // first virtual row (uniform)
  const bool active = v0 < P.vtotal;
  const int64_t tok = blockIdx.y;   // token of a multi-token launch (0 otherwise)
  // ---- the prologue's inputs are requested first -- before the row addressing, which
  // is a few hundred scalar instructions for paired segments, and before round 0 of the
  // weights, so that waiting for them never waits for the weight stream: one 16-byte
  // piece of each vector per held piece (cols <= 4096, a multiple of 32; indices past the
  // last piece repeat it)
  __shared__ float red[4];
  const int n = cols;
  const int np = n >> 3;
  uint4 qa[kNormPieces], qb[kNormPieces], qw[kNormPieces];
  if constexpr (PRO != Pro::kLoad) {
    const uint16_t* pa;
    if constexpr (PRO == Pro::kEmbedNorm) {
      int64_t t = P.token[tok];
      t = t < 0 ? 0 : (t >= P.vocab ? P.vocab - 1 : t);
      pa = reinterpret_cast<const uint16_t*>(P.embed) + t * P.embed_row;
    } else {
      pa = reinterpret_cast<const uint16_t*>(P.left) + tok * P.token_x;
    }
    const uint16_t* pb = reinterpret_cast<const uint16_t*>(P.right) + tok * P.token_x;
#pragma unroll
    for (int k = 0; k < kNormPieces; k++) {
      const int pi = (int)threadIdx.x + 256 * k;
      const int pc = pi < np ? pi : np - 1;
      qa[k] = reinterpret_cast<const uint4*>(pa)[pc];
      if constexpr (PRO != Pro::kEmbedNorm) qb[k] = reinterpret_cast<const uint4*>(pb)[pc];
      qw[k] = reinterpret_cast<const uint4*>(P.norm_w)[pc];
    }
  }
  // the token position of the RoPE / cache epilogues, requested with the prologue's
  // inputs so that the epilogue's table reads are its only dependent round trip
  const int32_t pos_raw = P.pos != nullptr ? P.pos[0] : 0;
  __builtin_amdgcn_sched_barrier(0);
  // MULTI: every segment's fields are read from the kernel arguments unconditionally and
  // the wave's segment is selected afterwards (scalar selects), so the argument loads go
  // out together instead of a second round trip behind the segment index; a
  // one-segment launch reads segment 0 only (fewer argument loads, fewer scalar
  // registers)
  int si = 0;
  if constexpr (MULTI) si = (P.nseg > 1 && v0 >= P.seg[1].vbegin ? 1 : 0) + (P.nseg > 2 && v0 >= P.seg[2].vbegin ? 1 : 0);
  const LeanSeg S = MULTI ? pick_seg(P.seg[0], P.seg[1], P.seg[2], si) : P.seg[0];
  const int kind = S.kind;
  const int srows = S.rows;
  const int lr0 = v0 - S.vbegin;
  const bool paired = kind == kSegRopeOut || kind == kSegRopeCache || kind == kSegSilu;

  // Physical row (and matrix) of row vr (0 .. ROWS * SUBS - 1) of this wave's block, the
  // mapping of paired_row: the block starts on a pair boundary (lr0 is a multiple of
  // ROWS * SUBS), so its rows are a few shifts away from its first pair P0, and for the
  // RoPE segments the block's pairs lie in one head (the host checks that half a head
  // is a whole number of blocks), whose index and in-head offset are one scalar
  // division per wave.  Rows past the segment read the block's first row, and a block
  // past the segment reads row 0 (in bounds; the values are never used).
  const int P0 = lr0 >> 1;
  const int half = P.head_dim >> 1;
  int h0 = 0, j0 = 0;
  if (kind == kSegRopeOut || kind == kSegRopeCache) {
    h0 = (int)((uint32_t)P0 / (uint32_t)half);
    j0 = P0 - h0 * half;
  }
  const bool any_row = lr0 < srows;
  const bool silu = kind == kSegSilu;
  const int rope_base = h0 * P.head_dim + j0;   // row of the block's first pair (RoPE segments)
  // (selects only, no branches: the row addressing stays a short straight run ahead of
  // the first weight loads)
  auto phys = [&](int vr, bool valid, bool& up, bool& odd) -> int {
    vr = valid ? vr : 0;
    const int blk = vr / (2 * SUBS), rem = vr % (2 * SUBS);   // SUBS is a power of two
    const bool o = paired && rem >= SUBS;
    const int poff = blk * SUBS + (o ? rem - SUBS : rem);
    const int pr = silu ? P0 + poff : rope_base + poff + (o ? half : 0);
    const int ph = paired ? pr : lr0 + vr;
    odd = o;
    up = o && silu && any_row;
    return any_row ? ph : 0;
  };
  // both matrices' base pointers in scalar registers, so the per-lane choice between them
  // is a select and not a vector load of the chosen kernel argument
  const uint8_t* const wlo = uniform_ptr(S.w);
  const uint8_t* const whi = uniform_ptr(S.w2);
  const uint8_t* wrow[ROWS];
  bool rv[ROWS];
#pragma unroll
  for (int i = 0; i < ROWS; i++) {
    const int vr = i * SUBS + sub;
    rv[i] = lr0 + vr < srows;
    bool up, odd;
    const int ph = phys(vr, rv[i], up, odd);
    wrow[i] = (up ? whi : wlo) + (size_t)ph * S.w_row;
  }
  const f16_t* srow[NS];
  bool sv[NS];
  if constexpr (kInt4) {
    const f16_t* const slo = uniform_ptr(S.s);
    const f16_t* const shi = uniform_ptr(S.s2);
#pragma unroll
    for (int k = 0; k < NS; k++) {
      const int vr = rs_row<ROWS>(l, GLEV, k) * SUBS + sub;
      sv[k] = lr0 + vr < srows;
      bool up, odd;
      const int ph = phys(vr, sv[k], up, odd);
      srow[k] = (up ? shi : slo) + (size_t)ph * S.s_row;
    }
  }
  auto fetch = [&](int r, Raw<B>* w, f16_t* sc) {
    uint32_t j = (uint32_t)(r * LPR + l);
    j = j < (uint32_t)nchunks ? j : (uint32_t)nchunks - 1;
#pragma unroll
    for (int i = 0; i < ROWS; i++) w[i] = load_raw<B>(wrow[i] + j * (uint32_t)B);
    if constexpr (kInt4) {
#pragma unroll
      for (int k = 0; k < NS; k++) sc[k] = srow[k][j >> 2];
    }
  };
  __builtin_amdgcn_sched_barrier(0);
  Raw<B> wc[ROWS];
  f16_t sc[NS];
  fetch(0, wc, sc);   // in bounds for inactive waves too (rows clamped)
  // nothing that consumes the prologue's loads may be scheduled above round 0's weight
  // loads: its wait would hold the weight stream back by a memory round trip
  __builtin_amdgcn_sched_barrier(0);

  // ---- activation vector into LDS
  if constexpr (PRO == Pro::kLoad) {
    const int xn = cols >> 3;
    for (int idx = threadIdx.x; idx < xn; idx += 256)
      reinterpret_cast<uint4*>(xs_lds)[idx] = reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(P.x) +
                                                                             tok * P.token_x)[idx];
  } else {
    // RMSNorm of the residual stream in the piece partition, reduction order and
    // rounding points of the standalone rms_norm / add_rms_norm kernels; workgroup 0
    // stores the residual.
    const bool writer = blockIdx.x == 0 && P.residual_out != nullptr;
    const int t = threadIdx.x;
    float rr[kNormPieces][8];
    float ss = 0.0f;
#pragma unroll
    for (int k = 0; k < kNormPieces; k++)
#pragma unroll
      for (int e = 0; e < 8; e++) {
        const float a = piece_f32<XT>(qa[k], e);
        float r;
        if constexpr (PRO == Pro::kAddNorm) r = round_bf16(a + piece_f32<XT>(qb[k], e));
        else if constexpr (PRO == Pro::kAddRmsNorm) r = round_to<XT>(a + piece_f32<XT>(qb[k], e));
        else r = a;
        rr[k][e] = r;
        if (8 * (t + 256 * k) + e < n) ss = __builtin_fmaf(r, r, ss);
      }
    const float total = block_sum256(ss, red);
    const float inv = 1.0f / __builtin_sqrtf(total / (float)n + P.eps);
#pragma unroll
    for (int k = 0; k < kNormPieces; k++) {
      const int pi = t + 256 * k;
      if (pi < np) {
        float o[8];
#pragma unroll
        for (int e = 0; e < 8; e++) {
          const float w = piece_f32<XT>(qw[k], e);
          o[e] = PRO == Pro::kAddNorm ? (rr[k][e] * inv) * w : (rr[k][e] * inv) * (w + 0.0f);
        }
        if (writer)
          reinterpret_cast<uint4*>(reinterpret_cast<XT*>(P.residual_out) + tok * P.token_x)[pi] = pack_piece<XT>(rr[k]);
        reinterpret_cast<uint4*>(xs_lds)[pi] = pack_piece<XT>(o);
      }
    }
  }
  lds_barrier();
  if (!active) return;

  // the row this lane stores and, for the RoPE segments, its cos / sin table entries:
  // requested now so that they arrive during the dot products instead of costing the
  // epilogue a memory round trip (a non-RoPE lane reads a weight byte pair instead, so
  // the loads are unconditional)
  const int frow = rs_row<ROWS>(l, log2c(ROWS), 0) * SUBS + sub;
  const bool fstore = (l >> log2c(ROWS)) == 0;
  const int fr = lr0 + frow;
  const bool ok = fstore && fr < srows;
  bool odd = false, up_unused;
  const int ph = phys(frow, fr < srows, up_unused, odd);
  const int64_t pos = (int64_t)__builtin_amdgcn_readfirstlane(pos_raw);
  const bool rope = (kind == kSegRopeOut || kind == kSegRopeCache) && pos >= 0 && pos < P.table_rows;
  const int hd = P.head_dim > 0 ? P.head_dim : 1;   // 0 for launches without RoPE segments
  const int rope_j = (ph % hd) - (odd ? (hd >> 1) : 0);
  const uint16_t* cos_p = rope ? reinterpret_cast<const uint16_t*>(P.cos) + pos * P.table_row + rope_j
                               : reinterpret_cast<const uint16_t*>(wlo);
  const uint16_t* sin_p = rope ? reinterpret_cast<const uint16_t*>(P.sin) + pos * P.table_row + rope_j
                               : reinterpret_cast<const uint16_t*>(wlo);
  const uint32_t cos_raw = *cos_p, sin_raw = *sin_p;

  float acc[NVG];
#pragma unroll
  for (int k = 0; k < NVG; k++) acc[k] = 0.0f;
  int r = 0;
  do {
    Raw<B> wn[ROWS];
    f16_t sn[NS];
    const bool more = r + 1 < rounds;
    if (more) fetch(r + 1, wn, sn);
    const int j = r * LPR + l;
    const bool cv = j < nchunks;
    uint32_t xw[16];
    {
      const uint4* xp = reinterpret_cast<const uint4*>(xs_lds + (cv ? j : 0) * 16);
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const uint4 v = xp[q];
        xw[4 * q] = v.x; xw[4 * q + 1] = v.y; xw[4 * q + 2] = v.z; xw[4 * q + 3] = v.w;
      }
    }
    float p[ROWS];
    chunk_dot_rows<F, XT, ROWS>(wc, xw, p);
#pragma unroll
    for (int i = 0; i < ROWS; i++) p[i] = (cv && rv[i]) ? p[i] : 0.0f;
    if constexpr (kInt4) {
      reduce_range<ROWS, 1, L>(p);
#pragma unroll
      for (int k = 0; k < NVG; k++) {
        const float t = p[k] * to_f32(sc[k]);
        acc[k] = acc[k] + ((cv && sv[k]) ? t : 0.0f);
      }
    } else {
#pragma unroll
      for (int i = 0; i < ROWS; i++) acc[i] = acc[i] + p[i];
    }
    if (more) {
#pragma unroll
      for (int i = 0; i < ROWS; i++) wc[i] = wn[i];
      if constexpr (kInt4) {
#pragma unroll
        for (int k = 0; k < NS; k++) sc[k] = sn[k];
      }
    }
  } while (++r < rounds);
  if constexpr (kInt4) reduce_range<NVG, L, LPR>(acc);
  else reduce_range<ROWS, 1, LPR>(acc);

  // ---- epilogue on the row held by this lane (same as gemv_kernel's fused epilogues)
  float v = acc[0];
  if (kind == kSegPlain) {
    if (ok) {
      if (S.bias != nullptr) v = round_to<XT>(v) + to_f32(reinterpret_cast<const XT*>(S.bias)[fr]);
      store<XT>(reinterpret_cast<XT*>(S.out) + tok * P.token_out + fr, v);
    }
    return;
  }
  if (S.bias != nullptr && ok) v = round_to<XT>(v) + to_f32(reinterpret_cast<const XT*>(S.bias)[ph]);
  const float val = round_to<XT>(v);
  const float pv = xor_partner<ROWS / 2 < 1 ? 1 : ROWS / 2>(val);   // the other half of the pair
  if (kind == kSegSilu) {
    if (ok && !odd) store<XT>(reinterpret_cast<XT*>(S.out) + tok * P.token_out + ph, silu_mul_val(val, pv));
    return;
  }
  const int D = P.head_dim;
  float o = val;
  if (rope) {
    const float c = lo_f32<XT>(cos_raw);
    const float sn = lo_f32<XT>(sin_raw);
    float o1, o2;
    if (odd) rope_pair<XT>(pv, val, c, sn, o1, o2);
    else rope_pair<XT>(val, pv, c, sn, o1, o2);
    o = odd ? o2 : o1;
  }
  if (ok) {
    if (kind == kSegRopeOut) {
      store<XT>(reinterpret_cast<XT*>(S.out) + tok * P.token_out + ph, o);
    } else if (pos >= 0 && pos < P.capacity) {
      const int64_t h = ph / D, d = ph - h * D;
      store<XT>(reinterpret_cast<XT*>(S.out) + tok * P.token_cache + h * P.cache_head + pos * D + d, o);
    }
  }
}

// fused_lean_kernel for TOK tokens of a batched step per workgroup (a copy, so that the
// one-token kernel's code stays as it is): every weight load feeds TOK tokens' dot
// products, each in the one-token order (token t's activation at LDS slice t, its own
// prologue and epilogue), so each token's outputs keep their bits.
template <Fmt F, typename XT, int LPR, int ROWS, Pro PRO, bool MULTI, int TOK>
__global__ __launch_bounds__(256) void fused_lean_tok_kernel(const LeanFused P) {
  constexpr bool kInt4 = F == Fmt::kInt4Sym;
  constexpr int B = FmtInfo<F>::kBytes;
  constexpr int L = kInt4 ? 4 : 1;
  constexpr int SUBS = 64 / LPR;
  constexpr int NVG = kInt4 ? (ROWS / L > 0 ? ROWS / L : 1) : ROWS;
  constexpr int NS = kInt4 ? NVG : 1;
  constexpr int GLEV = kInt4 ? (log2c(L) < log2c(ROWS) ? log2c(L) : log2c(ROWS)) : 0;
  static_assert(ROWS >= 2, "paired segments need two rows per wave");
  extern __shared__ uint32_t xs_lds[];
  const int lane = threadIdx.x & 63;
  const int sub = lane / LPR;
  const int l = lane % LPR;
  const int cols = P.cols;
  const int nchunks = cols >> 5;
  const int rounds = (nchunks + LPR - 1) / LPR;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int v0 = (int)(blockIdx.x * 4 + wave) * (ROWS * SUBS);   // first virtual row (uniform)
  const bool active = v0 < P.vtotal;
  const int64_t tok0 = (int64_t)blockIdx.y * TOK;   // first token of the workgroup
  // ---- the prologue's inputs are requested first -- before the row addressing, which
  // is a few hundred scalar instructions for paired segments, and before round 0 of the
  // weights, so that waiting for them never waits for the weight stream: one 16-byte
  // piece of each vector per held piece (cols <= 4096, a multiple of 32; indices past the
  // last piece repeat it)
  __shared__ float red[4];
  const int n = cols;
  const int np = n >> 3;
  uint4 qa[TOK][kNormPieces], qb[TOK][kNormPieces], qw[kNormPieces];
  if constexpr (PRO != Pro::kLoad) {
#pragma unroll
    for (int ti = 0; ti < TOK; ti++) {
      const int64_t tok = tok0 + ti;
      const uint16_t* pa;
      if constexpr (PRO == Pro::kEmbedNorm) {
        int64_t t = P.token[tok];
        t = t < 0 ? 0 : (t >= P.vocab ? P.vocab - 1 : t);
        pa = reinterpret_cast<const uint16_t*>(P.embed) + t * P.embed_row;
      } else {
        pa = reinterpret_cast<const uint16_t*>(P.left) + tok * P.token_x;
      }
      const uint16_t* pb = reinterpret_cast<const uint16_t*>(P.right) + tok * P.token_x;
#pragma unroll
      for (int k = 0; k < kNormPieces; k++) {
        const int pi = (int)threadIdx.x + 256 * k;
        const int pc = pi < np ? pi : np - 1;
        qa[ti][k] = reinterpret_cast<const uint4*>(pa)[pc];
        if constexpr (PRO != Pro::kEmbedNorm) qb[ti][k] = reinterpret_cast<const uint4*>(pb)[pc];
        if (ti == 0) qw[k] = reinterpret_cast<const uint4*>(P.norm_w)[pc];
      }
    }
  }
  // the token position of the RoPE / cache epilogues, requested with the prologue's
  // inputs so that the epilogue's table reads are its only dependent round trip
  const int32_t pos_raw = P.pos != nullptr ? P.pos[0] : 0;
  __builtin_amdgcn_sched_barrier(0);
  // MULTI: every segment's fields are read from the kernel arguments unconditionally and
  // the wave's segment is selected afterwards (scalar selects), so the argument loads go
  // out together instead of a second round trip behind the segment index; a
  // one-segment launch reads segment 0 only (fewer argument loads, fewer scalar
  // registers)
  int si = 0;
  if constexpr (MULTI) si = (P.nseg > 1 && v0 >= P.seg[1].vbegin ? 1 : 0) + (P.nseg > 2 && v0 >= P.seg[2].vbegin ? 1 : 0);
  const LeanSeg S = MULTI ? pick_seg(P.seg[0], P.seg[1], P.seg[2], si) : P.seg[0];
  const int kind = S.kind;
  const int srows = S.rows;
  const int lr0 = v0 - S.vbegin;
  const bool paired = kind == kSegRopeOut || kind == kSegRopeCache || kind == kSegSilu;

  // Physical row (and matrix) of row vr (0 .. ROWS * SUBS - 1) of this wave's block, the
  // mapping of paired_row: the block starts on a pair boundary (lr0 is a multiple of
  // ROWS * SUBS), so its rows are a few shifts away from its first pair P0, and for the
  // RoPE segments the block's pairs lie in one head (the host checks that half a head
  // is a whole number of blocks), whose index and in-head offset are one scalar
  // division per wave.  Rows past the segment read the block's first row, and a block
  // past the segment reads row 0 (in bounds; the values are never used).
  const int P0 = lr0 >> 1;
  const int half = P.head_dim >> 1;
  int h0 = 0, j0 = 0;
  if (kind == kSegRopeOut || kind == kSegRopeCache) {
    h0 = (int)((uint32_t)P0 / (uint32_t)half);
    j0 = P0 - h0 * half;
  }
  const bool any_row = lr0 < srows;
  const bool silu = kind == kSegSilu;
  const int rope_base = h0 * P.head_dim + j0;   // row of the block's first pair (RoPE segments)
  // (selects only, no branches: the row addressing stays a short straight run ahead of
  // the first weight loads)
  auto phys = [&](int vr, bool valid, bool& up, bool& odd) -> int {
    vr = valid ? vr : 0;
    const int blk = vr / (2 * SUBS), rem = vr % (2 * SUBS);   // SUBS is a power of two
    const bool o = paired && rem >= SUBS;
    const int poff = blk * SUBS + (o ? rem - SUBS : rem);
    const int pr = silu ? P0 + poff : rope_base + poff + (o ? half : 0);
    const int ph = paired ? pr : lr0 + vr;
    odd = o;
    up = o && silu && any_row;
    return any_row ? ph : 0;
  };
  // both matrices' base pointers in scalar registers, so the per-lane choice between them
  // is a select and not a vector load of the chosen kernel argument
  const uint8_t* const wlo = uniform_ptr(S.w);
  const uint8_t* const whi = uniform_ptr(S.w2);
  const uint8_t* wrow[ROWS];
  bool rv[ROWS];
#pragma unroll
  for (int i = 0; i < ROWS; i++) {
    const int vr = i * SUBS + sub;
    rv[i] = lr0 + vr < srows;
    bool up, odd;
    const int ph = phys(vr, rv[i], up, odd);
    wrow[i] = (up ? whi : wlo) + (size_t)ph * S.w_row;
  }
  const f16_t* srow[NS];
  bool sv[NS];
  if constexpr (kInt4) {
    const f16_t* const slo = uniform_ptr(S.s);
    const f16_t* const shi = uniform_ptr(S.s2);
#pragma unroll
    for (int k = 0; k < NS; k++) {
      const int vr = rs_row<ROWS>(l, GLEV, k) * SUBS + sub;
      sv[k] = lr0 + vr < srows;
      bool up, odd;
      const int ph = phys(vr, sv[k], up, odd);
      srow[k] = (up ? shi : slo) + (size_t)ph * S.s_row;
    }
  }
  auto fetch = [&](int r, Raw<B>* w, f16_t* sc) {
    uint32_t j = (uint32_t)(r * LPR + l);
    j = j < (uint32_t)nchunks ? j : (uint32_t)nchunks - 1;
#pragma unroll
    for (int i = 0; i < ROWS; i++) w[i] = load_raw<B>(wrow[i] + j * (uint32_t)B);
    if constexpr (kInt4) {
#pragma unroll
      for (int k = 0; k < NS; k++) sc[k] = srow[k][j >> 2];
    }
  };
  __builtin_amdgcn_sched_barrier(0);
  Raw<B> wc[ROWS];
  f16_t sc[NS];
  fetch(0, wc, sc);   // in bounds for inactive waves too (rows clamped)
  // nothing that consumes the prologue's loads may be scheduled above round 0's weight
  // loads: its wait would hold the weight stream back by a memory round trip
  __builtin_amdgcn_sched_barrier(0);

  // ---- activation vector into LDS
  if constexpr (PRO == Pro::kLoad) {
    const int xn = cols >> 3;
#pragma unroll
    for (int ti = 0; ti < TOK; ti++)
      for (int idx = threadIdx.x; idx < xn; idx += 256)
        reinterpret_cast<uint4*>(xs_lds)[ti * xn + idx] = reinterpret_cast<const uint4*>(
            reinterpret_cast<const uint16_t*>(P.x) + (tok0 + ti) * P.token_x)[idx];
  } else {
    // RMSNorm of the residual stream in the piece partition, reduction order and
    // rounding points of the standalone rms_norm / add_rms_norm kernels; workgroup 0
    // stores the residual.
    const bool writer = blockIdx.x == 0 && P.residual_out != nullptr;
    const int t = threadIdx.x;
#pragma unroll
    for (int ti = 0; ti < TOK; ti++) {
      const int64_t tok = tok0 + ti;
      float rr[kNormPieces][8];
      float ss = 0.0f;
#pragma unroll
      for (int k = 0; k < kNormPieces; k++)
#pragma unroll
        for (int e = 0; e < 8; e++) {
          const float a = piece_f32<XT>(qa[ti][k], e);
          float r;
          if constexpr (PRO == Pro::kAddNorm) r = round_bf16(a + piece_f32<XT>(qb[ti][k], e));
          else if constexpr (PRO == Pro::kAddRmsNorm) r = round_to<XT>(a + piece_f32<XT>(qb[ti][k], e));
          else r = a;
          rr[k][e] = r;
          if (8 * (t + 256 * k) + e < n) ss = __builtin_fmaf(r, r, ss);
        }
      const float total = block_sum256(ss, red);
      const float inv = 1.0f / __builtin_sqrtf(total / (float)n + P.eps);
#pragma unroll
      for (int k = 0; k < kNormPieces; k++) {
        const int pi = t + 256 * k;
        if (pi < np) {
          float o[8];
#pragma unroll
          for (int e = 0; e < 8; e++) {
            const float w = piece_f32<XT>(qw[k], e);
            o[e] = PRO == Pro::kAddNorm ? (rr[k][e] * inv) * w : (rr[k][e] * inv) * (w + 0.0f);
          }
          if (writer)
            reinterpret_cast<uint4*>(reinterpret_cast<XT*>(P.residual_out) + tok * P.token_x)[pi] = pack_piece<XT>(rr[k]);
          reinterpret_cast<uint4*>(xs_lds)[ti * np + pi] = pack_piece<XT>(o);
        }
      }
    }
  }
  lds_barrier();
  if (!active) return;

  // the row this lane stores and, for the RoPE segments, its cos / sin table entries:
  // requested now so that they arrive during the dot products instead of costing the
  // epilogue a memory round trip (a non-RoPE lane reads a weight byte pair instead, so
  // the loads are unconditional)
  const int frow = rs_row<ROWS>(l, log2c(ROWS), 0) * SUBS + sub;
  const bool fstore = (l >> log2c(ROWS)) == 0;
  const int fr = lr0 + frow;
  const bool ok = fstore && fr < srows;
  bool odd = false, up_unused;
  const int ph = phys(frow, fr < srows, up_unused, odd);
  const int64_t pos = (int64_t)__builtin_amdgcn_readfirstlane(pos_raw);
  const bool rope = (kind == kSegRopeOut || kind == kSegRopeCache) && pos >= 0 && pos < P.table_rows;
  const int hd = P.head_dim > 0 ? P.head_dim : 1;   // 0 for launches without RoPE segments
  const int rope_j = (ph % hd) - (odd ? (hd >> 1) : 0);
  const uint16_t* cos_p = rope ? reinterpret_cast<const uint16_t*>(P.cos) + pos * P.table_row + rope_j
                               : reinterpret_cast<const uint16_t*>(wlo);
  const uint16_t* sin_p = rope ? reinterpret_cast<const uint16_t*>(P.sin) + pos * P.table_row + rope_j
                               : reinterpret_cast<const uint16_t*>(wlo);
  const uint32_t cos_raw = *cos_p, sin_raw = *sin_p;

  float acc_t[TOK][NVG];
#pragma unroll
  for (int ti = 0; ti < TOK; ti++)
#pragma unroll
    for (int k = 0; k < NVG; k++) acc_t[ti][k] = 0.0f;
  int r = 0;
  do {
    Raw<B> wn[ROWS];
    f16_t sn[NS];
    const bool more = r + 1 < rounds;
    if (more) fetch(r + 1, wn, sn);
    const int j = r * LPR + l;
    const bool cv = j < nchunks;
#pragma unroll
    for (int ti = 0; ti < TOK; ti++) {
      float* acc = acc_t[ti];
      uint32_t xw[16];
      {
        const uint4* xp = reinterpret_cast<const uint4*>(xs_lds + ti * (cols >> 1) + (cv ? j : 0) * 16);
#pragma unroll
        for (int q = 0; q < 4; q++) {
          const uint4 v = xp[q];
          xw[4 * q] = v.x; xw[4 * q + 1] = v.y; xw[4 * q + 2] = v.z; xw[4 * q + 3] = v.w;
        }
      }
      float p[ROWS];
      chunk_dot_rows<F, XT, ROWS>(wc, xw, p);
#pragma unroll
      for (int i = 0; i < ROWS; i++) p[i] = (cv && rv[i]) ? p[i] : 0.0f;
      if constexpr (kInt4) {
        reduce_range<ROWS, 1, L>(p);
#pragma unroll
        for (int k = 0; k < NVG; k++) {
          const float t = p[k] * to_f32(sc[k]);
          acc[k] = acc[k] + ((cv && sv[k]) ? t : 0.0f);
        }
      } else {
#pragma unroll
        for (int i = 0; i < ROWS; i++) acc[i] = acc[i] + p[i];
      }
    }
    if (more) {
#pragma unroll
      for (int i = 0; i < ROWS; i++) wc[i] = wn[i];
      if constexpr (kInt4) {
#pragma unroll
        for (int k = 0; k < NS; k++) sc[k] = sn[k];
      }
    }
  } while (++r < rounds);
#pragma unroll
  for (int ti = 0; ti < TOK; ti++) {
    if constexpr (kInt4) reduce_range<NVG, L, LPR>(acc_t[ti]);
    else reduce_range<ROWS, 1, LPR>(acc_t[ti]);
  }

  // ---- epilogue on the row held by this lane, once per token of the workgroup
  auto epilogue = [&](float v, int64_t tok) __attribute__((always_inline)) {
  if (kind == kSegPlain) {
    if (ok) {
      if (S.bias != nullptr) v = round_to<XT>(v) + to_f32(reinterpret_cast<const XT*>(S.bias)[fr]);
      store<XT>(reinterpret_cast<XT*>(S.out) + tok * P.token_out + fr, v);
    }
    return;
  }
  if (S.bias != nullptr && ok) v = round_to<XT>(v) + to_f32(reinterpret_cast<const XT*>(S.bias)[ph]);
  const float val = round_to<XT>(v);
  const float pv = xor_partner<ROWS / 2 < 1 ? 1 : ROWS / 2>(val);   // the other half of the pair
  if (kind == kSegSilu) {
    if (ok && !odd) store<XT>(reinterpret_cast<XT*>(S.out) + tok * P.token_out + ph, silu_mul_val(val, pv));
    return;
  }
  const int D = P.head_dim;
  float o = val;
  if (rope) {
    const float c = lo_f32<XT>(cos_raw);
    const float sn = lo_f32<XT>(sin_raw);
    float o1, o2;
    if (odd) rope_pair<XT>(pv, val, c, sn, o1, o2);
    else rope_pair<XT>(val, pv, c, sn, o1, o2);
    o = odd ? o2 : o1;
  }
  if (ok) {
    if (kind == kSegRopeOut) {
      store<XT>(reinterpret_cast<XT*>(S.out) + tok * P.token_out + ph, o);
    } else if (pos >= 0 && pos < P.capacity) {
      const int64_t h = ph / D, d = ph - h * D;
      store<XT>(reinterpret_cast<XT*>(S.out) + tok * P.token_cache + h * P.cache_head + pos * D + d, o);
    }
  }
  };
#pragma unroll
  for (int ti = 0; ti < TOK; ti++) epilogue(acc_t[ti][0], tok0 + ti);
}


// Tokens per workgroup of the batched dense multi-matrix launch (gpt-oss QKV, eight
// sequences): two measured 2,262 tok/s, four 2,249, eight 2,079 (VALU-bound) and one
// 2,222 on one box.
#ifndef TT_FUSED_TOK
#define TT_FUSED_TOK 2
#endif

// Rows per wave of the lean fused kernel (paired segments need two).  Eight for the
// largest launches (the 1B gate/up, 16384 virtual rows: 9.06 -> 8.69 us against four):
// half the waves, each prologue shared by twice the rows.
inline int fused_rows_per_wave(int64_t vrows, int lpr) {
  const int64_t groups = vrows * lpr / 64;
  // four for the 64-lane rows of 2048 to 8191 lane groups (the 1B QKV, 3072 rows: 1,791 ->
  // 1,800 tok/s decode); the 32-lane gpt-oss QKV stays at two (743 -> 729 tok/s at four)
  if (lpr == 64 && groups >= 2048 && groups < 8192) return 4;
  return groups >= 16384 ? 8 : (groups >= 8192 ? 4 : 2);
}

LeanFused lean_params(const tt_fused_gemv* d, int per_batch) {
  LeanFused P{};
  P.nseg = d->count;
  int v = 0;
  for (int i = 0; i < d->count; i++) {
    const tt_fused_segment& g = d->seg[i];
    LeanSeg& S = P.seg[i];
    S.w = static_cast<const uint8_t*>(g.weight);
    S.w2 = static_cast<const uint8_t*>(g.weight2);
    S.s = static_cast<const f16_t*>(g.scales);
    S.s2 = static_cast<const f16_t*>(g.scales2);
    S.out = g.out;
    S.bias = g.bias;
    S.w_row = (uint32_t)g.w_row_bytes;
    S.s_row = (uint32_t)g.s_row;
    S.rows = (int)(g.kind == TT_SEG_SILU ? 2 * g.rows : g.rows);
    S.vbegin = v;
    S.kind = g.kind;
    v += (S.rows + per_batch - 1) / per_batch * per_batch;
  }
  P.vtotal = v;
  P.cols = (int)d->cols;
  P.head_dim = (int)d->head_dim;
  P.x = d->x;
  P.left = d->left;
  P.right = d->right;
  P.embed = d->embed;
  P.embed_row = d->embed_row;
  P.vocab = d->vocab;
  P.token = d->token;
  P.norm_w = d->norm_weight;
  P.eps = d->eps;
  P.residual_out = d->residual_out;
  P.pos = d->position;
  P.capacity = d->capacity;
  P.cache_head = d->cache_head;
  P.cos = d->cos_table;
  P.sin = d->sin_table;
  P.table_row = d->table_row;
  P.table_rows = d->table_rows;
  P.token_x = d->token_x;
  P.token_out = d->token_out;
  P.token_cache = d->token_cache;
  return P;
}

// The lean kernel covers int4 g128 and dense segments whose operands fit 32-bit
// offsets and whose activation vector fits the register-held prologue.  With RoPE
// segments half a head must hold whole wave blocks of pairs (at most 4 rows per wave
// times 4 lane groups, i.e. 8 pairs): head_dim a multiple of 16.
bool lean_fits(const tt_fused_gemv* d) {
  if (d->cols > 4096) return false;
  for (int i = 0; i < d->count; i++) {
    const tt_fused_segment& g = d->seg[i];
    const int64_t rows = g.rows;
    if (g.w_row_bytes >= ((int64_t)1 << 31) || rows * g.w_row_bytes >= ((int64_t)1 << 31)) return false;
    if (g.s_row >= ((int64_t)1 << 30)) return false;
    if ((g.kind == TT_SEG_ROPE_OUT || g.kind == TT_SEG_ROPE_CACHE) && d->head_dim % 16 != 0) return false;
  }
  return true;
}

template <Fmt F, typename XT, int LPR, Pro PRO>
int launch_lean_lpr(const tt_fused_gemv* d, hipStream_t st) {
  int64_t vrows = 0;
  for (int i = 0; i < d->count; i++) vrows += d->seg[i].kind == TT_SEG_SILU ? 2 * d->seg[i].rows : d->seg[i].rows;
  const int rpw = fused_rows_per_wave(vrows, LPR);
  const int per_batch = rpw * (64 / LPR);
  const LeanFused P = lean_params(d, per_batch);
  const int64_t waves = P.vtotal / per_batch;
  const size_t lds = (size_t)d->cols * 2;
  const unsigned ytok = (unsigned)(d->tokens > 1 ? d->tokens : 1);
  const dim3 grid((unsigned)((waves + 3) / 4), ytok);
  // dense multi-matrix launches of a batched step (the gpt-oss QKV of eight sequences):
  // TT_FUSED_TOK tokens per workgroup, so each weight row is streamed once per group of
  // tokens instead of once per token
  if constexpr (F != Fmt::kInt4Sym && LPR == 32) {
    constexpr int TK = TT_FUSED_TOK;
    if (TK > 1 && d->count > 1 && d->tokens >= TK && d->tokens % TK == 0) {
      const dim3 gt((unsigned)((waves + 3) / 4), (unsigned)(d->tokens / TK));
      const size_t ldst = (size_t)TK * d->cols * 2;
      if (rpw == 8) hipLaunchKernelGGL((fused_lean_tok_kernel<F, XT, LPR, 8, PRO, true, TK>), gt, dim3(256), ldst, st, P);
      else if (rpw == 4) hipLaunchKernelGGL((fused_lean_tok_kernel<F, XT, LPR, 4, PRO, true, TK>), gt, dim3(256), ldst, st, P);
      else hipLaunchKernelGGL((fused_lean_tok_kernel<F, XT, LPR, 2, PRO, true, TK>), gt, dim3(256), ldst, st, P);
      return check_launch(kWhat);
    }
  }
  if (d->count > 1) {
    if (rpw == 8) hipLaunchKernelGGL((fused_lean_kernel<F, XT, LPR, 8, PRO, true>), grid, dim3(256), lds, st, P);
    else if (rpw == 4) hipLaunchKernelGGL((fused_lean_kernel<F, XT, LPR, 4, PRO, true>), grid, dim3(256), lds, st, P);
    else hipLaunchKernelGGL((fused_lean_kernel<F, XT, LPR, 2, PRO, true>), grid, dim3(256), lds, st, P);
  } else {
    if (rpw == 8) hipLaunchKernelGGL((fused_lean_kernel<F, XT, LPR, 8, PRO, false>), grid, dim3(256), lds, st, P);
    else if (rpw == 4) hipLaunchKernelGGL((fused_lean_kernel<F, XT, LPR, 4, PRO, false>), grid, dim3(256), lds, st, P);
    else hipLaunchKernelGGL((fused_lean_kernel<F, XT, LPR, 2, PRO, false>), grid, dim3(256), lds, st, P);
  }
  return check_launch(kWhat);
}

template <Fmt F, typename XT, Pro PRO>
int launch_lean_f(const tt_fused_gemv* d, int lpr, hipStream_t st) {
  if (lpr == 64) return launch_lean_lpr<F, XT, 64, PRO>(d, st);
  if (lpr == 32) return launch_lean_lpr<F, XT, 32, PRO>(d, st);
  return launch_lean_lpr<F, XT, 16, PRO>(d, st);
}

template <typename XT, Pro PRO>
int launch_lean(const tt_fused_gemv* d, int lpr, hipStream_t st) {
  if (d->weight_format == TT_FMT_INT4_G) return launch_lean_f<Fmt::kInt4Sym, XT, PRO>(d, lpr, st);
  if (d->weight_dtype == TT_F16) return launch_lean_f<Fmt::kF16W, XT, PRO>(d, lpr, st);
  return launch_lean_f<Fmt::kBF16W, XT, PRO>(d, lpr, st);
}

// Highest key among n partials (256 threads), then token / value / bookkeeping; the
// position inputs are requested before the partials.
__global__ __launch_bounds__(256) void argmax_step_kernel(const uint64_t* partials, int n, int64_t* out_idx,
                                                          float* out_val, int32_t* pos, const int32_t* base,
                                                          int64_t* history, int32_t history_len) {
  __shared__ uint64_t red[4];
  int32_t p0 = 0, b0 = 0;
  if (threadIdx.x == 0 && pos != nullptr) {
    p0 = pos[0];
    if (base != nullptr) b0 = base[0];
  }
  const uint64_t k = block_max_u64(partials, n, red);
  if (threadIdx.x == 0) {
    const uint32_t o = (uint32_t)(k >> 32);
    const uint32_t bits = o == 0xffffffffu ? 0x7fc00000u : ((o & 0x80000000u) ? (o & 0x7fffffffu) : ~o);
    const int64_t token = (int64_t)(0xffffffffu - (uint32_t)k);
    out_idx[0] = token;
    if (out_val) out_val[0] = __builtin_bit_cast(float, bits);
    if (pos) {
      const int32_t i = p0 - b0;
      if (history && i >= 0 && i < history_len) history[i] = token;
      pos[0] = p0 + 1;
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
      TT_REQUIRE(aligned(d->left, 16) && aligned(d->right, 16) && aligned(d->norm_weight, 16),
                 "%s: the norm prologue reads 16-byte pieces: left, right and the weight must be 16-byte aligned",
                 kWhat);
      break;
    case TT_PRO_EMBED_NORM:
      TT_REQUIRE(d->embed && d->token && d->norm_weight && d->vocab > 0 && d->embed_row >= d->cols,
                 "%s: embedding prologue needs the table, the device token and the weight", kWhat);
      TT_REQUIRE(aligned(d->embed, 16) && d->embed_row % 8 == 0 && aligned(d->norm_weight, 16),
                 "%s: the norm prologue reads 16-byte pieces: embedding rows and the weight must be 16-byte aligned",
                 kWhat);
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
  TT_REQUIRE(d->tokens >= 0 && d->tokens <= 65535, "%s: bad token count", kWhat);
  if (d->tokens > 1) {
    TT_UNSUPPORTED(!lm_head && lean_fits(d), "%s: several tokens per launch need cols <= 4096 and 32-bit offsets",
                   kWhat);
    TT_REQUIRE(d->token_x >= d->cols && d->token_x % 8 == 0 && d->token_out >= 0 && d->token_cache >= 0,
               "%s: bad token strides", kWhat);
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
  if (!argmax && lean_fits(d)) return launch_lean<AT, PRO>(d, lpr, st);
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
