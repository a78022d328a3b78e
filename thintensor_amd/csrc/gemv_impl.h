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
#pragma once

#include "tt_abi_internal.h"
#include "tt_gemv.h"

namespace tt {

enum class SMode : int { kNone = 0, kRow = 1, kGroup = 2, kGroupAff = 3, kBlockE8 = 4 };

// Epilogue of a segment in the fused decode kernels (EPI instantiations only).
enum SegKind : int {
  kSegPlain = 0,      // store row values to out (+ bias)
  kSegRopeOut = 1,    // rows of heads, RoPE applied, stored to out
  kSegRopeCache = 2,  // rows of KV heads, RoPE applied, stored to the K cache at the position
  kSegCache = 3,      // rows of KV heads stored to the V cache at the position
  kSegSilu = 4,       // gate rows from w/s, up rows from w2/s2; out[i] = silu(gate_i) * up_i
};

struct Seg {
  const uint8_t* w;     // weight bytes of expert 0 / the matrix
  int64_t w_row;        // bytes between rows
  const void* s;        // scales
  int64_t s_row, s_grp; // scale element strides
  void* out;            // output (slot 0)
  int rows;             // virtual rows (kSegSilu: 2 x activation rows)
  int vbegin;           // first virtual row (batches never straddle segments)
  const void* bias;     // optional per-row bias in the output dtype: out = r(r(dot) + b)
  int kind;             // SegKind
  const uint8_t* w2;    // kSegSilu: up-projection weights and scales
  const void* s2;
};

// The segment of index si, every segment's fields read unconditionally first and the
// wanted one selected afterwards (uniform selects): the kernel-argument loads then go out
// in one batch instead of a second round trip behind the segment index.
__device__ __forceinline__ Seg pick_seg(const Seg a, const Seg b, const Seg c, int si) {
  Seg r;
  r.w = si == 0 ? a.w : (si == 1 ? b.w : c.w);
  r.w_row = si == 0 ? a.w_row : (si == 1 ? b.w_row : c.w_row);
  r.s = si == 0 ? a.s : (si == 1 ? b.s : c.s);
  r.s_row = si == 0 ? a.s_row : (si == 1 ? b.s_row : c.s_row);
  r.s_grp = si == 0 ? a.s_grp : (si == 1 ? b.s_grp : c.s_grp);
  r.out = si == 0 ? a.out : (si == 1 ? b.out : c.out);
  r.rows = si == 0 ? a.rows : (si == 1 ? b.rows : c.rows);
  r.vbegin = si == 0 ? a.vbegin : (si == 1 ? b.vbegin : c.vbegin);
  r.bias = si == 0 ? a.bias : (si == 1 ? b.bias : c.bias);
  r.kind = si == 0 ? a.kind : (si == 1 ? b.kind : c.kind);
  r.w2 = si == 0 ? a.w2 : (si == 1 ? b.w2 : c.w2);
  r.s2 = si == 0 ? a.s2 : (si == 1 ? b.s2 : c.s2);
  return r;
}

// Context of the fused prologue (activation vector built in the kernel) and the
// position-dependent epilogues.
struct FuseParams {
  const void* left;           // add+RMSNorm prologue: residual = bf16(left + right)
  const void* right;
  const void* embed;          // embedding prologue: residual = embed[token]
  int64_t embed_row, vocab;
  const int64_t* token;
  const void* norm_w;         // RMSNorm weight (activation dtype)
  float eps;
  void* residual_out;         // written by workgroup (0, 0)
  const int32_t* pos;         // decode position (device)
  int64_t capacity;           // KV cache tokens
  int64_t cache_head;         // elements between KV heads of one layer's cache
  const void* cos;            // RoPE tables [rows, table_row]
  const void* sin;
  int64_t table_row, table_rows;
  int head_dim;
};

// How the activation vector reaches LDS.
enum class Pro : int {
  kLoad = 0,       // copy x
  kAddNorm = 1,    // x = RMSNorm(bf16(left + right)) * w, residual stored
  kEmbedNorm = 2,  // x = RMSNorm(embed[token]) * w, residual (the embedding row) stored
  kAddRmsNorm = 3, // x = RMSNorm(round(left + right)) * w: add then rms_norm, residual stored
};

struct GemvParams {
  Seg seg[3];
  int nseg;
  int vtotal;              // virtual rows (segments padded to whole batches)
  const void* x;
  int64_t x_slot;          // activation elements between slots (0: shared vector)
  const void* experts;     // expert id per slot, int32 or int64 (nullptr: dense)
  int ishift;              // log2 of the id size in 32-bit words (0: int32, 1: int64)
  int64_t w_expert;        // bytes between experts
  int64_t s_expert;        // scale elements between experts
  int64_t out_slot;        // output elements between slots
  int64_t w_slot;          // bytes between slots without expert ids (split-K column slices)
  int64_t s_pair;          // affine: element offset of the second scale value
  int aff_zero;            // affine pair holds (s, z) instead of (s, m)
  int cols;
  uint64_t* am_partials;   // argmax epilogue: one key per wave (null: plain GEMV)
  FuseParams f;
};

// Order-preserving argmax key of a rounded logit at row `idx`: larger value wins,
// equal values (+0 == -0) go to the lower index, NaN beats every number (first NaN
// wins), matching torch.argmax on the rounded logits.
__device__ __forceinline__ uint64_t argmax_key(float v, uint32_t idx) {
  uint32_t b = __builtin_bit_cast(uint32_t, v);
  if ((b & 0x7fffffffu) == 0) b = 0;
  uint32_t o;
  if ((b & 0x7fffffffu) > 0x7f800000u) o = 0xffffffffu;
  else o = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  return ((uint64_t)o << 32) | (uint64_t)(0xffffffffu - idx);
}

constexpr int log2c(int v) { return v <= 1 ? 0 : 1 + log2c(v / 2); }

// Reduce per-lane values v[0..NV) over lane bits [M, MEND): reduce-scatter levels
// while more than one value is left, plain butterfly levels afterwards.
template <int NV, int M, int MEND>
__device__ __forceinline__ void reduce_range(float* v) {
  if constexpr (M < MEND) {
    if constexpr (NV > 1) {
      float t[NV / 2];
      rs_level<NV, M>(v, t);
#pragma unroll
      for (int i = 0; i < NV / 2; i++) v[i] = t[i];
      reduce_range<NV / 2, M * 2, MEND>(v);
    } else {
      v[0] = bfly<M>(v[0]);
      reduce_range<1, M * 2, MEND>(v);
    }
  }
}

// Row (within the batch) of value k held by lane l after reduce-scatter levels on
// the lowest `levels` lane bits of a batch of ROWS rows.
template <int ROWS>
__device__ __forceinline__ int rs_row(int l, int levels, int k) {
  int off = 0;
#pragma unroll
  for (int j = 0; j < log2c(ROWS); j++)
    if (j < levels) off += ((l >> j) & 1) * (ROWS >> (j + 1));
  return off + k;
}

template <Fmt F, SMode SM, typename ST, int ROWS, int NVG>
struct GemvBatch {
  bool active;
  int lr0, rows, kind;
  const uint8_t* wb;         // weight base of the segment (expert applied)
  const ST* sb;              // scale base of the segment (expert applied)
  int64_t s_row, s_grp;
  void* out;
  const void* bias;
  int64_t woffs[ROWS];       // byte offset of each batch row's weights from wb
  int rcl[ROWS];             // physical row of each batch row (clamped)
  bool rv[ROWS];
  int64_t soffs[NVG];        // element offset of each kept value's scale row from sb
};

// Physical row of virtual row v of a paired segment (RoPE pairs or gate/up pairs):
// virtual rows 2m*SUBS + sub and (2m + 1)*SUBS + sub of a block of 2*SUBS rows form
// pair m*SUBS + sub, so both halves of a pair land in the same lane group and the
// epilogue exchanges them with one cross-lane move.  RoPE: pair p of head h is
// (h*D + j, h*D + j + D/2) with j = p mod D/2; SiLU: pair p is (gate p, up p).
template <int SUBS>
__device__ __forceinline__ int paired_row(int v, int kind, int head_dim, bool& odd) {
  const int blk = v / (2 * SUBS), rem = v - blk * (2 * SUBS);
  odd = rem >= SUBS;
  const int pidx = blk * SUBS + (odd ? rem - SUBS : rem);
  if (kind == kSegSilu) return pidx;
  const int half = head_dim >> 1;
  const int h = pidx / half, j = pidx - h * half;
  return h * head_dim + j + (odd ? half : 0);
}

// One round's loads.  Scales stay in their storage type until the round is consumed,
// so issuing a fetch never waits for a load to return.
template <Fmt F, typename ST, int ROWS, int NVG>
struct GemvData {
  Raw<FmtInfo<F>::kBytes> w[ROWS];
  ST s[NVG], m[NVG];
  int e[ROWS];
};

template <Fmt F, SMode SM, typename XT, typename OT, typename ST, int LPR, int ROWS, int L, bool AM,
          Pro PRO = Pro::kLoad, bool EPI = false, int PF = 1, int MR = 1>
__global__ __launch_bounds__(256) void gemv_kernel(GemvParams P) {
  // MR > 1: MR activation rows (x + m * x_slot) share every weight load; output row m
  // at out + m * out_slot, each with the single-row reduction order.
  static_assert(MR == 1 || (PRO == Pro::kLoad && !EPI), "several activation rows only with a loaded x");
  extern __shared__ uint32_t xs_lds[];
  constexpr int B = FmtInfo<F>::kBytes;
  constexpr int SUBS = 64 / LPR;
  constexpr bool kGroup = SM == SMode::kGroup || SM == SMode::kGroupAff;
  constexpr int LG = kGroup ? L : 1;                        // lanes per quantisation group
  constexpr int NVG = ROWS / LG > 0 ? ROWS / LG : 1;        // values per lane after the group levels
  constexpr int GLEV = log2c(LG) < log2c(ROWS) ? log2c(LG) : log2c(ROWS);
  static_assert(ROWS <= LPR && LG <= LPR, "batch rows and groups must fit the lane group");
  using Batch = GemvBatch<F, SM, ST, ROWS, NVG>;
  using Data = GemvData<F, ST, ROWS, NVG>;

  const int slot = blockIdx.y;
  int64_t woff = (int64_t)slot * P.w_slot, soff = 0;
  if (P.experts != nullptr) {
    const int64_t e = load_expert(P.experts, P.ishift, slot);
    woff = e * P.w_expert;
    soff = e * P.s_expert;
  }
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int sub = lane / LPR;
  const int l = lane % LPR;
  const int nchunks = P.cols >> 5;
  const int rounds = (nchunks + LPR - 1) / LPR;
  const int per_iter = ROWS * SUBS;
  const int nwaves = gridDim.x * (blockDim.x >> 6);
  int grow[NVG];
#pragma unroll
  for (int k = 0; k < NVG; k++) grow[k] = rs_row<ROWS>(l, GLEV, k) * SUBS + sub;
  const int frow = rs_row<ROWS>(l, log2c(ROWS), 0) * SUBS + sub;  // row stored by this lane
  const bool fstore = (l >> log2c(ROWS)) == 0;
  uint64_t best[MR];
#pragma unroll
  for (int m = 0; m < MR; m++) best[m] = 0;

  auto setup = [&](int b, Batch& bt) {
    const int v0 = __builtin_amdgcn_readfirstlane(b * per_iter);
    bt.active = v0 < P.vtotal;
    int si = 0;
    if (P.nseg > 1 && v0 >= P.seg[1].vbegin) si = 1;
    if (P.nseg > 2 && v0 >= P.seg[2].vbegin) si = 2;
    si = __builtin_amdgcn_readfirstlane(si);
    const Seg S = pick_seg(P.seg[0], P.seg[1], P.seg[2], si);   // argument loads in one batch
    bt.lr0 = v0 - S.vbegin;
    bt.rows = S.rows;
    bt.kind = EPI ? S.kind : kSegPlain;
    bt.wb = S.w + woff;
    bt.sb = reinterpret_cast<const ST*>(S.s) + soff;
    bt.s_row = S.s_row;
    bt.s_grp = S.s_grp;
    bt.out = S.out;
    bt.bias = S.bias;
    if (!EPI || bt.kind == kSegPlain || bt.kind == kSegCache) {
#pragma unroll
      for (int i = 0; i < ROWS; i++) {
        const int r = i * SUBS + sub;
        bt.rv[i] = bt.lr0 + r < bt.rows;
        bt.rcl[i] = bt.rv[i] ? bt.lr0 + r : bt.rows - 1;
        bt.woffs[i] = (int64_t)bt.rcl[i] * S.w_row;
      }
#pragma unroll
      for (int k = 0; k < NVG; k++)
        bt.soffs[k] = (int64_t)(bt.lr0 + grow[k] < bt.rows ? bt.lr0 + grow[k] : bt.rows - 1) * S.s_row;
    } else if constexpr (EPI) {
      // paired segments: the up rows of a SiLU pair live in a second matrix, reached
      // by the byte / element distance between the two allocations
      const int64_t w2d = bt.kind == kSegSilu ? (int64_t)(S.w2 - S.w) : 0;
      const int64_t s2d = bt.kind == kSegSilu ? (int64_t)(reinterpret_cast<const ST*>(S.s2) - reinterpret_cast<const ST*>(S.s)) : 0;
#pragma unroll
      for (int i = 0; i < ROWS; i++) {
        const int r = i * SUBS + sub;
        bt.rv[i] = bt.lr0 + r < bt.rows;
        bool odd;
        const int ph = paired_row<SUBS>(bt.rv[i] ? bt.lr0 + r : bt.rows - 1, bt.kind, P.f.head_dim, odd);
        bt.rcl[i] = ph;
        bt.woffs[i] = (int64_t)ph * S.w_row + (odd ? w2d : 0);
      }
#pragma unroll
      for (int k = 0; k < NVG; k++) {
        bool odd;
        const int ph = paired_row<SUBS>(bt.lr0 + grow[k] < bt.rows ? bt.lr0 + grow[k] : bt.rows - 1, bt.kind,
                                        P.f.head_dim, odd);
        bt.soffs[k] = (int64_t)ph * S.s_row + (odd ? s2d : 0);
      }
    }
  };

  auto fetch = [&](const Batch& bt, int r, Data& d) {
    int j = r * LPR + l;
    j = j < nchunks ? j : nchunks - 1;
#pragma unroll
    for (int i = 0; i < ROWS; i++) d.w[i] = load_raw<B>(bt.wb + bt.woffs[i] + (int64_t)j * B);
    if constexpr (kGroup) {
#pragma unroll
      for (int k = 0; k < NVG; k++) {
        const int64_t off = bt.soffs[k] + (int64_t)(j / LG) * bt.s_grp;
        d.s[k] = bt.sb[off];
        if constexpr (SM == SMode::kGroupAff) d.m[k] = bt.sb[off + P.s_pair];
      }
    }
    if constexpr (SM == SMode::kBlockE8) {
#pragma unroll
      for (int i = 0; i < ROWS; i++) d.e[i] = reinterpret_cast<const uint8_t*>(bt.sb)[(int64_t)bt.rcl[i] * bt.s_row + j];
    }
  };

  // Activation loads are issued before the weight fetch and written to LDS once they
  // return, so a wave waits for memory once (weights, scales and x in flight together).
  // Piece idx (16 bytes) of the staged activations is piece idx - m * xn of row m; the
  // first 256 * kXR pieces go through registers, with indices clamped to the last piece
  // (duplicate loads and stores of the same value) so that no branch separates them.
  constexpr int kXR = 4;                  // 16-byte activation pieces per thread in registers
  const int xn = P.cols >> 3;             // 16-byte pieces per activation row
  const int xtotal = xn * MR;
  uint4 xreg[kXR];
  int xidx[kXR];
  if constexpr (PRO == Pro::kLoad) {
#pragma unroll
    for (int k = 0; k < kXR; k++) {
      const int idx = threadIdx.x + 256 * k;
      xidx[k] = idx < xtotal ? idx : xtotal - 1;
      const int m = MR == 1 ? 0 : xidx[k] / xn;
      const uint4* xg = reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(P.x) +
                                                       (int64_t)(slot + m) * P.x_slot);
      xreg[k] = xg[xidx[k] - m * xn];
    }
  }

  // The RMSNorm prologue's inputs (cols <= 4096, in the piece partition of tt_common.h)
  // are requested here too, ahead of the weights, as raw 16-byte pieces: indices past the
  // last piece repeat it (values discarded), so no branch separates the loads and waiting
  // for them never waits for the weight stream.
  uint4 qa[kNormPieces], qb[kNormPieces], qw[kNormPieces];
  if constexpr (PRO != Pro::kLoad) {
    const int np = P.cols >> 3;
    const uint16_t* pa;
    if constexpr (PRO == Pro::kEmbedNorm) {
      int64_t t = P.f.token[0];
      t = t < 0 ? 0 : (t >= P.f.vocab ? P.f.vocab - 1 : t);
      pa = reinterpret_cast<const uint16_t*>(P.f.embed) + t * P.f.embed_row;
    } else {
      pa = reinterpret_cast<const uint16_t*>(P.f.left);
    }
#pragma unroll
    for (int k = 0; k < kNormPieces; k++) {
      const int pi = (int)threadIdx.x + 256 * k;
      const int pc = pi < np ? pi : np - 1;
      qa[k] = reinterpret_cast<const uint4*>(pa)[pc];
      if constexpr (PRO != Pro::kEmbedNorm) qb[k] = reinterpret_cast<const uint4*>(P.f.right)[pc];
      qw[k] = reinterpret_cast<const uint4*>(P.f.norm_w)[pc];
    }
    __builtin_amdgcn_sched_barrier(0);   // raw bits only above: no use between the loads
  }

  int b = blockIdx.x * (blockDim.x >> 6) + wave;
  Batch cb;
  setup(b, cb);
  // PF == 1: one round in flight ahead of the one being computed.  PF > 1 (rounds <=
  // PF): every round of the next batch is fetched while the current batch computes.
  // The first fetch is unconditional: an inactive batch (past the last row) clamps every
  // row to the last row of the last segment, so its loads stay in bounds, and round 0
  // always exists (the host requires cols >= 32).
  Data cd[PF];
#pragma unroll
  for (int r = 0; r < PF; r++)
    if (r == 0 || r < rounds) fetch(cb, r, cd[r]);
  if constexpr (PRO == Pro::kLoad) {
    // LDS holds activation row m at uint4 offset m * xn.
    uint4* xl = reinterpret_cast<uint4*>(xs_lds);
#pragma unroll
    for (int k = 0; k < kXR; k++) xl[xidx[k]] = xreg[k];
    // the rest (several activation rows) in steps of kXR loads in flight per thread,
    // indices clamped as above
    for (int i0 = threadIdx.x + 256 * kXR; i0 < xtotal; i0 += 256 * kXR) {
#pragma unroll
      for (int k = 0; k < kXR; k++) {
        const int idx = i0 + 256 * k;
        xidx[k] = idx < xtotal ? idx : xtotal - 1;
        const int m = MR == 1 ? 0 : xidx[k] / xn;
        const uint4* xg = reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(P.x) +
                                                         (int64_t)(slot + m) * P.x_slot);
        xreg[k] = xg[xidx[k] - m * xn];
      }
#pragma unroll
      for (int k = 0; k < kXR; k++) xl[xidx[k]] = xreg[k];
    }
    __syncthreads();
  } else {
    // Build the activation vector: RMSNorm of the residual stream, with the same
    // thread partition, reduction order and rounding points as the standalone
    // rms_norm / add_rms_norm kernels (every workgroup computes the identical vector;
    // workgroup (0, 0) also stores the residual).
    __shared__ float red[4];
    const int n = P.cols;
    const XT* erow = nullptr;
    if constexpr (PRO == Pro::kEmbedNorm) {
      int64_t t = P.f.token[0];
      t = t < 0 ? 0 : (t >= P.f.vocab ? P.f.vocab - 1 : t);
      erow = reinterpret_cast<const XT*>(P.f.embed) + t * P.f.embed_row;
    }
    auto resid = [&](int i) -> float {
      if constexpr (PRO == Pro::kAddNorm) return norm_residual<XT>(P.f.left, P.f.right, i);
      else if constexpr (PRO == Pro::kAddRmsNorm) return round_to<XT>(ld<XT>(P.f.left, i) + ld<XT>(P.f.right, i));
      else return to_f32(erow[i]);
    };
    const bool writer = blockIdx.x == 0 && blockIdx.y == 0 && P.f.residual_out != nullptr;
    XT* xl = reinterpret_cast<XT*>(xs_lds);
    auto normed = [&](float r, float inv, float w) -> float {
      if constexpr (PRO == Pro::kAddNorm) return (r * inv) * w;
      else return (r * inv) * (w + 0.0f);
    };
    const int np = n >> 3;
    const int t = threadIdx.x;
    if (np <= 256 * kNormPieces) {
      // one pass over memory: the raw pieces requested before the weights
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
      const float inv = 1.0f / __builtin_sqrtf(total / (float)n + P.f.eps);
#pragma unroll
      for (int k = 0; k < kNormPieces; k++) {
        const int pi = t + 256 * k;
        if (pi < np) {
          float o[8];
#pragma unroll
          for (int e = 0; e < 8; e++) o[e] = normed(rr[k][e], inv, piece_f32<XT>(qw[k], e));
          if (writer) reinterpret_cast<uint4*>(P.f.residual_out)[pi] = pack_piece<XT>(rr[k]);
          reinterpret_cast<uint4*>(xs_lds)[pi] = pack_piece<XT>(o);
        }
      }
    } else {
      float ss = 0.0f;
      for (int pi = t; pi < np; pi += 256)
        for (int i = 8 * pi; i < 8 * pi + 8; i++) {
          const float r = resid(i);
          ss = __builtin_fmaf(r, r, ss);
        }
      const float total = block_sum256(ss, red);
      const float inv = 1.0f / __builtin_sqrtf(total / (float)n + P.f.eps);
      for (int pi = t; pi < np; pi += 256)
        for (int i = 8 * pi; i < 8 * pi + 8; i++) {
          const float r = resid(i);
          if (writer) store<XT>(reinterpret_cast<XT*>(P.f.residual_out) + i, r);
          store<XT>(xl + i, normed(r, inv, ld<XT>(P.f.norm_w, i)));
        }
    }
    __syncthreads();
  }

  // One round: chunk partials of the batch rows, scaled and accumulated in round order.
  auto consume = [&](const Batch& bt, const Data& d, int r, float (*accs)[ROWS]) {
    const int j = r * LPR + l;
    const bool cv = j < nchunks;
    uint32_t xws[MR][16];
#pragma unroll
    for (int m = 0; m < MR; m++) {
      const uint4* xp = reinterpret_cast<const uint4*>(xs_lds + m * (P.cols >> 1) + (cv ? j : 0) * 16);
#pragma unroll
      for (int q = 0; q < 4; q++) {
        uint4 v = xp[q];
        xws[m][4 * q] = v.x; xws[m][4 * q + 1] = v.y; xws[m][4 * q + 2] = v.z; xws[m][4 * q + 3] = v.w;
      }
    }
    float ps[MR][ROWS];
    chunk_dot_rows_multi<F, XT, ROWS, MR>(d.w, xws, ps);
#pragma unroll
    for (int m = 0; m < MR; m++) {
      float* acc = accs[m];
      float* p = ps[m];
      const uint32_t* xw = xws[m];
#pragma unroll
      for (int i = 0; i < ROWS; i++) p[i] = (cv && bt.rv[i]) ? p[i] : 0.0f;
      if constexpr (SM == SMode::kNone || SM == SMode::kRow) {
#pragma unroll
        for (int i = 0; i < ROWS; i++) acc[i] = acc[i] + p[i];
      } else if constexpr (SM == SMode::kBlockE8) {
#pragma unroll
        for (int i = 0; i < ROWS; i++) {
          const float t = p[i] * pow2i(d.e[i] - 127);
          acc[i] = acc[i] + ((cv && bt.rv[i]) ? t : 0.0f);
        }
      } else {
        float xsum = 0.0f;
        if constexpr (SM == SMode::kGroupAff) {
#pragma unroll
          for (int e = 0; e < 32; e++) xsum = xsum + xv<XT>(xw, e);
          xsum = cv ? xsum : 0.0f;
          reduce_range<1, 1, LG>(&xsum);
        }
        reduce_range<ROWS, 1, LG>(p);
#pragma unroll
        for (int k = 0; k < NVG; k++) {
          float t;
          const float sk = to_f32(d.s[k]);
          if constexpr (SM == SMode::kGroupAff) {
            float m = to_f32(d.m[k]);
            if (P.aff_zero) m = -(m * sk);
            t = __builtin_fmaf(xsum, m, p[k] * sk);
          } else {
            t = p[k] * sk;
          }
          // a group counts when its first chunk is in range (ragged last group)
          const bool ok = ((j & ~(LG - 1)) < nchunks) && (bt.lr0 + grow[k] < bt.rows);
          acc[k] = acc[k] + (ok ? t : 0.0f);
        }
      }
    }
  };

  // Row values of a finished batch: final lane reduction, then the epilogue.
  auto finish = [&](const Batch& bt, float (*accs)[ROWS]) {
#pragma unroll
    for (int m = 0; m < MR; m++) {
      float* acc = accs[m];
      if constexpr (kGroup) reduce_range<NVG, LG, LPR>(acc);
      else reduce_range<ROWS, 1, LPR>(acc);
      float v = acc[0];
      const bool ok = fstore && bt.lr0 + frow < bt.rows;
      if constexpr (SM == SMode::kRow) v = v * to_f32(bt.sb[(int64_t)(ok ? bt.lr0 + frow : 0) * bt.s_row]);
      if (!EPI || bt.kind == kSegPlain) {
        if (bt.bias != nullptr && ok) v = round_to<OT>(v) + to_f32(reinterpret_cast<const OT*>(bt.bias)[bt.lr0 + frow]);
        if (ok && bt.out != nullptr) store<OT>(reinterpret_cast<OT*>(bt.out) + (int64_t)(slot + m) * P.out_slot + bt.lr0 + frow, v);
      } else if constexpr (EPI) {
        // fused epilogues: the row value rounded to OT as the unfused operator would
        // store it, then RoPE / cache placement / SiLU on it
        bool odd = false;
        const int fr = bt.lr0 + frow;
        const int ph = bt.kind == kSegCache ? fr : paired_row<SUBS>(fr, bt.kind, P.f.head_dim, odd);
        if (bt.bias != nullptr && ok) v = round_to<OT>(v) + to_f32(reinterpret_cast<const OT*>(bt.bias)[ph]);
        const float val = round_to<OT>(v);
        const float pv = xor_partner<ROWS / 2 < 1 ? 1 : ROWS / 2>(val);   // the other half of the pair
        const int64_t pos = P.f.pos != nullptr ? (int64_t)P.f.pos[0] : 0;
        const int D = P.f.head_dim;
        if (bt.kind == kSegSilu) {
          if (ok && !odd) store<OT>(reinterpret_cast<OT*>(bt.out) + ph, silu_mul_val(val, pv));
        } else {
          float o = val;
          if (bt.kind != kSegCache && pos >= 0 && pos < P.f.table_rows) {
            const int half = D >> 1;
            const int j = (ph % D) - (odd ? half : 0);
            const float c = ld<OT>(P.f.cos, pos * P.f.table_row + j);
            const float sn = ld<OT>(P.f.sin, pos * P.f.table_row + j);
            float o1, o2;
            if (odd) rope_pair<OT>(pv, val, c, sn, o1, o2);
            else rope_pair<OT>(val, pv, c, sn, o1, o2);
            o = odd ? o2 : o1;
          }
          if (ok) {
            if (bt.kind == kSegRopeOut) {
              store<OT>(reinterpret_cast<OT*>(bt.out) + ph, o);
            } else if (pos >= 0 && pos < P.f.capacity) {
              const int64_t h = ph / D, d = ph - h * D;
              store<OT>(reinterpret_cast<OT*>(bt.out) + h * P.f.cache_head + pos * D + d, o);
            }
          }
        }
      }
      if constexpr (AM) {
        if (ok) {
          const uint64_t key = argmax_key(round_to<OT>(v), (uint32_t)(bt.lr0 + frow));
          best[m] = key > best[m] ? key : best[m];
        }
      }
    }
  };

  if constexpr (PF == 1) {
    while (cb.active) {
      Batch nb;
      nb.active = false;
      float acc[MR][ROWS];
#pragma unroll
      for (int m = 0; m < MR; m++)
#pragma unroll
        for (int i = 0; i < ROWS; i++) acc[m][i] = 0.0f;
      for (int r = 0; r < rounds; r++) {
        Data nd;
        if (r + 1 < rounds) {
          fetch(cb, r + 1, nd);
        } else {
          setup(b + nwaves, nb);
          if (nb.active) fetch(nb, 0, nd);
        }
        consume(cb, cd[0], r, acc);
        cd[0] = nd;
      }
      finish(cb, acc);
      cb = nb;
      b += nwaves;
    }
  } else {
    while (cb.active) {
      Batch nb;
      setup(b + nwaves, nb);
      Data nd[PF];
      if (nb.active) {
#pragma unroll
        for (int r = 0; r < PF; r++)
          if (r < rounds) fetch(nb, r, nd[r]);
      }
      float acc[MR][ROWS];
#pragma unroll
      for (int m = 0; m < MR; m++)
#pragma unroll
        for (int i = 0; i < ROWS; i++) acc[m][i] = 0.0f;
#pragma unroll
      for (int r = 0; r < PF; r++)
        if (r < rounds) consume(cb, cd[r], r, acc);
      finish(cb, acc);
      cb = nb;
#pragma unroll
      for (int r = 0; r < PF; r++) cd[r] = nd[r];
      b += nwaves;
    }
  }
  if constexpr (AM) {
#pragma unroll
    for (int m = 0; m < MR; m++) {
      const uint64_t bm = wave_max_u64(best[m]);
      if (lane == 0) P.am_partials[(int64_t)(blockIdx.x * (blockDim.x >> 6) + wave) * MR + m] = bm;
    }
  }
}

// ------------------------------------------------------------------ dispatch

// Workgroups of four waves; the grid is capped (waves loop over row batches) so that
// argmax partials fit kMaxGemvWaves keys.
constexpr int kMaxGemvBlocks = 2048;
constexpr int kMaxGemvWaves = 4 * kMaxGemvBlocks;

template <Fmt F, SMode SM, typename XT, typename OT, typename ST, int LPR, int ROWS, int L, Pro PRO = Pro::kLoad,
          bool EPI = false, int PF = 1, int MR = 1>
static int launch_one(GemvParams P, int slots, hipStream_t stream, const char* what) {
  constexpr int SUBS = 64 / LPR;
  constexpr int per_iter = ROWS * SUBS;
  int v = 0;
  for (int i = 0; i < P.nseg; i++) {
    P.seg[i].vbegin = v;
    v += (P.seg[i].rows + per_iter - 1) / per_iter * per_iter;
  }
  P.vtotal = v;
  const int batches = v / per_iter;
  int blocks = (batches + 3) / 4;
  if (blocks < 1) blocks = 1;
  if (blocks > kMaxGemvBlocks) blocks = kMaxGemvBlocks;
  const size_t lds = (size_t)P.cols * 2 * MR;
  if (P.am_partials == nullptr && slots == 1) {
    // Persistent grid of at most the workgroups the chip holds at once: waves loop
    // over row batches with the next batch in flight, instead of a second
    // generation of workgroups starting behind the first.
    static size_t cached_lds = ~(size_t)0;
    static int cached_cap = 0;
    if (cached_lds != lds) {
      int per_cu = 0, dev = 0, cus = 0;
      if (hipGetDevice(&dev) == hipSuccess &&
          hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
          hipOccupancyMaxActiveBlocksPerMultiprocessor(
              &per_cu, reinterpret_cast<const void*>(&gemv_kernel<F, SM, XT, OT, ST, LPR, ROWS, L, false, PRO, EPI, PF, MR>),
              256, lds) == hipSuccess &&
          per_cu > 0 && cus > 0) {
        cached_cap = per_cu * cus;
      } else {
        cached_cap = kMaxGemvBlocks;
      }
      cached_lds = lds;
    }
    if (blocks > cached_cap) blocks = cached_cap;
  }
  if (P.am_partials != nullptr) {
    if constexpr (SM == SMode::kNone) {
      // unused partial slots must not win the final reduction
      hipLaunchKernelGGL((gemv_kernel<F, SM, XT, OT, ST, LPR, ROWS, L, true, PRO, EPI, PF, MR>), dim3(blocks, slots),
                         dim3(256), lds, stream, P);
      return check_launch(what);
    }
    set_error("%s: argmax epilogue is only available for dense weights", what);
    return TT_ERR_UNSUPPORTED;
  }
  hipLaunchKernelGGL((gemv_kernel<F, SM, XT, OT, ST, LPR, ROWS, L, false, PRO, EPI, PF, MR>), dim3(blocks, slots),
                     dim3(256), lds, stream, P);
  return check_launch(what);
}

template <Fmt F, SMode SM, typename XT, typename OT, typename ST, int ROWS, int L, Pro PRO = Pro::kLoad, bool EPI = false,
          int PF = 1, int MR = 1>
static int launch_lpr(int lpr, const GemvParams& P, int slots, hipStream_t stream, const char* what) {
  switch (lpr) {
    case 64: return launch_one<F, SM, XT, OT, ST, 64, ROWS, L, PRO, EPI, PF, MR>(P, slots, stream, what);
    case 32:
      if constexpr (L <= 32) return launch_one<F, SM, XT, OT, ST, 32, ROWS, L, PRO, EPI, PF, MR>(P, slots, stream, what);
      break;
    case 16:
      if constexpr (L <= 16) return launch_one<F, SM, XT, OT, ST, 16, ROWS, L, PRO, EPI, PF, MR>(P, slots, stream, what);
      break;
    default: break;
  }
  set_error("%s: invalid lanes per row %d for a %d-chunk group", what, lpr, L);
  return TT_ERR_INVALID;
}

template <Fmt F, SMode SM, typename XT, typename OT, typename ST, int ROWS>
static int launch_group(int L, int lpr, const GemvParams& P, int slots, hipStream_t stream, const char* what) {
  switch (L) {
    case 1: return launch_lpr<F, SM, XT, OT, ST, ROWS, 1>(lpr, P, slots, stream, what);
    case 2: return launch_lpr<F, SM, XT, OT, ST, ROWS, 2>(lpr, P, slots, stream, what);
    case 4: return launch_lpr<F, SM, XT, OT, ST, ROWS, 4>(lpr, P, slots, stream, what);
    case 8: return launch_lpr<F, SM, XT, OT, ST, ROWS, 8>(lpr, P, slots, stream, what);
    case 16: return launch_lpr<F, SM, XT, OT, ST, ROWS, 16>(lpr, P, slots, stream, what);
    case 32: return launch_lpr<F, SM, XT, OT, ST, ROWS, 32>(lpr, P, slots, stream, what);
    case 64: return launch_lpr<F, SM, XT, OT, ST, ROWS, 64>(lpr, P, slots, stream, what);
  }
  set_error("%s: unsupported group of %d chunks", what, L);
  return TT_ERR_UNSUPPORTED;
}

template <Fmt F, SMode SM, typename ST, int ROWS>
static int launch_types(int x_dtype, int out_dtype, int L, int lpr, const GemvParams& P, int slots, hipStream_t stream,
                        const char* what) {
  constexpr bool kGroup = SM == SMode::kGroup || SM == SMode::kGroupAff;
  auto go = [&](auto xt, auto ot) -> int {
    using XT = decltype(xt);
    using OT = decltype(ot);
    if constexpr (kGroup) return launch_group<F, SM, XT, OT, ST, ROWS>(L, lpr, P, slots, stream, what);
    else return launch_lpr<F, SM, XT, OT, ST, ROWS, 1>(lpr, P, slots, stream, what);
  };
  if (x_dtype == TT_F16) {
    if (out_dtype == TT_F16) return go(f16_t{}, f16_t{});
    if (out_dtype == TT_F32) return go(f16_t{}, float{});
  } else if (x_dtype == TT_BF16) {
    if (out_dtype == TT_BF16) return go(bf16_t{}, bf16_t{});
    if (out_dtype == TT_F32) return go(bf16_t{}, float{});
  }
  set_error("%s: unsupported activation/output dtype pair (%d, %d); output must match the activation dtype or be fp32",
            what, x_dtype, out_dtype);
  return TT_ERR_UNSUPPORTED;
}

// Launch shape of the symmetric int4 group-128 GEMV (the decode hot path): rows per
// wave and rounds prefetched per batch.  Fewer rows per wave when the matrix is short,
// so that the grid still fills the chip; whole-batch prefetch when a row takes 2 to 4
// rounds, so a wave waits for memory once per batch instead of once per round.
// Paired (RoPE / SiLU) segments need at least two rows per wave.  The reduction order
// does not depend on either choice.
inline void int4_shape(int64_t rows, int rounds, bool paired, int* rows_per_wave, int* prefetch) {
  int rpw = rows >= 16384 ? 4 : (rows >= 4096 || paired ? 2 : 1);
  if (paired && rpw < 2) rpw = 2;
  int pf = rounds >= 2 && rounds <= 4 && rpw <= 2 ? 4 : 1;
  *rows_per_wave = rpw;
  *prefetch = pf;
}

template <typename XT, typename OT, Pro PRO, bool EPI>
static int launch_int4_g128(int lpr, int rows_per_wave, int prefetch, const GemvParams& P, hipStream_t st,
                            const char* what) {
  constexpr Fmt F = Fmt::kInt4Sym;
  constexpr SMode SM = SMode::kGroup;
  // whole-batch prefetch holds every round of a batch in registers
  TT_REQUIRE(prefetch == 1 || (P.cols / 32 + lpr - 1) / lpr <= prefetch, "%s: prefetch %d below the rounds per row",
             what, prefetch);
  if (rows_per_wave == 4) return launch_lpr<F, SM, XT, OT, f16_t, 4, 4, PRO, EPI, 1>(lpr, P, 1, st, what);
  if (rows_per_wave == 2) {
    if (prefetch == 4) return launch_lpr<F, SM, XT, OT, f16_t, 2, 4, PRO, EPI, 4>(lpr, P, 1, st, what);
    return launch_lpr<F, SM, XT, OT, f16_t, 2, 4, PRO, EPI, 1>(lpr, P, 1, st, what);
  }
  if constexpr (!EPI) {
    if (prefetch == 4) return launch_lpr<F, SM, XT, OT, f16_t, 1, 4, PRO, EPI, 4>(lpr, P, 1, st, what);
    return launch_lpr<F, SM, XT, OT, f16_t, 1, 4, PRO, EPI, 1>(lpr, P, 1, st, what);
  }
  set_error("%s: paired segments need two rows per wave", what);
  return TT_ERR_INVALID;
}

// Validates the common GEMV contract and fills group information.
inline int plan_groups(const char* what, int64_t cols, int64_t group_size, int* L, bool* row_mode) {
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


}  // namespace tt
