// Wave-level MoE top-k + softmax over router logits (the selection and scores of
// triton_kernels.py:2821-2851 / 2889-2919), in registers so that any wave of any kernel
// can run it: the router's finishing wave writes the result out, and the expert kernels
// of the decode step derive their own slot's expert from the logits with the same code.
#pragma once

#include "tt_common.h"

namespace tt {

// Ordered key of a router logit: larger value wins, equal values (+0 == -0) go to
// the lowest expert index.  NaN never wins through the key (see wave_topk_lanes).
__device__ __forceinline__ uint64_t topk_key(float v, uint32_t e) {
  uint32_t b = __builtin_bit_cast(uint32_t, v);
  if ((b & 0x7fffffffu) == 0) b = 0;
  const uint32_t o = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  return ((uint64_t)o << 32) | (uint64_t)(0xffffffffu - e);
}

__device__ __forceinline__ float lane_value(float a, float b, int i) {
  return i < 64 ? __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, a), i))
                : __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, b), i - 64));
}

// Slot s's expert and score sit in lane s % 64 of idx0 / score0 (s < 64) or idx1 /
// score1 (s >= 64).
struct TopkLanes {
  int idx0, idx1;
  float score0, score1;
};

// Top-k + softmax over E <= 128 logits held by one wave (expert e in lane e % 64,
// register e / 64).  Same result as scanning the experts in order for each slot:
// the first untaken expert starts the scan and a later one replaces it only when
// strictly greater -- so a NaN at the first untaken position is selected, any other
// NaN never is, and equal values keep the lowest index.  The denominator is summed
// sequentially in slot order (renormalize) or expert order, each term
// exp(v - max) with max the NaN-ignoring maximum over all experts.  Uses no LDS.
__device__ __forceinline__ TopkLanes wave_topk_lanes(float lg0, float lg1, int E, int top_k, bool renorm) {
  const int lane = lane_id();
  const bool v0 = lane < E, v1 = lane + 64 < E;
  float m = __builtin_bit_cast(float, 0xff800000u);
  if (v0) m = fmaxf(m, lg0);
  if (v1) m = fmaxf(m, lg1);
  m = fmaxf(m, xor_partner<1>(m));
  m = fmaxf(m, xor_partner<2>(m));
  m = fmaxf(m, xor_partner<4>(m));
  m = fmaxf(m, xor_partner<8>(m));
  m = fmaxf(m, xor_partner<16>(m));
  m = fmaxf(m, xor_partner<32>(m));
  float sel0 = 0.0f, sel1 = 0.0f;
  int id0 = 0, id1 = 0;
  const bool any_nan = __builtin_amdgcn_ballot_w64((v0 && __builtin_isnan(lg0)) || (v1 && __builtin_isnan(lg1))) != 0;
  if (E <= 64 && !any_nan && top_k <= 8) {
    // Without NaNs the keys (value, then lowest index) are distinct and slot s holds the
    // s-th largest: top_k wave maxima of the keys' value halves, each followed by a ballot
    // for the lowest lane holding it (taken and invalid lanes hold 0, below every valid
    // value half), as in wave_topk_expert.
    uint32_t mk = v0 ? (uint32_t)(topk_key(lg0, lane) >> 32) : 0u;
    auto umax = [](uint32_t a, float b) { const uint32_t u = __builtin_bit_cast(uint32_t, b); return u > a ? u : a; };
    for (int s = 0; s < top_k; s++) {
      uint32_t m = mk;
      m = umax(m, xor_partner<1>(__builtin_bit_cast(float, m)));
      m = umax(m, xor_partner<2>(__builtin_bit_cast(float, m)));
      m = umax(m, xor_partner<4>(__builtin_bit_cast(float, m)));
      m = umax(m, xor_partner<8>(__builtin_bit_cast(float, m)));
      m = umax(m, xor_partner<16>(__builtin_bit_cast(float, m)));
      m = umax(m, xor_partner<32>(__builtin_bit_cast(float, m)));
      const uint64_t hit = __builtin_amdgcn_ballot_w64(mk == m);
      const int e = (int)__builtin_ctzll(hit);
      const float val = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, lg0), e));
      if (lane == s) {
        sel0 = val;
        id0 = e;
      }
      if (lane == e) mk = 0u;
    }
  } else if (E <= 64 && !any_nan) {
    // Larger top_k: slot s is the expert with exactly s greater keys; every lane counts
    // the keys above its own, independently of the others, and slot s finds its lane by
    // a ballot.
    const uint64_t mine = topk_key(lg0, lane);
    int rank = 0;
    for (int f = 0; f < E; f++) {
      const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)mine, f);
      const uint32_t hi = __builtin_amdgcn_readlane((uint32_t)(mine >> 32), f);
      rank += (((uint64_t)hi << 32) | lo) > mine ? 1 : 0;
    }
    for (int s = 0; s < top_k; s++) {
      const uint64_t hit = __builtin_amdgcn_ballot_w64(v0 && rank == s);
      const int e = hit ? (int)__builtin_ctzll(hit) : 0;
      const float val = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, lg0), e));
      if (lane == s) {
        sel0 = val;
        id0 = e;
      }
    }
  } else {
    bool t0 = !v0, t1 = !v1;
    for (int s = 0; s < top_k; s++) {
      uint64_t k = 0, f = 0;
      if (!t0) {
        f = 0xffffffffu - (uint32_t)lane;
        if (!__builtin_isnan(lg0)) k = topk_key(lg0, lane);
      }
      if (!t1) {
        if (f == 0) f = 0xffffffffu - (uint32_t)(lane + 64);
        if (!__builtin_isnan(lg1)) {
          const uint64_t k1 = topk_key(lg1, lane + 64);
          k = k1 > k ? k1 : k;
        }
      }
      k = wave_max_u64(k);
      f = wave_max_u64(f);
      const int first = __builtin_amdgcn_readfirstlane((int)(0xffffffffu - (uint32_t)f));
      const float fv = lane_value(lg0, lg1, first);
      int bi = first;
      if (!__builtin_isnan(fv)) bi = __builtin_amdgcn_readfirstlane((int)(0xffffffffu - (uint32_t)k));
      const float bv = lane_value(lg0, lg1, bi);
      if (lane == bi) t0 = true;
      if (lane + 64 == bi) t1 = true;
      if (lane == (s & 63)) {
        if (s < 64) {
          sel0 = bv;
          id0 = bi;
        } else {
          sel1 = bv;
          id1 = bi;
        }
      }
    }
  }
  const float e0 = exp_f32(sel0 - m), e1 = exp_f32(sel1 - m);
  float den = 0.0f;
  if (renorm) {
    for (int s = 0; s < top_k; s++) den = den + lane_value(e0, e1, s);
  } else {
    const float a0 = exp_f32(lg0 - m), a1 = exp_f32(lg1 - m);
    for (int e = 0; e < E; e++) den = den + lane_value(a0, a1, e);
  }
  return TopkLanes{id0, id1, e0 / den, e1 / den};
}

// Expert of slot k of wave_topk_lanes's selection (the same rule, so the same expert),
// without the softmax.  With no NaN logit and E <= 64 the keys (value, then lowest index)
// are distinct and slot s holds the s-th largest, so k + 1 wave maxima over the untaken
// keys find it: the maximum of the keys' value halves, then the lowest lane holding it (a
// taken or invalid lane holds 0, below every valid value half: -inf orders as 0x007fffff).  Each SwiGLU wave calls
// this before its first weight request: a rank pass over all E keys cost the gpt-oss
// bs=1 decode ~4% (720 against 750 tok/s with the pass skipped in a timing copy).
// Otherwise the iterated scan of wave_topk_lanes, stopped at slot k.
__device__ __forceinline__ int wave_topk_expert(float lg0, float lg1, int E, int k) {
  const int lane = lane_id();
  const bool v0 = lane < E, v1 = lane + 64 < E;
  const bool any_nan = __builtin_amdgcn_ballot_w64((v0 && __builtin_isnan(lg0)) || (v1 && __builtin_isnan(lg1))) != 0;
  if (E <= 64 && !any_nan) {
    // the value half of the key (32-bit maxima), then the lowest index holding it
    uint32_t mine = v0 ? (uint32_t)(topk_key(lg0, lane) >> 32) : 0u;
    int e = 0;
    for (int s = 0; s <= k; s++) {
      uint32_t m = mine;
      auto umax = [](uint32_t a, float b) { const uint32_t u = __builtin_bit_cast(uint32_t, b); return u > a ? u : a; };
      m = umax(m, xor_partner<1>(__builtin_bit_cast(float, m)));
      m = umax(m, xor_partner<2>(__builtin_bit_cast(float, m)));
      m = umax(m, xor_partner<4>(__builtin_bit_cast(float, m)));
      m = umax(m, xor_partner<8>(__builtin_bit_cast(float, m)));
      m = umax(m, xor_partner<16>(__builtin_bit_cast(float, m)));
      m = umax(m, xor_partner<32>(__builtin_bit_cast(float, m)));
      const uint64_t hit = __builtin_amdgcn_ballot_w64(mine == m);
      e = (int)__builtin_ctzll(hit);
      if (lane == e) mine = 0u;
    }
    return e;
  }
  bool t0 = !v0, t1 = !v1;
  int bi = 0;
  for (int s = 0; s <= k; s++) {
    uint64_t key = 0, f = 0;
    if (!t0) {
      f = 0xffffffffu - (uint32_t)lane;
      if (!__builtin_isnan(lg0)) key = topk_key(lg0, lane);
    }
    if (!t1) {
      if (f == 0) f = 0xffffffffu - (uint32_t)(lane + 64);
      if (!__builtin_isnan(lg1)) {
        const uint64_t k1 = topk_key(lg1, lane + 64);
        key = k1 > key ? k1 : key;
      }
    }
    key = wave_max_u64(key);
    f = wave_max_u64(f);
    const int first = __builtin_amdgcn_readfirstlane((int)(0xffffffffu - (uint32_t)f));
    const float fv = lane_value(lg0, lg1, first);
    bi = first;
    if (!__builtin_isnan(fv)) bi = __builtin_amdgcn_readfirstlane((int)(0xffffffffu - (uint32_t)key));
    if (lane == bi) t0 = true;
    if (lane + 64 == bi) t1 = true;
  }
  return bi;
}

}  // namespace tt
