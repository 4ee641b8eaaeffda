// Sigmoid top-k expert selection of one token by one wave, shared by the
// router kernel, the fused router + gate/up decode kernel and the fused
// router + schedule kernel of the expert-major block
// (engine/klinear/router.py:47-85).
#pragma once

#include "lk_common.hpp"

namespace lk {

// ---------------------------------------------------------------------------
// sigmoid top-k router for one token, computed by one wave (all lanes).
// EPL experts per lane (lane l holds ids l*EPL .. l*EPL+EPL-1).
// Returns the expert id of selection `want` (-1 if want >= top_k). When
// idx_out is non-null, lanes < top_k write the selection and its weight;
// when sel_out is non-null (LDS), they also write the selection there.
//
// Each lane first sorts its EPL candidates by key (descending; equal keys keep
// the lower id first), so a selection round only compares the lanes' head
// entries: one wave max, one ballot (the lowest lane holding the max holds the
// lowest id, since ids grow with the lane) and the owner lane advancing its
// head. The rounds are a short dependent chain, which is what bounds a router
// that runs on one wave.

// The lane's EPL logits (addresses clamped in bounds; ids past the bank are
// masked by the selection).
template <int EPL>
__device__ inline void route_load(const float* __restrict__ v, int ne, float (&out)[EPL]) {
  const int lane = threadIdx.x & (kWave - 1);
#pragma unroll
  for (int j = 0; j < EPL; ++j) out[j] = v[min(lane * EPL + j, ne - 1)];
}

template <int EPL>
__device__ inline int64_t route_select_rounds(const float (&lg)[EPL], const float (&bs)[EPL],
                                              int ne, int top_k, int want, float scaling,
                                              int renorm, int64_t* __restrict__ idx_out,
                                              float* __restrict__ w_out, int32_t* sel_out) {
  const int lane = threadIdx.x & (kWave - 1);
  uint32_t key[EPL];
  float sc[EPL];
  int slot[EPL];
#pragma unroll
  for (int j = 0; j < EPL; ++j) {
    sc[j] = 1.0f / (1.0f + expf(-lg[j]));
    // ids past the bank sit behind every real expert: key 0 and the highest
    // slots; live keys are at least 1 (orderable() gives 0 only for one NaN
    // bit pattern, which then ties with the key above it)
    key[j] = lane * EPL + j < ne ? max(orderable(sc[j] + bs[j]), 1u) : 0u;
    slot[j] = j;
  }
#pragma unroll
  for (int a = 0; a < EPL; ++a)
#pragma unroll
    for (int b = EPL - 1; b > a; --b) {
      const bool sw = key[b] > key[b - 1];  // strict, so equal keys stay in id order
      const uint32_t k0 = key[b - 1], k1 = key[b];
      const float s0 = sc[b - 1], s1 = sc[b];
      const int q0 = slot[b - 1], q1 = slot[b];
      key[b - 1] = sw ? k1 : k0;
      key[b] = sw ? k0 : k1;
      sc[b - 1] = sw ? s1 : s0;
      sc[b] = sw ? s0 : s1;
      slot[b - 1] = sw ? q1 : q0;
      slot[b] = sw ? q0 : q1;
    }
  // Selection rounds. A lane's head is entry 0; the owner of a round shifts
  // its entries down and fills key 0 behind them. Live keys are at least 1
  // (set above), so a lane whose entries are used up, or that holds only ids
  // past the bank, never matches the round's maximum while a live candidate
  // is left (top_k <= ne). The shift is branch-free: one v_cndmask per entry.
  float ssum = 0.f;
  int64_t mine = -1;
  float my_score = 0.f;
  int64_t wanted = -1;
  // a caller that writes no outputs needs only the rounds up to `want`
  const bool outputs = idx_out != nullptr || sel_out != nullptr;
  const int rounds = outputs ? top_k : min(top_k, max(want + 1, 0));
  for (int rr = 0; rr < rounds; ++rr) {
    const uint32_t kb = key[0];
    const uint32_t kmax = wave_max_u32(kb);
    const uint64_t holders = __builtin_amdgcn_ballot_w64(kb == kmax);
    const int owner = static_cast<int>(__builtin_ctzll(holders | (1ull << 63)));
    const int q = __builtin_amdgcn_readlane(slot[0], owner);
    const float score = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(sc[0]), owner));
    const uint32_t sel = static_cast<uint32_t>(owner * EPL + q);
    // top_k <= ne guarantees a live candidate; stay in range regardless
    const uint32_t safe = sel < static_cast<uint32_t>(ne) ? sel : 0u;
    const bool own = lane == owner;
#pragma unroll
    for (int j = 0; j + 1 < EPL; ++j) {
      key[j] = own ? key[j + 1] : key[j];
      sc[j] = own ? sc[j + 1] : sc[j];
      slot[j] = own ? slot[j + 1] : slot[j];
    }
    key[EPL - 1] = own ? 0u : key[EPL - 1];
    ssum += score;
    mine = lane == rr ? static_cast<int64_t>(safe) : mine;
    my_score = lane == rr ? score : my_score;
    wanted = rr == want ? static_cast<int64_t>(safe) : wanted;
  }
  if (idx_out != nullptr && lane < top_k) {
    const float denom = ssum + 1e-20f;
    idx_out[lane] = mine;
    w_out[lane] = (renorm && top_k > 1) ? (my_score / denom) * scaling : my_score * scaling;
  }
  if (sel_out != nullptr && lane < top_k) sel_out[lane] = static_cast<int32_t>(mine);
  return wanted;
}

// ---------------------------------------------------------------------------
// Top-k (k <= 8) of up to 256 experts by merging sorted lists across the wave.
//
// The rounds above are a dependent chain of wave-wide max, ballot and readlane
// steps per selected expert. Here every lane builds a 32-bit merge key per
// expert: the choice key's high 24 bits and (255 - id) in the low 8, so that
// key order is choice order with ties to the lower id. A lane sorts its 4 merge
// keys, then six butterfly levels (partners at lane distance 1, 2, 4 and 8 by
// DPP, 16 and 32 by the permlane swaps) each keep the top 8 of the two lanes' sorted
// lists: the element-wise max of one list against the other reversed is a
// bitonic sequence holding the top 8 of the union, which a 12-exchange bitonic
// network sorts. After the last level every lane holds the wave's top 8.
//
// Dropping the choice key's low 8 bits makes the result exact only when no
// expert outside the selection shares the high 24 bits of the last selected
// one and no two selected experts share theirs: a ballot count checks both,
// and the rare token that fails (about 1 in 200 at N(0, 1) logits) takes the
// exact rounds. Scores, weights and their summation order are the rounds'.

__device__ inline void cmp_swap_desc(uint32_t& a, uint32_t& b) {
  const uint32_t hi = max(a, b), lo = min(a, b);
  a = hi;
  b = lo;
}

// A bitonic sequence of 8 -> descending order.
__device__ inline void bitonic_sort8(uint32_t (&v)[8]) {
  cmp_swap_desc(v[0], v[4]);
  cmp_swap_desc(v[1], v[5]);
  cmp_swap_desc(v[2], v[6]);
  cmp_swap_desc(v[3], v[7]);
  cmp_swap_desc(v[0], v[2]);
  cmp_swap_desc(v[1], v[3]);
  cmp_swap_desc(v[4], v[6]);
  cmp_swap_desc(v[5], v[7]);
  cmp_swap_desc(v[0], v[1]);
  cmp_swap_desc(v[2], v[3]);
  cmp_swap_desc(v[4], v[5]);
  cmp_swap_desc(v[6], v[7]);
}

// Keep the top 8 of this lane's sorted list and the partner's (both descending).
__device__ inline void merge_top8(uint32_t (&v)[8], const uint32_t (&p)[8]) {
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = max(v[i], p[7 - i]);
  bitonic_sort8(v);
}

template <int CTRL>
__device__ inline void merge_dpp(uint32_t (&v)[8]) {
  uint32_t p[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) p[i] = dpp_u32<CTRL>(v[i]);
  merge_top8(v, p);
}

// Partner lists at lane distance 16 and 32 come from the gfx950 permlane
// swaps (no LDS crossbar: a ds_bpermute between the two halves of the wave
// measured about 900 cycles per register here). Swapping a register with
// itself leaves the partner's value in the second result for even 16-lane
// rows (lower half) and in the first result for odd rows (upper half).
__device__ inline void merge_swap16(uint32_t (&v)[8]) {
  const bool odd = (threadIdx.x & 16) != 0;
  uint32_t p[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const auto r = __builtin_amdgcn_permlane16_swap(v[i], v[i], false, false);
    p[i] = odd ? r[0] : r[1];
  }
  merge_top8(v, p);
}

__device__ inline void merge_swap32(uint32_t (&v)[8]) {
  const bool upper = (threadIdx.x & 32) != 0;
  uint32_t p[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const auto r = __builtin_amdgcn_permlane32_swap(v[i], v[i], false, false);
    p[i] = upper ? r[0] : r[1];
  }
  merge_top8(v, p);
}

// The rounds' outputs from a selection held (identically) by every lane:
// merge keys `list` in selection order. Returns the id of selection `want`.
__device__ inline int64_t route_emit_merged(const uint32_t (&list)[8], const float (&sc)[4],
                                            int top_k, int want, float scaling, int renorm,
                                            int64_t* __restrict__ idx_out,
                                            float* __restrict__ w_out, int32_t* sel_out) {
  const int lane = threadIdx.x & (kWave - 1);
  int ids[8];
#pragma unroll
  for (int i = 0; i < 8; ++i)
    ids[i] = 255 - static_cast<int>(__builtin_amdgcn_readfirstlane(list[i]) & 0xFFu);
  int64_t wanted = -1;
#pragma unroll
  for (int i = 0; i < 8; ++i)
    if (i == want) wanted = ids[i];
  if (idx_out == nullptr && sel_out == nullptr) return wanted;
  // each selected score from the lane holding it (id / 4, slot id % 4), read
  // into a scalar; summed in selection order, as the rounds accumulate them
  float score[8];
  float ssum = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int slot = ids[i] & 3;
    const float pick = slot == 0 ? sc[0] : slot == 1 ? sc[1] : slot == 2 ? sc[2] : sc[3];
    score[i] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pick), ids[i] >> 2));
    if (i < top_k) ssum += score[i];
  }
  int id = ids[0];
  float mine = score[0];
#pragma unroll
  for (int i = 1; i < 8; ++i) {
    id = lane == i ? ids[i] : id;
    mine = lane == i ? score[i] : mine;
  }
  if (idx_out != nullptr && lane < top_k) {
    const float denom = ssum + 1e-20f;
    idx_out[lane] = id;
    w_out[lane] = (renorm && top_k > 1) ? (mine / denom) * scaling : mine * scaling;
  }
  if (sel_out != nullptr && lane < top_k) sel_out[lane] = id;
  return wanted;
}

template <int EPL>
__device__ inline int64_t route_select(const float (&lg)[EPL], const float (&bs)[EPL], int ne,
                                       int top_k, int want, float scaling, int renorm,
                                       int64_t* __restrict__ idx_out, float* __restrict__ w_out,
                                       int32_t* sel_out) {
  if constexpr (EPL == 4) {
    if (top_k <= 8 && ne <= 256) {  // wave-uniform
      const int lane = threadIdx.x & (kWave - 1);
      float sc[4];
      uint32_t key[4], v[8];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int id = lane * 4 + j;
        sc[j] = 1.0f / (1.0f + expf(-lg[j]));
        // the rounds' choice key (live keys >= 1, ids past the bank 0)
        key[j] = id < ne ? max(orderable(sc[j] + bs[j]), 1u) : 0u;
        v[j] = id < ne ? (key[j] & 0xFFFFFF00u) | static_cast<uint32_t>(255 - id) : 0u;
      }
      cmp_swap_desc(v[0], v[1]);
      cmp_swap_desc(v[2], v[3]);
      cmp_swap_desc(v[0], v[2]);
      cmp_swap_desc(v[1], v[3]);
      cmp_swap_desc(v[1], v[2]);
      {  // lane pairs: the union of two sorted 4-lists, as a bitonic 8
        uint32_t p[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) p[i] = dpp_u32<kQuadXor1>(v[i]);
#pragma unroll
        for (int i = 0; i < 4; ++i) v[4 + i] = p[3 - i];
        bitonic_sort8(v);
      }
      merge_dpp<kQuadXor2>(v);
      merge_dpp<kRowHalfMirror>(v);
      merge_dpp<kRowMirror>(v);
      merge_swap16(v);
      merge_swap32(v);
      // exact iff no other expert shares the high 24 bits of the last
      // selected one, and the selected ones have distinct high 24 bits
      uint32_t last = v[0];
#pragma unroll
      for (int i = 1; i < 8; ++i) last = i == top_k - 1 ? v[i] : last;
      const uint32_t thr = last & 0xFFFFFF00u;
      int at_or_above = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j)
        at_or_above += __builtin_popcountll(__builtin_amdgcn_ballot_w64(key[j] >= thr));
      bool distinct = true;
#pragma unroll
      for (int i = 0; i + 1 < 8; ++i)
        distinct = distinct && (i + 1 >= top_k || (v[i] >> 8) != (v[i + 1] >> 8));
      if (at_or_above == top_k && distinct)  // wave-uniform
        return route_emit_merged(v, sc, top_k, want, scaling, renorm, idx_out, w_out, sel_out);
    }
  }
  return route_select_rounds<EPL>(lg, bs, ne, top_k, want, scaling, renorm, idx_out, w_out,
                                  sel_out);
}

// The lane's logits and biases (zeros without a bias), every load issued
// before any is used.
template <int EPL>
__device__ inline void route_load_all(const float* __restrict__ logits,
                                      const float* __restrict__ bias, int ne, float (&lg)[EPL],
                                      float (&bs)[EPL]) {
  route_load<EPL>(logits, ne, lg);
  if (bias) {
    route_load<EPL>(bias, ne, bs);
  } else {
#pragma unroll
    for (int j = 0; j < EPL; ++j) bs[j] = 0.0f;
  }
}

template <int EPL>
__device__ inline int64_t route_token(const float* __restrict__ logits,
                                      const float* __restrict__ bias, int ne, int top_k, int want,
                                      float scaling, int renorm, int64_t* __restrict__ idx_out,
                                      float* __restrict__ w_out, int32_t* sel_out = nullptr) {
  float lg[EPL], bs[EPL];
  route_load_all<EPL>(logits, bias, ne, lg, bs);  // all loads first
  return route_select<EPL>(lg, bs, ne, top_k, want, scaling, renorm, idx_out, w_out, sel_out);
}

}  // namespace lk
