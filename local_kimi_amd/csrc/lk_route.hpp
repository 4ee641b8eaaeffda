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
__device__ inline int64_t route_select(const float (&lg)[EPL], const float (&bs)[EPL], int ne,
                                       int top_k, int want, float scaling, int renorm,
                                       int64_t* __restrict__ idx_out, float* __restrict__ w_out,
                                       int32_t* sel_out) {
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
