// Shared device/host helpers for the gfx950 W4A16 / MXFP4 kernels.
//
// bf16 is carried as uint16_t storage; all conversions are explicit so every
// rounding point matches the reference's torch semantics (round to nearest,
// ties to even).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "lk_w4a16.h"

namespace lk {

constexpr int kWave = 64;  // lanes per wavefront on CDNA

// ---------------------------------------------------------------------------
// error state (per host thread)

void set_error(const char* fmt, ...);
int fail_arg(const char* fmt, ...);
int check_launch(const char* what);

// Kernel-form selection of this process (lk_set_path). Every knob is 0
// ("auto") unless a caller forces a form; the library reads no environment.
enum Knob : int {
  kKnobMoeGemm = 0,       // 0 auto, 1 lds, 2 stream16, 3 stream64
  kKnobMoePersist,        // 0 auto, 1 off
  kKnobDenseGemm,         // 0 auto, 1 lds
  kKnobMxfp4Mfma,         // 0 auto, 1 fp4, 2 bf16
  kKnobMoeFusedSchedule,  // 0 auto, 1 off
  kKnobMoeSplitSwiglu,    // 0 auto, 1 off
  kKnobCount
};
int path_choice(Knob knob);

// Whether the token-major W2 + combine launch (w2_combine_rows) takes this
// shape: LK_OK, or LK_ERR_ARGUMENT with the reason set as the last error.
int w2_rows_check(int64_t routes, int64_t h, int64_t inter);
bool w2_rows_fits(int64_t routes, int64_t inter);

// W2 for every (token, route) row of `act` [tokens, routes, inter] plus the
// route-weighted combine and the shared expert (the last route; bank entry
// shared_id when shared_id >= 0), one launch: the token-major W2 kernels of
// the decode path (w4a16_gemv.hip).
int w2_combine_rows(const uint16_t* act, const int64_t* idx, int64_t idx_stride,
                    int64_t shared_id, const float* cw, int64_t cw_stride, const uint8_t* w2p,
                    const uint16_t* w2s, uint16_t* y, int64_t tokens, int64_t routes,
                    int64_t experts, int64_t h, int64_t inter, int64_t group, hipStream_t s);
// Up to three W4A16 matrices of one shape [n, k] and their outputs [m, n].
struct DenseMats {
  const uint8_t* packed[3];
  const uint16_t* scales[3];
  uint16_t* y[3];
};

// y_z = x . W_z^T for z < count in one launch of the decode K-split GEMV
// (w4a16_gemv.hip); the group size must already be checked.
int dense_multi(const uint16_t* x, const DenseMats& mats, int count, int64_t m, int64_t n,
                int64_t k, int64_t group_size, hipStream_t s, const char* name);

// LK_OK when k > 0 and group is a positive multiple of 32 that divides k.
int check_group(int64_t k, int64_t group);
// check_group, and group is a power of two.
int check_pow2_group(int64_t k, int64_t group);

#define LK_REQUIRE(cond, ...)          \
  do {                                 \
    if (!(cond)) {                     \
      return ::lk::fail_arg(__VA_ARGS__); \
    }                                  \
  } while (0)

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// ---------------------------------------------------------------------------
// bf16 helpers

__host__ __device__ inline float bf16_to_f32(uint16_t b) {
  return __builtin_bit_cast(float, static_cast<uint32_t>(b) << 16);
}

__host__ __device__ inline uint16_t f32_to_bf16(float f) {
  uint32_t u = __builtin_bit_cast(uint32_t, f);
  if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x007FFFFFu)) return 0x7FC0;  // NaN
  u += 0x7FFFu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

__device__ inline float round_bf16(float f) { return bf16_to_f32(f32_to_bf16(f)); }

// torch's F.silu on a bf16 tensor: fp32 x / (1 + exp(-x)), rounded to bf16.
__device__ inline float silu_f32(float x) { return x / (1.0f + expf(-x)); }

// silu for the fast kernels: x * 1 / (1 + 2^(-x log2 e)) on the hardware
// exp2 and reciprocal (about 1 ulp each, against the ~25 instructions of
// expf and an IEEE divide); the result is rounded to bf16 next, so it differs
// from silu_f32 by at most one bf16 ulp, in rare near-tie cases. Limits
// match: x -> +inf gives x, x -> -inf gives -0 (NaN at -inf, as x / inf).
__device__ inline float silu_fast_f32(float x) {
  const float e = __builtin_amdgcn_exp2f(x * -1.4426950408889634f);
  return x * __builtin_amdgcn_rcpf(1.0f + e);
}

// SwiGLU contract of the reference: bf16(bf16(silu(bf16(gate))) * bf16(up)).
__device__ inline uint16_t swiglu_bf16(float gate_acc, float up_acc) {
  const float g = round_bf16(gate_acc);
  const float u = round_bf16(up_acc);
  const float s = round_bf16(silu_fast_f32(g));
  return f32_to_bf16(s * u);
}

// ---------------------------------------------------------------------------
// int4 -> bf16 pair unpack.
//
// A dword of packed weights holds 8 consecutive reduction positions
// k0..k7 (k_p in bits [4p, 4p+4)). XOR with 0x8 maps the two's complement
// code q in [-8, 7] to u = q + 8 in [0, 15]; OR-ing u into the mantissa of
// bf16 128.0 (0x4300) gives the exact bf16 value 128 + u = q + 136. One
// v_and_or_b32 builds two such values, pairing (k_p, k_{p+4}) in (lo, hi).
// The activation operand is staged in the same (k_p, k_{p+4}) pair order, and
// the constant 136 * sum(x) is subtracted once per 32-wide chunk.

constexpr uint32_t kNibbleFlip = 0x88888888u;
constexpr uint32_t kPairMask = 0x000F000Fu;
constexpr uint32_t kBf16_128 = 0x43004300u;
constexpr float kCodeOffset = 136.0f;

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

__device__ inline float dot2_bf16(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                         __builtin_bit_cast(bf16x2_t, b), c, false);
}

// sum over the 8 codes of one packed dword against 4 staged x pairs
__device__ inline float dot8_int4(uint32_t w, const uint32_t (&xp)[4], float acc) {
  const uint32_t u = w ^ kNibbleFlip;
  acc = dot2_bf16((u & kPairMask) | kBf16_128, xp[0], acc);
  acc = dot2_bf16(((u >> 4) & kPairMask) | kBf16_128, xp[1], acc);
  acc = dot2_bf16(((u >> 8) & kPairMask) | kBf16_128, xp[2], acc);
  acc = dot2_bf16(((u >> 12) & kPairMask) | kBf16_128, xp[3], acc);
  return acc;
}

// Build the 4 staged x pairs for 8 consecutive bf16 activations (a dword j of
// a chunk): input words hold (x0,x1),(x2,x3),(x4,x5),(x6,x7); output pairs are
// (x0,x4),(x1,x5),(x2,x6),(x3,x7).
__device__ inline void pair_x8(const uint4 v, uint32_t (&out)[4]) {
  out[0] = (v.x & 0xFFFFu) | (v.z << 16);
  out[1] = (v.x >> 16) | (v.z & 0xFFFF0000u);
  out[2] = (v.y & 0xFFFFu) | (v.w << 16);
  out[3] = (v.y >> 16) | (v.w & 0xFFFF0000u);
}

__device__ inline float sum_x8(const uint4 v) {
  float s = 0.f;
  s += bf16_to_f32(v.x & 0xFFFFu) + bf16_to_f32(v.x >> 16);
  s += bf16_to_f32(v.y & 0xFFFFu) + bf16_to_f32(v.y >> 16);
  s += bf16_to_f32(v.z & 0xFFFFu) + bf16_to_f32(v.z >> 16);
  s += bf16_to_f32(v.w & 0xFFFFu) + bf16_to_f32(v.w >> 16);
  return s;
}

// ---------------------------------------------------------------------------
// wave64 DPP reductions

template <int CTRL>
__device__ inline float dpp_f32(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, true));
}
template <int CTRL>
__device__ inline uint32_t dpp_u32(uint32_t v) {
  return static_cast<uint32_t>(
      __builtin_amdgcn_update_dpp(0, static_cast<int>(v), CTRL, 0xF, 0xF, true));
}

constexpr int kQuadXor1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int kQuadXor2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int kRowHalfMirror = 0x141;  // lane i <-> 7-i within 8
constexpr int kRowMirror = 0x140;      // lane i <-> 15-i within 16

// Sum over each aligned group of 8 lanes; every lane of the group gets it.
__device__ inline float sum8(float v) {
  v += dpp_f32<kQuadXor1>(v);
  v += dpp_f32<kQuadXor2>(v);
  v += dpp_f32<kRowHalfMirror>(v);
  return v;
}

// Sum over each aligned group of 4 lanes.
__device__ inline float sum4(float v) {
  v += dpp_f32<kQuadXor1>(v);
  v += dpp_f32<kQuadXor2>(v);
  return v;
}

// Max over each 16-lane row (every lane of the row gets it).
__device__ inline uint32_t max16_u32(uint32_t v) {
  v = max(v, dpp_u32<kQuadXor1>(v));
  v = max(v, dpp_u32<kQuadXor2>(v));
  v = max(v, dpp_u32<kRowHalfMirror>(v));
  v = max(v, dpp_u32<kRowMirror>(v));
  return v;
}
__device__ inline uint32_t min16_u32(uint32_t v) {
  v = min(v, dpp_u32<kQuadXor1>(v));
  v = min(v, dpp_u32<kQuadXor2>(v));
  v = min(v, dpp_u32<kRowHalfMirror>(v));
  v = min(v, dpp_u32<kRowMirror>(v));
  return v;
}

// Wave-uniform max / min (result broadcast through SGPRs).
__device__ inline uint32_t wave_max_u32(uint32_t v) {
  v = max16_u32(v);
  uint32_t a = __builtin_amdgcn_readlane(v, 0), b = __builtin_amdgcn_readlane(v, 16);
  uint32_t c = __builtin_amdgcn_readlane(v, 32), d = __builtin_amdgcn_readlane(v, 48);
  return max(max(a, b), max(c, d));
}
__device__ inline uint32_t wave_min_u32(uint32_t v) {
  v = min16_u32(v);
  uint32_t a = __builtin_amdgcn_readlane(v, 0), b = __builtin_amdgcn_readlane(v, 16);
  uint32_t c = __builtin_amdgcn_readlane(v, 32), d = __builtin_amdgcn_readlane(v, 48);
  return min(min(a, b), min(c, d));
}

// fp32 -> uint32 key whose unsigned order is the float order.
__device__ inline uint32_t orderable(float f) {
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// ---------------------------------------------------------------------------
// global loads with a streaming hint (weights are read once per call)

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

__device__ inline uint4 load_stream_u4(const uint8_t* p) {
  const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

}  // namespace lk
