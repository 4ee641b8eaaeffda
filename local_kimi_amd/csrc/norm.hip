// RMSNorm, residual add + RMSNorm, and the gated RMSNorm of the KDA output,
// for gfx950 (wave64).
//
// engine/klinear/norm.py:9-52 and the residual adds of
// engine/klinear/layer.py:150-170. Decode runs these on one to a few rows
// (latency: one launch, a few hundred bytes per lane in flight); prefill on
// thousands of rows (HBM-bound: every byte read and written once).
//
// Work mapping. A row is split into 8-value chunks (16 bytes of bf16/fp16,
// 32 of fp32). LPR lanes own a row (16 for rows of at most 128 values, 64
// otherwise); lane j of the row takes chunks j, j + LPR, ... (IT chunks, the
// last ones masked), issuing every load of the row before the first use. The
// squares are summed per lane in chunk order, then over the row's lanes by a
// fixed DPP/shuffle butterfly, so every lane holds the same mean square and
// reruns are bit-identical. Blocks of 256 threads hold 256 / LPR rows.

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "lk_common.hpp"
#include "lk_norm.h"

namespace lk {
namespace {

constexpr int kNormThreads = 256;
constexpr int kNormMaxWidth = 8192;

// 8 values of one chunk as loaded from storage of a given dtype code. The
// dtype only picks the addresses (no branch between loads, so a lane's loads
// all go out before the first is used): fp32 takes two 16-byte words, the
// 16-bit types one, whose second load repeats the first (an L1 hit).
struct Chunk {
  uint4 lo, hi;  // hi holds values 4..7 only for fp32 storage
};

__device__ inline Chunk load_chunk(const void* base, int64_t chunk, int dt) {
  const uint4* p = static_cast<const uint4*>(base);
  const bool wide = dt == LK_DTYPE_F32;
  Chunk c;
  c.lo = p[wide ? 2 * chunk : chunk];
  c.hi = p[wide ? 2 * chunk + 1 : chunk];
  return c;
}

// The dtype conversions below select between the candidate results with the
// (launch-uniform) dtype code instead of branching on it: the kernels stay
// straight-line code a few KB long, which a cold instruction cache fetches in
// far less time than a branch tree over every dtype (a one-row decode launch
// is one wave walking that code once).
__device__ inline float half_bits_to_f32(uint32_t h, bool bf16) {
  const float as_bf16 = __uint_as_float(h << 16);
  const float as_f16 = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(h)));
  return bf16 ? as_bf16 : as_f16;
}

__device__ inline void unpack_chunk(const Chunk& c, int dt, float (&v)[8]) {
  const bool wide = dt == LK_DTYPE_F32, bf16 = dt == LK_DTYPE_BF16;
  const uint32_t w[8] = {c.lo.x, c.lo.y, c.lo.z, c.lo.w, c.hi.x, c.hi.y, c.hi.z, c.hi.w};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float a = half_bits_to_f32(w[j] & 0xFFFFu, bf16);
    const float b = half_bits_to_f32(w[j] >> 16, bf16);
    v[2 * j] = wide ? __uint_as_float(w[2 * j]) : a;
    v[2 * j + 1] = wide ? __uint_as_float(w[2 * j + 1]) : b;
  }
}

__device__ inline uint32_t f32_to_half_bits(float x, bool bf16) {
  const uint32_t as_f16 = __builtin_bit_cast(uint16_t, static_cast<_Float16>(x));
  return bf16 ? static_cast<uint32_t>(f32_to_bf16(x)) : as_f16;
}

__device__ inline float round_to(float x, int dt) {
  const float as_bf16 = round_bf16(x);
  const float as_f16 = static_cast<float>(static_cast<_Float16>(x));
  return dt == LK_DTYPE_BF16 ? as_bf16 : (dt == LK_DTYPE_F16 ? as_f16 : x);
}

__device__ inline void store_chunk(void* base, int64_t chunk, int dt, const float (&v)[8]) {
  const bool wide = dt == LK_DTYPE_F32, bf16 = dt == LK_DTYPE_BF16;
  uint32_t h[4];
#pragma unroll
  for (int j = 0; j < 4; ++j)
    h[j] = f32_to_half_bits(v[2 * j], bf16) | (f32_to_half_bits(v[2 * j + 1], bf16) << 16);
  // fp32 writes two 16-byte words; the 16-bit types write their one word
  // twice (the same bytes to the same address), so no store is conditional
  uint4* p = static_cast<uint4*>(base);
  const uint4 narrow = make_uint4(h[0], h[1], h[2], h[3]);
  p[wide ? 2 * chunk : chunk] =
      wide ? make_uint4(__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]),
                        __float_as_uint(v[3]))
           : narrow;
  p[wide ? 2 * chunk + 1 : chunk] =
      wide ? make_uint4(__float_as_uint(v[4]), __float_as_uint(v[5]), __float_as_uint(v[6]),
                        __float_as_uint(v[7]))
           : narrow;
}

template <int LPR>
__device__ inline float row_sum(float v) {
  v += dpp_f32<kQuadXor1>(v);
  v += dpp_f32<kQuadXor2>(v);
  v += dpp_f32<kRowHalfMirror>(v);
  v += dpp_f32<kRowMirror>(v);
  if constexpr (LPR == 64) {
    v += __shfl_xor(v, 16);
    v += __shfl_xor(v, 32);
  }
  return v;
}

__device__ inline float inv_rms(float sum_sq, int64_t width, float eps) {
  return 1.0f / sqrtf(sum_sq / static_cast<float>(width) + eps);
}

enum class NormKind { Plain, Add, Gated };

struct NormArgs {
  const void* x;       // rows of the norm's input (residual for Add, values for Gated)
  const void* delta;   // Add: the term added to x
  const void* gate;    // Gated: the gate rows
  const void* weight;
  void* sum_out;       // Add: the rounded sum
  void* y;
  int64_t rows, width;
  float eps;
  int in_dt;       // storage dtype of x (and delta)
  int round_dt;    // dtype the normalised values (Plain/Add) or inputs (Gated) round to
  int weight_dt, gate_dt, out_dt;
};

// XDT is the storage dtype of the input rows (and delta / sum), ODT the one
// dtype of weight, gate, rounding and output, when the launch has one; a
// negative value takes each dtype from the arguments at run time instead.
// The fixed forms fold every dtype decision at compile time.
constexpr int kRuntimeDtype = -1;

template <NormKind KIND, int LPR, int IT, int XDT, int ODT>
__global__ void __launch_bounds__(kNormThreads) norm_kernel(NormArgs a) {
  constexpr int kRowsPerBlock = kNormThreads / LPR;
  const int xdt = XDT >= 0 ? XDT : a.in_dt;
  const int wdt = ODT >= 0 ? ODT : a.weight_dt;
  const int gdt = ODT >= 0 ? ODT : a.gate_dt;
  const int rdt = ODT >= 0 ? ODT : a.round_dt;
  const int odt = ODT >= 0 ? ODT : a.out_dt;
  const int lane = static_cast<int>(threadIdx.x) % LPR;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + threadIdx.x / LPR;
  if (row >= a.rows) return;  // uniform per row group; the butterfly stays within it
  const int64_t chunks = a.width / 8;
  const int64_t first = row * chunks;

  // every load of the row first: input (and delta / gate), then the weight
  // (wide rows load the weight after the reduction, which keeps them in
  // registers)
  constexpr bool kEarlyWeight = IT <= 8;
  Chunk cx[IT], cd[IT], cw[kEarlyWeight ? IT : 1];
#pragma unroll
  for (int i = 0; i < IT; ++i) {
    const int64_t c = lane + static_cast<int64_t>(LPR) * i;
    const int64_t cc = c < chunks ? c : 0;
    cx[i] = load_chunk(a.x, first + cc, xdt);
    if constexpr (KIND == NormKind::Add) cd[i] = load_chunk(a.delta, first + cc, xdt);
    if constexpr (KIND == NormKind::Gated) cd[i] = load_chunk(a.gate, first + cc, gdt);
  }
  if constexpr (kEarlyWeight) {
#pragma unroll
    for (int i = 0; i < IT; ++i) {
      const int64_t c = lane + static_cast<int64_t>(LPR) * i;
      cw[i] = load_chunk(a.weight, c < chunks ? c : 0, wdt);
    }
  }

  float v[IT][8];
  float sq = 0.f;
#pragma unroll
  for (int i = 0; i < IT; ++i) {
    const bool ok = lane + static_cast<int64_t>(LPR) * i < chunks;
    unpack_chunk(cx[i], xdt, v[i]);
    if constexpr (KIND == NormKind::Add) {
      float d[8];
      unpack_chunk(cd[i], xdt, d);
#pragma unroll
      for (int j = 0; j < 8; ++j) v[i][j] = round_to(v[i][j] + d[j], xdt);
      if (ok) store_chunk(a.sum_out, first + lane + static_cast<int64_t>(LPR) * i, xdt, v[i]);
    }
    if constexpr (KIND == NormKind::Gated) {
#pragma unroll
      for (int j = 0; j < 8; ++j) v[i][j] = round_to(v[i][j], rdt);
    }
    float part = sq;
#pragma unroll
    for (int j = 0; j < 8; ++j) part = fmaf(v[i][j], v[i][j], part);
    sq = ok ? part : sq;
  }
  const float r = inv_rms(row_sum<LPR>(sq), a.width, a.eps);

#pragma unroll
  for (int i = 0; i < IT; ++i) {
    const int64_t c = lane + static_cast<int64_t>(LPR) * i;
    if (c >= chunks) continue;
    float w[8], out[8];
    if constexpr (kEarlyWeight) {
      unpack_chunk(cw[i], wdt, w);
    } else {
      unpack_chunk(load_chunk(a.weight, c, wdt), wdt, w);
    }
    if constexpr (KIND == NormKind::Gated) {
      float g[8];
      unpack_chunk(cd[i], gdt, g);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float sig = 1.0f / (1.0f + expf(-g[j]));
        out[j] = (v[i][j] * r) * w[j] * sig;
      }
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) out[j] = w[j] * round_to(v[i][j] * r, rdt);
    }
    store_chunk(a.y, first + c, odt, out);
  }
}

// rows of up to 16 chunks take 16 lanes each (4 rows per wave); wider rows a
// whole wave, IT chunks per lane
template <NormKind KIND, int XDT, int ODT>
int launch_width(const NormArgs& a, hipStream_t s) {
  const int64_t chunks = a.width / 8;
  if (chunks <= 16) {
    const dim3 grid(static_cast<unsigned>((a.rows + kNormThreads / 16 - 1) / (kNormThreads / 16)));
    norm_kernel<KIND, 16, 1, XDT, ODT><<<grid, kNormThreads, 0, s>>>(a);
    return check_launch("norm_kernel");
  }
  const int64_t its = (chunks + 63) / 64;
  const dim3 grid(static_cast<unsigned>((a.rows + kNormThreads / 64 - 1) / (kNormThreads / 64)));
#define LK_NORM_CASE(N)                                               \
  if (its <= N) {                                                     \
    norm_kernel<KIND, 64, N, XDT, ODT><<<grid, kNormThreads, 0, s>>>(a); \
    return check_launch("norm_kernel");                               \
  }
  LK_NORM_CASE(1)
  LK_NORM_CASE(2)
  LK_NORM_CASE(3)
  LK_NORM_CASE(4)
  LK_NORM_CASE(5)
  LK_NORM_CASE(6)
  LK_NORM_CASE(8)
  LK_NORM_CASE(12)
  LK_NORM_CASE(16)
#undef LK_NORM_CASE
  return fail_arg("row width too large for the norm kernels");
}

template <NormKind KIND>
int launch_norm(const NormArgs& a, hipStream_t s) {
  const bool one_out = a.weight_dt == a.round_dt && a.out_dt == a.round_dt &&
                       (KIND != NormKind::Gated || a.gate_dt == a.round_dt);
  if (one_out && a.in_dt == a.round_dt) {
    if (a.in_dt == LK_DTYPE_BF16) return launch_width<KIND, LK_DTYPE_BF16, LK_DTYPE_BF16>(a, s);
    if (a.in_dt == LK_DTYPE_F16) return launch_width<KIND, LK_DTYPE_F16, LK_DTYPE_F16>(a, s);
    if (a.in_dt == LK_DTYPE_F32) return launch_width<KIND, LK_DTYPE_F32, LK_DTYPE_F32>(a, s);
  }
  if constexpr (KIND == NormKind::Gated) {
    // fp32 values rounded to bf16 before the norm (the KDA output projection's input)
    if (one_out && a.in_dt == LK_DTYPE_F32 && a.round_dt == LK_DTYPE_BF16)
      return launch_width<KIND, LK_DTYPE_F32, LK_DTYPE_BF16>(a, s);
  }
  return launch_width<KIND, kRuntimeDtype, kRuntimeDtype>(a, s);
}

bool norm_dtype(int d) { return d == LK_DTYPE_F32 || d == LK_DTYPE_F16 || d == LK_DTYPE_BF16; }

// torch's promotion of x_dtype with weight_dtype over {fp32, fp16, bf16}
int promoted(int x_dt, int w_dt) { return x_dt == w_dt ? x_dt : LK_DTYPE_F32; }

int check_shape(int64_t rows, int64_t width, float eps) {
  LK_REQUIRE(rows >= 0 && width > 0, "norm rows must be >= 0 and the width positive");
  LK_REQUIRE(width % 8 == 0 && width <= kNormMaxWidth,
             "norm width must be a multiple of 8 up to %d, got %lld", kNormMaxWidth,
             (long long)width);
  LK_REQUIRE(rows <= (1LL << 32), "too many rows for one norm call");
  LK_REQUIRE(eps >= 0.f, "eps must be non-negative");
  return LK_OK;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace
}  // namespace lk

using namespace lk;

extern "C" {

int lk_rms_norm(const void* x, const void* weight, void* y, int64_t rows, int64_t hidden,
                float eps, int x_dtype, int weight_dtype, void* stream) {
  if (const int st = check_shape(rows, hidden, eps)) return st;
  LK_REQUIRE(norm_dtype(x_dtype) && norm_dtype(weight_dtype), "unsupported norm dtype code");
  if (rows == 0) return LK_OK;
  LK_REQUIRE(x && weight && y, "null pointer argument");
  LK_REQUIRE(aligned16(x) && aligned16(weight) && aligned16(y),
             "norm tensors must start on a 16-byte boundary");
  NormArgs a{x, nullptr, nullptr, weight, nullptr, y, rows, hidden, eps,
             x_dtype, x_dtype, weight_dtype, LK_DTYPE_F32, promoted(x_dtype, weight_dtype)};
  return launch_norm<NormKind::Plain>(a, as_stream(stream));
}

int lk_add_rms_norm(const void* residual, const void* delta, const void* weight, void* sum_out,
                    void* y, int64_t rows, int64_t hidden, float eps, int x_dtype,
                    int weight_dtype, void* stream) {
  if (const int st = check_shape(rows, hidden, eps)) return st;
  LK_REQUIRE(norm_dtype(x_dtype) && norm_dtype(weight_dtype), "unsupported norm dtype code");
  if (rows == 0) return LK_OK;
  LK_REQUIRE(residual && delta && weight && sum_out && y, "null pointer argument");
  LK_REQUIRE(aligned16(residual) && aligned16(delta) && aligned16(weight) && aligned16(sum_out) &&
                 aligned16(y),
             "norm tensors must start on a 16-byte boundary");
  NormArgs a{residual, delta, nullptr, weight, sum_out, y, rows, hidden, eps,
             x_dtype, x_dtype, weight_dtype, LK_DTYPE_F32, promoted(x_dtype, weight_dtype)};
  return launch_norm<NormKind::Add>(a, as_stream(stream));
}

int lk_rms_gated_norm(const void* values, const void* gate, const void* weight, void* y,
                      int64_t rows, int64_t dim, float eps, int values_dtype, int input_dtype,
                      int gate_dtype, int weight_dtype, void* stream) {
  if (const int st = check_shape(rows, dim, eps)) return st;
  LK_REQUIRE(norm_dtype(values_dtype) && norm_dtype(input_dtype) && norm_dtype(gate_dtype) &&
                 norm_dtype(weight_dtype),
             "unsupported norm dtype code");
  if (rows == 0) return LK_OK;
  LK_REQUIRE(values && gate && weight && y, "null pointer argument");
  LK_REQUIRE(aligned16(values) && aligned16(gate) && aligned16(weight) && aligned16(y),
             "norm tensors must start on a 16-byte boundary");
  NormArgs a{values, nullptr, gate, weight, nullptr, y, rows, dim, eps,
             values_dtype, input_dtype, weight_dtype, gate_dtype, input_dtype};
  return launch_norm<NormKind::Gated>(a, as_stream(stream));
}

}  // extern "C"
