// OCP MXFP4 codec on the GPU: E2M1 elements, low nibble first, one E8M0
// exponent per 32 values along K (engine/k3ref/dequant.py:18-73).
//
// Decode: value = e2m1[code] * 2**(e8m0 - 127) in fp32 (exact: the scale is a
// power of two), cast once to the output type, as dequantize_mxfp4 does.
// Encode (the reference has none): shared exponent floor(log2(amax)) - 2,
// biased and clamped to [0, 254], 127 for an all-zero block; elements
// w / 2**exp rounded to the E2M1 grid, ties to the even code, saturated to
// +-6, sign kept for zeros (OCP Microscaling Formats v1.0).

#include "lk_common.hpp"

namespace lk {
namespace {

constexpr int kMxGroup = 32;

__device__ inline float e2m1_value(uint32_t code) {
  // magnitudes 0, 0.5, 1, 1.5, 2, 3, 4, 6 by the 3 low bits; bit 3 is the sign
  const uint32_t mag = code & 7u;
  const float v = mag < 4u ? 0.5f * static_cast<float>(mag)
                           : static_cast<float>(2u << ((mag - 4u) >> 1)) *
                                 (1.0f + 0.5f * static_cast<float>(mag & 1u));
  return (code & 8u) ? -v : v;
}

// 2**(e - 127) as fp32: e = 0 is the subnormal 2**-127, e = 255 gives inf.
__device__ inline float e8m0_scale(uint32_t e) {
  return __builtin_bit_cast(float, e == 0u ? 0x00400000u : e << 23);
}

__device__ inline uint32_t e2m1_code(float v) {
  const float a = fminf(fabsf(v), 6.0f);
  uint32_t mag = 0;
  mag = a > 0.25f ? 1u : mag;
  mag = a >= 0.75f ? 2u : mag;
  mag = a > 1.25f ? 3u : mag;
  mag = a >= 1.75f ? 4u : mag;
  mag = a > 2.5f ? 5u : mag;
  mag = a >= 3.5f ? 6u : mag;
  mag = a > 5.0f ? 7u : mag;
  return mag | (signbit(v) ? 8u : 0u);
}

// One thread per (row, 32-value block).
__global__ void mxfp4_quantise_kernel(const uint16_t* __restrict__ w, uint8_t* __restrict__ packed,
                                      uint8_t* __restrict__ scale, int64_t n, int64_t k) {
  const int64_t blocks_per_row = k / kMxGroup;
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (gid >= n * blocks_per_row) return;
  const int64_t row = gid / blocks_per_row;
  const int64_t blk = gid - row * blocks_per_row;
  const uint16_t* src = w + row * k + blk * kMxGroup;
  float v[kMxGroup];
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < kMxGroup / 8; ++i) {
    const uint4 q = *reinterpret_cast<const uint4*>(src + 8 * i);
    const uint32_t words[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[8 * i + 2 * j] = bf16_to_f32(words[j] & 0xFFFFu);
      v[8 * i + 2 * j + 1] = bf16_to_f32(words[j] >> 16);
    }
  }
#pragma unroll
  for (int i = 0; i < kMxGroup; ++i) amax = fmaxf(amax, fabsf(v[i]));
  int biased = 127;
  if (amax > 0.f) {
    const int e = ilogbf(amax);  // floor(log2(amax)), subnormals included
    biased = min(254, max(0, e - 2 + 127));
  }
  // w / 2**(biased - 127) as an exact multiply by 2**(127 - biased)
  const float inv_scale = e8m0_scale(static_cast<uint32_t>(254 - biased));
  uint32_t out[4] = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int i = 0; i < kMxGroup; ++i) {
    const uint32_t code = e2m1_code(v[i] * inv_scale);
    out[i / 8] |= code << (4 * (i % 8));
  }
  *reinterpret_cast<uint4*>(packed + row * (k / 2) + blk * (kMxGroup / 2)) =
      make_uint4(out[0], out[1], out[2], out[3]);
  scale[row * blocks_per_row + blk] = static_cast<uint8_t>(biased);
}

// One thread per packed byte (two values).
__global__ void mxfp4_dequantise_kernel(const uint8_t* __restrict__ packed,
                                        const uint8_t* __restrict__ scale, void* __restrict__ out,
                                        int64_t n, int64_t k, int out_f32) {
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t half = k / 2;
  if (gid >= n * half) return;
  const int64_t row = gid / half;
  const int64_t j = gid - row * half;
  const uint32_t byte = packed[gid];
  const float s = e8m0_scale(scale[row * (k / kMxGroup) + (2 * j) / kMxGroup]);
  const float lo = e2m1_value(byte & 0xFu) * s;
  const float hi = e2m1_value(byte >> 4) * s;
  if (out_f32) {
    reinterpret_cast<float2*>(out)[gid] = make_float2(lo, hi);
  } else {
    reinterpret_cast<uint32_t*>(out)[gid] =
        static_cast<uint32_t>(f32_to_bf16(lo)) | (static_cast<uint32_t>(f32_to_bf16(hi)) << 16);
  }
}

// Reference variant of the GEMM: one thread per output, each weight decoded
// to the activation type (exact there), fp32 dot in k order.
__global__ void mxfp4_gemm_reference_kernel(const uint16_t* __restrict__ x,
                                            const uint8_t* __restrict__ packed,
                                            const uint8_t* __restrict__ scale,
                                            uint16_t* __restrict__ y, int64_t m, int64_t n,
                                            int64_t k, int act_f16) {
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (gid >= m * n) return;
  const int64_t row = gid / n;
  const int64_t col = gid - row * n;
  const uint16_t* xr = x + row * k;
  const uint8_t* wr = packed + col * (k / 2);
  const uint8_t* sr = scale + col * (k / kMxGroup);
  float acc = 0.f;
  for (int64_t kk = 0; kk < k; ++kk) {
    const uint32_t byte = wr[kk / 2];
    const float w = e2m1_value((kk & 1) ? (byte >> 4) : (byte & 0xFu)) * e8m0_scale(sr[kk / kMxGroup]);
    float wq, xv;
    if (act_f16) {
      wq = static_cast<float>(static_cast<_Float16>(w));
      xv = static_cast<float>(__builtin_bit_cast(_Float16, xr[kk]));
    } else {
      wq = bf16_to_f32(f32_to_bf16(w));
      xv = bf16_to_f32(xr[kk]);
    }
    acc = fmaf(xv, wq, acc);
  }
  y[gid] = act_f16 ? __builtin_bit_cast(uint16_t, static_cast<_Float16>(acc)) : f32_to_bf16(acc);
}

inline unsigned blocks_for(int64_t count, int threads) {
  return static_cast<unsigned>((count + threads - 1) / threads);
}

int check_mx_dims(int64_t n, int64_t k) {
  LK_REQUIRE(n > 0 && k > 0, "reduction and output dimensions must be nonzero");
  LK_REQUIRE(k % kMxGroup == 0, "MXFP4 reduction dimension must be divisible by 32");
  return LK_OK;
}

}  // namespace
}  // namespace lk

using namespace lk;

extern "C" {

int lk_mxfp4_quantise(const uint16_t* weight, uint8_t* packed, uint8_t* scale, int64_t n,
                      int64_t k, void* stream) {
  LK_REQUIRE(weight && packed && scale, "null pointer argument");
  if (int rc = check_mx_dims(n, k)) return rc;
  const int64_t work = n * (k / kMxGroup);
  mxfp4_quantise_kernel<<<blocks_for(work, 256), 256, 0, as_stream(stream)>>>(weight, packed,
                                                                              scale, n, k);
  return check_launch("lk_mxfp4_quantise");
}

int lk_mxfp4_dequantise(const uint8_t* packed, const uint8_t* scale, void* out, int64_t n,
                        int64_t k, int out_f32, void* stream) {
  LK_REQUIRE(packed && scale && out, "null pointer argument");
  if (int rc = check_mx_dims(n, k)) return rc;
  const int64_t work = n * (k / 2);
  mxfp4_dequantise_kernel<<<blocks_for(work, 256), 256, 0, as_stream(stream)>>>(
      packed, scale, out, n, k, out_f32);
  return check_launch("lk_mxfp4_dequantise");
}

int lk_mxfp4_gemm_reference(const uint16_t* x, const uint8_t* packed, const uint8_t* scale,
                            uint16_t* y, int64_t m, int64_t n, int64_t k, int act_f16,
                            void* stream) {
  LK_REQUIRE(packed && scale && y, "null pointer argument");
  LK_REQUIRE(m >= 0, "negative row count");
  if (int rc = check_mx_dims(n, k)) return rc;
  if (m == 0) return LK_OK;
  LK_REQUIRE(x != nullptr, "null activation pointer");
  mxfp4_gemm_reference_kernel<<<blocks_for(m * n, 256), 256, 0, as_stream(stream)>>>(
      x, packed, scale, y, m, n, k, act_f16);
  return check_launch("lk_mxfp4_gemm_reference");
}

}  // extern "C"
