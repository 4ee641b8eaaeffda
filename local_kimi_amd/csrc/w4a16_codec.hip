// W4A16 codec kernels, the one-thread-per-output reference-rounding kernels
// and the library's error state.
//
// quantise/dequantise restate engine/quant/w4a16.py:68-129 bit for bit.
// The *_reference kernels follow the reference's rounding contract exactly
// (weight decoded to bf16(q * s) before the fp32 multiply-add,
// engine/quant/triton_w4a16.py:105-113) and are registered as the
// "reference" variants; they are deliberately simple, not fast.

#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <atomic>

#include "lk_common.hpp"

namespace lk {

static thread_local char g_error[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
}

int fail_arg(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
  return LK_ERR_ARGUMENT;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: kernel launch failed: %s", what, hipGetErrorString(e));
    return LK_ERR_HIP;
  }
  g_error[0] = '\0';
  return LK_OK;
}

namespace {

struct KnobSpec {
  const char* name;
  const char* choices[4];  // index = value; choice 0 is "auto"
};

constexpr KnobSpec kKnobs[kKnobCount] = {
    {"moe_gemm", {"auto", "lds", "stream16", "stream64"}},
    {"moe_persist", {"auto", "off", nullptr, nullptr}},
    {"dense_gemm", {"auto", "lds", nullptr, nullptr}},
    {"mxfp4_mfma", {"auto", "fp4", "bf16", nullptr}},
    {"moe_fused_schedule", {"auto", "off", nullptr, nullptr}},
    {"moe_split_swiglu", {"auto", "off", nullptr, nullptr}},
};

std::atomic<int> g_knobs[kKnobCount];  // zero-initialised: "auto"

}  // namespace

int path_choice(Knob knob) { return g_knobs[knob].load(std::memory_order_relaxed); }

namespace {

constexpr float kQmax = 7.0f;
constexpr float kBf16Tiny = 1.17549435082228750797e-38f;  // 2^-126

// One thread per (row, group): absmax, stored bf16 scale, codes.
__global__ void quantise_kernel(const uint16_t* __restrict__ w, uint8_t* __restrict__ packed,
                                uint16_t* __restrict__ scales, int64_t n, int64_t k,
                                int64_t group) {
  const int64_t groups_per_row = k / group;
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (gid >= n * groups_per_row) return;
  const int64_t row = gid / groups_per_row;
  const int64_t g = gid - row * groups_per_row;
  const uint16_t* src = w + row * k + g * group;
  float absmax = 0.f;
  for (int64_t j = 0; j < group; ++j) absmax = fmaxf(absmax, fabsf(bf16_to_f32(src[j])));
  const float raw = absmax / kQmax;
  float scale = (absmax == 0.f) ? 1.0f : fmaxf(round_bf16(raw), kBf16Tiny);
  const uint16_t scale_bits = f32_to_bf16(scale);
  scale = bf16_to_f32(scale_bits);
  scales[row * groups_per_row + g] = scale_bits;
  uint8_t* dst = packed + row * (k / 2) + g * (group / 2);
  for (int64_t j = 0; j < group; j += 2) {
    float c0 = fminf(fmaxf(rintf(bf16_to_f32(src[j]) / scale), -kQmax), kQmax);
    float c1 = fminf(fmaxf(rintf(bf16_to_f32(src[j + 1]) / scale), -kQmax), kQmax);
    const uint32_t n0 = static_cast<uint32_t>(static_cast<int32_t>(c0)) & 0xFu;
    const uint32_t n1 = static_cast<uint32_t>(static_cast<int32_t>(c1)) & 0xFu;
    dst[j / 2] = static_cast<uint8_t>(n0 | (n1 << 4));
  }
}

__device__ inline int32_t nibble_code(uint32_t word, int p) {
  const int32_t v = static_cast<int32_t>((word >> (4 * p)) & 0xFu);
  return v >= 8 ? v - 16 : v;
}

// One thread per packed dword (8 outputs); bf16 output = bf16(q * s).
__global__ void dequantise_kernel(const uint8_t* __restrict__ packed,
                                  const uint16_t* __restrict__ scales,
                                  uint16_t* __restrict__ out, int64_t n, int64_t k,
                                  int64_t group) {
  const int64_t words_per_row = k / 8;
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (gid >= n * words_per_row) return;
  const int64_t row = gid / words_per_row;
  const int64_t wd = gid - row * words_per_row;
  const uint32_t word = reinterpret_cast<const uint32_t*>(packed + row * (k / 2))[wd];
  const float s = bf16_to_f32(scales[row * (k / group) + (wd * 8) / group]);
  uint16_t v[8];
#pragma unroll
  for (int p = 0; p < 8; ++p) v[p] = f32_to_bf16(static_cast<float>(nibble_code(word, p)) * s);
  uint4 o;
  o.x = v[0] | (static_cast<uint32_t>(v[1]) << 16);
  o.y = v[2] | (static_cast<uint32_t>(v[3]) << 16);
  o.z = v[4] | (static_cast<uint32_t>(v[5]) << 16);
  o.w = v[6] | (static_cast<uint32_t>(v[7]) << 16);
  reinterpret_cast<uint4*>(out + row * k)[wd] = o;
}

// float32 output = q * s exactly (the reference's dequantise(dtype=float32)).
__global__ void dequantise_f32_kernel(const uint8_t* __restrict__ packed,
                                      const uint16_t* __restrict__ scales,
                                      float* __restrict__ out, int64_t n, int64_t k,
                                      int64_t group) {
  const int64_t words_per_row = k / 8;
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (gid >= n * words_per_row) return;
  const int64_t row = gid / words_per_row;
  const int64_t wd = gid - row * words_per_row;
  const uint32_t word = reinterpret_cast<const uint32_t*>(packed + row * (k / 2))[wd];
  const float s = bf16_to_f32(scales[row * (k / group) + (wd * 8) / group]);
  float4 a, b;
  a.x = nibble_code(word, 0) * s;
  a.y = nibble_code(word, 1) * s;
  a.z = nibble_code(word, 2) * s;
  a.w = nibble_code(word, 3) * s;
  b.x = nibble_code(word, 4) * s;
  b.y = nibble_code(word, 5) * s;
  b.z = nibble_code(word, 6) * s;
  b.w = nibble_code(word, 7) * s;
  float4* dst = reinterpret_cast<float4*>(out + row * k + wd * 8);
  dst[0] = a;
  dst[1] = b;
}

// Dot product of one activation row with one packed weight row, weights
// rounded to bf16 first (the reference contract).
__device__ float dot_row_reference(const uint16_t* __restrict__ x,
                                   const uint8_t* __restrict__ prow,
                                   const uint16_t* __restrict__ srow, int64_t k,
                                   int64_t group) {
  float acc = 0.f;
  for (int64_t kk = 0; kk < k; kk += 8) {
    const uint32_t word = *reinterpret_cast<const uint32_t*>(prow + kk / 2);
    const float s = bf16_to_f32(srow[kk / group]);
#pragma unroll
    for (int p = 0; p < 8; ++p) {
      const float wv = round_bf16(static_cast<float>(nibble_code(word, p)) * s);
      acc = fmaf(bf16_to_f32(x[kk + p]), wv, acc);
    }
  }
  return acc;
}

__global__ void dense_reference_kernel(const uint16_t* __restrict__ x,
                                       const uint8_t* __restrict__ packed,
                                       const uint16_t* __restrict__ scales,
                                       uint16_t* __restrict__ y, int64_t m, int64_t n,
                                       int64_t k, int64_t group) {
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (gid >= m * n) return;
  const int64_t row = gid / n;
  const int64_t col = gid - row * n;
  const float acc = dot_row_reference(x + row * k, packed + col * (k / 2),
                                      scales + col * (k / group), k, group);
  y[gid] = f32_to_bf16(acc);
}

__global__ void grouped_reference_kernel(const uint16_t* __restrict__ x,
                                         const int64_t* __restrict__ idx,
                                         const uint8_t* __restrict__ packed,
                                         const uint16_t* __restrict__ scales,
                                         uint16_t* __restrict__ out, int64_t tokens,
                                         int64_t routes, int64_t experts, int64_t n, int64_t k,
                                         int64_t group) {
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (gid >= tokens * routes * n) return;
  const int64_t pair = gid / n;
  const int64_t col = gid - pair * n;
  const int64_t t = pair / routes;
  const int64_t e = idx[pair];
  if (e < 0 || e >= experts) {  // empty route: no read outside the bank
    out[gid] = 0;
    return;
  }
  const float acc = dot_row_reference(x + t * k, packed + (e * n + col) * (k / 2),
                                      scales + (e * n + col) * (k / group), k, group);
  out[gid] = f32_to_bf16(acc);
}

__global__ void silu_mul_kernel(const uint16_t* __restrict__ gate,
                                const uint16_t* __restrict__ up, uint16_t* __restrict__ out,
                                int64_t count) {
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (gid >= count) return;
  const float g = bf16_to_f32(gate[gid]);
  const float s = round_bf16(silu_f32(g));
  out[gid] = f32_to_bf16(s * bf16_to_f32(up[gid]));
}

// y[t, :] = bf16(bf16(sum_{r<R-1} eo[t,r,:] * cw[t,r]) + eo[t,R-1,:]), one
// thread per output element (klinear/moe.py:327-334).
__global__ void route_combine_kernel(const uint16_t* __restrict__ eo, const float* __restrict__ cw,
                                     uint16_t* __restrict__ y, int64_t tokens, int64_t routes,
                                     int64_t h) {
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (gid >= tokens * h) return;
  const int64_t t = gid / h;
  const int64_t col = gid - t * h;
  const uint16_t* base = eo + t * routes * h + col;
  float acc = 0.f;
  for (int64_t r = 0; r + 1 < routes; ++r) acc += bf16_to_f32(base[r * h]) * cw[t * routes + r];
  y[gid] = f32_to_bf16(round_bf16(acc) + bf16_to_f32(base[(routes - 1) * h]));
}

inline unsigned blocks_for(int64_t count, int threads) {
  return static_cast<unsigned>((count + threads - 1) / threads);
}

}  // namespace

int check_group(int64_t k, int64_t group) {
  LK_REQUIRE(k > 0, "reduction width must be positive, got %lld", (long long)k);
  LK_REQUIRE(group > 0 && group % 32 == 0, "group size must be a positive multiple of 32, got %lld",
             (long long)group);
  LK_REQUIRE(k % group == 0, "reduction width %lld must be divisible by group size %lld",
             (long long)k, (long long)group);
  return LK_OK;
}

int check_pow2_group(int64_t k, int64_t group) {
  if (int rc = check_group(k, group)) return rc;
  LK_REQUIRE((group & (group - 1)) == 0, "group size must be a power of two, got %lld",
             (long long)group);
  return LK_OK;
}

}  // namespace lk

using namespace lk;

extern "C" {

const char* lk_last_error(void) { return lk::g_error; }

int lk_abi_version(void) { return 2; }

int lk_set_path(const char* knob, const char* choice) {
  LK_REQUIRE(knob && choice, "null knob or choice");
  for (int k = 0; k < lk::kKnobCount; ++k) {
    const lk::KnobSpec& spec = lk::kKnobs[k];
    if (strcmp(knob, spec.name) != 0) continue;
    for (int v = 0; v < 4 && spec.choices[v]; ++v) {
      if (strcmp(choice, spec.choices[v]) == 0) {
        lk::g_knobs[k].store(v, std::memory_order_relaxed);
        return LK_OK;
      }
    }
    return lk::fail_arg("unknown choice '%s' for path knob '%s'", choice, knob);
  }
  return lk::fail_arg("unknown path knob '%s'", knob);
}

int lk_get_path(const char* knob) {
  if (!knob) return -1;
  for (int k = 0; k < lk::kKnobCount; ++k)
    if (strcmp(knob, lk::kKnobs[k].name) == 0) return lk::path_choice(static_cast<lk::Knob>(k));
  return -1;
}

int lk_w4a16_quantise(const uint16_t* weight, uint8_t* packed, uint16_t* scales, int64_t n,
                      int64_t k, int64_t group_size, void* stream) {
  LK_REQUIRE(weight && packed && scales, "null pointer argument");
  LK_REQUIRE(n > 0, "output features must be positive");
  if (int rc = check_group(k, group_size)) return rc;
  const int64_t work = n * (k / group_size);
  quantise_kernel<<<blocks_for(work, 256), 256, 0, as_stream(stream)>>>(weight, packed, scales,
                                                                         n, k, group_size);
  return check_launch("lk_w4a16_quantise");
}

int lk_w4a16_dequantise(const uint8_t* packed, const uint16_t* scales, void* out, int64_t n,
                        int64_t k, int64_t group_size, int out_f32, void* stream) {
  LK_REQUIRE(packed && scales && out, "null pointer argument");
  LK_REQUIRE(n > 0, "output features must be positive");
  if (int rc = check_group(k, group_size)) return rc;
  const int64_t work = n * (k / 8);
  if (out_f32)
    dequantise_f32_kernel<<<blocks_for(work, 256), 256, 0, as_stream(stream)>>>(
        packed, scales, static_cast<float*>(out), n, k, group_size);
  else
    dequantise_kernel<<<blocks_for(work, 256), 256, 0, as_stream(stream)>>>(
        packed, scales, static_cast<uint16_t*>(out), n, k, group_size);
  return check_launch("lk_w4a16_dequantise");
}

int lk_w4a16_dense_reference(const uint16_t* x, const uint8_t* packed, const uint16_t* scales,
                             uint16_t* y, int64_t m, int64_t n, int64_t k, int64_t group_size,
                             void* stream) {
  LK_REQUIRE(packed && scales && y && (m == 0 || x), "null pointer argument");
  LK_REQUIRE(n > 0 && m >= 0, "invalid dense dimensions m=%lld n=%lld", (long long)m,
             (long long)n);
  if (int rc = check_group(k, group_size)) return rc;
  if (m == 0) return LK_OK;
  dense_reference_kernel<<<blocks_for(m * n, 256), 256, 0, as_stream(stream)>>>(
      x, packed, scales, y, m, n, k, group_size);
  return check_launch("lk_w4a16_dense_reference");
}

int lk_w4a16_grouped_reference(const uint16_t* x, const int64_t* expert_indices,
                               const uint8_t* packed, const uint16_t* scales, uint16_t* out,
                               int64_t tokens, int64_t routes, int64_t experts, int64_t n,
                               int64_t k, int64_t group_size, void* stream) {
  LK_REQUIRE(packed && scales && out, "null pointer argument");
  LK_REQUIRE(routes > 0 && experts > 0 && n > 0 && tokens >= 0,
             "grouped W4A16 requires nonzero dimensions");
  if (int rc = check_group(k, group_size)) return rc;
  if (tokens == 0) return LK_OK;
  LK_REQUIRE(x && expert_indices, "null pointer argument");
  grouped_reference_kernel<<<blocks_for(tokens * routes * n, 256), 256, 0, as_stream(stream)>>>(
      x, expert_indices, packed, scales, out, tokens, routes, experts, n, k, group_size);
  return check_launch("lk_w4a16_grouped_reference");
}

int lk_route_combine(const uint16_t* expert_outputs, const float* combine_weights, uint16_t* y,
                     int64_t tokens, int64_t routes, int64_t h, void* stream) {
  LK_REQUIRE(tokens >= 0 && routes > 0 && h > 0, "invalid combine dimensions");
  if (tokens == 0) return LK_OK;
  LK_REQUIRE(expert_outputs && combine_weights && y, "null pointer argument");
  route_combine_kernel<<<blocks_for(tokens * h, 256), 256, 0, as_stream(stream)>>>(
      expert_outputs, combine_weights, y, tokens, routes, h);
  return check_launch("lk_route_combine");
}

int lk_silu_mul(const uint16_t* gate, const uint16_t* up, uint16_t* out, int64_t count,
                void* stream) {
  LK_REQUIRE(count >= 0, "negative element count");
  if (count == 0) return LK_OK;
  LK_REQUIRE(gate && up && out, "null pointer argument");
  silu_mul_kernel<<<blocks_for(count, 256), 256, 0, as_stream(stream)>>>(gate, up, out, count);
  return check_launch("lk_silu_mul");
}

}  // extern "C"
