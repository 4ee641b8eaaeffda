// W4A16 GEMV kernels for decode shapes (few tokens per weight row):
// dense, grouped (one expert per token-route), fused gate/up + SwiGLU,
// the sigmoid top-k router, the fused router + gate/up decode kernel and the
// W2 projection + route combine.
//
// Work mapping (shared by every kernel here): a wave covers 8 weight rows per
// load instruction; the 8 lanes of a row read 8 consecutive 16-byte chunks
// (8 x 128 B fully used cache lines per instruction). A chunk is 32 reduction
// positions. All of a lane's weight and scale loads for the row block are
// issued before the activations are staged, so the activation staging and the
// LDS barrier hide under the HBM latency. Activations live in LDS as bf16
// pairs in the unpack order (see lk_common.hpp) plus 136 * chunk sum.
// Each lane accumulates scale * (sum x*(q+136) - 136*sum x) per chunk, and the
// 8 lanes of a row are reduced with DPP. Scales are applied per chunk, so the
// decoded weight is q * s exactly (no bf16 rounding of q * s); the tests bound
// the resulting difference from the reference rounding.

#include <stdlib.h>

#include "lk_common.hpp"

namespace lk {
namespace {

constexpr int kWave = 64;

struct XStage {
  uint4* pair;  // [(tok * 4 + j) * cpr + c]
  float* off;   // [tok * cpr + c]
  int cpr;
};

__device__ inline XStage make_stage(void* smem, int ntok, int cpr) {
  XStage st;
  st.pair = reinterpret_cast<uint4*>(smem);
  st.off = reinterpret_cast<float*>(st.pair + static_cast<size_t>(ntok) * 4 * cpr);
  st.cpr = cpr;
  return st;
}

inline size_t stage_bytes(int ntok, int cpr) {
  return static_cast<size_t>(ntok) * cpr * (4 * sizeof(uint4) + sizeof(float));
}

// Stage nt activation rows (row stride `stride` elements) into LDS.
__device__ inline void stage_x(const uint16_t* __restrict__ x, int64_t stride, int nt,
                               const XStage st) {
  const int cpr = st.cpr;
  const int units = nt * cpr * 4;
  for (int u = threadIdx.x; u < units; u += blockDim.x) {
    const int j = u & 3;
    const int rest = u >> 2;
    const int tok = rest / cpr;
    const int c = rest - tok * cpr;
    const uint4 v = *reinterpret_cast<const uint4*>(x + tok * stride + c * 32 + j * 8);
    uint32_t p[4];
    pair_x8(v, p);
    st.pair[(tok * 4 + j) * cpr + c] = make_uint4(p[0], p[1], p[2], p[3]);
    const float s = sum4(sum_x8(v));
    if (j == 0) st.off[tok * cpr + c] = kCodeOffset * s;
  }
}

// Geometry of one lane's share of a row block.
template <int NR>
struct Rows {
  int64_t row[NR];
  bool ok[NR];
  __device__ inline Rows(int64_t row_base, int64_t n) {
    const int lane = threadIdx.x & (kWave - 1);
#pragma unroll
    for (int j = 0; j < NR; ++j) {
      row[j] = row_base + (lane >> 3) + 8 * j;
      ok[j] = row[j] < n;
    }
  }
};

struct Shape {
  int64_t bytes_row;  // k / 2
  int spr;            // scales per row (k / group)
  int gshift;         // log2(group / 32)
  int cpr;            // chunks per row (k / 32)
};

__device__ inline Shape make_shape(int64_t k, int64_t group) {
  Shape s;
  s.bytes_row = k >> 1;
  s.spr = static_cast<int>(k / group);
  s.gshift = __ffs(static_cast<int>(group >> 5)) - 1;
  s.cpr = static_cast<int>(k >> 5);
  return s;
}

// Registers holding one batch of ITERS chunk columns for MATS matrices x NR rows.
template <int MATS, int NR, int ITERS>
struct Batch {
  uint4 w[MATS][NR][ITERS];
  float s[MATS][NR][ITERS];

  __device__ inline void load(const uint8_t* const (&wp)[MATS], const uint16_t* const (&ws)[MATS],
                              const Rows<NR>& rows, const Shape& sh, int cbase) {
    const int ph = threadIdx.x & 7;
#pragma unroll
    for (int it = 0; it < ITERS; ++it) {
      const int c = cbase + ph + 8 * it;
#pragma unroll
      for (int m = 0; m < MATS; ++m) {
#pragma unroll
        for (int j = 0; j < NR; ++j) {
          if (c < sh.cpr && rows.ok[j]) {
            w[m][j][it] = load_stream_u4(wp[m] + rows.row[j] * sh.bytes_row + c * 16);
            s[m][j][it] = bf16_to_f32(ws[m][rows.row[j] * sh.spr + (c >> sh.gshift)]);
          } else {
            w[m][j][it] = make_uint4(0, 0, 0, 0);
            s[m][j][it] = 0.f;
          }
        }
      }
    }
  }

  template <int NTOK>
  __device__ inline void compute(const XStage& st, int nt, int cbase,
                                 float (&part)[MATS][NR][NTOK]) const {
    const int ph = threadIdx.x & 7;
#pragma unroll
    for (int it = 0; it < ITERS; ++it) {
      const int c = cbase + ph + 8 * it;
      if (c < st.cpr) {
#pragma unroll
        for (int tok = 0; tok < NTOK; ++tok) {
          if (tok < nt) {
            uint32_t xq[4][4];
#pragma unroll
            for (int jj = 0; jj < 4; ++jj) {
              const uint4 v = st.pair[(tok * 4 + jj) * st.cpr + c];
              xq[jj][0] = v.x;
              xq[jj][1] = v.y;
              xq[jj][2] = v.z;
              xq[jj][3] = v.w;
            }
            const float xo = st.off[tok * st.cpr + c];
#pragma unroll
            for (int m = 0; m < MATS; ++m) {
#pragma unroll
              for (int j = 0; j < NR; ++j) {
                float acc = 0.f;
                acc = dot8_int4(w[m][j][it].x, xq[0], acc);
                acc = dot8_int4(w[m][j][it].y, xq[1], acc);
                acc = dot8_int4(w[m][j][it].z, xq[2], acc);
                acc = dot8_int4(w[m][j][it].w, xq[3], acc);
                part[m][j][tok] = fmaf(s[m][j][it], acc - xo, part[m][j][tok]);
              }
            }
          }
        }
      }
    }
  }
};

template <int MATS, int NR, int NTOK>
__device__ inline void zero_and(float (&part)[MATS][NR][NTOK]) {
#pragma unroll
  for (int m = 0; m < MATS; ++m)
#pragma unroll
    for (int j = 0; j < NR; ++j)
#pragma unroll
      for (int t = 0; t < NTOK; ++t) part[m][j][t] = 0.f;
}

template <int MATS, int NR, int NTOK>
__device__ inline void reduce8(float (&part)[MATS][NR][NTOK]) {
#pragma unroll
  for (int m = 0; m < MATS; ++m)
#pragma unroll
    for (int j = 0; j < NR; ++j)
#pragma unroll
      for (int t = 0; t < NTOK; ++t) part[m][j][t] = sum8(part[m][j][t]);
}

// Full GEMV for one row block: loads first, then x staging, then compute.
// `x` rows are `nt` activation rows with stride `xstride`.
template <int MATS, int NR, int NTOK, int ITERS>
__device__ inline void gemv_block(const uint8_t* const (&wp)[MATS],
                                  const uint16_t* const (&ws)[MATS], const Rows<NR>& rows,
                                  const Shape& sh, const uint16_t* __restrict__ x,
                                  int64_t xstride, int nt, const XStage& st,
                                  float (&part)[MATS][NR][NTOK]) {
  Batch<MATS, NR, ITERS> b;
  b.load(wp, ws, rows, sh, 0);
  stage_x(x, xstride, nt, st);
  __syncthreads();
  zero_and(part);
  for (int cbase = 0;;) {
    b.template compute<NTOK>(st, nt, cbase, part);
    cbase += 8 * ITERS;
    if (cbase >= sh.cpr) break;
    b.load(wp, ws, rows, sh, cbase);
  }
  reduce8(part);
}

// ---------------------------------------------------------------------------
// dense: y[m, n]

template <int NR, int NTOK, int ITERS>
__global__ void __launch_bounds__(256)
dense_gemv_kernel(const uint16_t* __restrict__ x, const uint8_t* __restrict__ packed,
                  const uint16_t* __restrict__ scales, uint16_t* __restrict__ y, int64_t m,
                  int64_t n, int64_t k, int64_t group) {
  extern __shared__ uint4 smem[];
  const Shape sh = make_shape(k, group);
  const XStage st = make_stage(smem, NTOK, sh.cpr);
  const int64_t tok0 = static_cast<int64_t>(blockIdx.y) * NTOK;
  const int nt = static_cast<int>(min<int64_t>(NTOK, m - tok0));
  const int64_t row_base =
      (static_cast<int64_t>(blockIdx.x) * (blockDim.x / kWave) + threadIdx.x / kWave) * 8 * NR;
  const Rows<NR> rows(row_base, n);
  const uint8_t* const wp[1] = {packed};
  const uint16_t* const ws[1] = {scales};
  float part[1][NR][NTOK];
  gemv_block<1, NR, NTOK, ITERS>(wp, ws, rows, sh, x + tok0 * k, k, nt, st, part);
  const int ph = threadIdx.x & 7;
#pragma unroll
  for (int j = 0; j < NR; ++j)
#pragma unroll
    for (int t = 0; t < NTOK; ++t)
      if (((j * NTOK + t) & 7) == ph && rows.ok[j] && t < nt)
        y[(tok0 + t) * n + rows.row[j]] = f32_to_bf16(part[0][j][t]);
}

// ---------------------------------------------------------------------------
// grouped (MATS=1) and fused gate/up SwiGLU (MATS=2): one token-route per
// blockIdx.y, expert from the index table.

template <int MATS, int ITERS>
__global__ void __launch_bounds__(256)
grouped_gemv_kernel(const uint16_t* __restrict__ x, const int64_t* __restrict__ idx,
                    const uint8_t* __restrict__ p0, const uint16_t* __restrict__ s0,
                    const uint8_t* __restrict__ p1, const uint16_t* __restrict__ s1,
                    uint16_t* __restrict__ out, int64_t routes, int64_t experts, int64_t n,
                    int64_t k, int64_t group) {
  extern __shared__ uint4 smem[];
  const Shape sh = make_shape(k, group);
  const XStage st = make_stage(smem, 1, sh.cpr);
  const int64_t pair = blockIdx.y;
  const int64_t t = pair / routes;
  // An index outside the bank is an empty route: it reads expert 0 (always
  // in bounds) and writes zeros, rather than reading past the bank.
  const int64_t e_raw = idx[pair];
  const bool valid = e_raw >= 0 && e_raw < experts;
  const int64_t e = valid ? e_raw : 0;
  const int64_t row_base =
      (static_cast<int64_t>(blockIdx.x) * (blockDim.x / kWave) + threadIdx.x / kWave) * 8;
  const Rows<1> rows(row_base, n);
  const int64_t wstride = n * sh.bytes_row;
  const int64_t sstride = n * sh.spr;
  float part[MATS][1][1];
  if constexpr (MATS == 1) {
    const uint8_t* const wp[1] = {p0 + e * wstride};
    const uint16_t* const ws[1] = {s0 + e * sstride};
    gemv_block<1, 1, 1, ITERS>(wp, ws, rows, sh, x + t * k, k, 1, st, part);
  } else {
    const uint8_t* const wp[2] = {p0 + e * wstride, p1 + e * wstride};
    const uint16_t* const ws[2] = {s0 + e * sstride, s1 + e * sstride};
    gemv_block<2, 1, 1, ITERS>(wp, ws, rows, sh, x + t * k, k, 1, st, part);
  }
  if ((threadIdx.x & 7) == 0 && rows.ok[0]) {
    uint16_t v;
    if constexpr (MATS == 1) v = f32_to_bf16(part[0][0][0]);
    else v = swiglu_bf16(part[0][0][0], part[1][0][0]);
    out[pair * n + rows.row[0]] = valid ? v : static_cast<uint16_t>(0);
  }
}

// ---------------------------------------------------------------------------
// sigmoid top-k router for one token, computed by one wave (all lanes).
// EPL experts per lane (lane l holds ids l*EPL .. l*EPL+EPL-1).
// Returns the expert id of selection `want` (-1 if want >= top_k). When
// idx_out is non-null, lanes < top_k write the selection and its weight.

template <int EPL>
__device__ int64_t route_token(const float* __restrict__ logits, const float* __restrict__ bias,
                               int ne, int top_k, int want, float scaling, int renorm,
                               int64_t* __restrict__ idx_out, float* __restrict__ w_out) {
  const int lane = threadIdx.x & (kWave - 1);
  float s[EPL];
  uint32_t key[EPL];
#pragma unroll
  for (int j = 0; j < EPL; ++j) {
    const int id = lane * EPL + j;
    if (id < ne) {
      const float l = logits[id];
      s[j] = 1.0f / (1.0f + expf(-l));
      const float c = s[j] + (bias ? bias[id] : 0.0f);
      key[j] = orderable(c);
    } else {
      s[j] = 0.f;
      key[j] = 0u;
    }
  }
  float ssum = 0.f;
  int64_t mine = -1;
  float my_score = 0.f;
  int64_t wanted = -1;
  for (int rr = 0; rr < top_k; ++rr) {
    uint32_t kb = 0u;
    int jb = 0;
#pragma unroll
    for (int j = 0; j < EPL; ++j)
      if (key[j] > kb) {
        kb = key[j];
        jb = j;
      }
    const uint32_t kmax = wave_max_u32(kb);
    const uint32_t cand = (kb == kmax && kb != 0u) ? static_cast<uint32_t>(lane * EPL + jb) : 0xFFFFFFFFu;
    const uint32_t sel = wave_min_u32(cand);
    const int owner = static_cast<int>(sel / EPL);
    const int slot = static_cast<int>(sel % EPL);
    float local = 0.f;
#pragma unroll
    for (int j = 0; j < EPL; ++j)
      if (j == slot) {
        local = s[j];
        if (lane == owner) key[j] = 0u;
      }
    const float score = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(local), owner));
    ssum += score;
    if (lane == rr) {
      mine = sel;
      my_score = score;
    }
    if (rr == want) wanted = sel;
  }
  if (idx_out != nullptr && lane < top_k) {
    const float denom = ssum + 1e-20f;
    idx_out[lane] = mine;
    w_out[lane] = (renorm && top_k > 1) ? (my_score / denom) * scaling : my_score * scaling;
  }
  return wanted;
}

template <int EPL>
__global__ void __launch_bounds__(64)
router_kernel(const float* __restrict__ logits, const float* __restrict__ bias,
              int64_t* __restrict__ idx, float* __restrict__ w, int64_t experts, int top_k,
              float scaling, int renorm) {
  const int64_t t = blockIdx.x;
  route_token<EPL>(logits + t * experts, bias, static_cast<int>(experts), top_k, -1, scaling,
                   renorm, idx + t * top_k, w + t * top_k);
}

// ---------------------------------------------------------------------------
// decode: router + gate/up + SwiGLU for route r of token t in one kernel.
// blockIdx.y = t * (top_k + 1) + r; route top_k is the shared expert (bank
// entry experts - 1). Each wave recomputes the token's routing (a few hundred
// instructions) instead of waiting for a separate router launch.

template <int ITERS, int EPL>
__global__ void __launch_bounds__(256)
moe_gateup_kernel(const uint16_t* __restrict__ x, const float* __restrict__ logits,
                  const float* __restrict__ bias, const uint8_t* __restrict__ w1p,
                  const uint16_t* __restrict__ w1s, const uint8_t* __restrict__ w3p,
                  const uint16_t* __restrict__ w3s, uint16_t* __restrict__ act,
                  int64_t* __restrict__ idx_out, float* __restrict__ w_out, int64_t experts,
                  int64_t h, int64_t inter, int top_k, float scaling, int renorm,
                  int64_t group) {
  extern __shared__ uint4 smem[];
  const int routes = top_k + 1;
  const int64_t pair = blockIdx.y;
  const int64_t t = pair / routes;
  const int r = static_cast<int>(pair - t * routes);
  const int ne = static_cast<int>(experts - 1);
  int64_t e;
  if (r < top_k) {
    const bool writer = (r == 0 && blockIdx.x == 0 && threadIdx.x < kWave);
    e = route_token<EPL>(logits + t * ne, bias, ne, top_k, r, scaling, renorm,
                         writer ? idx_out + t * top_k : nullptr,
                         writer ? w_out + t * top_k : nullptr);
  } else {
    e = experts - 1;
  }
  const Shape sh = make_shape(h, group);
  const XStage st = make_stage(smem, 1, sh.cpr);
  const int64_t row_base =
      (static_cast<int64_t>(blockIdx.x) * (blockDim.x / kWave) + threadIdx.x / kWave) * 8;
  const Rows<1> rows(row_base, inter);
  const int64_t wstride = inter * sh.bytes_row;
  const int64_t sstride = inter * sh.spr;
  const uint8_t* const wp[2] = {w1p + e * wstride, w3p + e * wstride};
  const uint16_t* const ws[2] = {w1s + e * sstride, w3s + e * sstride};
  float part[2][1][1];
  gemv_block<2, 1, 1, ITERS>(wp, ws, rows, sh, x + t * h, h, 1, st, part);
  if ((threadIdx.x & 7) == 0 && rows.ok[0])
    act[pair * inter + rows.row[0]] = swiglu_bf16(part[0][0][0], part[1][0][0]);
}

// ---------------------------------------------------------------------------
// W2 + combine: blockIdx.y = token, rows of H from blockIdx.x. Routes are
// processed in batches of RB with all of a batch's loads in flight at once.
// Route r's expert is idx[t * idx_stride + r]; when shared_id >= 0 the last
// route uses shared_id instead. Combine weight of route r < routes-1 is
// cw[t * cw_stride + r]; the last route is added with weight 1.

template <int ITERS, int RB>
__global__ void __launch_bounds__(256)
w2_combine_kernel(const uint16_t* __restrict__ act, const int64_t* __restrict__ idx,
                  int64_t idx_stride, int64_t shared_id, const float* __restrict__ cw,
                  int64_t cw_stride, const uint8_t* __restrict__ w2p,
                  const uint16_t* __restrict__ w2s, uint16_t* __restrict__ y, int routes,
                  int64_t experts, int64_t h, int64_t inter, int64_t group) {
  extern __shared__ uint4 smem[];
  const int64_t t = blockIdx.y;
  const Shape sh = make_shape(inter, group);
  const XStage st = make_stage(smem, routes, sh.cpr);
  const int64_t row_base =
      (static_cast<int64_t>(blockIdx.x) * (blockDim.x / kWave) + threadIdx.x / kWave) * 8;
  const Rows<1> rows(row_base, h);
  const int64_t wstride = h * sh.bytes_row;
  const int64_t sstride = h * sh.spr;
  const uint16_t* xa = act + t * routes * inter;
  // expert of route r; indices outside the bank read expert 0 and count as 0
  auto expert_of = [&](int r, bool& valid) -> int64_t {
    const int64_t e = (shared_id >= 0 && r == routes - 1) ? shared_id : idx[t * idx_stride + r];
    valid = e >= 0 && e < experts;
    return valid ? e : 0;
  };

  float routed = 0.f;
  float last = 0.f;
  bool staged = false;
  for (int rb0 = 0; rb0 < routes; rb0 += RB) {
    Batch<1, 1, ITERS> b[RB];
#pragma unroll
    for (int q = 0; q < RB; ++q) {
      const int r = rb0 + q;
      if (r < routes) {
        bool valid;
        const int64_t e = expert_of(r, valid);
        const uint8_t* const wp[1] = {w2p + e * wstride};
        const uint16_t* const ws[1] = {w2s + e * sstride};
        b[q].load(wp, ws, rows, sh, 0);
      }
    }
    if (!staged) {
      stage_x(xa, inter, routes, st);
      __syncthreads();
      staged = true;
    }
#pragma unroll
    for (int q = 0; q < RB; ++q) {
      const int r = rb0 + q;
      if (r < routes) {
        bool valid;
        const int64_t e = expert_of(r, valid);
        const uint8_t* const wp[1] = {w2p + e * wstride};
        const uint16_t* const ws[1] = {w2s + e * sstride};
        float part[1][1][1] = {{{0.f}}};
        XStage sr = st;
        sr.pair += static_cast<size_t>(r) * 4 * sh.cpr;
        sr.off += static_cast<size_t>(r) * sh.cpr;
        for (int cbase = 0;;) {
          b[q].template compute<1>(sr, 1, cbase, part);
          cbase += 8 * ITERS;
          if (cbase >= sh.cpr) break;
          b[q].load(wp, ws, rows, sh, cbase);
        }
        const float eo = valid ? round_bf16(sum8(part[0][0][0])) : 0.f;
        if (r < routes - 1) routed += eo * cw[t * cw_stride + r];
        else last = eo;
      }
    }
  }
  if ((threadIdx.x & 7) == 0 && rows.ok[0])
    y[t * h + rows.row[0]] = f32_to_bf16(round_bf16(routed) + last);
}

// ---------------------------------------------------------------------------
// host-side dispatch

int waves_per_block() {
  static int w = [] {
    const char* v = getenv("LK_GEMV_WAVES");
    int n = v ? atoi(v) : 1;
    return (n == 1 || n == 2 || n == 4) ? n : 1;
  }();
  return w;
}

int pick_iters(int cpr) {
  const int need = (cpr + 7) / 8;
  static const int kIters[] = {1, 2, 3, 4, 5, 6, 8, 9, 12, 16};
  for (int it : kIters)
    if (it >= need) return it;
  return 16;
}

#define LK_ITERS_CASES(ITERS_VAR, BODY) \
  switch (ITERS_VAR) {                  \
    case 1: { constexpr int IT = 1; BODY; } break;   \
    case 2: { constexpr int IT = 2; BODY; } break;   \
    case 3: { constexpr int IT = 3; BODY; } break;   \
    case 4: { constexpr int IT = 4; BODY; } break;   \
    case 5: { constexpr int IT = 5; BODY; } break;   \
    case 6: { constexpr int IT = 6; BODY; } break;   \
    case 8: { constexpr int IT = 8; BODY; } break;   \
    case 9: { constexpr int IT = 9; BODY; } break;   \
    case 12: { constexpr int IT = 12; BODY; } break; \
    default: { constexpr int IT = 16; BODY; } break; \
  }

int check_pow2_group(int64_t k, int64_t group) {
  if (int rc = check_group(k, group)) return rc;
  LK_REQUIRE((group & (group - 1)) == 0, "group size must be a power of two, got %lld",
             (long long)group);
  return LK_OK;
}

constexpr size_t kMaxLds = 64 * 1024;

}  // namespace
}  // namespace lk

using namespace lk;

extern "C" {

int lk_w4a16_dense(const uint16_t* x, const uint8_t* packed, const uint16_t* scales, uint16_t* y,
                   int64_t m, int64_t n, int64_t k, int64_t group_size, void* stream) {
  LK_REQUIRE(packed && scales && y, "null pointer argument");
  LK_REQUIRE(m >= 0 && n > 0, "invalid dense dimensions m=%lld n=%lld", (long long)m,
             (long long)n);
  if (int rc = check_pow2_group(k, group_size)) return rc;
  if (m == 0) return LK_OK;
  LK_REQUIRE(x != nullptr, "null activation pointer");
  const int cpr = static_cast<int>(k / 32);
  int ntok = m >= 8 ? 8 : m >= 4 ? 4 : m >= 2 ? 2 : 1;
  while (ntok > 1 && stage_bytes(ntok, cpr) > kMaxLds) ntok /= 2;
  LK_REQUIRE(stage_bytes(ntok, cpr) <= kMaxLds, "reduction width %lld too large", (long long)k);
  const int nw = waves_per_block();
  const int64_t rows_per_block = nw * 8;
  dim3 grid(static_cast<unsigned>((n + rows_per_block - 1) / rows_per_block),
            static_cast<unsigned>((m + ntok - 1) / ntok));
  const size_t lds = stage_bytes(ntok, cpr);
  hipStream_t s = as_stream(stream);
  const int iters = pick_iters(cpr);
#define LK_DENSE_LAUNCH(NT)                                                                 \
  LK_ITERS_CASES(iters, (dense_gemv_kernel<1, NT, IT><<<grid, nw * kWave, lds, s>>>(        \
                            x, packed, scales, y, m, n, k, group_size)))
  switch (ntok) {
    case 1: LK_DENSE_LAUNCH(1); break;
    case 2: LK_DENSE_LAUNCH(2); break;
    case 4: LK_DENSE_LAUNCH(4); break;
    default: LK_DENSE_LAUNCH(8); break;
  }
#undef LK_DENSE_LAUNCH
  return check_launch("lk_w4a16_dense");
}

static int grouped_common(const uint16_t* x, const int64_t* idx, const uint8_t* p0,
                          const uint16_t* s0, const uint8_t* p1, const uint16_t* s1,
                          uint16_t* out, int64_t tokens, int64_t routes, int64_t experts,
                          int64_t n, int64_t k, int64_t group, void* stream, bool swiglu,
                          const char* name) {
  LK_REQUIRE(p0 && s0 && out && (!swiglu || (p1 && s1)), "null pointer argument");
  LK_REQUIRE(routes > 0 && experts > 0 && n > 0 && tokens >= 0,
             "grouped W4A16 requires nonzero dimensions");
  if (int rc = check_pow2_group(k, group)) return rc;
  if (tokens == 0) return LK_OK;
  LK_REQUIRE(x && idx, "null pointer argument");
  const int64_t pairs = tokens * routes;
  LK_REQUIRE(pairs <= 65535, "%s: at most 65535 token-routes per call, got %lld", name,
             (long long)pairs);
  const int cpr = static_cast<int>(k / 32);
  LK_REQUIRE(stage_bytes(1, cpr) <= kMaxLds, "reduction width %lld too large", (long long)k);
  const int nw = waves_per_block();
  const int64_t rows_per_block = nw * 8;
  dim3 grid(static_cast<unsigned>((n + rows_per_block - 1) / rows_per_block),
            static_cast<unsigned>(pairs));
  const size_t lds = stage_bytes(1, cpr);
  hipStream_t s = as_stream(stream);
  const int iters = pick_iters(cpr);
  if (swiglu) {
    LK_ITERS_CASES(iters, (grouped_gemv_kernel<2, IT><<<grid, nw * kWave, lds, s>>>(
                              x, idx, p0, s0, p1, s1, out, routes, experts, n, k, group)));
  } else {
    LK_ITERS_CASES(iters, (grouped_gemv_kernel<1, IT><<<grid, nw * kWave, lds, s>>>(
                              x, idx, p0, s0, p0, s0, out, routes, experts, n, k, group)));
  }
  return check_launch(name);
}

int lk_w4a16_grouped(const uint16_t* x, const int64_t* expert_indices, const uint8_t* packed,
                     const uint16_t* scales, uint16_t* out, int64_t tokens, int64_t routes,
                     int64_t experts, int64_t n, int64_t k, int64_t group_size, void* stream) {
  return grouped_common(x, expert_indices, packed, scales, nullptr, nullptr, out, tokens, routes,
                        experts, n, k, group_size, stream, false, "lk_w4a16_grouped");
}

int lk_w4a16_swiglu(const uint16_t* x, const int64_t* expert_indices, const uint8_t* w1_packed,
                    const uint16_t* w1_scales, const uint8_t* w3_packed,
                    const uint16_t* w3_scales, uint16_t* out, int64_t tokens, int64_t routes,
                    int64_t experts, int64_t n, int64_t k, int64_t group_size, void* stream) {
  return grouped_common(x, expert_indices, w1_packed, w1_scales, w3_packed, w3_scales, out,
                        tokens, routes, experts, n, k, group_size, stream, true,
                        "lk_w4a16_swiglu");
}

static int w2_combine_launch(const uint16_t* act, const int64_t* idx, int64_t idx_stride,
                             int64_t shared_id, const float* cw, int64_t cw_stride,
                             const uint8_t* w2p, const uint16_t* w2s, uint16_t* y,
                             int64_t tokens, int64_t routes, int64_t experts, int64_t h,
                             int64_t inter, int64_t group, hipStream_t s) {
  const int cpr = static_cast<int>(inter / 32);
  LK_REQUIRE(stage_bytes(static_cast<int>(routes), cpr) <= kMaxLds,
             "routes x reduction width too large for one block (%lld x %lld)",
             (long long)routes, (long long)inter);
  LK_REQUIRE(tokens <= 65535, "at most 65535 tokens per call");
  const int nw = waves_per_block();
  const int64_t rows_per_block = nw * 8;
  dim3 grid(static_cast<unsigned>((h + rows_per_block - 1) / rows_per_block),
            static_cast<unsigned>(tokens));
  const size_t lds = stage_bytes(static_cast<int>(routes), cpr);
  const int iters = pick_iters(cpr);
  if (iters <= 4) {
    LK_ITERS_CASES(iters, (w2_combine_kernel<IT, 9><<<grid, nw * kWave, lds, s>>>(
                              act, idx, idx_stride, shared_id, cw, cw_stride, w2p, w2s, y,
                              static_cast<int>(routes), experts, h, inter, group)));
  } else {
    LK_ITERS_CASES(iters, (w2_combine_kernel<IT, 3><<<grid, nw * kWave, lds, s>>>(
                              act, idx, idx_stride, shared_id, cw, cw_stride, w2p, w2s, y,
                              static_cast<int>(routes), experts, h, inter, group)));
  }
  return check_launch("w2_combine");
}

int lk_w4a16_w2_combine(const uint16_t* activated, const int64_t* expert_indices,
                        const float* combine_weights, const uint8_t* w2_packed,
                        const uint16_t* w2_scales, uint16_t* y, int64_t tokens, int64_t routes,
                        int64_t experts, int64_t h, int64_t i, int64_t group_size,
                        void* stream) {
  LK_REQUIRE(w2_packed && w2_scales && y, "null pointer argument");
  LK_REQUIRE(routes > 0 && experts > 0 && h > 0 && tokens >= 0,
             "fused W2 combine requires nonzero route and weight dimensions");
  if (int rc = check_pow2_group(i, group_size)) return rc;
  if (tokens == 0) return LK_OK;
  LK_REQUIRE(activated && expert_indices && combine_weights, "null pointer argument");
  return w2_combine_launch(activated, expert_indices, routes, -1, combine_weights, routes,
                           w2_packed, w2_scales, y, tokens, routes, experts, h, i, group_size,
                           as_stream(stream));
}

int lk_moe_router(const float* logits, const float* bias, int64_t* expert_indices,
                  float* weights, int64_t tokens, int64_t experts, int64_t top_k,
                  float routed_scaling_factor, int renormalize, void* stream) {
  LK_REQUIRE(experts > 0 && experts <= 1024, "router supports 1..1024 experts, got %lld",
             (long long)experts);
  LK_REQUIRE(top_k > 0 && top_k <= 32 && top_k <= experts, "invalid top_k %lld",
             (long long)top_k);
  LK_REQUIRE(tokens >= 0, "negative token count");
  if (tokens == 0) return LK_OK;
  LK_REQUIRE(logits && expert_indices && weights, "null pointer argument");
  LK_REQUIRE(tokens <= 2147483647LL, "too many tokens");
  hipStream_t s = as_stream(stream);
  const int k = static_cast<int>(top_k);
  if (experts <= 256)
    router_kernel<4><<<static_cast<unsigned>(tokens), 64, 0, s>>>(
        logits, bias, expert_indices, weights, experts, k, routed_scaling_factor, renormalize);
  else
    router_kernel<16><<<static_cast<unsigned>(tokens), 64, 0, s>>>(
        logits, bias, expert_indices, weights, experts, k, routed_scaling_factor, renormalize);
  return check_launch("lk_moe_router");
}

static int moe_gateup_launch(const uint16_t* x, const float* logits, const float* bias,
                             const uint8_t* w1_packed, const uint16_t* w1_scales,
                             const uint8_t* w3_packed, const uint16_t* w3_scales,
                             int64_t* expert_indices, float* weights, uint16_t* activated,
                             int64_t tokens, int64_t experts, int64_t h, int64_t i,
                             int64_t top_k, float routed_scaling_factor, int renormalize,
                             int64_t group_size, hipStream_t s) {
  const int64_t routes = top_k + 1;
  LK_REQUIRE(tokens * routes <= 65535, "at most 65535 token-routes per call");
  const int cpr = static_cast<int>(h / 32);
  LK_REQUIRE(stage_bytes(1, cpr) <= kMaxLds, "hidden size %lld too large", (long long)h);
  const int nw = waves_per_block();
  const int64_t rows_per_block = nw * 8;
  dim3 grid(static_cast<unsigned>((i + rows_per_block - 1) / rows_per_block),
            static_cast<unsigned>(tokens * routes));
  const size_t lds = stage_bytes(1, cpr);
  const int iters = pick_iters(cpr);
  const int k = static_cast<int>(top_k);
  if (experts - 1 <= 256) {
    LK_ITERS_CASES(iters, (moe_gateup_kernel<IT, 4><<<grid, nw * kWave, lds, s>>>(
                              x, logits, bias, w1_packed, w1_scales, w3_packed, w3_scales,
                              activated, expert_indices, weights, experts, h, i, k,
                              routed_scaling_factor, renormalize, group_size)));
  } else {
    LK_ITERS_CASES(iters, (moe_gateup_kernel<IT, 16><<<grid, nw * kWave, lds, s>>>(
                              x, logits, bias, w1_packed, w1_scales, w3_packed, w3_scales,
                              activated, expert_indices, weights, experts, h, i, k,
                              routed_scaling_factor, renormalize, group_size)));
  }
  return check_launch("moe gate/up");
}

static int moe_check(const uint8_t* w1_packed, const uint16_t* w1_scales,
                     const uint8_t* w3_packed, const uint16_t* w3_scales, int64_t* expert_indices,
                     float* weights, uint16_t* activated, int64_t tokens, int64_t experts,
                     int64_t h, int64_t i, int64_t top_k, int64_t group_size) {
  LK_REQUIRE(w1_packed && w1_scales && w3_packed && w3_scales && expert_indices && weights &&
                 activated,
             "null pointer argument");
  LK_REQUIRE(experts >= 2 && experts - 1 <= 1024, "experts (routed + shared) must be 2..1025");
  LK_REQUIRE(top_k > 0 && top_k <= 32 && top_k <= experts - 1, "invalid top_k %lld",
             (long long)top_k);
  LK_REQUIRE(h > 0 && i > 0 && tokens >= 0, "invalid dimensions");
  if (int rc = check_pow2_group(h, group_size)) return rc;
  if (int rc = check_pow2_group(i, group_size)) return rc;
  return LK_OK;
}

int lk_w4a16_moe_gateup(const uint16_t* x, const float* logits, const float* bias,
                        const uint8_t* w1_packed, const uint16_t* w1_scales,
                        const uint8_t* w3_packed, const uint16_t* w3_scales,
                        int64_t* expert_indices, float* weights, uint16_t* activated,
                        int64_t tokens, int64_t experts, int64_t h, int64_t i, int64_t top_k,
                        float routed_scaling_factor, int renormalize, int64_t group_size,
                        void* stream) {
  if (int rc = moe_check(w1_packed, w1_scales, w3_packed, w3_scales, expert_indices, weights,
                         activated, tokens, experts, h, i, top_k, group_size))
    return rc;
  if (tokens == 0) return LK_OK;
  LK_REQUIRE(x && logits, "null pointer argument");
  return moe_gateup_launch(x, logits, bias, w1_packed, w1_scales, w3_packed, w3_scales,
                           expert_indices, weights, activated, tokens, experts, h, i, top_k,
                           routed_scaling_factor, renormalize, group_size, as_stream(stream));
}

int lk_w4a16_moe_decode(const uint16_t* x, const float* logits, const float* bias,
                        const uint8_t* w1_packed, const uint16_t* w1_scales,
                        const uint8_t* w3_packed, const uint16_t* w3_scales,
                        const uint8_t* w2_packed, const uint16_t* w2_scales, uint16_t* y,
                        int64_t* expert_indices, float* weights, uint16_t* activated,
                        int64_t tokens, int64_t experts, int64_t h, int64_t i, int64_t top_k,
                        float routed_scaling_factor, int renormalize, int64_t group_size,
                        void* stream) {
  if (int rc = moe_check(w1_packed, w1_scales, w3_packed, w3_scales, expert_indices, weights,
                         activated, tokens, experts, h, i, top_k, group_size))
    return rc;
  LK_REQUIRE(w2_packed && w2_scales && y, "null pointer argument");
  if (tokens == 0) return LK_OK;
  LK_REQUIRE(x && logits, "null pointer argument");
  hipStream_t s = as_stream(stream);
  if (int rc = moe_gateup_launch(x, logits, bias, w1_packed, w1_scales, w3_packed, w3_scales,
                                 expert_indices, weights, activated, tokens, experts, h, i, top_k,
                                 routed_scaling_factor, renormalize, group_size, s))
    return rc;
  return w2_combine_launch(activated, expert_indices, top_k, experts - 1, weights, top_k,
                           w2_packed, w2_scales, y, tokens, top_k + 1, experts, h, i, group_size,
                           s);
}

}  // extern "C"
