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
#include "lk_route.hpp"

namespace lk {
namespace {


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

// Write 8 activations (one dword j of chunk c of token tok) in pair order.
__device__ inline void stage_unit(const uint4 v, int tok, int c, int j, const XStage& st) {
  uint32_t p[4];
  pair_x8(v, p);
  st.pair[(tok * 4 + j) * st.cpr + c] = make_uint4(p[0], p[1], p[2], p[3]);
  const float s = sum4(sum_x8(v));  // the 4 units of a chunk sit in one lane quad
  if (j == 0) st.off[tok * st.cpr + c] = kCodeOffset * s;
}

// Activation staging in two phases so that every global load is in flight
// before the first one is used: issue() loads up to UPT 16-byte units per
// thread (addresses clamped in bounds, no branches), commit() writes them to
// LDS. Units beyond UPT * blockDim (large multi-token stagings only) are
// staged by a plain loop in commit().
template <int UPT>
struct XLoader {
  uint4 v[UPT];

  __device__ inline void issue(const uint16_t* __restrict__ x, int64_t stride, int nt,
                               int cpr) {
    const int units = nt * cpr * 4;
#pragma unroll
    for (int i = 0; i < UPT; ++i) {
      if (static_cast<int>(i * blockDim.x) < units) {  // uniform across the block
        const int u = min(static_cast<int>(threadIdx.x + i * blockDim.x), units - 1);
        const int j = u & 3;
        const int rest = u >> 2;
        const int tok = rest / cpr;
        const int c = rest - tok * cpr;
        v[i] = *reinterpret_cast<const uint4*>(x + tok * stride + c * 32 + j * 8);
      }
    }
  }

  __device__ inline void commit(const uint16_t* __restrict__ x, int64_t stride, int nt,
                                const XStage& st) const {
    const int cpr = st.cpr;
    const int units = nt * cpr * 4;
#pragma unroll
    for (int i = 0; i < UPT; ++i) {
      const int u = threadIdx.x + i * blockDim.x;
      if (u < units) {
        const int rest = u >> 2;
        const int tok = rest / cpr;
        stage_unit(v[i], tok, rest - tok * cpr, u & 3, st);
      }
    }
    for (int u = threadIdx.x + UPT * blockDim.x; u < units; u += blockDim.x) {
      const int rest = u >> 2;
      const int tok = rest / cpr;
      const int c = rest - tok * cpr;
      stage_unit(*reinterpret_cast<const uint4*>(x + tok * stride + c * 32 + (u & 3) * 8), tok,
                 c, u & 3, st);
    }
  }
};

constexpr int kUpt = 8;

// Geometry of one lane's share of a row block.
template <int NR>
struct Rows {
  int64_t row[NR];   // this lane's weight rows
  int64_t rowc[NR];  // the same, clamped into [0, n) for branch-free loads
  bool ok[NR];
  __device__ inline Rows(int64_t row_base, int64_t n) {
    const int lane = threadIdx.x & (kWave - 1);
#pragma unroll
    for (int j = 0; j < NR; ++j) {
      row[j] = row_base + (lane >> 3) + 8 * j;
      ok[j] = row[j] < n;
      rowc[j] = ok[j] ? row[j] : n - 1;
    }
  }
};

struct Shape {
  int64_t bytes_row;  // k / 2
  int spr;            // scales per row (k / group)
  int gshift;         // log2(group / 32)
  int cpr;            // chunks per row (k / 32)
};

// group is a power of two >= 32 (host-checked): shifts, not a 64-bit divide
// in every kernel's prologue ahead of its first load
__device__ inline Shape make_shape(int64_t k, int64_t group) {
  Shape s;
  s.bytes_row = k >> 1;
  s.gshift = __ffs(static_cast<int>(group >> 5)) - 1;
  s.spr = static_cast<int>(k >> (s.gshift + 5));
  s.cpr = static_cast<int>(k >> 5);
  return s;
}

// Registers holding one batch of ITERS chunk columns for MATS matrices x NR
// rows. load() issues every load of the batch without branches (addresses
// clamped in bounds) and keeps the scales as raw bf16 bits, so no load result
// is needed before the compute phase and all loads stay in flight together.
template <int MATS, int NR, int ITERS>
struct Batch {
  uint4 w[MATS][NR][ITERS];
  uint16_t s[MATS][NR][ITERS];

  __device__ inline void load(const uint8_t* const (&wp)[MATS], const uint16_t* const (&ws)[MATS],
                              const Rows<NR>& rows, const Shape& sh, int cbase) {
    const int ph = threadIdx.x & 7;
#pragma unroll
    for (int it = 0; it < ITERS; ++it) {
      const int c = min(cbase + ph + 8 * it, sh.cpr - 1);
#pragma unroll
      for (int m = 0; m < MATS; ++m) {
#pragma unroll
        for (int j = 0; j < NR; ++j) {
          w[m][j][it] = load_stream_u4(wp[m] + rows.rowc[j] * sh.bytes_row + c * 16);
          s[m][j][it] = ws[m][rows.rowc[j] * sh.spr + (c >> sh.gshift)];
        }
      }
    }
  }

  template <int NTOK>
  __device__ inline void compute(const XStage& st, int nt, int cbase, const Rows<NR>& rows,
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
                const float sc = rows.ok[j] ? bf16_to_f32(s[m][j][it]) : 0.f;
                part[m][j][tok] = fmaf(sc, acc - xo, part[m][j][tok]);
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
  XLoader<kUpt> xl;
  xl.issue(x, xstride, nt, sh.cpr);
  Batch<MATS, NR, ITERS> b;
  b.load(wp, ws, rows, sh, 0);
  xl.commit(x, xstride, nt, st);
  __syncthreads();
  zero_and(part);
  for (int cbase = 0;;) {
    b.template compute<NTOK>(st, nt, cbase, rows, part);
    cbase += 8 * ITERS;
    if (cbase >= sh.cpr) break;
    b.load(wp, ws, rows, sh, cbase);
  }
  reduce8(part);
}

// ---------------------------------------------------------------------------
// K-split GEMV core (decode shapes).
//
// A block of KW waves covers 8*NR weight rows; its waves split the reduction
// axis. Lane (rg = lane >> 3, ph = lane & 7) of wave w owns the 32-wide chunk
// columns c = w*8 + ph + 8*KW*i (i < CI) and the rows row0 + rg + 8*j (j < NR).
// Each lane loads its own activation chunk(s) straight into registers (the 8
// lanes sharing a chunk hit the same addresses, which the memory pipeline
// merges), then every weight and scale load, all before first use. Partial
// sums are reduced over the 8 chunk lanes with DPP and over the block's waves
// through LDS in fixed wave order, so results are bit-reproducible.

constexpr int kMaxKWaves = 16;

template <int MATS, int NR, int NTOK, int CI>
struct KSplit {
  uint4 xv[NTOK][CI][4];
  uint4 w[MATS][NR][CI];
  uint16_t s[MATS][NR][CI];
  float part[MATS][NR][NTOK];

  __device__ inline static int chunk(int wave, int kw, int i) {
    return wave * 8 + (threadIdx.x & 7) + 8 * kw * i;
  }

  // activation chunks of nt tokens (row stride xstride), clamped in bounds
  __device__ inline void load_x(const uint16_t* __restrict__ x, int64_t xstride, int nt,
                                int wave, int kw, int cpr) {
#pragma unroll
    for (int t = 0; t < NTOK; ++t) {
      const int tc = min(t, nt - 1);
#pragma unroll
      for (int i = 0; i < CI; ++i) {
        const int c = min(chunk(wave, kw, i), cpr - 1);
        const uint4* src = reinterpret_cast<const uint4*>(x + tc * xstride + c * 32);
#pragma unroll
        for (int q = 0; q < 4; ++q) xv[t][i][q] = src[q];
      }
    }
  }

  __device__ inline void load_w(const uint8_t* const (&wp)[MATS], const uint16_t* const (&ws)[MATS],
                                const Rows<NR>& rows, const Shape& sh, int wave, int kw) {
#pragma unroll
    for (int i = 0; i < CI; ++i) {
      const int c = min(chunk(wave, kw, i), sh.cpr - 1);
#pragma unroll
      for (int m = 0; m < MATS; ++m)
#pragma unroll
        for (int j = 0; j < NR; ++j) {
          w[m][j][i] = load_stream_u4(wp[m] + rows.rowc[j] * sh.bytes_row + c * 16);
          s[m][j][i] = ws[m][rows.rowc[j] * sh.spr + (c >> sh.gshift)];
        }
    }
  }

  __device__ inline void compute(const Rows<NR>& rows, int nt, int wave, int kw, int cpr) {
#pragma unroll
    for (int m = 0; m < MATS; ++m)
#pragma unroll
      for (int j = 0; j < NR; ++j)
#pragma unroll
        for (int t = 0; t < NTOK; ++t) part[m][j][t] = 0.f;
#pragma unroll
    for (int i = 0; i < CI; ++i) {
      const bool cval = chunk(wave, kw, i) < cpr;
#pragma unroll
      for (int t = 0; t < NTOK; ++t) {
        uint32_t xp[4][4];
        float xs = 0.f;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          pair_x8(xv[t][i][q], xp[q]);
          xs += sum_x8(xv[t][i][q]);
        }
        const float xo = kCodeOffset * xs;
#pragma unroll
        for (int m = 0; m < MATS; ++m)
#pragma unroll
          for (int j = 0; j < NR; ++j) {
            // two independent chains per chunk for more ILP
            float a0 = dot8_int4(w[m][j][i].x, xp[0], 0.f);
            float a1 = dot8_int4(w[m][j][i].y, xp[1], 0.f);
            a0 = dot8_int4(w[m][j][i].z, xp[2], a0);
            a1 = dot8_int4(w[m][j][i].w, xp[3], a1);
            const float sc = (cval && rows.ok[j] && t < nt) ? bf16_to_f32(s[m][j][i]) : 0.f;
            part[m][j][t] = fmaf(sc, (a0 + a1) - xo, part[m][j][t]);
          }
      }
    }
  }

  // DPP over the 8 chunk lanes, then LDS over the block's waves. After the
  // barrier, red[v][idx] holds wave v's partial for idx = ((m*NR + j)*NTOK + t)*8 + rg.
  __device__ inline void reduce_to_lds(float (*red)[MATS * NR * NTOK * 8], int wave) {
    const int lane = threadIdx.x & (kWave - 1);
#pragma unroll
    for (int m = 0; m < MATS; ++m)
#pragma unroll
      for (int j = 0; j < NR; ++j)
#pragma unroll
        for (int t = 0; t < NTOK; ++t) {
          const float v = sum8(part[m][j][t]);
          if ((lane & 7) == 0) red[wave][((m * NR + j) * NTOK + t) * 8 + (lane >> 3)] = v;
        }
    __syncthreads();
  }
};

// Sum of idx over the kw waves, fixed order.
template <int W>
__device__ inline float wave_total(const float (*red)[W], int kw, int idx) {
  float acc = 0.f;
  for (int v = 0; v < kw; ++v) acc += red[v][idx];
  return acc;
}

struct KGeom {
  int kw;  // waves per block along K
  int ci;  // chunks per lane
};

inline KGeom kgeom(int64_t k) {
  const int cpr = static_cast<int>(k / 32);
  KGeom g;
  g.kw = min(kMaxKWaves, (cpr + 7) / 8);
  g.ci = (cpr + 8 * g.kw - 1) / (8 * g.kw);
  return g;
}

// dense: y[tok, n] for NTOK tokens per block (blockIdx.y = token block); up
// to three matrices of one shape in one launch (blockIdx.z picks the matrix:
// the fused QKV projection at decode)
template <int NR, int NTOK, int CI, bool MULTI>
__global__ void __launch_bounds__(1024)
dense_ksplit_kernel(const uint16_t* __restrict__ x, DenseMats mats, int64_t m, int64_t n,
                    int64_t k, int64_t group) {
  __shared__ float red[kMaxKWaves][NR * NTOK * 8];
  const int kw = blockDim.x / kWave;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const Shape sh = make_shape(k, group);
  // one matrix: its pointers straight from the kernel arguments
  const int z = MULTI ? static_cast<int>(blockIdx.z) : 0;
  const int64_t tok0 = static_cast<int64_t>(blockIdx.y) * NTOK;
  const int nt = static_cast<int>(min<int64_t>(NTOK, m - tok0));
  const int64_t row0 = static_cast<int64_t>(blockIdx.x) * 8 * NR;
  const Rows<NR> rows(row0, n);
  const uint8_t* const wp[1] = {mats.packed[z]};
  const uint16_t* const ws[1] = {mats.scales[z]};
  uint16_t* __restrict__ y = mats.y[z];
  KSplit<1, NR, NTOK, CI> ks;
  ks.load_x(x + tok0 * k, k, nt, wave, kw, sh.cpr);
  ks.load_w(wp, ws, rows, sh, wave, kw);
  ks.compute(rows, nt, wave, kw, sh.cpr);
  ks.reduce_to_lds(red, wave);
  const int idx = threadIdx.x;
  if (idx < NR * NTOK * 8) {
    const int rg = idx & 7, t = (idx >> 3) % NTOK, j = (idx >> 3) / NTOK;
    const int64_t row = row0 + rg + 8 * j;
    if (t < nt && row < n) y[(tok0 + t) * n + row] = f32_to_bf16(wave_total(red, kw, idx));
  }
}

// grouped (MATS=1) / fused gate-up SwiGLU (MATS=2): blockIdx.y = token-route
template <int MATS, int NR, int CI>
__global__ void __launch_bounds__(1024)
grouped_ksplit_kernel(const uint16_t* __restrict__ x, const int64_t* __restrict__ idx,
                      const uint8_t* __restrict__ p0, const uint16_t* __restrict__ s0,
                      const uint8_t* __restrict__ p1, const uint16_t* __restrict__ s1,
                      uint16_t* __restrict__ out, int64_t routes, int64_t experts, int64_t n,
                      int64_t k, int64_t group) {
  __shared__ float red[kMaxKWaves][MATS * NR * 8];
  const int kw = blockDim.x / kWave;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const Shape sh = make_shape(k, group);
  const int64_t pair = blockIdx.y;
  const int64_t t = static_cast<uint32_t>(pair) / static_cast<uint32_t>(routes);
  KSplit<MATS, NR, 1, CI> ks;
  ks.load_x(x + t * k, k, 1, wave, kw, sh.cpr);
  // an index outside the bank is an empty route: read expert 0, write zeros
  const int64_t e_raw = idx[pair];
  const bool valid = e_raw >= 0 && e_raw < experts;
  const int64_t e = valid ? e_raw : 0;
  const int64_t row0 = static_cast<int64_t>(blockIdx.x) * 8 * NR;
  const Rows<NR> rows(row0, n);
  const int64_t wstride = n * sh.bytes_row;
  const int64_t sstride = n * sh.spr;
  if constexpr (MATS == 1) {
    const uint8_t* const wp[1] = {p0 + e * wstride};
    const uint16_t* const ws[1] = {s0 + e * sstride};
    ks.load_w(wp, ws, rows, sh, wave, kw);
  } else {
    const uint8_t* const wp[2] = {p0 + e * wstride, p1 + e * wstride};
    const uint16_t* const ws[2] = {s0 + e * sstride, s1 + e * sstride};
    ks.load_w(wp, ws, rows, sh, wave, kw);
  }
  ks.compute(rows, 1, wave, kw, sh.cpr);
  ks.reduce_to_lds(red, wave);
  const int o = threadIdx.x;
  if (o < NR * 8) {
    const int rg = o & 7, j = o >> 3;
    const int64_t row = row0 + rg + 8 * j;
    if (row < n) {
      uint16_t v;
      if constexpr (MATS == 1) {
        v = f32_to_bf16(wave_total(red, kw, j * 8 + rg));
      } else {
        v = swiglu_bf16(wave_total(red, kw, j * 8 + rg), wave_total(red, kw, (NR + j) * 8 + rg));
      }
      out[pair * n + row] = valid ? v : static_cast<uint16_t>(0);
    }
  }
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
  const int64_t t = static_cast<uint32_t>(pair) / static_cast<uint32_t>(routes);
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
// sigmoid top-k router (route_token in lk_route.hpp), one wave per token

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
// Grouped top-k router (engine/klinear/router.py:62-80), one wave per token:
// the experts split into `groups` equal groups; a group's score is the sum of
// its two largest choice scores (sigmoid + bias; the largest alone for
// one-expert groups); the topk_group best groups are kept (ties to the lower
// group) and every expert of the other groups gets choice 0.0 (a masked fill,
// not -inf: such an expert still outranks a kept one whose choice is
// negative). The top_k selection then runs on the masked choices exactly as
// the ungrouped router does (descending, ties to the lower id), and the
// weights are the unbiased sigmoid scores, summed in selection order for the
// renormalisation.
constexpr int kGroupedMaxExperts = 1024;
constexpr int kGroupedEpl = kGroupedMaxExperts / kWave;

__global__ void __launch_bounds__(kWave)
router_grouped_kernel(const float* __restrict__ logits, const float* __restrict__ bias,
                      int64_t* __restrict__ idx, float* __restrict__ w, int experts, int top_k,
                      int groups, int topk_group, float scaling, int renorm) {
  __shared__ float choice[kGroupedMaxExperts];
  __shared__ float score[kGroupedMaxExperts];
  const int lane = threadIdx.x;
  const int64_t t = blockIdx.x;
  const float* lg = logits + t * experts;
  for (int e = lane; e < experts; e += kWave) {
    const float sc = 1.0f / (1.0f + expf(-lg[e]));
    score[e] = sc;
    choice[e] = sc + (bias != nullptr ? bias[e] : 0.f);
  }
  __syncthreads();
  const int per = experts / groups;
  // one lane per group: the sum of the group's two largest choices
  uint32_t gkey = 0u;
  if (lane < groups) {
    float t1 = -INFINITY, t2 = -INFINITY;
    for (int j = 0; j < per; ++j) {
      const float v = choice[lane * per + j];
      if (v > t1) {
        t2 = t1;
        t1 = v;
      } else if (v > t2) {
        t2 = v;
      }
    }
    gkey = max(orderable(per >= 2 ? t1 + t2 : t1), 1u);  // live groups rank above lanes past them
  }
  uint64_t kept = 0;
  for (int rr = 0; rr < topk_group; ++rr) {
    const uint32_t kmax = wave_max_u32(gkey);
    const uint64_t holders = __builtin_amdgcn_ballot_w64(gkey == kmax);
    const int owner = static_cast<int>(__builtin_ctzll(holders | (1ull << 63)));
    kept |= 1ull << owner;
    if (lane == owner) gkey = 0u;
  }
  // lane l holds experts l * epl .. l * epl + epl - 1 (contiguous, so among
  // lanes holding equal keys the lowest lane holds the lowest id)
  const int epl = (experts + kWave - 1) / kWave;
  uint32_t key[kGroupedEpl];
#pragma unroll
  for (int j = 0; j < kGroupedEpl; ++j) {
    const int e = lane * epl + j;
    const bool live = j < epl && e < experts;
    const float c = live ? choice[e] : 0.f;
    key[j] = live ? max(orderable(((kept >> (e / per)) & 1ull) ? c : 0.0f), 1u) : 0u;
  }
  float ssum = 0.f, my_score = 0.f;
  int64_t mine = -1;
  for (int rr = 0; rr < top_k; ++rr) {
    uint32_t best = 0u;
    int bj = 0;
#pragma unroll
    for (int j = 0; j < kGroupedEpl; ++j) {
      if (key[j] > best) {  // strict: equal keys keep the lower id
        best = key[j];
        bj = j;
      }
    }
    const uint32_t kmax = wave_max_u32(best);
    const uint64_t holders = __builtin_amdgcn_ballot_w64(best == kmax);
    const int owner = static_cast<int>(__builtin_ctzll(holders | (1ull << 63)));
    const int j_own = __builtin_amdgcn_readlane(bj, owner);
    const int sel = min(owner * epl + j_own, experts - 1);  // top_k <= experts: always live
    const float sc = score[sel];
    if (lane == owner) {
#pragma unroll
      for (int j = 0; j < kGroupedEpl; ++j) key[j] = j == bj ? 0u : key[j];
    }
    ssum += sc;
    if (lane == rr) {
      mine = sel;
      my_score = sc;
    }
  }
  if (lane < top_k) {
    const float denom = ssum + 1e-20f;
    idx[t * top_k + lane] = mine;
    w[t * top_k + lane] = (renorm && top_k > 1) ? (my_score / denom) * scaling : my_score * scaling;
  }
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
  const int64_t t = static_cast<uint32_t>(pair) / static_cast<uint32_t>(routes);
  const int r = static_cast<int>(pair - t * routes);
  const int ne = static_cast<int>(experts - 1);
  const Shape sh = make_shape(h, group);
  const XStage st = make_stage(smem, 1, sh.cpr);
  // the token's activations do not depend on routing: load them first
  XLoader<kUpt> xl;
  xl.issue(x + t * h, h, 1, sh.cpr);
  int64_t e;
  if (r < top_k) {
    const bool writer = (r == 0 && blockIdx.x == 0 && threadIdx.x < kWave);
    e = route_token<EPL>(logits + t * ne, bias, ne, top_k, r, scaling, renorm,
                         writer ? idx_out + t * top_k : nullptr,
                         writer ? w_out + t * top_k : nullptr);
    if (e < 0 || e >= ne) e = 0;  // unreachable for top_k <= ne; keeps reads in the bank
  } else {
    e = experts - 1;
  }
  const int64_t row_base =
      (static_cast<int64_t>(blockIdx.x) * (blockDim.x / kWave) + threadIdx.x / kWave) * 8;
  const Rows<1> rows(row_base, inter);
  const int64_t wstride = inter * sh.bytes_row;
  const int64_t sstride = inter * sh.spr;
  const uint8_t* const wp[2] = {w1p + e * wstride, w3p + e * wstride};
  const uint16_t* const ws[2] = {w1s + e * sstride, w3s + e * sstride};
  Batch<2, 1, ITERS> b;
  b.load(wp, ws, rows, sh, 0);
  xl.commit(x + t * h, h, 1, st);
  __syncthreads();
  float part[2][1][1];
  zero_and(part);
  for (int cbase = 0;;) {
    b.template compute<1>(st, 1, cbase, rows, part);
    cbase += 8 * ITERS;
    if (cbase >= sh.cpr) break;
    b.load(wp, ws, rows, sh, cbase);
  }
  reduce8(part);
  if ((threadIdx.x & 7) == 0 && rows.ok[0])
    act[pair * inter + rows.row[0]] = swiglu_bf16(part[0][0][0], part[1][0][0]);
}

// decode gate/up + SwiGLU with the router, K-split form. blockIdx.y =
// t * (top_k + 1) + r; route top_k is the shared expert (bank entry
// experts - 1). Activations are loaded before routing (they do not depend on
// it); every wave recomputes the token's routing so no extra launch or block
// barrier is needed before the weight loads.
template <int NR, int CI, int EPL>
__global__ void __launch_bounds__(1024)
moe_gateup_ksplit_kernel(const uint16_t* __restrict__ x, const float* __restrict__ logits,
                         const float* __restrict__ bias, const uint8_t* __restrict__ w1p,
                         const uint16_t* __restrict__ w1s, const uint8_t* __restrict__ w3p,
                         const uint16_t* __restrict__ w3s, uint16_t* __restrict__ act,
                         int64_t* __restrict__ idx_out, float* __restrict__ w_out,
                         int64_t experts, int64_t h, int64_t inter, int top_k, float scaling,
                         int renorm, int64_t group) {
  __shared__ float red[kMaxKWaves][2 * NR * 8];
  const int kw = blockDim.x / kWave;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int routes = top_k + 1;
  const int64_t pair = blockIdx.y;
  const int64_t t = static_cast<uint32_t>(pair) / static_cast<uint32_t>(routes);
  const int r = static_cast<int>(pair - t * routes);
  const int ne = static_cast<int>(experts - 1);
  const Shape sh = make_shape(h, group);
  __shared__ int64_t routed_expert;
  // the router's logits are the first loads of the routing wave, then every
  // wave's activation chunks (they do not depend on routing)
  const bool router = r < top_k && wave == 0;  // wave-uniform
  float lg[EPL], bs[EPL];
  if (router) route_load_all<EPL>(logits + t * ne, bias, ne, lg, bs);
  KSplit<2, NR, 1, CI> ks;
  ks.load_x(x + t * h, h, 1, wave, kw, sh.cpr);
  int64_t e;
  if (r < top_k) {  // block-uniform
    if (router) {  // one wave routes; the others wait at the barrier
      const bool writer = (r == 0 && blockIdx.x == 0);
      const int64_t sel = route_select<EPL>(lg, bs, ne, top_k, r, scaling, renorm,
                                            writer ? idx_out + t * top_k : nullptr,
                                            writer ? w_out + t * top_k : nullptr, nullptr);
      if ((threadIdx.x & (kWave - 1)) == 0) routed_expert = sel;
    }
    __syncthreads();
    e = routed_expert;
    if (e < 0 || e >= ne) e = 0;  // unreachable for top_k <= ne; keeps reads in the bank
  } else {
    e = experts - 1;
  }
  const int64_t row0 = static_cast<int64_t>(blockIdx.x) * 8 * NR;
  const Rows<NR> rows(row0, inter);
  const int64_t wstride = inter * sh.bytes_row;
  const int64_t sstride = inter * sh.spr;
  const uint8_t* const wp[2] = {w1p + e * wstride, w3p + e * wstride};
  const uint16_t* const ws[2] = {w1s + e * sstride, w3s + e * sstride};
  ks.load_w(wp, ws, rows, sh, wave, kw);
  ks.compute(rows, 1, wave, kw, sh.cpr);
  ks.reduce_to_lds(red, wave);
  const int o = threadIdx.x;
  if (o < NR * 8) {
    const int rg = o & 7, j = o >> 3;
    const int64_t row = row0 + rg + 8 * j;
    if (row < inter)
      act[pair * inter + row] =
          swiglu_bf16(wave_total(red, kw, j * 8 + rg), wave_total(red, kw, (NR + j) * 8 + rg));
  }
}

// ---------------------------------------------------------------------------
// W2 + combine: blockIdx.y = token, blockIdx.x = 8 rows of H. The block's
// W waves split the routes (wave w takes routes w, w + W, ...), so each wave
// keeps at most RPW routes of weight loads in flight; all waves share the
// staged activations of every route. A wave issues its routes' loads last
// route first: the last route (the shared expert when shared_id >= 0) needs
// no expert id, so its weights are requested before the ids written by the
// gate/up kernel arrive. Route outputs are rounded to
// bf16 and combined by one wave in route order: weighted fp32 sum of routes
// 0..R-2, rounded to bf16, plus the last route (the shared expert) with
// weight 1. Route r's expert is idx[t * idx_stride + r]; when shared_id >= 0
// the last route uses shared_id. Indices outside the bank read expert 0 and
// count as 0.

constexpr int kW2Waves = 4;

template <int ITERS, int RPW, int W>
__global__ void __launch_bounds__(W * kWave)
w2_combine_kernel(const uint16_t* __restrict__ act, const int64_t* __restrict__ idx,
                  int64_t idx_stride, int64_t shared_id, const float* __restrict__ cw,
                  int64_t cw_stride, const uint8_t* __restrict__ w2p,
                  const uint16_t* __restrict__ w2s, uint16_t* __restrict__ y, int routes,
                  int64_t experts, int64_t h, int64_t inter, int64_t group) {
  extern __shared__ uint4 smem[];
  const int64_t t = blockIdx.y;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const Shape sh = make_shape(inter, group);
  const XStage st = make_stage(smem, routes, sh.cpr);
  // expert ids of this wave's routes: wave-uniform scalar loads, all issued
  // before any weight load; the shared expert's id is known without a load
  int64_t e_of[RPW];
#pragma unroll
  for (int q = 0; q < RPW; ++q) {
    const int r = min(wave + W * q, routes - 1);
    if (shared_id >= 0 && r == routes - 1)  // wave-uniform branch
      e_of[q] = shared_id;
    else
      e_of[q] = idx[t * idx_stride + r];
  }
  float* eo_lds = reinterpret_cast<float*>(st.off + static_cast<size_t>(routes) * sh.cpr);
  const uint16_t* xa = act + t * routes * inter;

  XLoader<kUpt> xl;
  xl.issue(xa, inter, routes, sh.cpr);
  // the combine weights are loaded now and parked in LDS with the activations,
  // so the final combine does not wait on global memory (routes <= 32)
  __shared__ float cw_lds[32];
  const float cw_mine =
      static_cast<int>(threadIdx.x) + 1 < routes ? cw[t * cw_stride + threadIdx.x] : 0.f;

  const int64_t row_base = static_cast<int64_t>(blockIdx.x) * 8;
  const Rows<1> rows(row_base, h);
  const int64_t wstride = h * sh.bytes_row;
  const int64_t sstride = h * sh.spr;
  Batch<1, 1, ITERS> b[RPW];
  bool valid[RPW];
#pragma unroll
  for (int q = RPW - 1; q >= 0; --q) {
    valid[q] = e_of[q] >= 0 && e_of[q] < experts;
    const int64_t e = valid[q] ? e_of[q] : 0;
    const uint8_t* const wp[1] = {w2p + e * wstride};
    const uint16_t* const ws[1] = {w2s + e * sstride};
    b[q].load(wp, ws, rows, sh, 0);
  }
  xl.commit(xa, inter, routes, st);
  if (static_cast<int>(threadIdx.x) + 1 < routes) cw_lds[threadIdx.x] = cw_mine;
  __syncthreads();

#pragma unroll
  for (int q = RPW - 1; q >= 0; --q) {  // in load order
    const int r = wave + W * q;
    if (r < routes) {  // wave-uniform
      const int64_t e = valid[q] ? e_of[q] : 0;
      const uint8_t* const wp[1] = {w2p + e * wstride};
      const uint16_t* const ws[1] = {w2s + e * sstride};
      XStage sr = st;
      sr.pair += static_cast<size_t>(r) * 4 * sh.cpr;
      sr.off += static_cast<size_t>(r) * sh.cpr;
      float part[1][1][1] = {{{0.f}}};
      for (int cbase = 0;;) {
        b[q].template compute<1>(sr, 1, cbase, rows, part);
        cbase += 8 * ITERS;
        if (cbase >= sh.cpr) break;
        b[q].load(wp, ws, rows, sh, cbase);
      }
      const float eo = valid[q] ? round_bf16(sum8(part[0][0][0])) : 0.f;
      const int lane = threadIdx.x & (kWave - 1);
      if ((lane & 7) == 0) eo_lds[r * 8 + (lane >> 3)] = eo;
    }
  }
  __syncthreads();
  if (threadIdx.x < 8) {
    const int rl = threadIdx.x;
    float routed = 0.f;
    for (int r = 0; r + 1 < routes; ++r) routed += eo_lds[r * 8 + rl] * cw_lds[r];
    const int64_t row = row_base + rl;
    if (row < h) y[t * h + row] = f32_to_bf16(round_bf16(routed) + eo_lds[(routes - 1) * 8 + rl]);
  }
}

// ---------------------------------------------------------------------------
// W2 + combine for reduction width inter = 32 chunks of 32, one block per CU:
// blockIdx.x covers rows row0 .. row0 + rb - 1 of H (the host picks
// rb = H / CUs rounded up; with 8-row blocks, 288 for H = 2304, some CUs run
// two blocks and finish last) and blockIdx.y is the token. The block's W
// waves take routes w, w + W, ... (RPW at most); the decode launch uses one
// wave per route. (The waves sharing a SIMD issue their loads later: per-wave
// timestamps show routes 4-7 and 8 finishing 0.8 and 1.5 us after routes 0-3;
// three or four waves with three or four routes each measured slower still,
// 15.9 and 16.5 against 14.65 us per decode step.) Lane (hf, c) =
// (lane >> 5, lane & 31) owns chunk c of each route's activation row, loaded
// straight into registers before the expert ids arrive (no LDS staging), and
// rows row0 + 2j + hf (j < J) of the route's expert; a wave issues its last
// route first, which is the shared expert's (no id needed) when it has it.
// A row sum is reduced over the 32 lanes of its half-wave in a fixed order;
// route outputs pass through LDS to the combine, which rounds as the other
// W2 kernels do.
constexpr int kW2RouteCpr = 32;

template <int J, int W, int RPW>
__global__ void __launch_bounds__(W * kWave)
w2_route_kernel(const uint16_t* __restrict__ act, const int64_t* __restrict__ idx,
                int64_t idx_stride, int64_t shared_id, const float* __restrict__ cw,
                int64_t cw_stride, const uint8_t* __restrict__ w2p,
                const uint16_t* __restrict__ w2s, uint16_t* __restrict__ y, int routes,
                int64_t experts, int64_t h, int64_t inter, int64_t group, int rb) {
  __shared__ float eo_lds[kMaxKWaves][2 * J];
  __shared__ float cw_lds[kMaxKWaves];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int lane = threadIdx.x & (kWave - 1);
  const int hf = lane >> 5, c = lane & 31;
  const int64_t t = blockIdx.y;
  const int64_t row0 = static_cast<int64_t>(blockIdx.x) * rb;
  const int64_t row_end = min(row0 + rb, h);
  // loads that do not depend on the expert ids go first: every route's
  // activation chunk, the combine weights
  uint4 xv[RPW][4];
#pragma unroll
  for (int q = RPW - 1; q >= 0; --q) {
    const int r = min(wave + W * q, routes - 1);
    const uint4* xs = reinterpret_cast<const uint4*>(act + (t * routes + r) * inter + c * 32);
#pragma unroll
    for (int u = 0; u < 4; ++u) xv[q][u] = xs[u];
  }
  const float cw_mine =
      static_cast<int>(threadIdx.x) + 1 < routes ? cw[t * cw_stride + threadIdx.x] : 0.f;
  const int64_t bytes_row = inter >> 1;
  const int gshift = __ffs(static_cast<int>(group >> 5)) - 1;
  const int spr = static_cast<int>(inter >> (gshift + 5));
  uint4 w[RPW][J];
  uint16_t sc[RPW][J];
  bool valid[RPW];
  bool ok[J];
  int64_t rc[J];
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int64_t row = row0 + 2 * j + hf;
    ok[j] = row < row_end;
    rc[j] = ok[j] ? row : row_end - 1;  // in bounds, branch-free
  }
#pragma unroll
  for (int q = RPW - 1; q >= 0; --q) {
    const int r = min(wave + W * q, routes - 1);
    int64_t e;
    if (shared_id >= 0 && r == routes - 1)  // wave-uniform: the shared expert needs no load
      e = shared_id;
    else
      e = idx[t * idx_stride + r];
    valid[q] = e >= 0 && e < experts;
    const int64_t ec = valid[q] ? e : 0;
    const uint8_t* wb = w2p + ec * h * bytes_row + c * 16;
    const uint16_t* sb = w2s + ec * h * spr + (c >> gshift);
#pragma unroll
    for (int j = 0; j < J; ++j) {
      w[q][j] = load_stream_u4(wb + rc[j] * bytes_row);
      sc[q][j] = sb[rc[j] * spr];
    }
  }
  if (static_cast<int>(threadIdx.x) + 1 < routes) cw_lds[threadIdx.x] = cw_mine;
#pragma unroll
  for (int q = RPW - 1; q >= 0; --q) {  // in load order
    const int r = wave + W * q;
    if (r < routes) {  // wave-uniform
      uint32_t xp[4][4];
      float xsum = 0.f;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        pair_x8(xv[q][u], xp[u]);
        xsum += sum_x8(xv[q][u]);
      }
      const float xo = kCodeOffset * xsum;
#pragma unroll
      for (int j = 0; j < J; ++j) {
        float a0 = dot8_int4(w[q][j].x, xp[0], 0.f);
        float a1 = dot8_int4(w[q][j].y, xp[1], 0.f);
        a0 = dot8_int4(w[q][j].z, xp[2], a0);
        a1 = dot8_int4(w[q][j].w, xp[3], a1);
        float v = bf16_to_f32(sc[q][j]) * ((a0 + a1) - xo);
        v = sum8(v);                    // 8 lanes
        v += dpp_f32<kRowMirror>(v);    // 16 lanes
        v += __shfl_xor(v, 16);         // the 32 lanes of the half-wave
        if (c == 0 && ok[j]) eo_lds[r][2 * j + hf] = valid[q] ? round_bf16(v) : 0.f;
      }
    }
  }
  __syncthreads();
  if (static_cast<int>(threadIdx.x) < rb) {
    const int i = threadIdx.x;
    const int64_t row = row0 + i;
    if (row < h) {
      float routed = 0.f;
      for (int q = 0; q + 1 < routes; ++q) routed += eo_lds[q][i] * cw_lds[q];
      y[t * h + row] = f32_to_bf16(round_bf16(routed) + eo_lds[routes - 1][i]);
    }
  }
}

// ---------------------------------------------------------------------------
// host-side dispatch

// The LDS-staged GEMVs (reductions wider than 8192) run one wave of 8 rows per
// block; 2 and 4 waves measured no faster.
constexpr int kGemvWaves = 1;

int device_cus() {
  static int cache[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 0;
  if (dev < 64 && cache[dev] > 0) return cache[dev];
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    return 0;
  if (dev < 64) cache[dev] = cus;
  return cus;
}

// The token-major W2 + combine kernels and the shapes each takes: the
// route-per-wave kernel for reduction width 1024 (32 chunks) and up to 16
// routes; the LDS-staged kernel for up to 8 * kW2Waves routes whose staged
// activations and route outputs fit one block's 64 KiB of LDS.
enum W2Form { kW2None = 0, kW2Route, kW2Lds };

int w2_rows_form(int64_t routes, int64_t inter) {
  if (routes <= 0 || inter <= 0 || inter % 32) return kW2None;
  const int64_t cpr = inter / 32;
  if (cpr == kW2RouteCpr && routes <= kMaxKWaves) return kW2Route;
  const int64_t lds = routes * cpr * static_cast<int64_t>(4 * sizeof(uint4) + sizeof(float)) +
                      routes * 8 * static_cast<int64_t>(sizeof(float));
  if (routes <= 8 * kW2Waves && lds <= static_cast<int64_t>(64 * 1024)) return kW2Lds;
  return kW2None;
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

constexpr size_t kMaxLds = 64 * 1024;

// ---------------------------------------------------------------------------
// Router logits (engine/klinear/router.py:50-51): logits[t, e] =
// sum_k fp32(x[t, k]) * fp32(w[e, k]) for bf16 x and a bf16 or fp32 router
// weight w (each product of a bf16 x with a bf16 w is exact in fp32). One wave
// per (expert row, tile of up to kLogitTokens tokens): lane l holds the
// 8-value chunks l, l + 64, ... of the expert's row (loaded once for the
// tile: one 16-byte load per chunk for bf16, two for fp32), and for each
// token of the tile loads the same chunks of x, sums them in chunk order, then
// the wave reduces in a fixed order (DPP within 8 lanes, then the 8 group sums
// in lane order). Every output therefore has the same summation order whatever
// the batch size, so a token's logits (and its routing) do not depend on the
// batch, and reruns are bit-identical.
constexpr int kLogitWaves = 4;
constexpr int kLogitIters = 8;   // chunks per lane: h <= 64 * 8 * 8 = 4096
constexpr int kLogitTokens = 16;  // tokens per wave (the weight row is reused)

// WORDS = 16-byte loads per 8-value weight chunk: 1 (bf16) or 2 (fp32)
template <int WORDS>
struct LogitRow {
  uint4 v[kLogitIters][WORDS];
  // value j (0..7) of chunk i as fp32
  __device__ inline float at(int i, int j) const {
    if constexpr (WORDS == 1) {
      const uint32_t b[4] = {v[i][0].x, v[i][0].y, v[i][0].z, v[i][0].w};
      return bf16_to_f32((j & 1) ? (b[j >> 1] >> 16) : (b[j >> 1] & 0xFFFFu));
    } else {
      const uint4 q = v[i][j >> 2];
      const uint32_t b[4] = {q.x, q.y, q.z, q.w};
      return __uint_as_float(b[j & 3]);
    }
  }
};

template <int WORDS>
__device__ inline float logit_dot(const uint4 (&xv)[kLogitIters], const LogitRow<WORDS>& wr,
                                  int lane, int64_t chunks) {
  // a chunk past the row keeps acc (a select, not a branch, so the loads
  // stay batched)
  float acc = 0.f;
#pragma unroll
  for (int i = 0; i < kLogitIters; ++i) {
    const bool ok = lane + kWave * i < chunks;
    const uint32_t a[4] = {xv[i].x, xv[i].y, xv[i].z, xv[i].w};
    float part = acc;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      part = fmaf(bf16_to_f32(a[j] & 0xFFFFu), wr.at(i, 2 * j), part);
      part = fmaf(bf16_to_f32(a[j] >> 16), wr.at(i, 2 * j + 1), part);
    }
    acc = ok ? part : acc;
  }
  acc = sum8(acc);
  float total = 0.f;
#pragma unroll
  for (int gidx = 0; gidx < 8; ++gidx)
    total += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(acc), gidx * 8));
  return total;
}

template <int WORDS>
__global__ void __launch_bounds__(kLogitWaves * 64)
router_logits_kernel(const uint16_t* __restrict__ x, const void* __restrict__ w,
                     float* __restrict__ logits, int64_t tokens, int64_t experts, int64_t h) {
  const int wave = static_cast<int>(threadIdx.x) / kWave;
  const int lane = static_cast<int>(threadIdx.x) & (kWave - 1);
  const int64_t e = static_cast<int64_t>(blockIdx.x) * kLogitWaves + wave;
  const int64_t t0 = static_cast<int64_t>(blockIdx.y) * kLogitTokens;
  if (e >= experts) return;  // wave-uniform
  const int64_t chunks = h / 8;
  const int nt = static_cast<int>(min<int64_t>(kLogitTokens, tokens - t0));
  const uint4* wrow = reinterpret_cast<const uint4*>(w) + e * chunks * WORDS;
  LogitRow<WORDS> wv;
  uint4 xv[kLogitIters];
  const uint4* xr = reinterpret_cast<const uint4*>(x + t0 * h);
#pragma unroll
  for (int i = 0; i < kLogitIters; ++i) {
    const int64_t c = lane + kWave * i;
    const int64_t cc = c < chunks ? c : 0;
    xv[i] = xr[cc];
#pragma unroll
    for (int q = 0; q < WORDS; ++q) wv.v[i][q] = wrow[cc * WORDS + q];
  }
  for (int t = 0; t < nt; ++t) {
    const float total = logit_dot<WORDS>(xv, wv, lane, chunks);
    if (t + 1 < nt) {  // the next token's chunks (wave-uniform)
      const uint4* xn = reinterpret_cast<const uint4*>(x + (t0 + t + 1) * h);
#pragma unroll
      for (int i = 0; i < kLogitIters; ++i) {
        const int64_t c = lane + kWave * i;
        xv[i] = xn[c < chunks ? c : 0];
      }
    }
    if (lane == 0) logits[(t0 + t) * experts + e] = total;
  }
}

}  // namespace
}  // namespace lk

using namespace lk;

extern "C" {

constexpr int kNR = 2;  // weight rows per lane in the K-split kernels

int lk_router_logits(const uint16_t* x, const void* w, float* logits, int64_t tokens,
                     int64_t experts, int64_t h, int weight_f32, void* stream) {
  LK_REQUIRE(w && logits, "null pointer argument");
  LK_REQUIRE(experts > 0 && h > 0 && tokens >= 0, "invalid router dimensions");
  LK_REQUIRE(weight_f32 == 0 || weight_f32 == 1, "weight_f32 must be 0 (bf16) or 1 (fp32)");
  LK_REQUIRE(h % 8 == 0 && h <= 64 * 8 * kLogitIters,
             "router logits need hidden %% 8 == 0 and hidden <= %d, got %lld", 64 * 8 * kLogitIters,
             (long long)h);
  const int64_t token_tiles = (tokens + kLogitTokens - 1) / kLogitTokens;
  LK_REQUIRE(token_tiles <= 65535 && experts <= 4 * 65535LL,
             "too many tokens or experts for one call");
  if (tokens == 0) return LK_OK;
  LK_REQUIRE(x != nullptr, "null activation pointer");
  dim3 grid(static_cast<unsigned>((experts + kLogitWaves - 1) / kLogitWaves),
            static_cast<unsigned>(token_tiles));
  if (weight_f32)
    router_logits_kernel<2><<<grid, kLogitWaves * kWave, 0, as_stream(stream)>>>(x, w, logits, tokens,
                                                                                experts, h);
  else
    router_logits_kernel<1><<<grid, kLogitWaves * kWave, 0, as_stream(stream)>>>(x, w, logits, tokens,
                                                                                experts, h);
  return check_launch("lk_router_logits");
}

}  // extern "C"

namespace lk {

// The K-split GEMV over `count` matrices of one shape in one launch (K <=
// 8192), or one LDS-staged launch per matrix beyond that.
int dense_multi(const uint16_t* x, const DenseMats& mats, int count, int64_t m, int64_t n,
                int64_t k, int64_t group_size, hipStream_t s, const char* name) {
  const KGeom g = kgeom(k);
  const int ntok = m >= 4 ? 4 : m >= 2 ? 2 : 1;
  LK_REQUIRE((m + ntok - 1) / ntok <= 65535, "too many tokens for one call");
  if (g.ci <= 2) {
    dim3 grid(static_cast<unsigned>((n + 8 * kNR - 1) / (8 * kNR)),
              static_cast<unsigned>((m + ntok - 1) / ntok), static_cast<unsigned>(count));
    const int threads = g.kw * kWave;
#define LK_DENSE_KS(NT, CIV)                                                                  \
  do {                                                                                         \
    if (count > 1)                                                                             \
      dense_ksplit_kernel<kNR, NT, CIV, true><<<grid, threads, 0, s>>>(x, mats, m, n, k,        \
                                                                       group_size);            \
    else                                                                                       \
      dense_ksplit_kernel<kNR, NT, CIV, false><<<grid, threads, 0, s>>>(x, mats, m, n, k,       \
                                                                        group_size);           \
  } while (0)
    if (g.ci == 1) {
      if (ntok == 1) LK_DENSE_KS(1, 1); else if (ntok == 2) LK_DENSE_KS(2, 1); else LK_DENSE_KS(4, 1);
    } else {
      if (ntok == 1) LK_DENSE_KS(1, 2); else if (ntok == 2) LK_DENSE_KS(2, 2); else LK_DENSE_KS(4, 2);
    }
#undef LK_DENSE_KS
    return check_launch(name);
  }
  // very wide reductions (K > 8192): LDS-staged kernel
  const int cpr = static_cast<int>(k / 32);
  int nt2 = m >= 8 ? 8 : m >= 4 ? 4 : m >= 2 ? 2 : 1;
  while (nt2 > 1 && stage_bytes(nt2, cpr) > kMaxLds) nt2 /= 2;
  LK_REQUIRE(stage_bytes(nt2, cpr) <= kMaxLds, "reduction width %lld too large", (long long)k);
  const int nw = kGemvWaves;
  dim3 grid(static_cast<unsigned>((n + nw * 8 - 1) / (nw * 8)),
            static_cast<unsigned>((m + nt2 - 1) / nt2));
  const size_t lds = stage_bytes(nt2, cpr);
  const int iters = pick_iters(cpr);
  for (int z = 0; z < count; ++z) {
    const uint8_t* packed = mats.packed[z];
    const uint16_t* scales = mats.scales[z];
    uint16_t* y = mats.y[z];
#define LK_DENSE_LAUNCH(NT)                                                                 \
  LK_ITERS_CASES(iters, (dense_gemv_kernel<1, NT, IT><<<grid, nw * kWave, lds, s>>>(        \
                            x, packed, scales, y, m, n, k, group_size)))
    switch (nt2) {
      case 1: LK_DENSE_LAUNCH(1); break;
      case 2: LK_DENSE_LAUNCH(2); break;
      case 4: LK_DENSE_LAUNCH(4); break;
      default: LK_DENSE_LAUNCH(8); break;
    }
#undef LK_DENSE_LAUNCH
    if (int rc = check_launch(name)) return rc;
  }
  return LK_OK;
}

}  // namespace lk

extern "C" {

int lk_w4a16_dense(const uint16_t* x, const uint8_t* packed, const uint16_t* scales, uint16_t* y,
                   int64_t m, int64_t n, int64_t k, int64_t group_size, void* stream) {
  LK_REQUIRE(packed && scales && y, "null pointer argument");
  LK_REQUIRE(m >= 0 && n > 0, "invalid dense dimensions m=%lld n=%lld", (long long)m,
             (long long)n);
  if (int rc = check_pow2_group(k, group_size)) return rc;
  if (m == 0) return LK_OK;
  LK_REQUIRE(x != nullptr, "null activation pointer");
  DenseMats mats{};
  mats.packed[0] = packed;
  mats.scales[0] = scales;
  mats.y[0] = y;
  return dense_multi(x, mats, 1, m, n, k, group_size, as_stream(stream), "lk_w4a16_dense");
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
  hipStream_t s = as_stream(stream);
  const KGeom g = kgeom(k);
  if (g.ci <= 2) {
    dim3 grid(static_cast<unsigned>((n + 8 * kNR - 1) / (8 * kNR)), static_cast<unsigned>(pairs));
    const int threads = g.kw * kWave;
#define LK_GROUPED_KS(MATS, CIV)                                                      \
  grouped_ksplit_kernel<MATS, kNR, CIV><<<grid, threads, 0, s>>>(x, idx, p0, s0,      \
      swiglu ? p1 : p0, swiglu ? s1 : s0, out, routes, experts, n, k, group)
    if (swiglu) {
      if (g.ci == 1) LK_GROUPED_KS(2, 1); else LK_GROUPED_KS(2, 2);
    } else {
      if (g.ci == 1) LK_GROUPED_KS(1, 1); else LK_GROUPED_KS(1, 2);
    }
#undef LK_GROUPED_KS
    return check_launch(name);
  }
  const int cpr = static_cast<int>(k / 32);
  LK_REQUIRE(stage_bytes(1, cpr) <= kMaxLds, "reduction width %lld too large", (long long)k);
  const int nw = kGemvWaves;
  const int64_t rows_per_block = nw * 8;
  dim3 grid(static_cast<unsigned>((n + rows_per_block - 1) / rows_per_block),
            static_cast<unsigned>(pairs));
  const size_t lds = stage_bytes(1, cpr);
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
  const int form = w2_rows_form(routes, inter);
  if (form == kW2None) return w2_rows_check(routes, h, inter);
  LK_REQUIRE(tokens <= 65535, "at most 65535 tokens per call");
  const int cpr = static_cast<int>(inter / 32);
  if (form == kW2Route) {
    // rows of H per block: one block per CU where 16 rows per block cover H
    const int cus = device_cus();
    const int64_t per_cu = cus > 0 ? (h + cus - 1) / cus : int64_t{16};
    const int rb = static_cast<int>(per_cu < 16 ? per_cu : 16);
    const int jn = (rb + 1) / 2;
    dim3 g3(static_cast<unsigned>((h + rb - 1) / rb), static_cast<unsigned>(tokens));
    const int rr = static_cast<int>(routes);
#define LK_W2_RT(JV)                                                                        \
  w2_route_kernel<JV, kMaxKWaves, 1><<<g3, rr * kWave, 0, s>>>(                            \
      act, idx, idx_stride, shared_id, cw, cw_stride, w2p, w2s, y, rr, experts, h, inter, group, rb)
    if (jn <= 1) LK_W2_RT(1);
    else if (jn <= 2) LK_W2_RT(2);
    else if (jn <= 3) LK_W2_RT(3);
    else if (jn <= 5) LK_W2_RT(5);
    else LK_W2_RT(8);
#undef LK_W2_RT
    return check_launch("w2_combine");
  }
  const size_t lds = stage_bytes(static_cast<int>(routes), cpr) + routes * 8 * sizeof(float);
  dim3 grid(static_cast<unsigned>((h + 7) / 8), static_cast<unsigned>(tokens));
  const int iters = pick_iters(cpr);
  const int r = static_cast<int>(routes);
  if (routes <= 3 * kW2Waves) {
    LK_ITERS_CASES(iters, (w2_combine_kernel<IT, 3, kW2Waves><<<grid, kW2Waves * kWave, lds, s>>>(
                              act, idx, idx_stride, shared_id, cw, cw_stride, w2p, w2s, y, r,
                              experts, h, inter, group)));
  } else {
    LK_ITERS_CASES(iters, (w2_combine_kernel<IT, 8, kW2Waves><<<grid, kW2Waves * kWave, lds, s>>>(
                              act, idx, idx_stride, shared_id, cw, cw_stride, w2p, w2s, y, r,
                              experts, h, inter, group)));
  }
  return check_launch("w2_combine");
}

}  // extern "C"

namespace lk {
int w2_rows_check(int64_t routes, int64_t h, int64_t inter) {
  LK_REQUIRE(h > 0, "invalid hidden size %lld", (long long)h);
  LK_REQUIRE(w2_rows_form(routes, inter) != kW2None,
             "token-major W2 + combine takes up to %d routes at intermediate size 1024, or up "
             "to %d routes with routes x (intermediate / 32 x 68 + 32) <= 65536 bytes; got %lld "
             "routes at intermediate size %lld",
             kMaxKWaves, 8 * kW2Waves, (long long)routes, (long long)inter);
  return LK_OK;
}

bool w2_rows_fits(int64_t routes, int64_t inter) { return w2_rows_form(routes, inter) != kW2None; }

int w2_combine_rows(const uint16_t* act, const int64_t* idx, int64_t idx_stride,
                    int64_t shared_id, const float* cw, int64_t cw_stride, const uint8_t* w2p,
                    const uint16_t* w2s, uint16_t* y, int64_t tokens, int64_t routes,
                    int64_t experts, int64_t h, int64_t inter, int64_t group, hipStream_t s) {
  return w2_combine_launch(act, idx, idx_stride, shared_id, cw, cw_stride, w2p, w2s, y, tokens,
                           routes, experts, h, inter, group, s);
}
}  // namespace lk

extern "C" {

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

int lk_moe_router_grouped(const float* logits, const float* bias, int64_t* expert_indices,
                          float* weights, int64_t tokens, int64_t experts, int64_t top_k,
                          int64_t num_expert_group, int64_t topk_group,
                          float routed_scaling_factor, int renormalize, void* stream) {
  LK_REQUIRE(experts > 0 && experts <= kGroupedMaxExperts,
             "router supports 1..%d experts, got %lld", kGroupedMaxExperts, (long long)experts);
  LK_REQUIRE(top_k > 0 && top_k <= 32 && top_k <= experts, "invalid top_k %lld",
             (long long)top_k);
  LK_REQUIRE(num_expert_group >= 1 && num_expert_group <= kWave,
             "num_expert_group must be 1..%d, got %lld", kWave, (long long)num_expert_group);
  LK_REQUIRE(experts % num_expert_group == 0,
             "num_experts must be divisible by num_expert_group");
  LK_REQUIRE(topk_group >= 1 && topk_group <= num_expert_group,
             "topk_group must be 1..num_expert_group, got %lld", (long long)topk_group);
  LK_REQUIRE(tokens >= 0, "negative token count");
  if (tokens == 0) return LK_OK;
  LK_REQUIRE(logits && expert_indices && weights, "null pointer argument");
  LK_REQUIRE(tokens <= 2147483647LL, "too many tokens");
  router_grouped_kernel<<<static_cast<unsigned>(tokens), kWave, 0, as_stream(stream)>>>(
      logits, bias, expert_indices, weights, static_cast<int>(experts), static_cast<int>(top_k),
      static_cast<int>(num_expert_group), static_cast<int>(topk_group), routed_scaling_factor,
      renormalize);
  return check_launch("lk_moe_router_grouped");
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
  const KGeom g = kgeom(h);
  if (g.ci <= 2) {
    dim3 grid(static_cast<unsigned>((i + 8 * kNR - 1) / (8 * kNR)),
              static_cast<unsigned>(tokens * routes));
    const int threads = g.kw * kWave;
    const int kk = static_cast<int>(top_k);
#define LK_MOE_KS(CIV, EPLV)                                                              \
  moe_gateup_ksplit_kernel<kNR, CIV, EPLV><<<grid, threads, 0, s>>>(                      \
      x, logits, bias, w1_packed, w1_scales, w3_packed, w3_scales, activated, expert_indices, \
      weights, experts, h, i, kk, routed_scaling_factor, renormalize, group_size)
    if (experts - 1 <= 256) {
      if (g.ci == 1) LK_MOE_KS(1, 4); else LK_MOE_KS(2, 4);
    } else {
      if (g.ci == 1) LK_MOE_KS(1, 16); else LK_MOE_KS(2, 16);
    }
#undef LK_MOE_KS
    return check_launch("moe gate/up");
  }
  const int cpr = static_cast<int>(h / 32);
  LK_REQUIRE(stage_bytes(1, cpr) <= kMaxLds, "hidden size %lld too large", (long long)h);
  const int nw = kGemvWaves;
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

int64_t lk_w4a16_moe_decode_workspace(int64_t tokens, int64_t experts, int64_t h, int64_t i,
                                      int64_t top_k) {
  if (tokens < 0 || experts < 2 || h <= 0 || i <= 0 || top_k <= 0 || top_k > 32 ||
      top_k > experts - 1)
    return -1;
  if (w2_rows_form(top_k + 1, i) == kW2None) return -1;
  return tokens * (top_k + 1) * i * static_cast<int64_t>(sizeof(uint16_t));
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
  // checked before any launch: the second stage must take this shape
  if (int rc = w2_rows_check(top_k + 1, h, i)) return rc;
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
