// Expert-major W4A16 kernels on the matrix cores (bf16 MFMA 16x16x32):
//
//  * the route schedule: a stable counting sort of the [T, R] route table by
//    expert -- counts, offsets, the permutation (sorted position -> entry
//    t * R + r, row-major within an expert) and a list of 64-row tiles. It is
//    the table form of engine/kernels/moe_grouped.py:77-95 (sorted union of
//    experts, occurrences in row-major order); routes outside [0, E) collect
//    in a last bucket whose tiles write zeros;
//  * one GEMM kernel family for every multi-token W4A16 product: grouped
//    gate/up + SwiGLU over expert tiles (rows gathered through the
//    permutation), the grouped down projection scattered back to (token,
//    route) rows, and the dense / fused-QKV GEMM;
//  * the route combine and the expert-major MoE block built from them.
//
// MFMA operand mapping (v_mfma_f32_16x16x32_bf16, wave64): lane l holds
// A[m = l%16][8(l/16) + i] and B[8(l/16) + i][n = l%16] for i = 0..7 and
// receives D[4(l/16) + i][l%16]. One packed weight dword (8 codes) unpacks
// into exactly one B operand in the (k_p, k_{p+4}) pair order of
// lk_common.hpp, and the activation fragments are staged in LDS in that
// order. Decoded weights are q + 136 (exact in bf16); every group's partial
// product comes from a fresh accumulator and is corrected and scaled once:
//   y += s_g * (sum_{k in g} x * (q + 136) - 136 * sum_{k in g} x).
// The positions of one MFMA must share a group: with G >= 128 a lane's 16
// contiguous packed bytes (32 codes) feed the 4 MFMAs of one 128-wide k-step;
// with G = 32 or 64 each MFMA covers 32 consecutive codes and a lane loads
// one dword per MFMA.

#include <stdlib.h>
#include <string.h>

#include <mutex>

#include "lk_common.hpp"
#include "lk_route.hpp"

namespace lk {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------
// route schedule

constexpr int kSchedThreads = 512;
constexpr int kSchedWaves = kSchedThreads / kWave;
constexpr int kTileRows = 64;       // rows per tile of the LDS-staged GEMM
constexpr int kSmallTileRows = 16;  // rows per tile of the streaming GEMM
constexpr int kMaxBuckets = 513;  // experts + 1 (the last bucket collects invalid routes)

struct RouteTable {
  const int64_t* idx;  // [T, kcols]
  int64_t kcols;
  int64_t routes;   // entries per token (R)
  int64_t experts;  // bank entries (E)
  int64_t shared;   // when >= 0: expert of route R - 1 (not read from idx)

  __device__ inline int bucket(int64_t entry) const {
    const int64_t t = entry / routes;
    const int64_t r = entry - t * routes;
    const int64_t e = (shared >= 0 && r == routes - 1) ? shared : idx[t * kcols + r];
    return (e >= 0 && e < experts) ? static_cast<int>(e) : static_cast<int>(experts);
  }
};

struct Schedule {
  int32_t* rank;        // [n] rank of an entry within its bucket and chunk
  int32_t* hist;        // [chunks, E + 1] entries per bucket per chunk
  int32_t* offsets;     // [E + 2] bucket starts; offsets[E + 1] = n
  int32_t* perm;        // [n] sorted position -> entry
  int32_t* tiles;       // [max_tiles, 4] (expert or -1, first row, rows, 0)
  int32_t* tile_count;  // [1]
  int tile_rows;        // rows per tile (16 or 64)
  // 64-row lists only, when non-null: the same tiles with each bucket's last
  // tile of at most 16 rows merged into the 64-row tile before it (tiles of
  // up to 80 rows), so that every entry is work for the direct-load GEMMs
  int32_t* mtiles;       // [max_tiles, 4]
  int32_t* mtile_count;  // [1]
};

// Tiles of a bucket of `cnt` entries in the merged 64-row list.
__host__ __device__ inline int merged_tiles(int cnt) {
  const int q = cnt / 64, r = cnt % 64;
  return cnt == 0 ? 0 : (q == 0 || r > 16) ? q + 1 : q;
}

__device__ inline int wave_inclusive_scan(int v) {
  const int lane = threadIdx.x & (kWave - 1);
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    const int o = __shfl_up(v, d, kWave);
    if (lane >= d) v += o;
  }
  return v;
}

// Places the entries of one chunk: tot[b] = entries of bucket b overall,
// before[b] = entries of bucket b in earlier chunks. Block 0 also writes the
// bucket offsets and the tile lists. One wave takes the three prefix sums
// over the buckets in one pass (entries, tile_rows-row tiles, merged 64-row
// tiles): one barrier before the writes instead of a scan and barriers each.
__device__ void place_chunk(int64_t n, int nb, const int* tot, const int* before, int* start,
                            int* tbefore, int* mbefore, bool valid, int64_t entry, int b,
                            int rank, const Schedule& sc) {
  const int tshift = sc.tile_rows == kTileRows ? 6 : 4;  // 64- or 16-row tiles
  if (threadIdx.x < kWave) {
    const int lane = threadIdx.x;
    const int per = (nb + kWave - 1) / kWave;
    const int b0 = min(nb, lane * per);
    const int b1 = min(nb, b0 + per);
    int se = 0, st = 0, sm = 0;
    for (int i = b0; i < b1; ++i) {
      const int c = tot[i];
      se += c;
      st += (c + (1 << tshift) - 1) >> tshift;
      sm += merged_tiles(c);
    }
    const int ie = wave_inclusive_scan(se);
    const int it = wave_inclusive_scan(st);
    const int im = wave_inclusive_scan(sm);
    int re = ie - se, rt = it - st, rm = im - sm;
    for (int i = b0; i < b1; ++i) {
      const int c = tot[i];
      start[i] = re;
      tbefore[i] = rt;
      mbefore[i] = rm;
      re += c;
      rt += (c + (1 << tshift) - 1) >> tshift;
      rm += merged_tiles(c);
    }
    if (lane == kWave - 1 && blockIdx.x == 0) {
      *sc.tile_count = it;
      if (sc.mtiles != nullptr) *sc.mtile_count = im;
    }
  }
  __syncthreads();
  if (valid) sc.perm[start[b] + before[b] + rank] = static_cast<int32_t>(entry);
  if (blockIdx.x != 0) return;
  for (int i = threadIdx.x; i < nb; i += blockDim.x) sc.offsets[i] = start[i];
  if (threadIdx.x == 0) sc.offsets[nb] = static_cast<int32_t>(n);
  const int tr = 1 << tshift;
  for (int bb = threadIdx.x; bb < nb; bb += blockDim.x) {
    const int cnt = tot[bb];
    const int expert = bb < nb - 1 ? bb : -1;
    int4* out = reinterpret_cast<int4*>(sc.tiles) + tbefore[bb];
    for (int row = 0; row < cnt; row += tr, ++out)
      *out = make_int4(expert, start[bb] + row, min(tr, cnt - row), 0);
  }
  if (sc.mtiles == nullptr) return;  // uniform over the block
  for (int bb = threadIdx.x; bb < nb; bb += blockDim.x) {
    const int cnt = tot[bb];
    const int mt = merged_tiles(cnt);
    const int expert = bb < nb - 1 ? bb : -1;
    int4* out = reinterpret_cast<int4*>(sc.mtiles) + mbefore[bb];
    for (int j = 0; j < mt; ++j)
      out[j] = make_int4(expert, start[bb] + 64 * j, j + 1 < mt ? 64 : cnt - 64 * j, 0);
  }
}

// One chunk of kSchedThreads entries per block: per-wave bitmaps of the
// lanes holding each bucket give every entry its rank among the equal
// entries before it in the chunk (stable, row-major). With a single chunk
// the placement follows in the same launch.
__global__ void __launch_bounds__(kSchedThreads)
schedule_count_kernel(const RouteTable rt, int64_t n, Schedule sc) {
  __shared__ uint32_t bits[kSchedWaves * kMaxBuckets * 2];
  __shared__ int pre[kSchedWaves * kMaxBuckets];
  __shared__ int tot[kMaxBuckets], before[kMaxBuckets], start[kMaxBuckets], mbefore[kMaxBuckets],
      tbefore[kMaxBuckets];
  const int nb = static_cast<int>(rt.experts) + 1;
  for (int i = threadIdx.x; i < kSchedWaves * nb * 2; i += kSchedThreads) bits[i] = 0u;
  __syncthreads();
  const int lane = threadIdx.x & (kWave - 1);
  const int w = threadIdx.x / kWave;
  const int64_t entry = static_cast<int64_t>(blockIdx.x) * kSchedThreads + threadIdx.x;
  const bool valid = entry < n;
  const int b = valid ? rt.bucket(entry) : 0;
  if (valid) atomicOr(&bits[(w * nb + b) * 2 + (lane >> 5)], 1u << (lane & 31));
  __syncthreads();
  for (int bb = threadIdx.x; bb < nb; bb += kSchedThreads) {
    int run = 0;
    for (int ww = 0; ww < kSchedWaves; ++ww) {
      pre[ww * nb + bb] = run;
      run += __popc(bits[(ww * nb + bb) * 2]) + __popc(bits[(ww * nb + bb) * 2 + 1]);
    }
    tot[bb] = run;
    before[bb] = 0;
    if (gridDim.x > 1) sc.hist[static_cast<int64_t>(blockIdx.x) * nb + bb] = run;
  }
  __syncthreads();
  int rank = 0;
  if (valid) {
    const uint32_t lo = bits[(w * nb + b) * 2];
    const uint32_t hi = bits[(w * nb + b) * 2 + 1];
    const int below = lane < 32 ? __popc(lo & ((1u << lane) - 1u))
                                : __popc(lo) + __popc(hi & ((1u << (lane - 32)) - 1u));
    rank = pre[w * nb + b] + below;
  }
  if (gridDim.x == 1) {
    place_chunk(n, nb, tot, before, start, tbefore, mbefore, valid, entry, b, rank, sc);
  } else if (valid) {
    sc.rank[entry] = rank;
  }
}

__global__ void __launch_bounds__(kSchedThreads)
schedule_place_kernel(const RouteTable rt, int64_t n, int chunks, Schedule sc) {
  __shared__ int tot[kMaxBuckets], before[kMaxBuckets], start[kMaxBuckets], mbefore[kMaxBuckets],
      tbefore[kMaxBuckets];
  const int nb = static_cast<int>(rt.experts) + 1;
  const int c = blockIdx.x;
  for (int bb = threadIdx.x; bb < nb; bb += kSchedThreads) {
    // the chunk histograms in batches of 16 independent loads (one at a
    // time, each waited for, was 36 round trips for 2048 tokens)
    int pre = 0, all = 0;
    for (int c0 = 0; c0 < chunks; c0 += 16) {
      int h[16];
#pragma unroll
      for (int i = 0; i < 16; ++i)
        h[i] = c0 + i < chunks ? sc.hist[static_cast<int64_t>(c0 + i) * nb + bb] : 0;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        pre += c0 + i < c ? h[i] : 0;
        all += h[i];
      }
    }
    tot[bb] = all;
    before[bb] = pre;
  }
  __syncthreads();
  const int64_t entry = static_cast<int64_t>(c) * kSchedThreads + threadIdx.x;
  const bool valid = entry < n;
  const int b = valid ? rt.bucket(entry) : 0;
  const int rank = valid ? sc.rank[entry] : 0;
  place_chunk(n, nb, tot, before, start, tbefore, mbefore, valid, entry, b, rank, sc);
}

// Schedule of up to kFuseThreads token-routes over at most 257 bank entries
// in one block and one launch (schedule_count_kernel needs a second launch
// past one chunk of kSchedThreads): the same stable ranking (an entry's rank
// among the equal entries before it), so the same tables. With ROUTE, the
// block first routes the batch (engine/klinear/router.py:47-85), one token
// per wave, writing the selections and weights to the caller's tables and the
// selections to LDS, and schedules from LDS: one launch instead of the
// router's and the schedule's. The routing then runs on one CU, one token per
// wave: 4 tokens take 7.3 us here against 9.7 us for the two launches; with
// the merged-list selection 12 tokens take 64.0-64.2 against 64.9-65.1 us per
// step and 16 tokens the same either way (73.1-73.7 against 73.3-73.4 us), so
// ROUTE serves batches of at most kFuseRouteTokens (one wave each); larger
// ones route on a grid of one block per token.
constexpr int kFuseThreads = 1024;
constexpr int kFuseWaves = kFuseThreads / kWave;
constexpr int kFuseRouteTokens = 16;
constexpr int kFuseBuckets = 258;  // 256 routed experts, the shared one, invalid routes

template <bool ROUTE>
__global__ void __launch_bounds__(kFuseThreads)
schedule_one_kernel(const RouteTable rt, int64_t n, Schedule sc, const float* __restrict__ logits,
                    const float* __restrict__ bias, int64_t* __restrict__ idx,
                    float* __restrict__ wts, int top_k, float scaling, int renorm) {
  __shared__ int32_t sel[ROUTE ? kFuseThreads : 1];  // [tokens][top_k] selections
  __shared__ uint32_t bits[kFuseWaves * kFuseBuckets * 2];
  __shared__ int pre[kFuseWaves * kFuseBuckets];
  __shared__ int tot[kFuseBuckets], before[kFuseBuckets], start[kFuseBuckets],
      mbefore[kFuseBuckets], tbefore[kFuseBuckets];
  const int lane = threadIdx.x & (kWave - 1);
  const int w = threadIdx.x / kWave;
  const int nb = static_cast<int>(rt.experts) + 1;  // bank entries and the invalid bucket
  for (int i = threadIdx.x; i < kFuseWaves * nb * 2; i += kFuseThreads) bits[i] = 0u;
  const int entry = threadIdx.x;
  const bool valid = entry < n;
  int b = 0;
  if constexpr (ROUTE) {
    // the bank's last entry is the shared expert (route top_k of every token)
    const int ne = static_cast<int>(rt.experts) - 1;
    const int tokens = static_cast<int>(n) / (top_k + 1);
    if (w < tokens)
      route_token<4>(logits + static_cast<int64_t>(w) * ne, bias, ne, top_k, -1, scaling, renorm,
                     idx + static_cast<int64_t>(w) * top_k, wts + static_cast<int64_t>(w) * top_k,
                     sel + w * top_k);
    __syncthreads();
    if (valid) {
      const int t = entry / (top_k + 1), r = entry - t * (top_k + 1);
      const int e = r == top_k ? ne : sel[t * top_k + r];
      b = (e >= 0 && e <= ne) ? e : ne + 1;
    }
  } else {
    if (valid) b = rt.bucket(entry);
    __syncthreads();
  }
  if (valid) atomicOr(&bits[(w * nb + b) * 2 + (lane >> 5)], 1u << (lane & 31));
  __syncthreads();
  for (int bb = threadIdx.x; bb < nb; bb += kFuseThreads) {
    int run = 0;
    for (int ww = 0; ww < kFuseWaves; ++ww) {
      pre[ww * nb + bb] = run;
      run += __popc(bits[(ww * nb + bb) * 2]) + __popc(bits[(ww * nb + bb) * 2 + 1]);
    }
    tot[bb] = run;
    before[bb] = 0;
  }
  __syncthreads();
  int rank = 0;
  if (valid) {
    const uint32_t lo = bits[(w * nb + b) * 2];
    const uint32_t hi = bits[(w * nb + b) * 2 + 1];
    const int below = lane < 32 ? __popc(lo & ((1u << lane) - 1u))
                                : __popc(lo) + __popc(hi & ((1u << (lane - 32)) - 1u));
    rank = pre[w * nb + b] + below;
  }
  place_chunk(n, nb, tot, before, start, tbefore, mbefore, valid, entry, b, rank, sc);
}

// ---------------------------------------------------------------------------
// W4A16 GEMM on the matrix cores

// weight format x activation type; kFmtMxF8: MXFP4 weights x activations
// split into fp8 hi + lo with per-32 E8M0 exponents (scaled fp4 MFMA)
enum : int { kFmtW4A16 = 0, kFmtMxBf16 = 1, kFmtMxF16 = 2, kFmtMxF8 = 3 };
enum : int { kActSwiglu = 0, kActSitu = 1 };                   // two-matrix epilogues

struct GemmArgs {
  const uint16_t* a;         // activations (bf16, or fp16 for kFmtMxF16), rows of k
  const uint8_t* a_hi;       // kFmtMxF8: fp8 hi codes, rows of k bytes
  const uint8_t* a_lo;       // kFmtMxF8: fp8 lo codes
  const uint16_t* a_sc;      // kFmtMxF8: per-32 exponents, byte 0 hi, byte 1 lo
  // 64-row expert-major launches with 128-wide k-steps (gate/up gather, down
  // scatter; W4A16 G = 128 or MXFP4 on bf16 MFMA) load activations into LDS
  // with direct loads: W4A16 from a_pair (rows of a with every 8-value chunk
  // in the weight decode's k order) and a_neg (-136 * sum(x) per row and
  // 128-wide group), MXFP4 from a. a_rows bounds both buffers.
  const uint16_t* a_pair;
  const float* a_neg;
  int64_t a_rows;
  // W4A16 gate/up on those launches: write the activations paired (the down
  // GEMM's a_pair) and their group sums here (its a_neg); null: plain rows
  float* out_neg;
  const int32_t* perm;       // sorted position -> entry (gather / scatter modes)
  const int32_t* tiles;      // [*, 4] tile list (schedule modes)
  const int32_t* tile_count;
  // the merged 64-row list of the same schedule (tails of <= 16 rows joined
  // to the tile before them): what the direct-load launches walk
  const int32_t* mtiles;
  const int32_t* mtile_count;
  const uint8_t* wp[3];      // packed weights per output matrix (two-matrix: gate, up)
  const void* ws[3];         // scales: bf16 (W4A16) or E8M0 bytes (MXFP4)
  uint16_t* out[3];
  int64_t n, k, group;
  int64_t wstride;           // packed bytes per expert
  int64_t sstride;           // scale elements per expert
  int64_t routes;            // entries per token (gather: token = entry / routes)
  int dense_rows;            // rows of a dense product
  int col_blocks;            // column blocks per output matrix
  int outputs;               // output matrices (3 for fused QKV, else 1)
  int act;                   // two-matrix epilogue (kActSwiglu / kActSitu)
  int tail16;                // 64-row launches: tiles of <= 16 rows take the 16-row path
  float situ_beta, situ_linear_beta;  // SiTU parameters; linear_beta <= 0: none
  // persistent gate/up launches of small batches that route and schedule the
  // batch themselves (no router or schedule launch before them): the
  // router's inputs, the outputs block 0 writes, and the batch
  const float* rt_logits;
  const float* rt_bias;
  int64_t* rt_idx;
  float* rt_w;
  int rt_tokens, rt_routed, rt_top_k, rt_renorm;
  float rt_scaling;
  // nonzero: the selections come from rt_idx (written by the router launch)
  // and the block only ranks them
  int rt_from_idx;
  // where block 0 also writes the schedule (perm, tiles, count) for a later
  // launch of the same block (the split SwiGLU's down GEMM); null: not needed
  int32_t* rt_perm_out;
  int32_t* rt_tiles_out;
  int32_t* rt_count_out;
};

template <typename T>
__device__ inline T pick3(const T (&v)[3], int i) {
  return i == 0 ? v[0] : (i == 1 ? v[1] : v[2]);
}

constexpr int kSub = 4;       // 16-row MFMA subtiles per 64-row tile
constexpr int kGemmWaves = 4;
constexpr uint32_t kOnesBf16x2 = 0x3F803F80u;  // (1.0, 1.0) in bf16

typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef int v8i32_t __attribute__((ext_vector_type(8)));

// ((w ^ 0x88888888) >> 4j) & 0x000F000F | 0x43004300 rewritten as
// ((w >> 4j) & 0x000F000F) ^ 0x43084308: every nibble of the flip is 8 and the
// flipped bit never overlaps the bf16 128.0 bits, so each output is one shift
// and one three-input bit op.
constexpr uint32_t kFlip128 = kBf16_128 | (kNibbleFlip & kPairMask);  // 0x43084308
__device__ inline bf16x8_t unpack_q8(uint32_t w) {
  const u32x4_t v = {(w & kPairMask) ^ kFlip128, ((w >> 4) & kPairMask) ^ kFlip128,
                     ((w >> 8) & kPairMask) ^ kFlip128, ((w >> 12) & kPairMask) ^ kFlip128};
  return __builtin_bit_cast(bf16x8_t, v);
}

// 2**(e - 127) as fp32 for an E8M0 byte (e = 0: the subnormal 2**-127, 255: inf)
__device__ inline float e8m0_to_f32(uint32_t e) {
  return __builtin_bit_cast(float, e == 0u ? 0x00400000u : e << 23);
}

// 8 E2M1 codes (natural order, low nibble first) times 2**(e - 127), exact in
// bf16 / fp16 within range: the gfx950 scaled convert, two codes per byte.
__device__ inline u32x4_t unpack_fp4x8_bf16(uint32_t w, float scale) {
  const u32x4_t v = {
      __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 0)),
      __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 1)),
      __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 2)),
      __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 3))};
  return v;
}
__device__ inline u32x4_t unpack_fp4x8_f16(uint32_t w, float scale) {
  const u32x4_t v = {
      __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, scale, 0)),
      __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, scale, 1)),
      __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, scale, 2)),
      __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, scale, 3))};
  return v;
}

// K3's SiTU (engine/kernels/moe_grouped.py:163-178): gate and up rounded to
// bf16 first (they are linear outputs), fp32 math, one rounding at the end.
__device__ inline uint16_t situ_bf16(float gate_acc, float up_acc, float beta, float lbeta) {
  const float g = round_bf16(gate_acc);
  float u = round_bf16(up_acc);
  const float ag = beta * tanhf(g / beta) * (1.0f / (1.0f + expf(-g)));
  if (lbeta > 0.f) u = lbeta * tanhf(u / lbeta);
  return f32_to_bf16(ag * u);
}

// fp32 sum of 8 bf16 activations: four dot2 against (1, 1), exact products
__device__ inline float sum_x8_dot(const uint4 v) {
  float s = dot2_bf16(v.x, kOnesBf16x2, 0.f);
  s = dot2_bf16(v.y, kOnesBf16x2, s);
  s = dot2_bf16(v.z, kOnesBf16x2, s);
  return dot2_bf16(v.w, kOnesBf16x2, s);
}

// ---- direct global -> LDS loads (buffer_load ... lds)
// One wave-wide load: lane L's 16 (or 4) bytes at voff + soff of the buffer
// land in LDS at lds + 16 L (4 L); lds and soff are wave-uniform. Issued from
// inline asm so that the compiler does not order LDS reads behind it: the
// caller waits for it (s_waitcnt vmcnt) before the barrier that publishes
// the LDS buffer, and the "memory" clobber keeps the loads issued after it
// in program order (which that vmcnt count relies on).
__device__ inline uint32_t lds_offset(const void* p) {
  return static_cast<uint32_t>(
      reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const char*)(p)));
}
// raw buffer descriptor of `bytes` bytes at `base` (stride 0; loads at or
// past `bytes` return zeros)
__device__ inline u32x4_t buffer_rsrc(const void* base, int64_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  const uint32_t n = bytes < 0xFFFFFFFFll ? static_cast<uint32_t>(bytes) : 0xFFFFFFFFu;
  return u32x4_t{static_cast<uint32_t>(a), static_cast<uint32_t>(a >> 32) & 0xFFFFu, n,
                 0x00020000u};
}
__device__ inline void lds_direct16(u32x4_t rs, const void* lds, uint32_t voff, uint32_t soff) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
               ::"s"(__builtin_amdgcn_readfirstlane(lds_offset(lds))), "v"(voff), "s"(rs),
                 "s"(__builtin_amdgcn_readfirstlane(soff))
               : "memory");
}
__device__ inline void lds_direct4(u32x4_t rs, const void* lds, uint32_t voff, uint32_t soff) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dword %1, %2, %3 offen lds"
               ::"s"(__builtin_amdgcn_readfirstlane(lds_offset(lds))), "v"(voff), "s"(rs),
                 "s"(__builtin_amdgcn_readfirstlane(soff))
               : "memory");
}

// Rows of bf16 activations for the direct-load W4A16 GEMM: each 8-value chunk
// in the weight decode's k order (x0 x4, x1 x5, x2 x6, x3 x7, as the
// streaming kernel stages it) and -136 * sum(x) per 128-wide group, summed
// in the staging's order: one 16-lane DPP row per (row, group), lane c on
// chunk c, so the sums are bit-identical to the in-kernel staging's.
// Unit u of the pairing (row u / (k / 128), group u % (k / 128)) by one
// 16-lane row: lane c pairs chunk c and the row sums the group (live is
// uniform over the row; a dead row loads unit 0 and stores nothing).
__device__ inline void pair_unit(const uint16_t* __restrict__ x, uint16_t* __restrict__ xp,
                                 float* __restrict__ neg, uint32_t unit, bool live) {
  const uint32_t u = live ? unit : 0u;
  const int64_t off = static_cast<int64_t>(u) * 128 + (threadIdx.x & 15) * 8;
  const uint4 v = *reinterpret_cast<const uint4*>(x + off);
  uint32_t q[4];
  pair_x8(v, q);
  float sx = sum8(sum_x8_dot(v));
  sx += dpp_f32<kRowMirror>(sx);
  if (live) {
    *reinterpret_cast<uint4*>(xp + off) = make_uint4(q[0], q[1], q[2], q[3]);
    if ((threadIdx.x & 15) == 0) neg[u] = -kCodeOffset * sx;
  }
}

__global__ void __launch_bounds__(256)
pair_rows_kernel(const uint16_t* __restrict__ x, uint16_t* __restrict__ xp,
                 float* __restrict__ neg, uint32_t units) {
  // unit = row * (k / 128) + group, so its chunk sits at 128 unit + 8 c
  const uint32_t unit = (blockIdx.x * 256u + threadIdx.x) >> 4;
  pair_unit(x, xp, neg, unit, unit < units);  // uniform over each 16-lane row
}

// The router and the activation pairing of a prefill-sized batch in one
// launch: block t routes token t in its first wave (route_token, as the
// router kernel does: engine/klinear/router.py:47-85) and pairs token t's
// k / 128 groups in its 16-lane rows (pair_unit, as pair_rows_kernel does),
// so the selections, weights and paired rows are those two launches' bits.
constexpr int kRoutePairThreads = 320;

template <int EPL>
__global__ void __launch_bounds__(kRoutePairThreads)
route_pair_kernel(const float* __restrict__ logits, const float* __restrict__ bias,
                  int64_t* __restrict__ idx, float* __restrict__ w, int experts, int top_k,
                  float scaling, int renorm, const uint16_t* __restrict__ x,
                  uint16_t* __restrict__ xp, float* __restrict__ neg, int groups) {
  const int64_t t = blockIdx.x;
  if (threadIdx.x < kWave)
    route_token<EPL>(logits + t * experts, bias, experts, top_k, -1, scaling, renorm,
                     idx + t * top_k, w + t * top_k);
  for (int gq = threadIdx.x >> 4; gq < groups; gq += kRoutePairThreads / 16)  // per 16-lane row
    pair_unit(x, xp, neg, static_cast<uint32_t>(t * groups + gq), true);
}

// Zero line read by ring reloads past the last k-step. Every wave reads the
// same line, so after its first read it stays in each CU's vector L1 (one line
// per wave spread over L2 measured 5% slower on batched decode).
__device__ __align__(256) uint8_t g_tail_pad[256];

// One 128-wide k-step of a lane's weights: 4 packed dwords (one per MFMA) and
// the scale of the group each MFMA belongs to, per matrix and column tile.
// WIDE: one 16-byte load of 32 consecutive codes; dword t feeds MFMA t. For
// W4A16 (G >= 128) the step lies in one group; for MXFP4 the 32 codes are
// exactly one E8M0 block, so one scale byte serves all four dwords.
// Otherwise each MFMA covers 32 consecutive codes (one dword per lane).
template <int FMT, int MATS, int NT, bool WIDE>
struct WeightStep {
  uint32_t w[MATS][NT][4];
  uint32_t s[MATS][NT][4];  // bf16 bits (W4A16) or E8M0 byte (MXFP4)

  // gshift = log2(group): scale indices by shifts (a runtime 64-bit divide
  // here costs ~100 scalar instructions per reload). A step past the end
  // (step >= ksteps) still issues its loads, so the loads in flight are the same
  // on every path, but reads the shared zero line instead of weights.
  __device__ inline void load(const uint8_t* const (&wrow)[MATS][NT],
                              const void* const (&srow)[MATS][NT], int step, int jq, int64_t k,
                              int gshift, int ksteps, const uint8_t* dummy) {
    const bool live = step < ksteps;
#pragma unroll
    for (int mi = 0; mi < MATS; ++mi) {
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        if constexpr (WIDE) {
          const uint8_t* wp = live ? wrow[mi][nt] + static_cast<int64_t>(step) * 64 + jq * 16 : dummy;
          const uint4 v = *reinterpret_cast<const uint4*>(wp);
          w[mi][nt][0] = v.x;
          w[mi][nt][1] = v.y;
          w[mi][nt][2] = v.z;
          w[mi][nt][3] = v.w;
          if constexpr (FMT == kFmtW4A16) {
            const uint16_t* sp = live ? static_cast<const uint16_t*>(srow[mi][nt]) +
                                            ((static_cast<int64_t>(step) * 128) >> gshift)
                                      : reinterpret_cast<const uint16_t*>(dummy);
            s[mi][nt][0] = *sp;
          } else {
            const uint8_t* sp = live ? static_cast<const uint8_t*>(srow[mi][nt]) +
                                           static_cast<int64_t>(step) * 4 + jq
                                     : dummy;
            s[mi][nt][0] = *sp;
          }
        } else {
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const int64_t k0 = static_cast<int64_t>(step) * 128 + 32 * t;
            const bool in = live && k0 < k;  // sub-steps past k are skipped
            const uint8_t* wp = in ? wrow[mi][nt] + k0 / 2 + jq * 4 : dummy;
            w[mi][nt][t] = *reinterpret_cast<const uint32_t*>(wp);
            if constexpr (FMT == kFmtW4A16) {
              const uint16_t* sp = in ? static_cast<const uint16_t*>(srow[mi][nt]) + (k0 >> gshift)
                                      : reinterpret_cast<const uint16_t*>(dummy);
              s[mi][nt][t] = *sp;
            } else {
              const uint8_t* sp = in ? static_cast<const uint8_t*>(srow[mi][nt]) + (k0 >> 5) : dummy;
              s[mi][nt][t] = *sp;
            }
          }
        }
      }
    }
  }
};

// Block = 4 waves over one 64-row tile x (64 * NT) columns; each wave owns NT
// 16-column MFMA tiles of every matrix and all active 16-row subtiles.
// Activations go through LDS (double buffered, one barrier per 128-wide
// k-step; only the tile's real rows are staged); weights go straight from HBM
// into registers two k-steps ahead.
// W4A16: a group's MFMA chain starts from C = -136 * sum(x) (staged with the
// activations), so closing the group is one FMA per output: tot += s_g * acc.
// MXFP4: the scale is applied by the decode, one chain over all of k.
template <int FMT, int MATS, int NT, bool WIDE, bool GATHER, bool SCATTER, bool DENSE>
__global__ void __launch_bounds__(kGemmWaves * kWave, 2)
w4a16_gemm_kernel(const GemmArgs g) {
  constexpr bool kMx = FMT != kFmtW4A16;
  static_assert(!(kMx && WIDE), "MXFP4 groups are 32 wide");
  constexpr int kThreads = kGemmWaves * kWave;
  constexpr int kUPT = kTileRows * 16 / kThreads;  // 16-byte activation units per thread
  constexpr int kBN = kGemmWaves * NT * 16;
  __shared__ uint4 a_lds[2][kSub * 4 * kWave];
  // W4A16: -136 * sum(x) per (row, group-in-step); WIDE: one group part per step
  __shared__ __attribute__((aligned(16))) float off_lds[2][4 * kTileRows];

  // blocks of one tile sit on one XCD (block ids are dealt round robin to the 8 XCDs)
  const int per_tile = g.col_blocks * g.outputs;
  const int id = blockIdx.x;
  const int grp = id / (8 * per_tile);
  const int rem = id - grp * 8 * per_tile;
  const int tile = grp * 8 + (rem & 7);
  const int cb_all = rem >> 3;
  const int osel = cb_all / g.col_blocks;
  const int cb = cb_all - osel * g.col_blocks;
  int expert, row0, rows;
  if constexpr (DENSE) {
    row0 = tile * kTileRows;
    if (row0 >= g.dense_rows) return;
    rows = min(kTileRows, g.dense_rows - row0);
    expert = 0;
  } else {
    if (tile >= *g.tile_count) return;
    const int4 d = reinterpret_cast<const int4*>(g.tiles)[tile];
    expert = d.x;
    row0 = d.y;
    rows = d.z;
  }
  const int64_t N = g.n, K = g.k;
  uint16_t* const out = pick3(g.out, osel);
  const int tid = threadIdx.x;
  if (expert < 0) {  // routes outside the bank produce zero rows
    for (int i = tid; i < rows * kBN; i += kThreads) {
      const int m = i / kBN;
      const int64_t col = static_cast<int64_t>(cb) * kBN + (i - m * kBN);
      if (col < N) {
        const int64_t orow = SCATTER ? g.perm[row0 + m] : row0 + m;
        out[orow * N + col] = 0;
      }
    }
    return;
  }

  const int lane = tid & (kWave - 1);
  const int wv = tid / kWave;
  const int jq = lane >> 4;
  const int ln = lane & 15;
  const int64_t rowb = K / 2;
  const int64_t spr = K / g.group;
  const int ksteps = static_cast<int>((K + 127) / 128);
  const int mt_act = (rows + 15) >> 4;
  const int cg = static_cast<int>(g.group / 32);  // narrow W4A16 groups: MFMAs per group

  const uint8_t* wrow[MATS][NT];
  const void* srow[MATS][NT];
  int64_t col[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    col[nt] = static_cast<int64_t>(cb) * kBN + (wv * NT + nt) * 16 + ln;
    const int64_t cc = col[nt] < N ? col[nt] : N - 1;
#pragma unroll
    for (int mi = 0; mi < MATS; ++mi) {
      wrow[mi][nt] = pick3(g.wp, osel + mi) + expert * g.wstride + cc * rowb;
      if constexpr (kMx)
        srow[mi][nt] = static_cast<const uint8_t*>(pick3(g.ws, osel + mi)) + expert * g.sstride +
                       cc * spr;
      else
        srow[mi][nt] = static_cast<const uint16_t*>(pick3(g.ws, osel + mi)) +
                       expert * g.sstride + cc * spr;
    }
  }

  // activation rows this thread stages (unit u: row u / 16, 8-code unit u % 16);
  // rows past the tile's end are neither loaded nor staged (their outputs are
  // never stored and MFMA rows are independent)
  const uint16_t* arow[kUPT];
  bool aok[kUPT];
#pragma unroll
  for (int i = 0; i < kUPT; ++i) {
    const int m = (tid + i * kThreads) >> 4;
    aok[i] = m < rows;
    const int mm = aok[i] ? m : 0;
    int64_t r;
    if constexpr (GATHER) r = g.perm[row0 + mm] / g.routes;
    else r = row0 + mm;
    arow[i] = g.a + r * K;
  }
  uint4 av[kUPT];
  auto load_a = [&](int step) {
#pragma unroll
    for (int i = 0; i < kUPT; ++i) {
      if (aok[i]) {
        const int c = (tid + i * kThreads) & 15;
        const int64_t k0 = static_cast<int64_t>(step) * 128 + c * 8;
        const uint4 v = *reinterpret_cast<const uint4*>(arow[i] + (k0 < K ? k0 : 0));
        const uint32_t msk = k0 < K ? 0xFFFFFFFFu : 0u;
        av[i] = make_uint4(v.x & msk, v.y & msk, v.z & msk, v.w & msk);
      }
    }
  };
  // LDS fragment (subtile ms, MFMA t) is 64 x 16 bytes read by lane l at
  // position (l/16) * 16 + ((l%16) ^ (4t + l/16)); the xor spreads one row's
  // 16 writes over distinct banks.
  auto commit_a = [&](int buf) {
#pragma unroll
    for (int i = 0; i < kUPT; ++i) {
      if (aok[i]) {  // uniform over the 16 lanes of one row (the DPP row)
        const int u = tid + i * kThreads;
        const int m = u >> 4, c = u & 15;
        const int t = WIDE ? (c & 3) : (c >> 2);
        const int j = WIDE ? (c >> 2) : (c & 3);
        uint4* dst = &a_lds[buf][((m >> 4) * 4 + t) * kWave + j * 16 + ((m & 15) ^ (4 * t + j))];
        if constexpr (kMx) {
          *dst = av[i];  // natural order: the fp4 decode keeps codes in order
        } else {
          uint32_t p[4];
          pair_x8(av[i], p);
          *dst = make_uint4(p[0], p[1], p[2], p[3]);
          float sx = sum_x8_dot(av[i]);
          if constexpr (WIDE) {
            sx = sum8(sx);
            sx += dpp_f32<kRowMirror>(sx);  // the 16 units of a row sit in one 16-lane row
            if (c == 0) off_lds[buf][m] = -kCodeOffset * sx;
          } else {
            // a group is cg consecutive sub-steps = 4 * cg consecutive units
            sx = sum4(sx);
            if (cg == 2) sx += dpp_f32<kRowHalfMirror>(sx);
            if ((c & (4 * cg - 1)) == 0)
              off_lds[buf][(t / cg) * kTileRows + m] = -kCodeOffset * sx;
          }
        }
      }
    }
  };

  f32x4_t tot[MATS][NT][kSub], acc[MATS][NT][kSub];
  const f32x4_t zero4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int mi = 0; mi < MATS; ++mi)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
      for (int ms = 0; ms < kSub; ++ms) {
        tot[mi][nt][ms] = zero4;
        acc[mi][nt][ms] = zero4;
      }

  const int gshift = __builtin_ctzll(static_cast<unsigned long long>(g.group));
  WeightStep<FMT, MATS, NT, WIDE> w0, w1, w2;
  // every reload is issued (steps past the end read a zero line), so the
  // number of loads in flight is the same on every path
  const uint8_t* const dummy = g_tail_pad;
  w0.load(wrow, srow, 0, jq, K, gshift, ksteps, dummy);
  w1.load(wrow, srow, 1, jq, K, gshift, ksteps, dummy);
  load_a(0);
  commit_a(0);
  __syncthreads();
  for (int step = 0; step < ksteps; ++step) {
    const int buf = step & 1;
    const bool more = step + 1 < ksteps;
    w2.load(wrow, srow, step + 2, jq, K, gshift, ksteps, dummy);
    if (more) load_a(step + 1);

    if constexpr (kMx) {
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        if (static_cast<int64_t>(step) * 128 + 32 * t >= K) break;
        u32x4_t af[kSub];
#pragma unroll
        for (int ms = 0; ms < kSub; ++ms)
          if (ms < mt_act) {
            const uint4 q = a_lds[buf][(ms * 4 + t) * kWave + jq * 16 + (ln ^ (4 * t + jq))];
            af[ms] = u32x4_t{q.x, q.y, q.z, q.w};
          }
#pragma unroll
        for (int mi = 0; mi < MATS; ++mi)
#pragma unroll
          for (int nt = 0; nt < NT; ++nt) {
            const float sc = e8m0_to_f32(w0.s[mi][nt][t]);
            if constexpr (FMT == kFmtMxBf16) {
              const bf16x8_t bv =
                  __builtin_bit_cast(bf16x8_t, unpack_fp4x8_bf16(w0.w[mi][nt][t], sc));
#pragma unroll
              for (int ms = 0; ms < kSub; ++ms)
                if (ms < mt_act)
                  tot[mi][nt][ms] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                      __builtin_bit_cast(bf16x8_t, af[ms]), bv, tot[mi][nt][ms], 0, 0, 0);
            } else {
              const f16x8_t bv =
                  __builtin_bit_cast(f16x8_t, unpack_fp4x8_f16(w0.w[mi][nt][t], sc));
#pragma unroll
              for (int ms = 0; ms < kSub; ++ms)
                if (ms < mt_act)
                  tot[mi][nt][ms] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                      __builtin_bit_cast(f16x8_t, af[ms]), bv, tot[mi][nt][ms], 0, 0, 0);
            }
          }
      }
    } else if constexpr (WIDE) {
      const bool first = (static_cast<int64_t>(step) * 128) % g.group == 0;
      const bool last = (static_cast<int64_t>(step + 1) * 128) % g.group == 0;
      f32x4_t neg[kSub];
#pragma unroll
      for (int ms = 0; ms < kSub; ++ms)
        neg[ms] = ms < mt_act ? *reinterpret_cast<const f32x4_t*>(&off_lds[buf][ms * 16 + jq * 4])
                              : zero4;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        bf16x8_t af[kSub];
#pragma unroll
        for (int ms = 0; ms < kSub; ++ms)
          if (ms < mt_act)
            af[ms] = __builtin_bit_cast(
                bf16x8_t, a_lds[buf][(ms * 4 + t) * kWave + jq * 16 + (ln ^ (4 * t + jq))]);
#pragma unroll
        for (int mi = 0; mi < MATS; ++mi)
#pragma unroll
          for (int nt = 0; nt < NT; ++nt) {
            const bf16x8_t bv = unpack_q8(w0.w[mi][nt][t]);
#pragma unroll
            for (int ms = 0; ms < kSub; ++ms)
              if (ms < mt_act) {
                // G > 128: later steps of a group continue its chain plus their offset
                const f32x4_t c = t > 0 ? acc[mi][nt][ms]
                                        : (first ? neg[ms] : acc[mi][nt][ms] + neg[ms]);
                acc[mi][nt][ms] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[ms], bv, c, 0, 0, 0);
              }
          }
      }
      if (last) {
#pragma unroll
        for (int mi = 0; mi < MATS; ++mi)
#pragma unroll
          for (int nt = 0; nt < NT; ++nt) {
            const float sc = bf16_to_f32(static_cast<uint16_t>(w0.s[mi][nt][0]));
#pragma unroll
            for (int ms = 0; ms < kSub; ++ms)
              if (ms < mt_act) tot[mi][nt][ms] += sc * acc[mi][nt][ms];
          }
      }
    } else {
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        if (static_cast<int64_t>(step) * 128 + 32 * t >= K) break;
        const bool first = (t % cg) == 0;
        const bool last = ((t + 1) % cg) == 0;
        bf16x8_t af[kSub];
        f32x4_t neg[kSub];
#pragma unroll
        for (int ms = 0; ms < kSub; ++ms) {
          neg[ms] = zero4;
          if (ms < mt_act) {
            af[ms] = __builtin_bit_cast(
                bf16x8_t, a_lds[buf][(ms * 4 + t) * kWave + jq * 16 + (ln ^ (4 * t + jq))]);
            if (first)
              neg[ms] = *reinterpret_cast<const f32x4_t*>(
                  &off_lds[buf][(t / cg) * kTileRows + ms * 16 + jq * 4]);
          }
        }
#pragma unroll
        for (int mi = 0; mi < MATS; ++mi)
#pragma unroll
          for (int nt = 0; nt < NT; ++nt) {
            const bf16x8_t bv = unpack_q8(w0.w[mi][nt][t]);
            const float sc = bf16_to_f32(static_cast<uint16_t>(w0.s[mi][nt][t]));
#pragma unroll
            for (int ms = 0; ms < kSub; ++ms)
              if (ms < mt_act) {
                const f32x4_t c = first ? neg[ms] : acc[mi][nt][ms];
                acc[mi][nt][ms] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[ms], bv, c, 0, 0, 0);
                if (last) tot[mi][nt][ms] += sc * acc[mi][nt][ms];
              }
          }
      }
    }
    if (more) commit_a(buf ^ 1);
    w0 = w1;
    w1 = w2;
    __syncthreads();
  }

#pragma unroll
  for (int ms = 0; ms < kSub; ++ms) {
    if (ms >= mt_act) continue;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int m = ms * 16 + jq * 4 + i;
      if (m >= rows) continue;
      const int64_t orow = SCATTER ? static_cast<int64_t>(g.perm[row0 + m]) : row0 + m;
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        if (col[nt] >= N) continue;
        uint16_t v;
        if constexpr (MATS == 2) {
          v = g.act == kActSitu
                  ? situ_bf16(tot[0][nt][ms][i], tot[1][nt][ms][i], g.situ_beta,
                              g.situ_linear_beta)
                  : swiglu_bf16(tot[0][nt][ms][i], tot[1][nt][ms][i]);
        } else if constexpr (FMT == kFmtMxF16) {
          v = __builtin_bit_cast(uint16_t, static_cast<_Float16>(tot[0][nt][ms][i]));
        } else {
          v = f32_to_bf16(tot[0][nt][ms][i]);
        }
        out[orow * N + col[nt]] = v;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Streaming GEMM over tiles of at most 16 rows (decode batches)

constexpr int kStWaves = 8;
constexpr int kStDepth = 6;                      // k-steps of weights in flight per wave
constexpr int kStMaxLds = 150 * 1024;            // LDS a streaming block may take
constexpr int kStPassSteps = 4;                  // k-steps per activation pass (64-row tiles)
constexpr int64_t kMaxDirectBytes = 0xFFFFFFFFll;  // direct-load sources: 32-bit byte offsets

template <int FMT>
__device__ inline uint16_t store_value(float v) {
  if constexpr (FMT == kFmtMxF16) return __builtin_bit_cast(uint16_t, static_cast<_Float16>(v));
  else return f32_to_bf16(v);
}

// LDS bytes of one streaming block with 16 * mt-row tiles: mt == 1 keeps all
// k-steps of the tile's activations (one buffer); mt > 1 double-buffers
// passes of kStPassSteps k-steps. Per (k-step, 16-row subtile): 4 MFMA
// fragments of 64 x 16 bytes and W4A16's -136 * sum(x) per (group, row).
inline size_t stream_lds_bytes(int64_t k, int mt) {
  const int64_t ksteps = (k + 127) / 128;
  const int64_t ps = mt == 1 ? ksteps : kStPassSteps;
  const int64_t nbuf = mt == 1 ? 1 : 2;
  return static_cast<size_t>(nbuf * ps * mt) * (4 * kWave * sizeof(uint4) + 4 * 16 * sizeof(float));
}

// s_waitcnt vmcnt(N) from inline asm (the compiler does not count the
// direct loads, so it cannot place this wait itself)
template <int N>
__device__ inline void wait_vmcnt() {
  static_assert(N >= 0 && N <= 63, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Slot swizzle of row m in the direct-load activation layout: (m & 15) with
// its two 2-bit halves swapped.
__device__ inline int row_swizzle(int m) { return ((m >> 2) & 3) | ((m & 3) << 2); }

// One tile of <= 16 * MT rows x kBN columns of a streaming block (below).
// MT = 1: all k-steps of the activations resident; MT = 4 or 5: passes of
// kStPassSteps (5: 3) k-steps, double buffered. DIRECT: activations come in by
// direct loads (see GemmArgs::a_pair).
template <int FMT, int MATS, int NT, int MT, bool WIDE, bool GATHER, bool SCATTER, bool DENSE,
          bool DIRECT = false>
__device__ __forceinline__ void stream_tile(const GemmArgs& g, const int expert, const int row0,
                                            const int rows, const int cb, const int osel) {
  constexpr bool kMx = FMT != kFmtW4A16;
  constexpr bool kF8 = FMT == kFmtMxF8;
  static_assert(!(FMT == kFmtMxF16 && WIDE), "fp16 activations use the narrow layout");
  static_assert(!kF8 || WIDE, "the scaled fp4 MFMA takes 16-byte weight loads (k % 128 == 0)");
  constexpr int kThreads = kStWaves * kWave;
  constexpr int kBN = kStWaves * NT * 16;
  constexpr int kRows = 16 * MT;
  constexpr int kNBuf = MT == 1 ? 1 : 2;
  constexpr int kPS = MT == 5 ? 3 : kStPassSteps;  // k-steps per pass (MT > 1)
  constexpr int kPassUnits = MT == 1 ? 1 : (kRows * kPS * 16 + kThreads - 1) / kThreads;
  constexpr bool kDirect = DIRECT;
  static_assert(!kDirect || (WIDE && (FMT == kFmtW4A16 || FMT == kFmtMxBf16) &&
                             (DENSE ? !GATHER && !SCATTER : GATHER != SCATTER)),
                "direct loads: 128-wide k-steps of a dense product or an expert-major gather "
                "or scatter");
  static_assert(MT == 1 || MT == 4 || (MT == 5 && kDirect), "tile heights 16, 64, direct 80");
  extern __shared__ uint4 smem[];
  __shared__ int64_t row_index[kRows];  // activation row of each tile row
  __shared__ int64_t out_row[kRows];    // output row of each tile row
  const int64_t N = g.n, K = g.k;
  uint16_t* const out = pick3(g.out, osel);
  const int tid = threadIdx.x;

  // the tile's sorted-position lookups, issued ahead of the weight loads so
  // that waiting for them never waits for weights. Direct loads fill every
  // tile row: rows past `rows` read the tile's first row (never stored).
  const int table_rows = kDirect ? kRows : rows;
  const int src_m = kDirect && tid >= rows ? 0 : tid;
  int32_t pos = 0;
  if ((GATHER || SCATTER) && tid < table_rows) pos = g.perm[row0 + src_m];
  const int lane = tid & (kWave - 1);
  const int wv = tid / kWave;
  const int jq = lane >> 4;
  const int ln = lane & 15;
  const int64_t rowb = K / 2;
  const int64_t spr = K / g.group;
  const int ksteps = static_cast<int>((K + 127) / 128);
  const int ps = MT == 1 ? ksteps : kPS;  // k-steps per pass
  const int cg = static_cast<int>(g.group / 32);
  const int mt_act = (rows + 15) >> 4;
  uint4* const afrag = smem;  // [kNBuf][ps][MT][4][64]
  float* const offs = reinterpret_cast<float*>(smem + kNBuf * ps * MT * 4 * kWave);  // [kNBuf][ps][MT][4][16]

  // 1. this wave's first kStDepth k-steps of weights
  const uint8_t* wrow[MATS][NT];
  const void* srow[MATS][NT];
  int64_t col[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    col[nt] = static_cast<int64_t>(cb) * kBN + (wv * NT + nt) * 16 + ln;
    const int64_t cc = col[nt] < N ? col[nt] : N - 1;
#pragma unroll
    for (int mi = 0; mi < MATS; ++mi) {
      wrow[mi][nt] = pick3(g.wp, osel + mi) + expert * g.wstride + cc * rowb;
      if constexpr (kMx)
        srow[mi][nt] = static_cast<const uint8_t*>(pick3(g.ws, osel + mi)) + expert * g.sstride +
                       cc * spr;
      else
        srow[mi][nt] = static_cast<const uint16_t*>(pick3(g.ws, osel + mi)) +
                       expert * g.sstride + cc * spr;
    }
  }
  constexpr int kRing = MT == 1 ? kStDepth : kPS;
  const int gshift = __builtin_ctzll(static_cast<unsigned long long>(g.group));
  WeightStep<FMT, MATS, NT, WIDE> w[kRing];
  // every ring slot is refilled unconditionally (steps past the end read a
  // zero line): the loads in flight are then the same on every path and the
  // compiler waits only for the slot it needs, not for the whole ring
  const uint8_t* const dummy = g_tail_pad;
  // 16-row tiles issue the ring now; 64-row tiles issue it after the first
  // pass's activation loads (below), which then do not wait behind it
  if constexpr (MT == 1) {
#pragma unroll
    for (int j = 0; j < kRing; ++j) w[j].load(wrow, srow, j, jq, K, gshift, ksteps, dummy);
  }

  // 2. the tile's activation and output rows (one lookup per row, shared
  // through LDS; the epilogue then reads no global memory)
  if (tid < table_rows) {
    row_index[tid] = GATHER ? static_cast<int64_t>(pos / g.routes) : row0 + src_m;
    out_row[tid] = SCATTER ? static_cast<int64_t>(pos) : row0 + tid;
  }
  __syncthreads();

  // unit u of a pass: ((local step * kRows) + row slot m) * 16 + c, so the 16
  // units of one (row, step) sit in one 16-lane DPP row; slots m >= rows are
  // skipped (their MFMA rows are never stored)
  constexpr int kRowShift = MT == 1 ? 4 : 6;
  static_assert(kDirect || kRows == (1 << kRowShift), "staged tiles have 16 or 64 rows");
  auto unit_live = [&](int u) { return ((u >> 4) & (kRows - 1)) < rows; };
  // kFmtMxF8: unit c < 8 is 16 fp8 hi codes (k = 16c..16c+15 of the step),
  // c >= 8 the lo codes of chunk c - 8; units c < 4 also carry the row's
  // exponent word of 32-block c. MFMA lane (row, kb) takes k = 16kb.. and
  // 64 + 16kb.. of hi (slots t = 0, 1) and of lo (t = 2, 3), and the exponent
  // word of block kb (byte 0 hi, byte 1 lo).
  auto unit_load = [&](int p, int u) -> uint4 {
    const int c = u & 15;
    const int m = (u >> 4) & (kRows - 1);
    const int ls = u >> (4 + kRowShift);
    if constexpr (kF8) {
      const int64_t k0 = static_cast<int64_t>(p * ps + ls) * 128 + (c & 7) * 16;  // k % 128 == 0
      return *reinterpret_cast<const uint4*>((c < 8 ? g.a_hi : g.a_lo) + row_index[m] * K + k0);
    }
    const int64_t k0 = static_cast<int64_t>(p * ps + ls) * 128 + c * 8;
    uint4 v = *reinterpret_cast<const uint4*>(g.a + row_index[m] * K + (k0 < K ? k0 : 0));
    if (k0 >= K) v = make_uint4(0u, 0u, 0u, 0u);
    return v;
  };
  auto unit_scale = [&](int p, int u) -> uint32_t {  // kFmtMxF8 units c < 4 only
    const int c = u & 15;
    const int m = (u >> 4) & (kRows - 1);
    const int ls = u >> (4 + kRowShift);
    if (!kF8 || c >= 4) return 0u;
    return g.a_sc[row_index[m] * (K / 32) + static_cast<int64_t>(p * ps + ls) * 4 + c];
  };
  auto unit_store = [&](int b, int u, const uint4 v, uint32_t sv) {  // uniform per 16-lane row
    const int c = u & 15;
    const int m = (u >> 4) & (kRows - 1);
    const int ls = u >> (4 + kRowShift);
    const int ms = m >> 4, mr = m & 15;
    const int frag = ((b * ps + ls) * MT + ms) * 4;
    if constexpr (kF8) {
      const int kb = c & 3;
      const int t = (c >> 2);  // 0, 1: hi halves; 2, 3: lo halves
      afrag[(frag + t) * kWave + kb * 16 + (mr ^ (4 * t + kb))] = v;
      if (c < 4) reinterpret_cast<uint32_t*>(offs)[(frag + c) * 16 + mr] = sv;
      return;
    }
    (void)sv;
    const int t = WIDE ? (c & 3) : (c >> 2);
    const int j = WIDE ? (c >> 2) : (c & 3);
    uint4* dst = &afrag[(frag + t) * kWave + j * 16 + (mr ^ (4 * t + j))];
    if constexpr (kMx) {
      *dst = v;
    } else {
      uint32_t q[4];
      pair_x8(v, q);
      *dst = make_uint4(q[0], q[1], q[2], q[3]);
      float sx = sum_x8_dot(v);
      if constexpr (WIDE) {
        sx = sum8(sx);
        sx += dpp_f32<kRowMirror>(sx);
        if (c == 0) offs[frag * 16 + mr] = -kCodeOffset * sx;
      } else {
        sx = sum4(sx);
        if (cg == 2) sx += dpp_f32<kRowHalfMirror>(sx);
        if ((c & (4 * cg - 1)) == 0) offs[(frag + t / cg) * 16 + mr] = -kCodeOffset * sx;
      }
    }
  };
  auto pass_steps = [&](int p) { return min(ps, ksteps - p * ps); };

  // Direct-load layout: a k-step's activations are [tile row m][slot] of 16
  // bytes, chunk c (k = 8c..8c+7 of the step) of row m in slot c ^ rs(m),
  // rs(m) = (m & 15) with its two 2-bit halves swapped, so 16 lanes of one
  // load read one row's 256 contiguous bytes and an MFMA fragment read (16
  // rows, one chunk each) is free of bank conflicts (measured by the
  // SQ_LDS_BANK_CONFLICT counter on this access pattern: the plain c ^ (m & 15)
  // costs 4 conflict cycles per 16-byte read, this one none). One load
  // fills a block of 4 rows of one k-step (lane L: row 4 blk + L / 16, chunk
  // (L & 15) ^ (row & 15)). MT > 1: wave wv fills blocks wv, wv + 8, ... of
  // every k-step of a pass. MT == 1 (one pass over all k-steps): wave wv
  // fills block wv & 3 of k-steps wv / 4, wv / 4 + 2, ...
  // W4A16's group sums come in by 4-byte loads of 64 tile rows (lane = row;
  // lanes past the tile read row 0 into padding) to offs[buffer][ls][row]:
  // MT > 1: wave n loads step n / kNegLoads, rows 64 (n % kNegLoads) ..;
  // MT == 1: waves take the steps round robin.
  // MT > 1: a wave issues its direct loads before its kPS steps of weight
  // refills (2 MATS NT loads each), so vmcnt(kAfter) at the pass end covers
  // them; MT == 1 issues them after the ring and waits for everything.
  constexpr int kBlocks = kRows / 4;                                      // per k-step
  constexpr int kPw = MT == 1 ? 1 : (kBlocks + kStWaves - 1) / kStWaves;  // blocks per wave
  constexpr int kNegLoads = (kRows + 63) / 64;                            // per k-step
  constexpr int kNegStride = kNegLoads * 64;                              // floats per k-step
  constexpr int kAfter = kPS * 2 * MATS * NT;
  static_assert(!kDirect || MT == 1 || kPS * kNegLoads <= kStWaves, "one sum load per wave");
  static_assert(kNegLoads <= 2, "at most 128 tile rows");
  [[maybe_unused]] uint32_t voff[kPw] = {};
  [[maybe_unused]] uint32_t voff_neg0 = 0, voff_neg1 = 0;  // rows lane, 64 + lane
  [[maybe_unused]] u32x4_t rs_a = {0u, 0u, 0u, 0u}, rs_n = {0u, 0u, 0u, 0u};
  if constexpr (kDirect) {
    rs_a = buffer_rsrc(FMT == kFmtW4A16 ? g.a_pair : g.a, g.a_rows * K * 2);
#pragma unroll
    for (int h = 0; h < kPw; ++h) {
      const int blk = MT == 1 ? (wv & 3) : min(wv + kStWaves * h, kBlocks - 1);
      const int m = blk * 4 + jq;
      voff[h] = static_cast<uint32_t>(row_index[m] * K * 2 + ((lane & 15) ^ row_swizzle(m)) * 16);
    }
    if constexpr (FMT == kFmtW4A16) {
      rs_n = buffer_rsrc(g.a_neg, g.a_rows * (K / 128) * 4);
      voff_neg0 = static_cast<uint32_t>(row_index[lane < kRows ? lane : 0] * (K / 128) * 4);
      if constexpr (kNegLoads > 1)
        voff_neg1 = static_cast<uint32_t>(row_index[64 + lane < kRows ? 64 + lane : 0] * (K / 128) * 4);
    }
  }
  auto direct_pass = [&](int p, int b) {
    if constexpr (kDirect) {
      const int steps = pass_steps(p);
      if constexpr (MT == 1) {
        for (int ls = wv >> 2; ls < steps; ls += 2)
          lds_direct16(rs_a, afrag + (ls * kRows + (wv & 3) * 4) * 16, voff[0],
                       static_cast<uint32_t>(ls) * 256u);
        if constexpr (FMT == kFmtW4A16) {
          for (int ls = wv; ls < steps; ls += kStWaves)
            lds_direct4(rs_n, offs + ls * kNegStride, voff_neg0, static_cast<uint32_t>(ls) * 4u);
        }
      } else {
#pragma unroll
        for (int h = 0; h < kPw; ++h) {
          const int blk = wv + kStWaves * h;
          if (blk < kBlocks) {
#pragma unroll
            for (int ls = 0; ls < kPS; ++ls)
              if (ls < steps)
                lds_direct16(rs_a, afrag + ((b * ps + ls) * kRows + blk * 4) * 16, voff[h],
                             static_cast<uint32_t>(p * ps + ls) * 256u);
          }
        }
        if constexpr (FMT == kFmtW4A16) {
          const int ls = wv / kNegLoads, hh = wv % kNegLoads;
          if (ls < steps)
            lds_direct4(rs_n, offs + (b * ps + ls) * kNegStride + hh * 64,
                        hh == 0 ? voff_neg0 : voff_neg1,
                        static_cast<uint32_t>(p * ps + ls) * 4u);
        }
      }
    }
  };

  // 3. stage the first pass. 64-row tiles: all of its units in one batch of
  // loads, then the weight ring, then the stores (the stores wait for the
  // activation loads alone); direct loads: the pass, then the ring
  if constexpr (kDirect && MT == 1) {
    direct_pass(0, 0);  // the ring is already in flight
    wait_vmcnt<0>();
  } else if constexpr (kDirect) {
    direct_pass(0, 0);
#pragma unroll
    for (int j = 0; j < kRing; ++j) w[j].load(wrow, srow, j, jq, K, gshift, ksteps, dummy);
    wait_vmcnt<kAfter>();
  } else if constexpr (MT > 1) {
    uint4 v0[kPassUnits];
    uint32_t s0[kPassUnits];
    const int units0 = pass_steps(0) * kRows * 16;
#pragma unroll
    for (int q = 0; q < kPassUnits; ++q) {
      const int u = q * kThreads + tid;
      if (u < units0 && unit_live(u)) {
        v0[q] = unit_load(0, u);
        s0[q] = unit_scale(0, u);
      }
    }
#pragma unroll
    for (int j = 0; j < kRing; ++j) w[j].load(wrow, srow, j, jq, K, gshift, ksteps, dummy);
#pragma unroll
    for (int q = 0; q < kPassUnits; ++q) {
      const int u = q * kThreads + tid;
      if (u < units0 && unit_live(u)) unit_store(0, u, v0[q], s0[q]);
    }
  } else {
    constexpr int kBatch = 6;
    const int units = pass_steps(0) * kRows * 16;
    for (int u0 = 0; u0 < units; u0 += kBatch * kThreads) {
      uint4 v[kBatch];
      uint32_t sv[kBatch];
#pragma unroll
      for (int b = 0; b < kBatch; ++b) {
        const int u = u0 + b * kThreads + tid;
        if (u < units && unit_live(u)) {
          v[b] = unit_load(0, u);
          sv[b] = unit_scale(0, u);
        }
      }
#pragma unroll
      for (int b = 0; b < kBatch; ++b) {
        const int u = u0 + b * kThreads + tid;
        if (u < units && unit_live(u)) unit_store(0, u, v[b], sv[b]);
      }
    }
  }
  __syncthreads();

  // 4. stream: slot j of the ring holds step base + j and is refilled with
  // step base + j + kStDepth once consumed
  const f32x4_t zero4 = {0.f, 0.f, 0.f, 0.f};
  f32x4_t tot[MATS][NT][MT], acc[MATS][NT][MT];
#pragma unroll
  for (int mi = 0; mi < MATS; ++mi)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
      for (int ms = 0; ms < MT; ++ms) {
        tot[mi][nt][ms] = zero4;
        acc[mi][nt][ms] = zero4;
      }
  // LDS slot of this lane's MFMA fragment (subtile ms, sub-step t) of local
  // k-step ls in buffer b: the swizzled fragment blocks of the staged layout,
  // or the row-major layout of direct loads (this lane's row within a subtile
  // is ln, so its swizzle is rs(ln))
  [[maybe_unused]] const int rsw = row_swizzle(ln);
  auto a_slot = [&](int b, int ls, int ms, int t) -> int {
    if constexpr (kDirect) return ((b * ps + ls) * kRows + ms * 16 + ln) * 16 + ((4 * jq + t) ^ rsw);
    else return (((b * ps + ls) * MT + ms) * 4 + t) * kWave + jq * 16 + (ln ^ (4 * t + jq));
  };
  // one k-step: weights wj (a ring slot), activation buffer b, local step ls.
  // Every subtile is computed (no per-MFMA branch): rows past the tile read
  // stale LDS and produce rows that are never stored (MFMA rows are independent).
  auto compute_step = [&](const WeightStep<FMT, MATS, NT, WIDE>& wj, int step, int b, int ls) {
    const int frag0 = (b * ps + ls) * MT * 4;
    if constexpr (kF8) {
      // two scaled MFMAs per 16x16 tile and k-step: fp8 hi, then fp8 lo, each
      // times the raw fp4 weights with their E8M0 block exponents
      v8i32_t ahi[MT], alo[MT];
      int32_t sa[MT];
#pragma unroll
      for (int ms = 0; ms < MT; ++ms) {
        const int f = frag0 + ms * 4;
        const uint4 h0 = afrag[(f + 0) * kWave + jq * 16 + (ln ^ (0 + jq))];
        const uint4 h1 = afrag[(f + 1) * kWave + jq * 16 + (ln ^ (4 + jq))];
        const uint4 l0 = afrag[(f + 2) * kWave + jq * 16 + (ln ^ (8 + jq))];
        const uint4 l1 = afrag[(f + 3) * kWave + jq * 16 + (ln ^ (12 + jq))];
        ahi[ms] = v8i32_t{static_cast<int>(h0.x), static_cast<int>(h0.y), static_cast<int>(h0.z),
                          static_cast<int>(h0.w), static_cast<int>(h1.x), static_cast<int>(h1.y),
                          static_cast<int>(h1.z), static_cast<int>(h1.w)};
        alo[ms] = v8i32_t{static_cast<int>(l0.x), static_cast<int>(l0.y), static_cast<int>(l0.z),
                          static_cast<int>(l0.w), static_cast<int>(l1.x), static_cast<int>(l1.y),
                          static_cast<int>(l1.z), static_cast<int>(l1.w)};
        sa[ms] = reinterpret_cast<const int32_t*>(offs)[(f + jq) * 16 + ln];
      }
#pragma unroll
      for (int mi = 0; mi < MATS; ++mi)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          const v8i32_t bw = {static_cast<int>(wj.w[mi][nt][0]), static_cast<int>(wj.w[mi][nt][1]),
                              static_cast<int>(wj.w[mi][nt][2]), static_cast<int>(wj.w[mi][nt][3]),
                              0, 0, 0, 0};
          const int sb = static_cast<int>(wj.s[mi][nt][0]);
#pragma unroll
          for (int ms = 0; ms < MT; ++ms) {
            tot[mi][nt][ms] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                ahi[ms], bw, tot[mi][nt][ms], 0, 4, 0, sa[ms], 0, sb);
            tot[mi][nt][ms] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                alo[ms], bw, tot[mi][nt][ms], 0, 4, 1, sa[ms], 0, sb);
          }
        }
    } else if constexpr (kMx && WIDE) {
      // k % 128 == 0: every sub-step is real; the lane's block scale is decoded once
      float sc[MATS][NT];
#pragma unroll
      for (int mi = 0; mi < MATS; ++mi)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) sc[mi][nt] = e8m0_to_f32(wj.s[mi][nt][0]);
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        bf16x8_t af[MT];
#pragma unroll
        for (int ms = 0; ms < MT; ++ms)
          af[ms] = __builtin_bit_cast(
              bf16x8_t, afrag[a_slot(b, ls, ms, t)]);
#pragma unroll
        for (int mi = 0; mi < MATS; ++mi)
#pragma unroll
          for (int nt = 0; nt < NT; ++nt) {
            const bf16x8_t bv =
                __builtin_bit_cast(bf16x8_t, unpack_fp4x8_bf16(wj.w[mi][nt][t], sc[mi][nt]));
#pragma unroll
            for (int ms = 0; ms < MT; ++ms)
              tot[mi][nt][ms] =
                  __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[ms], bv, tot[mi][nt][ms], 0, 0, 0);
          }
      }
    } else if constexpr (kMx) {
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        if (static_cast<int64_t>(step) * 128 + 32 * t >= K) break;
#pragma unroll
        for (int ms = 0; ms < MT; ++ms) {
          const uint4 q = afrag[(frag0 + ms * 4 + t) * kWave + jq * 16 + (ln ^ (4 * t + jq))];
          const u32x4_t av = {q.x, q.y, q.z, q.w};
#pragma unroll
          for (int mi = 0; mi < MATS; ++mi)
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
              const float sc = e8m0_to_f32(wj.s[mi][nt][t]);
              if constexpr (FMT == kFmtMxBf16)
                tot[mi][nt][ms] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                    __builtin_bit_cast(bf16x8_t, av),
                    __builtin_bit_cast(bf16x8_t, unpack_fp4x8_bf16(wj.w[mi][nt][t], sc)),
                    tot[mi][nt][ms], 0, 0, 0);
              else
                tot[mi][nt][ms] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                    __builtin_bit_cast(f16x8_t, av),
                    __builtin_bit_cast(f16x8_t, unpack_fp4x8_f16(wj.w[mi][nt][t], sc)),
                    tot[mi][nt][ms], 0, 0, 0);
            }
        }
      }
    } else if constexpr (WIDE) {
      // G == 128: the step is one whole group; its chain starts from the offset
      f32x4_t neg[MT];
#pragma unroll
      for (int ms = 0; ms < MT; ++ms)
        neg[ms] = *reinterpret_cast<const f32x4_t*>(
            &offs[kDirect ? (b * ps + ls) * kNegStride + ms * 16 + jq * 4
                          : (frag0 + ms * 4) * 16 + jq * 4]);
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        bf16x8_t af[MT];
#pragma unroll
        for (int ms = 0; ms < MT; ++ms)
          af[ms] = __builtin_bit_cast(
              bf16x8_t, afrag[a_slot(b, ls, ms, t)]);
#pragma unroll
        for (int mi = 0; mi < MATS; ++mi)
#pragma unroll
          for (int nt = 0; nt < NT; ++nt) {
            const bf16x8_t bv = unpack_q8(wj.w[mi][nt][t]);
#pragma unroll
            for (int ms = 0; ms < MT; ++ms)
              acc[mi][nt][ms] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                  af[ms], bv, t > 0 ? acc[mi][nt][ms] : neg[ms], 0, 0, 0);
          }
      }
#pragma unroll
      for (int mi = 0; mi < MATS; ++mi)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          const float sc = bf16_to_f32(static_cast<uint16_t>(wj.s[mi][nt][0]));
#pragma unroll
          for (int ms = 0; ms < MT; ++ms) tot[mi][nt][ms] += sc * acc[mi][nt][ms];
        }
    } else {
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        if (static_cast<int64_t>(step) * 128 + 32 * t >= K) break;
        const bool first = (t % cg) == 0;
        const bool last = ((t + 1) % cg) == 0;
        bf16x8_t af[MT];
        f32x4_t neg[MT];
#pragma unroll
        for (int ms = 0; ms < MT; ++ms) {
          af[ms] = __builtin_bit_cast(
              bf16x8_t, afrag[(frag0 + ms * 4 + t) * kWave + jq * 16 + (ln ^ (4 * t + jq))]);
          neg[ms] = first ? *reinterpret_cast<const f32x4_t*>(
                                &offs[(frag0 + ms * 4 + t / cg) * 16 + jq * 4])
                          : zero4;
        }
#pragma unroll
        for (int mi = 0; mi < MATS; ++mi)
#pragma unroll
          for (int nt = 0; nt < NT; ++nt) {
            const bf16x8_t bv = unpack_q8(wj.w[mi][nt][t]);
            const float sc = bf16_to_f32(static_cast<uint16_t>(wj.s[mi][nt][t]));
#pragma unroll
            for (int ms = 0; ms < MT; ++ms) {
              acc[mi][nt][ms] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                  af[ms], bv, first ? neg[ms] : acc[mi][nt][ms], 0, 0, 0);
              if (last) tot[mi][nt][ms] += sc * acc[mi][nt][ms];
            }
          }
      }
    }
  };

  if constexpr (MT == 1) {
    // 16-row tiles: all activations are resident; a ring kStDepth deep. No exit
    // inside a round and every refill issued: steps past the end skip only
    // their compute (LDS reads and MFMAs, no vector-memory loads), so every path
    // around the loop carries the same loads and each step waits only for its
    // own slot instead of draining the ring.
    for (int base = 0; base < ksteps; base += kStDepth) {
#pragma unroll
      for (int j = 0; j < kStDepth; ++j) {
        const int step = base + j;
        if (step < ksteps) compute_step(w[j], step, 0, step);
        w[j].load(wrow, srow, step + kStDepth, jq, K, gshift, ksteps, dummy);
      }
    }
  } else {
    // 64- and 80-row tiles: passes of kPS k-steps; the ring is one pass deep
    // (its first kPS slots), so slot j serves local step j
    // No exit inside a pass (see the 16-row loop): a partial last pass skips
    // the compute of its missing steps only.
    const int passes = (ksteps + ps - 1) / ps;
    uint4 vnext[kPassUnits];  // the next pass, in flight during this one
    uint32_t snext[kPassUnits];
    for (int p = 0; p < passes; ++p) {
      const int b = p % kNBuf;
      const bool more = p + 1 < passes;
      const int units1 = more ? pass_steps(p + 1) * kRows * 16 : 0;
      if constexpr (kDirect) {
        // the next pass's buffer was retired by the previous pass's barrier
        if (more) direct_pass(p + 1, (p + 1) % kNBuf);
      } else if (more) {
#pragma unroll
        for (int q = 0; q < kPassUnits; ++q) {
          const int u = q * kThreads + tid;
          if (u < units1 && unit_live(u)) {
            vnext[q] = unit_load(p + 1, u);
            snext[q] = unit_scale(p + 1, u);
          }
        }
      }
#pragma unroll
      for (int j = 0; j < kPS; ++j) {
        const int step = p * ps + j;
        if (step < ksteps) compute_step(w[j], step, b, j);
        w[j].load(wrow, srow, step + kPS, jq, K, gshift, ksteps, dummy);
      }
      if (more) {
        // publish the next pass; the barrier also retires this pass's buffer,
        // which the pass after next overwrites
        if constexpr (kDirect) {
          wait_vmcnt<kAfter>();  // this wave's direct loads landed
        } else {
#pragma unroll
          for (int q = 0; q < kPassUnits; ++q) {
            const int u = q * kThreads + tid;
            if (u < units1 && unit_live(u)) unit_store((p + 1) % kNBuf, u, vnext[q], snext[q]);
          }
        }
        __syncthreads();
      }
    }
  }

  auto out_value = [&](int nt, int ms, int i) -> uint16_t {
    if constexpr (MATS == 2)
      return g.act == kActSitu ? situ_bf16(tot[0][nt][ms][i], tot[1][nt][ms][i], g.situ_beta,
                                           g.situ_linear_beta)
                               : swiglu_bf16(tot[0][nt][ms][i], tot[1][nt][ms][i]);
    else
      return store_value<FMT>(tot[0][nt][ms][i]);
  };
  if constexpr (kDirect) {
    // the tile goes through LDS ([row][column], rows padded by 8 values so
    // that the 2-byte writes of 4 rows spread over the banks) and out as
    // 16-byte chunks, a row's block columns contiguous. W4A16 gate/up with
    // out_neg: each chunk paired and the 128-wide group sums written too, in
    // the staging's order (the block's kBN = 128 columns are one group; the
    // 16 chunks of a row sit in one 16-lane DPP row).
    constexpr int kPitch = kBN + 8;
    constexpr int kChunks = kBN / 8;
    static_assert(kChunks % 16 == 0 && kThreads % 16 == 0, "chunks of a row fill DPP rows");
    uint16_t* const otile = reinterpret_cast<uint16_t*>(smem);
    __syncthreads();  // every wave has read its last activations
#pragma unroll
    for (int ms = 0; ms < MT; ++ms) {
      if (ms >= mt_act) break;
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
          otile[(ms * 16 + jq * 4 + i) * kPitch + (wv * NT + nt) * 16 + ln] = out_value(nt, ms, i);
    }
    __syncthreads();
    constexpr bool kPairOut = FMT == kFmtW4A16 && MATS == 2;
    static_assert(!kPairOut || kBN == 128, "paired output: one group per block");
    for (int u = tid; u < kRows * kChunks; u += kThreads) {
      const int m = u / kChunks, c = u - m * kChunks;
      const uint4 v = *reinterpret_cast<const uint4*>(otile + m * kPitch + c * 8);
      const int64_t c0 = static_cast<int64_t>(cb) * kBN + c * 8;
      const bool live = m < rows && c0 < N;
      if constexpr (kPairOut) {
        if (g.out_neg) {
          uint32_t q[4];
          pair_x8(v, q);
          float sx = sum8(sum_x8_dot(v));
          sx += dpp_f32<kRowMirror>(sx);
          if (live) {
            *reinterpret_cast<uint4*>(out + out_row[m] * N + c0) = make_uint4(q[0], q[1], q[2], q[3]);
            if (c == 0) g.out_neg[out_row[m] * (N / 128) + cb] = -kCodeOffset * sx;
          }
          continue;
        }
      }
      if (live) *reinterpret_cast<uint4*>(out + out_row[m] * N + c0) = v;
    }
  } else {
#pragma unroll
    for (int ms = 0; ms < MT; ++ms) {
      if (ms >= mt_act) break;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int m = ms * 16 + jq * 4 + i;
        if (m >= rows) continue;
        const int64_t orow = out_row[m];
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          if (col[nt] >= N) continue;
          out[orow * N + col[nt]] = out_value(nt, ms, i);
        }
      }
    }
  }
}

// Block = 8 waves over one tile of <= 16 * MT rows x (8 * 16 * NT) columns.
// The block stages the tile's activation rows in LDS (MT == 1: the whole
// reduction once, one barrier; MT > 1: passes of kStPassSteps k-steps,
// double buffered, the next pass loaded while the current one computes, one
// barrier per pass); every wave streams its own columns over all of k with
// kStDepth k-steps of weights in flight and stores its outputs itself.
template <int FMT, int MATS, int NT, int MT, bool WIDE, bool GATHER, bool SCATTER, bool DENSE,
          bool DDIRECT = false>
__global__ void __launch_bounds__(kStWaves * kWave, 2)
w4a16_stream_kernel(const GemmArgs g) {
  constexpr int kThreads = kStWaves * kWave;
  constexpr int kBN = kStWaves * NT * 16;
  constexpr int kRows = 16 * MT;

  const int per_tile = g.col_blocks * g.outputs;
  const int id = blockIdx.x;
  int tile, cb_all;
  if (DENSE && per_tile % 8 == 0) {
    // dense products: XCD x (block ids are dealt round robin to the 8 XCDs)
    // takes the band of per_tile / 8 column blocks from x * band and walks the
    // row tiles with it, so the band's weights stay in that XCD's L2 while
    // each row tile is read once per XCD (tile-major within the band keeps
    // the blocks in flight on a few row tiles)
    const int band = per_tile >> 3;
    const int j = id >> 3;
    tile = j / band;
    cb_all = (id & 7) * band + (j - tile * band);
  } else {
    // a tile's column blocks sit on one XCD
    const int grp = id / (8 * per_tile);
    const int rem = id - grp * 8 * per_tile;
    tile = grp * 8 + (rem & 7);
    cb_all = rem >> 3;
  }
  const int osel = cb_all / g.col_blocks;
  const int cb = cb_all - osel * g.col_blocks;
  int expert, row0, rows;
  if constexpr (DENSE) {
    row0 = tile * kRows;
    if (row0 >= g.dense_rows) return;
    rows = min(kRows, g.dense_rows - row0);
    expert = 0;
  } else {
    // the descriptor load does not wait for the count (the list holds max_tiles entries)
    const int4 d = reinterpret_cast<const int4*>(g.tiles)[tile];
    if (tile >= *g.tile_count) return;
    expert = d.x;
    row0 = d.y;
    rows = d.z;
  }
  const int64_t N = g.n;
  uint16_t* const out = pick3(g.out, osel);
  const int tid = threadIdx.x;
  if (expert < 0) {  // routes outside the bank produce zero rows
    for (int i = tid; i < rows * kBN; i += kThreads) {
      const int m = i / kBN;
      const int64_t col = static_cast<int64_t>(cb) * kBN + (i - m * kBN);
      if (col < N) {
        const int64_t orow = SCATTER ? g.perm[row0 + m] : row0 + m;
        out[orow * N + col] = 0;
      }
    }
    return;
  }
  // 64-row gather / scatter launches with 128-wide k-steps take their
  // activations by direct loads, in every tile path below
  // (DDIRECT: a dense product whose rows are loaded directly, W4A16 from the
  // paired copy)
  constexpr bool kDirect = MT > 1 && WIDE && (FMT == kFmtW4A16 || FMT == kFmtMxBf16) &&
                           (DENSE ? DDIRECT : GATHER != SCATTER);
  if constexpr (kDirect) {
    // the merged list: an expert's last tile of <= 16 rows is already part of
    // the 64-row tile before it, one pass over the expert's weights for up to
    // 80 rows (and every entry of the list is a tile with rows to compute, so
    // consecutive entries, which go to consecutive XCDs, carry equal work)
    if (rows > 64) {
      stream_tile<FMT, MATS, NT, 5, WIDE, GATHER, SCATTER, DENSE, true>(g, expert, row0, rows, cb,
                                                                        osel);
      return;
    }
  }
  // a tile of at most 16 rows (an expert's last rows) takes the 16-row path:
  // a quarter of the MFMAs and all of its activations resident (the host
  // sets tail16 when they fit the launch's LDS)
  if constexpr (MT > 1) {
    if (rows <= 16 && g.tail16) {
      stream_tile<FMT, MATS, NT, 1, WIDE, GATHER, SCATTER, DENSE, kDirect>(g, expert, row0, rows,
                                                                           cb, osel);
      return;
    }
  }
  stream_tile<FMT, MATS, NT, MT, WIDE, GATHER, SCATTER, DENSE, kDirect>(g, expert, row0, rows, cb,
                                                                        osel);
}

// ---------------------------------------------------------------------------
// Persistent streaming GEMM over 16-row tiles (decode batches; 16-byte
// weight loads). The grid is one resident block (8 waves) per CU slot. Block b
// takes an equal contiguous range of units (tile, 16-column group) in tile
// order, and its waves claim the units of the range one at a time, in order,
// so there are no rounds of blocks and a CU's waves finish together. Each
// wave keeps DEPTH k-steps of weights in flight across its units:
// the loads of a unit's first k-steps are issued while the previous unit's
// last k-steps are computed, so the weight stream never drains between tiles.
// The block's tiles (segments) are staged in LDS once, nbuf at a time (a range
// covering more tiles advances in phases with a block barrier between them),
// only their own rows when a phase holds few; their activation loads are
// issued before the weight ring, so staging does not wait behind the ring.
// Tile descriptors and output rows sit in LDS: the per-unit epilogue touches
// no global memory but its stores.
constexpr int kPsMaxSegs = 8;     // tiles one block may cover (checked on the host)
constexpr int kPsHalfMax = 12;    // staging units per thread and LDS buffer (k-steps <= 24)
constexpr int kPsSwiHalfMax = 4;  // the same for activations staged through the SwiGLU (k-steps <= 8)
constexpr int kPsBatch = 6;       // staging units in flight per thread in a later phase

// Eight SwiGLU outputs from eight bf16 gate and eight bf16 up values (the
// gate/up GEMM's outputs, already rounded to bf16): swiglu_bf16's steps after
// its two input roundings, which leave bf16 values unchanged, so the result
// is the fused epilogue's bits.
__device__ inline uint32_t swiglu_bf16_pair(uint32_t gate2, uint32_t up2) {
  const float g0 = __uint_as_float(gate2 << 16), g1 = __uint_as_float(gate2 & 0xFFFF0000u);
  const float u0 = __uint_as_float(up2 << 16), u1 = __uint_as_float(up2 & 0xFFFF0000u);
  const uint32_t lo = f32_to_bf16(round_bf16(silu_fast_f32(g0)) * u0);
  const uint32_t hi = f32_to_bf16(round_bf16(silu_fast_f32(g1)) * u1);
  return lo | (hi << 16);
}

__device__ inline uint4 swiglu_x8(const uint4 gate, const uint4 up) {
  return make_uint4(swiglu_bf16_pair(gate.x, up.x), swiglu_bf16_pair(gate.y, up.y),
                    swiglu_bf16_pair(gate.z, up.z), swiglu_bf16_pair(gate.w, up.w));
}
constexpr int kPsEarlyPairs = 1;  // ring pairs issued before the first staging completes

template <int FMT>
__device__ inline void ps_stage_store(uint4* afrag, float* offs, int frag, int c, int mr,
                                      const uint4 v) {
  const int t = c & 3, j = c >> 2;  // 16-byte unit c of the step feeds MFMA t, lane block j
  uint4* dst = &afrag[(frag + t) * kWave + j * 16 + (mr ^ (4 * t + j))];
  if constexpr (FMT != kFmtW4A16) {
    *dst = v;
  } else {
    uint32_t q[4];
    pair_x8(v, q);
    *dst = make_uint4(q[0], q[1], q[2], q[3]);
    float sx = sum8(sum_x8_dot(v));
    sx += dpp_f32<kRowMirror>(sx);  // the 16 units of a (row, step) sit in one 16-lane row
    if (c == 0) offs[frag * 16 + mr] = -kCodeOffset * sx;
  }
}

// Two consecutive 128-wide k-steps (2q, 2q + 1) of a lane's weights for the
// persistent kernel: per matrix and column tile, the two 16-byte code loads
// are issued back to back (they are the two halves of one 128-byte line of
// the weight row, so the line is fetched once: requested apart, each half
// costs a fetch of its own), and one scale load serves both steps (W4A16
// G = 128: the bf16 pair, low half = step 2q; MXFP4: eight E8M0 bytes, four
// per step). Whole-dword scale loads keep the ring free of narrow loads, whose
// zero-extension the compiler otherwise places at the loop latch, where it
// waits for every load in flight.
template <int FMT, int MATS, int NT>
struct PsPair {
  static constexpr int kSw = FMT == kFmtW4A16 ? 1 : 2;  // scale dwords per pair
  uint32_t w[2][MATS][NT][4];
  uint32_t s[MATS][NT][kSw];

  __device__ inline void load(const uint8_t* const (&wrow)[MATS][NT],
                              const void* const (&srow)[MATS][NT], int step0, int jq, int ksteps,
                              const uint8_t* dummy) {
    const bool live = step0 < ksteps;  // step0 even, ksteps even; past the end: the zero line
#pragma unroll
    for (int mi = 0; mi < MATS; ++mi)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        const void* sp;
        if constexpr (FMT == kFmtW4A16)
          sp = static_cast<const uint16_t*>(srow[mi][nt]) + step0;
        else
          sp = static_cast<const uint8_t*>(srow[mi][nt]) + static_cast<int64_t>(step0) * 4;
        if (!live) sp = dummy;
        if constexpr (kSw == 1) {
          s[mi][nt][0] = *static_cast<const uint32_t*>(sp);
        } else {
          const uint2 v = *static_cast<const uint2*>(sp);
          s[mi][nt][0] = v.x;
          s[mi][nt][1] = v.y;
        }
      }
#pragma unroll
    for (int mi = 0; mi < MATS; ++mi)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const uint8_t* wp =
              live ? wrow[mi][nt] + static_cast<int64_t>(step0 + h) * 64 + jq * 16 : dummy;
          const uint4 v = *reinterpret_cast<const uint4*>(wp);
          w[h][mi][nt][0] = v.x;
          w[h][mi][nt][1] = v.y;
          w[h][mi][nt][2] = v.z;
          w[h][mi][nt][3] = v.w;
        }
  }
};

//
// Split SwiGLU (SPLIT, SWI; decode batches of the MoE block): the gate/up
// GEMM runs with SPLIT, its units one matrix wide (16 columns of w1, or of
// w3, for a tile), and writes the two products rounded to bf16 side by side,
// [rows, 2n] (gate then up). The down GEMM runs with SWI: its activation
// rows are those [rows, 2k] pairs, and the staging applies the SwiGLU
// (swiglu_x8) before the values go into LDS. Units of half the bytes shorten
// the tail of the gate/up launch, where the last units of each block stream
// alone; the SwiGLU is applied to the same bf16-rounded values as in the
// fused epilogue, so the block's output is the same bits.
// Routing and schedule of a small batch inside each block of the persistent
// gate/up GEMM (ROUTED): wave w routes token w (at most kStWaves tokens;
// engine/klinear/router.py:47-85; block 0 writes the selections and weights
// for the launches that follow), or, with rt_from_idx, the block reads the
// router launch's selections. Then the block ranks the at most kRoutedEntries
// token-routes (shared expert as route top_k; two per thread) into the 16-row
// schedule in LDS, as the schedule kernels do: a bitmap of each bucket's
// entries per 64-entry group, the buckets' entry and tile counts scanned in
// bucket order by one wave, and an entry's rank the entries of its bucket in
// earlier groups plus the popcount of the lower lanes of its own (stable,
// row-major). Bucket routed + 1 collects invalid selections (expert -1:
// zeros). No schedule launch; block 0 also writes the tables where a later
// launch reads them (rt_tiles_out).
constexpr int kRoutedEntries = 2 * kStWaves * kWave;  // 1024

// LDS words of the selections (tokens x top_k, padded to 16 bytes)
__host__ __device__ inline int routed_sel_words(int tokens, int top_k) {
  return (tokens * top_k + 3) & ~3;
}

// LDS words of the routing scratch for n token-routes over nb buckets:
// selections, the tile list (at most n tiles), the permutation, the tile
// count, then the ranking's bitmaps, counts and starts
__host__ __device__ inline int routed_scratch_words(int tokens, int top_k, int nb) {
  const int n = tokens * (top_k + 1);
  const int nw = (n + kWave - 1) / kWave;
  return routed_sel_words(tokens, top_k) + 4 * n + n + 1 + 3 * nw * nb + 3 * nb;
}

// Bucket entry and tile counts of the nb buckets (cnt(i)), scanned in bucket
// order by one wave (a lane takes a run of buckets): bucket starts, first
// tiles and the tile count.
template <typename Count>
__device__ void routed_bucket_scan(int nb, int lane, Count cnt, int* bstart, int* btile,
                                   int32_t* r_count) {
  const int per = (nb + kWave - 1) / kWave;
  const int b0 = min(nb, lane * per), b1 = min(nb, b0 + per);
  int se = 0, st = 0;
  for (int i = b0; i < b1; ++i) {
    const int c = cnt(i);
    se += c;
    st += (c + 15) >> 4;
  }
  const int ie = wave_inclusive_scan(se);
  const int it = wave_inclusive_scan(st);
  int re = ie - se, rt = it - st;
  for (int i = b0; i < b1; ++i) {
    const int c = cnt(i);
    bstart[i] = re;
    btile[i] = rt;
    re += c;
    rt += (c + 15) >> 4;
  }
  if (lane == kWave - 1) *r_count = it;
}

__device__ void route_schedule_block(const GemmArgs& g, int32_t* r_sel, int4* r_tiles,
                                     int32_t* r_perm, int32_t* r_count) {
  constexpr int kThreads = kStWaves * kWave;
  const int tid = threadIdx.x;
  const int wave = tid / kWave, lane = tid & (kWave - 1);
  const int ne = g.rt_routed, top_k = g.rt_top_k, tokens = g.rt_tokens;
  const int routes = top_k + 1;
  const int n = tokens * routes;  // <= kRoutedEntries (host-checked)
  const int nb = ne + 2;          // experts 0 .. ne (ne: shared), invalid
  const bool writer = blockIdx.x == 0;
  const int nw = (n + kWave - 1) / kWave;
  uint32_t* const mask = reinterpret_cast<uint32_t*>(r_count + 1);  // [nw][nb][2]
  if (nw > 1)  // the several waves' bitmaps, cleared while the logits arrive
    for (int i = tid; i < 2 * nw * nb; i += kThreads) mask[i] = 0u;
  // the selection rounds (compact code, run once per block from a cold
  // instruction cache) rather than the merge network: the same choices
  auto select = [&](int t, const float (&lg)[4], const float (&bs)[4]) {
    route_select_rounds<4>(lg, bs, ne, top_k, -1, g.rt_scaling, g.rt_renorm,
                           writer ? g.rt_idx + static_cast<int64_t>(t) * top_k : nullptr,
                           writer ? g.rt_w + static_cast<int64_t>(t) * top_k : nullptr,
                           r_sel + t * top_k);
  };
  if (g.rt_from_idx) {  // block-uniform: the router launch's selections
    for (int i = tid; i < tokens * top_k; i += kThreads)
      r_sel[i] = static_cast<int32_t>(g.rt_idx[i]);
  } else if (wave < tokens) {  // one token per wave (at most kStWaves, host-checked)
    float lg0[4], bs[4];
    route_load_all<4>(g.rt_logits + static_cast<int64_t>(wave) * ne, g.rt_bias, ne, lg0, bs);
    select(wave, lg0, bs);
  }
  __syncthreads();
  if (nw == 1) {  // block-uniform: wave 0 ranks the entries alone
    if (wave == 0) {
      int* const bstart = reinterpret_cast<int*>(mask + 2 * nb);        // [nb]
      int* const btile = bstart + nb;                                   // [nb]
      const bool live = lane < n;
      int b = 0;
      if (live) {
        const int t = lane / routes, r = lane - t * routes;
        const int x = r == top_k ? ne : r_sel[t * top_k + r];
        b = (x >= 0 && x <= ne) ? x : ne + 1;
      }
      for (int i = lane; i < 2 * nb; i += kWave) mask[i] = 0u;
      __builtin_amdgcn_s_waitcnt(0);  // one wave: its LDS operations in order
      if (live) atomicOr(&mask[2 * b + (lane >> 5)], 1u << (lane & 31));
      __builtin_amdgcn_s_waitcnt(0);
      routed_bucket_scan(nb, lane,
                         [&](int i) { return __popc(mask[2 * i]) + __popc(mask[2 * i + 1]); },
                         bstart, btile, r_count);
      __builtin_amdgcn_s_waitcnt(0);
      if (live) {
        const uint32_t lo = mask[2 * b], hi = mask[2 * b + 1];
        const int before = lane < 32 ? __popc(lo & ((1u << lane) - 1u))
                                     : __popc(lo) + __popc(hi & ((1u << (lane - 32)) - 1u));
        const int same = __popc(lo) + __popc(hi);
        const int pos = bstart[b] + before;
        r_perm[pos] = lane;
        if ((before & 15) == 0)
          r_tiles[btile[b] + (before >> 4)] =
              make_int4(b <= ne ? b : -1, pos, min(16, same - before), 0);
      }
    }
  } else {  // entries tid and tid + 512: 64-entry group e / 64 keeps its bitmaps
    int* const pre = reinterpret_cast<int*>(mask + 2 * nw * nb);  // [nw][nb]
    int* const tot = pre + nw * nb;                               // [nb]
    int* const bstart = tot + nb;                                 // [nb]
    int* const btile = bstart + nb;                               // [nb]
    const bool two = n > kThreads;  // block-uniform: a second entry per thread
    auto bucket_of = [&](int e) {
      const int t = e / routes, r = e - t * routes;
      const int x = r == top_k ? ne : r_sel[t * top_k + r];
      return (x >= 0 && x <= ne) ? x : ne + 1;
    };
    int bk[2] = {0, 0};
    if (tid < n) {
      bk[0] = bucket_of(tid);
      atomicOr(&mask[(wave * nb + bk[0]) * 2 + (lane >> 5)], 1u << (lane & 31));
    }
    if (two && tid + kThreads < n) {
      bk[1] = bucket_of(tid + kThreads);
      atomicOr(&mask[((wave + kStWaves) * nb + bk[1]) * 2 + (lane >> 5)], 1u << (lane & 31));
    }
    __syncthreads();
    // each bucket's entries in the groups before each group, and in all
    for (int bb = tid; bb < nb; bb += kThreads) {
      int run = 0;
      for (int w = 0; w < nw; ++w) {
        pre[w * nb + bb] = run;
        run += __popc(mask[(w * nb + bb) * 2]) + __popc(mask[(w * nb + bb) * 2 + 1]);
      }
      tot[bb] = run;
    }
    __syncthreads();
    if (wave == 0)
      routed_bucket_scan(nb, lane, [&](int i) { return tot[i]; }, bstart, btile, r_count);
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int e = tid + kThreads * k;
      if ((k == 0 || two) && e < n) {
        const int grp = e / kWave, b = bk[k];
        const uint32_t lo = mask[(grp * nb + b) * 2], hi = mask[(grp * nb + b) * 2 + 1];
        const int below = lane < 32 ? __popc(lo & ((1u << lane) - 1u))
                                    : __popc(lo) + __popc(hi & ((1u << (lane - 32)) - 1u));
        const int rank = pre[grp * nb + b] + below;
        const int pos = bstart[b] + rank;
        r_perm[pos] = e;
        if ((rank & 15) == 0)
          r_tiles[btile[b] + (rank >> 4)] =
              make_int4(b <= ne ? b : -1, pos, min(16, tot[b] - rank), 0);
      }
    }
  }
  __syncthreads();
  if (writer && g.rt_tiles_out != nullptr) {
    const int count = *r_count;
    for (int i = tid; i < n; i += kThreads) g.rt_perm_out[i] = r_perm[i];
    for (int i = tid; i < count; i += kThreads)
      reinterpret_cast<int4*>(g.rt_tiles_out)[i] = r_tiles[i];
    if (tid == 0) *g.rt_count_out = count;
  }
}

template <int FMT, int MATS, int DEPTH, bool GATHER, bool SCATTER, bool SPLIT = false,
          bool SWI = false, bool ROUTED = false>
__global__ void __launch_bounds__(kStWaves * kWave)
w4a16_persist_kernel(const GemmArgs g, int nbuf) {
  static_assert(FMT == kFmtW4A16 || FMT == kFmtMxBf16, "bf16 activations, 16-byte weight loads");
  static_assert(!ROUTED || (GATHER && !SWI), "routing feeds the gate/up GEMM");
  static_assert(DEPTH % 2 == 0, "the ring holds pairs of k-steps");
  static_assert(!SPLIT || MATS == 1, "split units hold one matrix");
  static_assert(!SWI || (MATS == 1 && !SPLIT), "SwiGLU staging feeds the down GEMM");
  constexpr int kPairs = DEPTH / 2;
  static_assert(kPsEarlyPairs < kPairs, "the staging barrier sits inside the first round");
  // units are 16 columns (one MFMA column tile per matrix): at 64 tokens of
  // the Kimi-Linear layer the down GEMM takes 40.5 us with them against
  // 43.1 us with 32-column units, whose longer last units stretch the tail
  constexpr int NT = 1;
  constexpr int kHalfCap = SWI ? kPsSwiHalfMax : kPsHalfMax;
  constexpr bool kMx = FMT != kFmtW4A16;
  extern __shared__ uint4 smem[];
  __shared__ int64_t seg_row[kPsMaxSegs][16];  // activation row of tile row m
  __shared__ int32_t seg_out[kPsMaxSegs][16];  // output row of tile row m
  __shared__ int32_t seg_exp[kPsMaxSegs], seg_rows[kPsMaxSegs];
  __shared__ int32_t next_unit;  // the block's next unclaimed unit

  const int64_t N = g.n, K = g.k;
  const int ksteps = static_cast<int>(K >> 7);  // k % 128 == 0
  const int rounds = ksteps / DEPTH;  // DEPTH divides ksteps (host-checked)
  const int cgs1 = static_cast<int>((N + NT * 16 - 1) / (NT * 16));  // column groups per matrix
  const int cgs = SPLIT ? 2 * cgs1 : cgs1;
  // ROUTED: the batch's selections and schedule, computed by every block in
  // the activation LDS before any staging (at most kRoutedEntries routes;
  // the layout of routed_scratch_words)
  const int r_n = ROUTED ? g.rt_tokens * (g.rt_top_k + 1) : 0;
  int32_t* const r_sel = reinterpret_cast<int32_t*>(smem);  // [tokens][top_k]
  int4* const r_tiles =
      reinterpret_cast<int4*>(smem) + (ROUTED ? routed_sel_words(g.rt_tokens, g.rt_top_k) / 4 : 0);
  int32_t* const r_perm = reinterpret_cast<int32_t*>(r_tiles + r_n);  // at most n tiles
  int32_t* const r_count = r_perm + r_n;  // then the ranking scratch
  if constexpr (ROUTED) route_schedule_block(g, r_sel, r_tiles, r_perm, r_count);
  const int total = (ROUTED ? *r_count : *g.tile_count) * cgs;
  const int per = (total + static_cast<int>(gridDim.x) - 1) / static_cast<int>(gridDim.x);
  // ranges go to XCDs in contiguous runs (block b runs on XCD b % 8): the
  // blocks on one XCD take consecutive ranges, so an expert's consecutive
  // tiles, which read the same weights, meet in that XCD's L2 instead of
  // each fetching them from HBM
  const int grid = static_cast<int>(gridDim.x);
  const int bid = static_cast<int>(blockIdx.x);
  const int range = grid % 8 == 0 ? (bid % 8) * (grid / 8) + bid / 8 : bid;
  const int ub = range * per;
  const int ue = min(ub + per, total);
  if (ub >= ue) return;  // block-uniform
  const int t_first = ub / cgs;
  const int nseg = min((ue - 1) / cgs - t_first + 1, kPsMaxSegs);
  const int phases = (nseg + nbuf - 1) / nbuf;

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int jq = lane >> 4;
  const int ln = lane & 15;
  const int64_t rowb = K / 2;
  const int64_t spr = K / g.group;
  const uint8_t* const dummy = g_tail_pad;
  uint4* const afrag = smem;  // [nbuf][ksteps][4][64]
  float* const offs = reinterpret_cast<float*>(smem + nbuf * ksteps * 4 * kWave);  // [nbuf][ksteps][4][16]

  // 1. descriptors and row tables of the block's tiles
  if (tid == 0) next_unit = ub;
  if (tid < nseg * 16) {
    const int s = tid >> 4, m = tid & 15;
    const int4 d = ROUTED ? r_tiles[t_first + s] : reinterpret_cast<const int4*>(g.tiles)[t_first + s];
    if (m == 0) {
      seg_exp[s] = d.x;
      seg_rows[s] = d.z;
    }
    if (m < d.z) {
      const int32_t p = ROUTED ? r_perm[d.y + m] : (GATHER || SCATTER) ? g.perm[d.y + m] : d.y + m;
      seg_row[s][m] = GATHER ? p / g.routes : static_cast<int64_t>(d.y) + m;
      seg_out[s][m] = SCATTER ? p : d.y + m;
    }
  }
  __syncthreads();

  // Staging of phase p (the activation rows of segments p * nbuf .. into
  // buffers 0 .. nbuf - 1): thread tid owns 16-byte chunk sc of row sm at the
  // k-steps of parity sl, so buffer sb takes half = ksteps / 2 units per
  // thread, unit ii at k-step 2 ii + sl. Buffer and unit are compile-time in
  // the unrolled loops, so each unit is one load at a fixed offset from the
  // buffer's row pointer and one store: the staging runs once per block with
  // a cold instruction cache, so its code is kept short. Rows past a tile's
  // end (and buffers past the block's last tile) stage the block's first row:
  // their MFMA rows are never stored. Every staged load is stored, so no load
  // is left outstanding on any path (the compiler would otherwise wait for
  // every load in flight inside the weight loop).
  const int sc = tid & 15, sm = (tid >> 4) & 15, sl = tid >> 8;
  const int half = ksteps >> 1;  // ksteps is even (DEPTH is); half <= kHalfCap (host-checked)
  const int64_t astride = SWI ? 2 * K : K;  // SWI: gate values, then up values
  const uint16_t* rp[2];
  auto stage_rows = [&](int p) {
#pragma unroll
    for (int sb = 0; sb < 2; ++sb) {
      const int s = p * nbuf + sb;
      const bool ok = sb < nbuf && s < nseg && sm < seg_rows[s];
      const int64_t row = ok ? seg_row[s][sm] : seg_row[0][0];
      rp[sb] = g.a + row * astride + sl * 128 + sc * 8;
    }
  };
  // buffers holding a tile of the block in phase p (block-uniform; the same
  // predicate guards a buffer's loads and its stores)
  auto stage_live = [&](int p, int sb) { return sb < nbuf && p * nbuf + sb < nseg; };
  auto stage_loads = [&](int p, uint4 (&v)[2][kHalfCap]) {
#pragma unroll
    for (int sb = 0; sb < 2; ++sb)
#pragma unroll
      for (int ii = 0; ii < kHalfCap; ++ii)
        if (stage_live(p, sb) && ii < half)
          v[sb][ii] = *reinterpret_cast<const uint4*>(rp[sb] + ii * 256);
  };
  auto stage_stores = [&](int p, const uint4 (&v)[2][kHalfCap]) {
#pragma unroll
    for (int sb = 0; sb < 2; ++sb) {
      if (!stage_live(p, sb)) continue;
      const int fb = sb * ksteps + sl;
#pragma unroll
      for (int ii = 0; ii < kHalfCap; ++ii)
        if (ii < half) ps_stage_store<FMT>(afrag, offs, (fb + 2 * ii) * 4, sc, sm, v[sb][ii]);
    }
  };
  // Compact staging: only the tiles' own rows (most decode tiles hold a few
  // rows of their 16). Each 16-lane group takes (tile, row, k-step) items of
  // the phase's tiles, rows of the first tile first, spread over the block's
  // 32 groups, two items per pass; rows past a tile's end are not staged
  // (their MFMA rows are never stored). The passes are a short rolled loop
  // (it runs once per phase with a cold instruction cache: an unrolled form
  // of the SwiGLU staging took 2-3 us longer), each pass's loads issued
  // before the previous pass is stored. SWI stages through the SwiGLU this
  // way always; the other forms when the phase holds at most kCompactItems
  // items, else every row of both buffers at once (stage_loads).
  struct CPass {
    uint4 gv[2], uv[2];
    int frag[2], row[2];
    bool ok[2];
  };
  constexpr int kGroups = kStWaves * kWave / 16;
  constexpr int kCompactItems = 8 * kGroups;  // four passes
  const int sgid = tid >> 4;
  // item j < 2 tiles x 16 rows x 24 k-steps + one pass = 832: j / ksteps as
  // (j * ceil(2^16 / ksteps)) >> 16, exact there
  const int kinv = (65536 + ksteps - 1) / ksteps;
  auto cs_count = [&](int p, int& n0) {
    const int s0 = p * nbuf;
    n0 = s0 < nseg ? seg_rows[s0] * ksteps : 0;
    return n0 + (nbuf > 1 && s0 + 1 < nseg ? seg_rows[s0 + 1] * ksteps : 0);
  };
  auto cs_load = [&](int p, int j0, CPass& sp) {
    int n0;
    const int n = cs_count(p, n0);
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int j = j0 + q * kGroups;
      const int sb = j < n0 ? 0 : 1;
      const int jj = j - sb * n0;
      const int r = (jj * kinv) >> 16;
      const int step = jj - r * ksteps;
      sp.ok[q] = j < n;
      sp.frag[q] = (sb * ksteps + step) * 4;
      sp.row[q] = r;
      if (sp.ok[q]) {
        const uint16_t* a = g.a + seg_row[p * nbuf + sb][r] * astride + step * 128 + sc * 8;
        sp.gv[q] = *reinterpret_cast<const uint4*>(a);
        if constexpr (SWI) sp.uv[q] = *reinterpret_cast<const uint4*>(a + K);
      }
    }
  };
  auto cs_store = [&](const CPass& sp) {
#pragma unroll
    for (int q = 0; q < 2; ++q)
      if (sp.ok[q])
        ps_stage_store<FMT>(afrag, offs, sp.frag[q], sc, sp.row[q],
                            SWI ? swiglu_x8(sp.gv[q], sp.uv[q]) : sp.gv[q]);
  };
  // stores the pass `cur` (loaded from item sgid) and the rest of phase p
  auto cs_drain = [&](int p, CPass& cur) {
    int n0;
    const int n = cs_count(p, n0);
    for (int j0 = sgid + 2 * kGroups;; j0 += 2 * kGroups) {
      CPass nxt;
      const bool more = j0 < n;
      if (more) cs_load(p, j0, nxt);
      cs_store(cur);
      if (!more) break;
      cur = nxt;
    }
  };
  auto cs_compact = [&](int p) {
    int n0;
    return SWI || cs_count(p, n0) <= kCompactItems;
  };

  // Waves claim the block's units in order, one at a time, when their ring
  // reaches a new unit: a wave that streams faster takes more units (the waves
  // of a CU do not get equal shares of its memory bandwidth). A claim at or
  // past ue means no unit.
  auto claim = [&]() -> int {
    int u = 0;
    if (lane == 0) u = atomicAdd(&next_unit, 1);
    return __builtin_amdgcn_readfirstlane(u);
  };
  auto unit_tile = [&](int u, int& s, int& cgi) {
    const int t = u / cgs;
    s = t - t_first;
    cgi = u - t * cgs;
  };
  const uint8_t* lw[MATS][NT];
  const void* lsr[MATS][NT];
  auto set_ptrs = [&](int u) {
    int s, cgi;
    unit_tile(u, s, cgi);
    const int64_t e = max(seg_exp[s], 0);  // invalid routes: read expert 0, store zeros
    const bool second = SPLIT && cgi >= cgs1;  // SPLIT: a unit of the second matrix
    if (second) cgi -= cgs1;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const int64_t col = static_cast<int64_t>(cgi) * (NT * 16) + nt * 16 + ln;
      const int64_t cc = col < N ? col : N - 1;
#pragma unroll
      for (int mi = 0; mi < MATS; ++mi) {
        const uint8_t* wpm = SPLIT ? (second ? g.wp[1] : g.wp[0]) : g.wp[mi];
        const void* wsm = SPLIT ? (second ? g.ws[1] : g.ws[0]) : g.ws[mi];
        lw[mi][nt] = wpm + e * g.wstride + cc * rowb;
        if constexpr (kMx)
          lsr[mi][nt] = static_cast<const uint8_t*>(wsm) + e * g.sstride + cc * spr;
        else
          lsr[mi][nt] = static_cast<const uint16_t*>(wsm) + e * g.sstride + cc * spr;
      }
    }
  };

  // 2. the first phase's activation loads, then the first kPsEarlyPairs
  // pairs of k-steps of weights; the rest of the first round goes out once the
  // activations are staged, so the activation rows that miss L2 do not queue
  // behind every CU's whole first round
  uint4 sv[2][kHalfCap];
  CPass csp;
  const bool compact0 = cs_compact(0);  // block-uniform
  if (compact0) {
    cs_load(0, sgid, csp);
  } else if constexpr (!SWI) {
    stage_rows(0);
    stage_loads(0, sv);
  }
  PsPair<FMT, MATS, NT> w[kPairs];
  int lu = claim(), lr = 0;  // load cursor: unit, round
  if (lu < ue) set_ptrs(lu);
  // slot by slot, in the order the loop refills them, so the loop's per-slot
  // waits hold on entry as well
#pragma unroll
  for (int j = 0; j < kPairs; ++j) {
    if (j == kPsEarlyPairs) {
      if (compact0)
        cs_drain(0, csp);
      else if constexpr (!SWI)
        stage_stores(0, sv);
      __syncthreads();
    }
    w[j].load(lw, lsr, lu < ue ? 2 * j : ksteps, jq, ksteps, dummy);
    __builtin_amdgcn_sched_barrier(0);
  }
  int issued = lu;  // the unit of the round whose loads were issued last
  if (++lr == rounds) {
    lr = 0;
    lu = claim();
    if (lu < ue) set_ptrs(lu);
  }

  // 3. stream
  const f32x4_t zero4 = {0.f, 0.f, 0.f, 0.f};
  f32x4_t tot[MATS][NT], acc[MATS][NT];
#pragma unroll
  for (int mi = 0; mi < MATS; ++mi)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      tot[mi][nt] = zero4;
      acc[mi][nt] = zero4;
    }
  int cu = issued, cr = 0;  // compute cursor: unit, round
  int cseg = 0, ccg = 0;
  if (cu < ue) unit_tile(cu, cseg, ccg);

  // step 2q + h of pair wj (h = 0, 1), activation fragments from frag0
  auto compute_step = [&](const PsPair<FMT, MATS, NT>& wj, int h, int frag0) {
    if constexpr (kMx) {
      float sc[MATS][NT];
#pragma unroll
      for (int mi = 0; mi < MATS; ++mi)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) sc[mi][nt] = e8m0_to_f32((wj.s[mi][nt][h] >> (8 * jq)) & 0xFFu);
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const bf16x8_t af = __builtin_bit_cast(
            bf16x8_t, afrag[(frag0 + t) * kWave + jq * 16 + (ln ^ (4 * t + jq))]);
#pragma unroll
        for (int mi = 0; mi < MATS; ++mi)
#pragma unroll
          for (int nt = 0; nt < NT; ++nt)
            tot[mi][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                af, __builtin_bit_cast(bf16x8_t, unpack_fp4x8_bf16(wj.w[h][mi][nt][t], sc[mi][nt])),
                tot[mi][nt], 0, 0, 0);
      }
    } else {
      // the bf16 scale is decoded first, by an instruction the register
      // allocator cannot recompute later: the ring register holding the
      // loaded dword is then dead before the slot is refilled (otherwise the
      // refill needs a copy at the loop head, which waits for every load)
      float sc[MATS][NT];
#pragma unroll
      for (int mi = 0; mi < MATS; ++mi)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          if (h)
            asm("v_and_b32 %0, 0xffff0000, %1" : "=v"(sc[mi][nt]) : "v"(wj.s[mi][nt][0]));
          else
            asm("v_lshlrev_b32 %0, 16, %1" : "=v"(sc[mi][nt]) : "v"(wj.s[mi][nt][0]));
        }
      const f32x4_t neg = *reinterpret_cast<const f32x4_t*>(&offs[frag0 * 16 + jq * 4]);
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const bf16x8_t af = __builtin_bit_cast(
            bf16x8_t, afrag[(frag0 + t) * kWave + jq * 16 + (ln ^ (4 * t + jq))]);
#pragma unroll
        for (int mi = 0; mi < MATS; ++mi)
#pragma unroll
          for (int nt = 0; nt < NT; ++nt)
            acc[mi][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                af, unpack_q8(wj.w[h][mi][nt][t]), t > 0 ? acc[mi][nt] : neg, 0, 0, 0);
      }
#pragma unroll
      for (int mi = 0; mi < MATS; ++mi)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) tot[mi][nt] += sc[mi][nt] * acc[mi][nt];
    }
  };

  uint16_t* const out = g.out[0];
  for (int p = 0; p < phases; ++p) {
    if (p > 0) {  // every wave is done with the previous phase's buffers
      __syncthreads();
      // a later phase (blocks covering more tiles than buffers): batches of
      // kPsBatch units, in a rolled loop to keep registers for the ring
      if (cs_compact(p)) {
        cs_load(p, sgid, csp);
        cs_drain(p, csp);
      } else if constexpr (!SWI) {
        stage_rows(p);
        for (int sb = 0; sb < nbuf; ++sb) {
          if (!stage_live(p, sb)) continue;
          for (int i0 = 0; i0 < half; i0 += kPsBatch) {
            uint4 pv[kPsBatch];
#pragma unroll
            for (int b = 0; b < kPsBatch; ++b)
              if (i0 + b < half)
                pv[b] = *reinterpret_cast<const uint4*>(rp[sb] + (i0 + b) * 256);
#pragma unroll
            for (int b = 0; b < kPsBatch; ++b)
              if (i0 + b < half)
                ps_stage_store<FMT>(afrag, offs, (sb * ksteps + sl + 2 * (i0 + b)) * 4, sc, sm,
                                    pv[b]);
          }
        }
      }
      __syncthreads();
    }
    const int seg_end = min(nseg, (p + 1) * nbuf);
    while (cu < ue && cseg < seg_end) {
      const int fbase = (cseg - p * nbuf) * ksteps;
      // one round: DEPTH k-steps of the current unit (DEPTH divides the
      // k-steps); every slot is refilled, past the wave's last unit from the
      // shared zero line
#pragma unroll
      for (int j = 0; j < kPairs; ++j) {
        const int step = cr * DEPTH + 2 * j;
        compute_step(w[j], 0, (fbase + step) * 4);
        compute_step(w[j], 1, (fbase + step + 1) * 4);
        // pair order is kept (each pair waits for its own loads only) and the
        // refill follows the pair's compute, so its registers are reused
        __builtin_amdgcn_sched_barrier(0);
        w[j].load(lw, lsr, lu < ue ? lr * DEPTH + 2 * j : ksteps, jq, ksteps, dummy);
        __builtin_amdgcn_sched_barrier(0);
      }
      issued = lu;
      if (++lr == rounds) {
        lr = 0;
        lu = claim();
        if (lu < ue) set_ptrs(lu);
      }
      if (++cr == rounds) {  // the unit is complete: store it
        const int rows = seg_rows[cseg];
        const bool zero = seg_exp[cseg] < 0;
        // SPLIT: rows of [gate | up], 2n wide
        const bool second = SPLIT && ccg >= cgs1;
        const int ocg = second ? ccg - cgs1 : ccg;
        const int64_t ostride = SPLIT ? 2 * N : N;
        const int64_t ocol0 = second ? N : 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int m = jq * 4 + i;
          if (m >= rows) continue;
          const int64_t orow = seg_out[cseg][m];
#pragma unroll
          for (int nt = 0; nt < NT; ++nt) {
            const int64_t col = static_cast<int64_t>(ocg) * (NT * 16) + nt * 16 + ln;
            if (col >= N) continue;
            uint16_t v;
            if constexpr (MATS == 2)
              v = g.act == kActSitu ? situ_bf16(tot[0][nt][i], tot[1][nt][i], g.situ_beta,
                                                g.situ_linear_beta)
                                    : swiglu_bf16(tot[0][nt][i], tot[1][nt][i]);
            else
              v = store_value<FMT>(tot[0][nt][i]);
            out[orow * ostride + ocol0 + col] = zero ? static_cast<uint16_t>(0) : v;
          }
        }
#pragma unroll
        for (int mi = 0; mi < MATS; ++mi)
#pragma unroll
          for (int nt = 0; nt < NT; ++nt) tot[mi][nt] = zero4;
        cr = 0;
        cu = issued;  // the load cursor is one round ahead: its last round's unit
        if (cu < ue) unit_tile(cu, cseg, ccg);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// fp8 hi/lo split of bf16 activations for the scaled fp4 MFMA. Per block of
// 32 values along k: x ~= hi * 2^e_hi + lo * 2^e_lo with OCP E4M3 codes
// (nearest, ties to even; magnitudes under 2^-6 flush to signed zero) and
// e = clamp(E(block max) - 7, -127, 127), E = the float exponent field - 127,
// so the scaled block max lies in [128, 256) and never saturates. lo encodes
// the exact residual x - hi * 2^e_hi the same way. hi and lo together keep
// the 8 significant bits of a bf16 value. One thread per (row, block).

__device__ inline uint32_t e4m3_code(float v) {
  const uint32_t u = __float_as_uint(v);
  const uint32_t sign = (u >> 24) & 0x80u;
  const uint32_t a = u & 0x7FFFFFFFu;
  if (a < 0x3C800000u) return sign;  // below 2^-6
  const uint32_t r = a + 0x7FFFFu + ((a >> 20) & 1u);
  return sign | ((((r >> 23) - 120u) & 15u) << 3) | ((r >> 20) & 7u);
}

// value of a code produced by e4m3_code (normal or signed zero)
__device__ inline float e4m3_value(uint32_t c) {
  const uint32_t e = (c >> 3) & 15u;
  const uint32_t sign = (c & 0x80u) << 24;
  return __uint_as_float(e == 0u ? sign : sign | ((e + 120u) << 23) | ((c & 7u) << 20));
}

__device__ inline int split_exponent(float amax) {
  const int field = static_cast<int>((__float_as_uint(amax) >> 23) & 0xFFu);
  return min(max(field - 134, -127), 127);
}

__global__ void __launch_bounds__(256)
mx_split_kernel(const uint16_t* __restrict__ x, uint8_t* __restrict__ hi, uint8_t* __restrict__ lo,
                uint16_t* __restrict__ sc, int64_t blocks) {
  const int64_t b = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (b >= blocks) return;
  const uint4* src = reinterpret_cast<const uint4*>(x + b * 32);
  float v[32];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const uint4 w = src[q];
    const uint32_t d[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[q * 8 + 2 * j] = __uint_as_float(d[j] << 16);
      v[q * 8 + 2 * j + 1] = __uint_as_float(d[j] & 0xFFFF0000u);
    }
  }
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(v[i]));
  const int e1 = split_exponent(amax);
  const float inv1 = __uint_as_float(static_cast<uint32_t>(127 - e1) << 23);
  const float s1 = e8m0_to_f32(static_cast<uint32_t>(e1 + 127));
  uint32_t h[8] = {0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u};
  float ramax = 0.f;
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    const uint32_t c = e4m3_code(v[i] * inv1);
    h[i >> 2] |= c << (8 * (i & 3));
    v[i] -= e4m3_value(c) * s1;  // exact residual
    ramax = fmaxf(ramax, fabsf(v[i]));
  }
  const int e2 = split_exponent(ramax);
  const float inv2 = __uint_as_float(static_cast<uint32_t>(127 - e2) << 23);
  uint32_t l[8] = {0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u};
#pragma unroll
  for (int i = 0; i < 32; ++i) l[i >> 2] |= e4m3_code(v[i] * inv2) << (8 * (i & 3));
  uint4* dh = reinterpret_cast<uint4*>(hi + b * 32);
  uint4* dl = reinterpret_cast<uint4*>(lo + b * 32);
  dh[0] = make_uint4(h[0], h[1], h[2], h[3]);
  dh[1] = make_uint4(h[4], h[5], h[6], h[7]);
  dl[0] = make_uint4(l[0], l[1], l[2], l[3]);
  dl[1] = make_uint4(l[4], l[5], l[6], l[7]);
  sc[b] = static_cast<uint16_t>((e1 + 127) | ((e2 + 127) << 8));
}

int split_launch(const uint16_t* x, uint8_t* hi, uint8_t* lo, uint16_t* sc, int64_t rows, int64_t k,
                 hipStream_t s) {
  const int64_t blocks = rows * (k / 32);
  if (blocks == 0) return LK_OK;
  LK_REQUIRE((blocks + 255) / 256 < (1LL << 31), "too many rows for the fp8 split");
  mx_split_kernel<<<static_cast<unsigned>((blocks + 255) / 256), 256, 0, s>>>(x, hi, lo, sc, blocks);
  return check_launch("mxfp4 activation split");
}

// ---------------------------------------------------------------------------
// route combine over entry-ordered expert outputs eo [T * (top_k + 1), H]:
// y[t] = bf16(bf16(sum_{r < top_k} w[t, r] * eo[t, r]) + eo[t, top_k]),
// 8 columns per thread.
__global__ void __launch_bounds__(256)
moe_combine_kernel(const uint16_t* __restrict__ eo, const float* __restrict__ w,
                   uint16_t* __restrict__ y, int64_t tokens, int top_k, int64_t h) {
  const int64_t per = h / 8;
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (gid >= tokens * per) return;
  const int64_t t = gid / per;
  const int64_t c8 = (gid - t * per) * 8;
  const int64_t routes = top_k + 1;
  const uint16_t* base = eo + t * routes * h + c8;
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  // routes in batches of 8 independent loads (the shared route's with the
  // first batch), summed in route order
  const uint4 sv = *reinterpret_cast<const uint4*>(base + top_k * h);
  for (int r0 = 0; r0 < top_k; r0 += 8) {
    uint4 v[8];
    float wr[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int r = min(r0 + i, top_k - 1);
      v[i] = *reinterpret_cast<const uint4*>(base + r * h);
      wr[i] = w[t * top_k + r];
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      // a route past top_k adds +0 (acc starts at +0 and never holds -0, so
      // this leaves every bit as the loop over top_k routes would)
      const bool ok = r0 + i < top_k;
      const uint32_t q[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        acc[2 * j] += ok ? bf16_to_f32(q[j] & 0xFFFFu) * wr[i] : 0.f;
        acc[2 * j + 1] += ok ? bf16_to_f32(q[j] >> 16) * wr[i] : 0.f;
      }
    }
  }
  const uint32_t sq[4] = {sv.x, sv.y, sv.z, sv.w};
  uint32_t o[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t lo = f32_to_bf16(round_bf16(acc[2 * j]) + bf16_to_f32(sq[j] & 0xFFFFu));
    const uint32_t hi = f32_to_bf16(round_bf16(acc[2 * j + 1]) + bf16_to_f32(sq[j] >> 16));
    o[j] = lo | (hi << 16);
  }
  *reinterpret_cast<uint4*>(y + t * h + c8) = make_uint4(o[0], o[1], o[2], o[3]);
}

// offsets[0, n) = 0 and *count = 0 (an empty route table)
__global__ void fill_i32_kernel(int32_t* offsets, int64_t n, int32_t* count) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) offsets[i] = 0;
  if (i == 0) *count = 0;
}

// ---------------------------------------------------------------------------
// host side

inline size_t align_up(size_t v) { return (v + 255) & ~static_cast<size_t>(255); }

struct SchedLayout {
  size_t rank, hist, total;
  int chunks;
  int64_t max_tiles;
};

int64_t max_tiles_for(int64_t entries, int64_t experts, int tile_rows) {
  return (experts + 1 < entries ? experts + 1 : entries) + entries / tile_rows + 1;
}

// The layout holds the tile list of the smaller (16-row) tiles, which bounds both.
SchedLayout sched_layout(int64_t entries, int64_t experts) {
  SchedLayout l;
  l.chunks = static_cast<int>((entries + kSchedThreads - 1) / kSchedThreads);
  l.max_tiles = max_tiles_for(entries, experts, kSmallTileRows);
  l.rank = 0;
  l.hist = align_up(static_cast<size_t>(entries) * 4);
  l.total = l.hist + align_up(static_cast<size_t>(l.chunks) * (experts + 1) * 4);
  return l;
}

// Private buffers of one expert-major call, carved from the caller's workspace.
// bytes of one fp8 split region (hi, lo, exponent words) of `elems` values
size_t split_bytes(int64_t elems) {
  const size_t e = static_cast<size_t>(elems);
  return align_up(e) * 2 + align_up(e / 16);
}

struct MoeLayout {
  SchedLayout sched;
  size_t offsets, perm, tiles, count, mtiles, act, eo, x_split, act_split;
  size_t x_pair, x_neg, act_neg;  // paired W4A16 input and group sums (direct loads)
  size_t total;
};

// Pointers into one fp8 split region of `elems` values: hi, lo, exponent words.
struct SplitBufs {
  uint8_t* hi;
  uint8_t* lo;
  uint16_t* sc;
};

SplitBufs split_bufs(char* base, int64_t elems) {
  SplitBufs b;
  b.hi = reinterpret_cast<uint8_t*>(base);
  b.lo = b.hi + align_up(static_cast<size_t>(elems));
  b.sc = reinterpret_cast<uint16_t*>(b.lo + align_up(static_cast<size_t>(elems)));
  return b;
}

MoeLayout moe_layout(int64_t entries, int64_t experts, int64_t act_cols, int64_t out_cols,
                     int64_t split_x_elems = 0, int64_t pair_rows = 0, int act_mult = 1) {
  MoeLayout l;
  l.sched = sched_layout(entries, experts);
  size_t at = l.sched.total;
  l.offsets = at;
  at += align_up(static_cast<size_t>(experts + 2) * 4);
  l.perm = at;
  at += align_up(static_cast<size_t>(entries) * 4);
  l.tiles = at;
  at += align_up(static_cast<size_t>(l.sched.max_tiles) * 16);
  l.count = at;  // the tile count, and at +4 bytes the merged 64-row list's
  at += 256;
  // the merged 64-row tile list (direct-load expert GEMMs); its launches read
  // descriptors up to the bound rounded up to 8 tiles before checking the count
  l.mtiles = at;
  at += align_up(static_cast<size_t>((max_tiles_for(entries, experts, kTileRows) + 7) / 8 * 8) * 16);
  // (act_mult 2: the split SwiGLU's [gate | up] rows)
  l.act = at;
  at += align_up(static_cast<size_t>(entries) * act_cols * 2 * act_mult);
  l.eo = at;
  at += align_up(static_cast<size_t>(entries) * out_cols * 2);
  // fp8 hi/lo splits of the gathered input and of the activations (MXFP4 on
  // the scaled fp4 MFMA only): hi and lo bytes plus one exponent word per 32
  l.x_split = at;
  at += split_bytes(split_x_elems);
  l.act_split = at;
  if (split_x_elems > 0) at += split_bytes(entries * act_cols);
  // W4A16 64-row launches: the gathered input (pair_rows rows of out_cols)
  // paired for direct loads, its group sums and the activations' group sums
  // (the gate/up GEMM writes the activations paired in place)
  const bool pairs = pair_rows > 0;
  l.x_pair = at;
  if (pairs) at += align_up(static_cast<size_t>(pair_rows) * out_cols * 2);
  l.x_neg = at;
  if (pairs) at += align_up(static_cast<size_t>(pair_rows) * (out_cols / 128) * 4);
  l.act_neg = at;
  if (pairs) at += align_up(static_cast<size_t>(entries) * (act_cols / 128) * 4);
  l.total = at;
  return l;
}

// Whether one block routes and schedules the batch (schedule_one_kernel with
// routing): at most kFuseRouteTokens tokens, 256 routed experts (four per
// lane) and kFuseThreads token-routes. The path knob moe_fused_schedule=off
// takes the router and schedule launches instead (the same tables).
bool route_schedule_fits(int64_t tokens, int64_t routed, int64_t top_k) {
  if (path_choice(kKnobMoeFusedSchedule) == 1) return false;
  return routed >= 1 && routed <= 256 && top_k >= 1 && top_k <= 32 && top_k <= routed &&
         tokens <= kFuseRouteTokens && tokens * (top_k + 1) <= kFuseThreads;
}

int route_schedule_launch(const float* logits, const float* bias, int64_t* idx, float* weights,
                          int64_t tokens, int64_t routed, int64_t top_k, float scaling,
                          int renormalize, int32_t* offsets, int32_t* perm, int32_t* tiles,
                          int32_t* tile_count, int tile_rows, int32_t* mtiles,
                          int32_t* mtile_count, hipStream_t s) {
  Schedule sc{};
  sc.offsets = offsets;
  sc.perm = perm;
  sc.tiles = tiles;
  sc.tile_count = tile_count;
  sc.tile_rows = tile_rows;
  sc.mtiles = tile_rows == kTileRows ? mtiles : nullptr;
  sc.mtile_count = mtile_count;
  const RouteTable rt{idx, top_k, top_k + 1, routed + 1, routed};
  schedule_one_kernel<true><<<1, kFuseThreads, 0, s>>>(rt, tokens * (top_k + 1), sc, logits, bias,
                                                       idx, weights, static_cast<int>(top_k),
                                                       scaling, renormalize);
  return check_launch("moe router + schedule");
}

int schedule_launch(const RouteTable& rt, int64_t entries, char* ws, const SchedLayout& sl,
                    int32_t* offsets, int32_t* perm, int32_t* tiles, int32_t* tile_count,
                    int tile_rows, hipStream_t s, int32_t* mtiles = nullptr,
                    int32_t* mtile_count = nullptr) {
  Schedule sc{};
  sc.rank = reinterpret_cast<int32_t*>(ws + sl.rank);
  sc.hist = reinterpret_cast<int32_t*>(ws + sl.hist);
  sc.offsets = offsets;
  sc.perm = perm;
  sc.tiles = tiles;
  sc.tile_count = tile_count;
  sc.tile_rows = tile_rows;
  sc.mtiles = tile_rows == kTileRows ? mtiles : nullptr;
  sc.mtile_count = mtile_count;
  // one block of 16 waves where one chunk of kSchedThreads would not cover
  // the table (otherwise the chunk kernel, at 8 waves, is the faster one launch)
  if (entries > kSchedThreads && entries <= kFuseThreads && rt.experts + 1 <= kFuseBuckets &&
      path_choice(kKnobMoeFusedSchedule) != 1) {
    schedule_one_kernel<false><<<1, kFuseThreads, 0, s>>>(rt, entries, sc, nullptr, nullptr, nullptr,
                                                          nullptr, 0, 0.f, 0);
    return check_launch("moe schedule");
  }
  schedule_count_kernel<<<sl.chunks, kSchedThreads, 0, s>>>(rt, entries, sc);
  if (sl.chunks > 1)
    schedule_place_kernel<<<sl.chunks, kSchedThreads, 0, s>>>(rt, entries, sl.chunks, sc);
  return check_launch("moe schedule");
}

// Paired copy + group sums of `rows` bf16 rows of k (k % 128 == 0) for the
// direct-load W4A16 GEMM.
int pair_rows_launch(const uint16_t* x, uint16_t* xp, float* neg, int64_t rows, int64_t k,
                     hipStream_t s) {
  const int64_t units = rows * (k / 128);
  if (units == 0) return LK_OK;
  LK_REQUIRE(k % 128 == 0 && units < (1LL << 27), "pairing: unsupported size");
  pair_rows_kernel<<<static_cast<unsigned>((units + 15) / 16), 256, 0, s>>>(
      x, xp, neg, static_cast<uint32_t>(units));
  return check_launch("moe activation pairing");
}

// route_pair_kernel over `tokens` tokens of k (k % 128 == 0, at most 256
// routed experts; validated by the caller)
int route_pair_launch(const float* logits, const float* bias, int64_t* idx, float* w,
                      int64_t tokens, int64_t routed, int64_t top_k, float scaling, int renorm,
                      const uint16_t* x, uint16_t* xp, float* neg, int64_t k, hipStream_t s) {
  LK_REQUIRE(k % 128 == 0 && tokens * (k / 128) < (1LL << 27) && routed <= 256 &&
                 tokens <= 2147483647LL,
             "router + pairing: unsupported size");
  route_pair_kernel<4><<<static_cast<unsigned>(tokens), kRoutePairThreads, 0, s>>>(
      logits, bias, idx, w, static_cast<int>(routed), static_cast<int>(top_k), scaling, renorm,
      x, xp, neg, static_cast<int>(k / 128));
  return check_launch("moe router + activation pairing");
}

enum class Mode { Gather, Scatter, GatherScatter, Dense };

template <int FMT, int MATS, int NT, bool WIDE>
void gemm_dispatch_mode(const GemmArgs& g, Mode mode, unsigned blocks, hipStream_t s) {
  constexpr int T = kGemmWaves * kWave;
  if constexpr (FMT == kFmtMxF16) {  // fp16 activations: the plain MXFP4 GEMM only
    w4a16_gemm_kernel<FMT, MATS, NT, false, false, false, true><<<blocks, T, 0, s>>>(g);
    return;
  } else {
    switch (mode) {
      case Mode::Gather:
        w4a16_gemm_kernel<FMT, MATS, NT, WIDE, true, false, false><<<blocks, T, 0, s>>>(g);
        break;
      case Mode::Scatter:
        w4a16_gemm_kernel<FMT, MATS, NT, WIDE, false, true, false><<<blocks, T, 0, s>>>(g);
        break;
      case Mode::GatherScatter:
        w4a16_gemm_kernel<FMT, MATS, NT, WIDE, true, true, false><<<blocks, T, 0, s>>>(g);
        break;
      case Mode::Dense:
        w4a16_gemm_kernel<FMT, MATS, NT, WIDE, false, false, true><<<blocks, T, 0, s>>>(g);
        break;
    }
  }
}

// Launches the GEMM over `tiles` row tiles (an upper bound in schedule
// modes); `wide_cols` picks two 16-column tiles per wave.
template <int FMT, int MATS>
int gemm_launch(GemmArgs g, Mode mode, int64_t tiles, bool wide_cols, hipStream_t s,
                const char* what) {
  if constexpr (FMT == kFmtW4A16) {
    LK_REQUIRE(g.k % 32 == 0 && g.group % 32 == 0 && (g.group & (g.group - 1)) == 0,
               "%s: unsupported reduction width / group size", what);
  } else {
    LK_REQUIRE(g.k % 32 == 0 && g.group == 32, "%s: MXFP4 needs k %% 32 == 0", what);
    LK_REQUIRE(FMT != kFmtMxF16 || (mode == Mode::Dense && MATS == 1),
               "%s: fp16 activations are supported by the plain MXFP4 GEMM only", what);
  }
  const bool wide = FMT == kFmtW4A16 && g.group >= 128;
  wide_cols = wide_cols && MATS == 1;  // two matrices x two column tiles exceed 256 VGPRs
  const int nt = wide_cols ? 2 : 1;
  const int bn = kGemmWaves * nt * 16;
  g.col_blocks = static_cast<int>((g.n + bn - 1) / bn);
  const int64_t groups8 = (tiles + 7) / 8;
  const int64_t blocks = groups8 * 8 * g.col_blocks * g.outputs;
  LK_REQUIRE(blocks > 0 && blocks < (1LL << 31), "%s: too many blocks", what);
  const unsigned nb = static_cast<unsigned>(blocks);
  if constexpr (MATS == 1) {
    if (wide) {
      if (wide_cols) gemm_dispatch_mode<FMT, 1, 2, FMT == kFmtW4A16>(g, mode, nb, s);
      else gemm_dispatch_mode<FMT, 1, 1, FMT == kFmtW4A16>(g, mode, nb, s);
    } else {
      if (wide_cols) gemm_dispatch_mode<FMT, 1, 2, false>(g, mode, nb, s);
      else gemm_dispatch_mode<FMT, 1, 1, false>(g, mode, nb, s);
    }
  } else {
    if (wide) gemm_dispatch_mode<FMT, MATS, 1, FMT == kFmtW4A16>(g, mode, nb, s);
    else gemm_dispatch_mode<FMT, MATS, 1, false>(g, mode, nb, s);
  }
  return check_launch(what);
}

template <int FMT, int MATS, int MT, bool WIDE, bool GATHER, bool SCATTER, bool DENSE,
          bool DDIRECT = false>
void stream_one(const GemmArgs& g, unsigned blocks, size_t lds, hipStream_t s) {
  constexpr int NT = MATS == 2 ? 1 : 2;
  auto* fn = &w4a16_stream_kernel<FMT, MATS, NT, MT, WIDE, GATHER, SCATTER, DENSE, DDIRECT>;
  static bool limit_set = false;  // the attribute is per function; set once per process
  if (!limit_set) {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(fn),
                              hipFuncAttributeMaxDynamicSharedMemorySize, kStMaxLds);
    limit_set = true;
  }
  fn<<<blocks, kStWaves * kWave, lds, s>>>(g);
}

// moe_persist=off takes the per-tile streaming kernel for 16-row tiles.
bool persist_disabled() { return path_choice(kKnobMoePersist) == 1; }

template <int FMT, int MATS, int MT, bool WIDE>
void stream_dispatch(const GemmArgs& g, Mode mode, unsigned blocks, size_t lds, hipStream_t s,
                     bool dense_direct = false) {
  if constexpr (FMT == kFmtMxF16) {
    stream_one<FMT, MATS, MT, false, false, false, true>(g, blocks, lds, s);
  } else {
    switch (mode) {
      case Mode::Gather: stream_one<FMT, MATS, MT, WIDE, true, false, false>(g, blocks, lds, s); break;
      case Mode::Scatter: stream_one<FMT, MATS, MT, WIDE, false, true, false>(g, blocks, lds, s); break;
      case Mode::GatherScatter:
        stream_one<FMT, MATS, MT, WIDE, true, true, false>(g, blocks, lds, s);
        break;
      case Mode::Dense:
        if constexpr (MT > 1 && WIDE && (FMT == kFmtW4A16 || FMT == kFmtMxBf16)) {
          if (dense_direct) {
            stream_one<FMT, MATS, MT, WIDE, false, false, true, true>(g, blocks, lds, s);
            break;
          }
        }
        stream_one<FMT, MATS, MT, WIDE, false, false, true>(g, blocks, lds, s);
        break;
    }
  }
}

// Whether the streaming kernel with 16 * mt-row tiles covers this reduction
// (W4A16 groups of 32, 64 or 128, or MXFP4; wider groups use the LDS-staged kernel).
bool stream_fits(int64_t k, int mt, int64_t group, bool mx) {
  if (!mx && group > 128) return false;
  return stream_lds_bytes(k, mt) <= static_cast<size_t>(kStMaxLds);
}

// ---- persistent 16-row streaming GEMM: host side ----

constexpr int kPsMaxLds = 160 * 1024 - 2048;  // dynamic LDS of one persistent block

template <int FMT, int MATS, int DEPTH, bool GATHER, bool SCATTER, bool SPLIT, bool SWI,
          bool ROUTED = false>
int persist_one(const GemmArgs& g, int nbuf, size_t lds, int64_t tiles_bound, hipStream_t s,
                bool launch) {
  auto* fn = &w4a16_persist_kernel<FMT, MATS, DEPTH, GATHER, SCATTER, SPLIT, SWI, ROUTED>;
  struct Cfg {
    int device = -1, blocks_per_cu = 0, cus = 0;
    size_t lds = 0;
  };
  // per device (the attribute is per function); filled and read under one
  // lock, so threads making their first calls at once see a whole entry
  static Cfg cfg[16];
  static std::mutex cfg_lock;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 16) return -1;
  Cfg c;
  {
    std::lock_guard<std::mutex> hold(cfg_lock);
    c = cfg[dev];
  }
  if (c.device != dev || c.lds != lds) {
    // a failed query leaves no error behind for the fallback kernel's launch check
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(fn),
                            hipFuncAttributeMaxDynamicSharedMemorySize, kPsMaxLds) != hipSuccess) {
      (void)hipGetLastError();
      return -1;
    }
    int per_cu = 0, cus = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, kStWaves * kWave, lds) !=
            hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        per_cu < 1 || cus < 1) {
      (void)hipGetLastError();
      return -1;
    }
    c = Cfg{dev, per_cu, cus, lds};
    std::lock_guard<std::mutex> hold(cfg_lock);
    cfg[dev] = c;
  }
  const int64_t grid = static_cast<int64_t>(c.cus) * c.blocks_per_cu;
  if (grid <= 0) return -1;
  constexpr int NT = 1;  // 16-column units, as in the kernel
  const int64_t cgs = (SPLIT ? 2 : 1) * ((g.n + NT * 16 - 1) / (NT * 16));
  // a block's range covers at most (per - 1) / cgs + 2 tiles; its tables hold kPsMaxSegs
  const int64_t per = (tiles_bound * cgs + grid - 1) / grid;
  if ((per - 1) / cgs + 2 > kPsMaxSegs) return -1;
  if (tiles_bound * cgs >= (1LL << 31)) return -1;
  if (launch) fn<<<static_cast<unsigned>(grid), kStWaves * kWave, lds, s>>>(g, nbuf);
  return 0;
}

template <int FMT, int MATS, bool GATHER, bool SCATTER, bool SPLIT, bool SWI,
          bool ROUTED = false>
int persist_depth(const GemmArgs& g, int nbuf, size_t lds, int64_t tiles_bound, hipStream_t s,
                  bool launch) {
  // the ring depth divides the k-steps (at least one whole round per unit)
  const int64_t ksteps = g.k / 128;
  if (ksteps >= 6 && ksteps % 6 == 0)
    return persist_one<FMT, MATS, 6, GATHER, SCATTER, SPLIT, SWI, ROUTED>(g, nbuf, lds,
                                                                          tiles_bound, s, launch);
  if (ksteps >= 8 && ksteps % 8 == 0)
    return persist_one<FMT, MATS, 8, GATHER, SCATTER, SPLIT, SWI, ROUTED>(g, nbuf, lds,
                                                                          tiles_bound, s, launch);
  if (ksteps >= 4 && ksteps % 4 == 0)
    return persist_one<FMT, MATS, 4, GATHER, SCATTER, SPLIT, SWI, ROUTED>(g, nbuf, lds,
                                                                          tiles_bound, s, launch);
  return -1;
}

// Forms of the persistent GEMM: one launch per product (fused gate/up with
// its SwiGLU epilogue, or a single matrix), or the split SwiGLU pair of the
// MoE block (gate/up as one-matrix units writing [rows, 2n], then the down
// GEMM staging its activations through the SwiGLU).
enum class PsForm { Plain, SplitGateUp, SwiDown };

// Launches the persistent 16-row GEMM when it applies (schedule modes, 16-byte
// weight loads, the block's tiles fit in LDS) and returns the launch status;
// returns kPsNotApplicable when it does not, so the caller takes the per-tile
// streaming kernel. With launch == false it only answers whether it applies
// (0) or not (kPsNotApplicable).
constexpr int kPsNotApplicable = -1000;
template <int FMT, int MATS>
int persist_launch(const GemmArgs& g, Mode mode, int64_t tiles_bound, hipStream_t s,
                   const char* what, PsForm form = PsForm::Plain, bool launch = true) {
  if constexpr (FMT != kFmtW4A16 && FMT != kFmtMxBf16) {
    return kPsNotApplicable;
  } else {
    if (persist_disabled() || mode == Mode::Dense || g.outputs != 1) return kPsNotApplicable;
    // W4A16: G = 128 and an even number of groups per row (dword scale pairs stay in the row)
    if (g.k % 128 != 0 || (FMT == kFmtW4A16 && (g.group != 128 || g.k % 256 != 0)))
      return kPsNotApplicable;
    const size_t one = stream_lds_bytes(g.k, 1);
    const int nbuf = 2 * one <= static_cast<size_t>(kPsMaxLds) ? 2 : (one <= static_cast<size_t>(kPsMaxLds) ? 1 : 0);
    if (nbuf == 0) return kPsNotApplicable;
    const size_t lds = nbuf * one;
    // a launch that routes keeps its routing scratch in the activation LDS
    const bool routed = g.rt_logits != nullptr || g.rt_from_idx;
    if (routed) {
      const int n = g.rt_tokens * (g.rt_top_k + 1);
      if (FMT == kFmtMxF16 || n > kRoutedEntries || g.rt_tokens < 1 ||
          (!g.rt_from_idx && g.rt_tokens > kStWaves) ||
          g.rt_routed > 256 ||
          static_cast<size_t>(routed_scratch_words(g.rt_tokens, g.rt_top_k, g.rt_routed + 2)) * 4 >
              lds)
        return kPsNotApplicable;
    }
    // a phase's activations are staged from one batch of registers per thread
    const int half_cap = form == PsForm::SwiDown ? kPsSwiHalfMax : kPsHalfMax;
    if (g.k / 128 > 2 * half_cap) return kPsNotApplicable;
    int rc = -1;
    if constexpr (MATS == 1) {
      if (form == PsForm::SplitGateUp) {
        if (mode != Mode::Gather || g.act != kActSwiglu) return kPsNotApplicable;
        if (routed)  // the block routes (or ranks) and schedules the batch itself
          rc = persist_depth<FMT, 1, true, false, true, false, true>(g, nbuf, lds, tiles_bound, s,
                                                                     launch);
        else
          rc = persist_depth<FMT, 1, true, false, true, false>(g, nbuf, lds, tiles_bound, s, launch);
      } else if (form == PsForm::SwiDown) {
        if (mode != Mode::Scatter || g.act != kActSwiglu) return kPsNotApplicable;
        rc = persist_depth<FMT, 1, false, true, false, true>(g, nbuf, lds, tiles_bound, s, launch);
      }
    }
    if (form == PsForm::Plain) {
      switch (mode) {
        case Mode::Gather:
          rc = persist_depth<FMT, MATS, true, false, false, false>(g, nbuf, lds, tiles_bound, s, launch);
          break;
        case Mode::Scatter:
          rc = persist_depth<FMT, MATS, false, true, false, false>(g, nbuf, lds, tiles_bound, s, launch);
          break;
        case Mode::GatherScatter:
          if constexpr (MATS == 2) {
            if (routed) {  // the block routes (or ranks) and schedules the batch itself
              rc = persist_depth<FMT, MATS, true, true, false, false, true>(g, nbuf, lds,
                                                                            tiles_bound, s, launch);
              break;
            }
          }
          rc = persist_depth<FMT, MATS, true, true, false, false>(g, nbuf, lds, tiles_bound, s, launch);
          break;
        default: break;
      }
    }
    if (rc < 0) return kPsNotApplicable;
    return launch ? check_launch(what) : 0;
  }
}

template <int FMT, int MATS>
int stream_launch(GemmArgs g, Mode mode, int64_t tiles, int mt, hipStream_t s, const char* what) {
  constexpr int NT = MATS == 2 ? 1 : 2;
  // W4A16 G == 128 (wider groups use the LDS-staged kernel) or MXFP4 with k % 128 == 0
  const bool wide = FMT == kFmtW4A16 ? g.group >= 128 : (FMT == kFmtMxBf16 && g.k % 128 == 0);
  constexpr bool kWideOk = FMT != kFmtMxF16;
  const size_t lds = stream_lds_bytes(g.k, mt);
  LK_REQUIRE(lds <= static_cast<size_t>(kStMaxLds), "%s: reduction width too large", what);
  // 64-row launches: tiles of <= 16 rows run the 16-row path when all of
  // their activations fit the LDS the launch takes anyway
  g.tail16 = mt > 1 && stream_lds_bytes(g.k, 1) <= lds ? 1 : 0;
  // 64-row gather / scatter launches load activations directly (byte
  // offsets of 32 bits; W4A16 from the paired copy)
  if (mt > 1 && wide && FMT != kFmtMxF8 && (mode == Mode::Gather || mode == Mode::Scatter)) {
    LK_REQUIRE(g.a_rows > 0 && g.a_rows * g.k * 2 <= static_cast<int64_t>(kMaxDirectBytes),
               "%s: activations out of range for direct loads", what);
    LK_REQUIRE(FMT != kFmtW4A16 || (g.a_pair && g.a_neg), "%s: paired activations missing", what);
    LK_REQUIRE(g.n % 8 == 0 && (!g.out_neg || (MATS == 2 && g.n % 128 == 0)),
               "%s: output width %lld unsupported for direct loads", what, (long long)g.n);
    LK_REQUIRE(g.mtiles && g.mtile_count, "%s: merged tile list missing", what);
    g.tiles = g.mtiles;
    g.tile_count = g.mtile_count;
  }
  // dense 64-row launches load their rows directly as well when they can:
  // MXFP4 from the rows themselves, W4A16 from a paired copy with its group
  // sums (a_pair / a_neg, made by the caller's pre-pass)
  const bool dense_direct = mt > 1 && wide && mode == Mode::Dense && g.n % 8 == 0 &&
                            g.a_rows > 0 &&
                            g.a_rows * g.k * 2 <= static_cast<int64_t>(kMaxDirectBytes) &&
                            (FMT == kFmtMxBf16 || (FMT == kFmtW4A16 && g.a_pair && g.a_neg));
  g.col_blocks = static_cast<int>((g.n + kStWaves * NT * 16 - 1) / (kStWaves * NT * 16));
  const int64_t blocks = (tiles + 7) / 8 * 8 * g.col_blocks * g.outputs;
  LK_REQUIRE(blocks > 0 && blocks < (1LL << 31), "%s: too many blocks", what);
  const unsigned nb = static_cast<unsigned>(blocks);
  if constexpr (FMT == kFmtMxF8) {  // 16-byte weight loads only
    LK_REQUIRE(g.k % 128 == 0, "%s: the scaled fp4 MFMA needs k %% 128 == 0", what);
    if (mt == 1) stream_dispatch<FMT, MATS, 1, true>(g, mode, nb, lds, s);
    else stream_dispatch<FMT, MATS, 4, true>(g, mode, nb, lds, s);
  } else if (mt == 1) {
    if (wide) {
      const int rc = persist_launch<FMT, MATS>(g, mode, tiles, s, what);
      if (rc != kPsNotApplicable) return rc;
    }
    if (wide) stream_dispatch<FMT, MATS, 1, kWideOk>(g, mode, nb, lds, s);
    else stream_dispatch<FMT, MATS, 1, false>(g, mode, nb, lds, s);
  } else {
    if (wide) stream_dispatch<FMT, MATS, 4, kWideOk>(g, mode, nb, lds, s, dense_direct);
    else stream_dispatch<FMT, MATS, 4, false>(g, mode, nb, lds, s);
  }
  return check_launch(what);
}

// Wider column blocks once there are enough tiles to fill the machine.
bool wide_cols_for(int64_t tiles, int64_t n) { return tiles * ((n + 63) / 64) >= 2048; }

// Dense products (dense GEMM, fused QKV, MXFP4 GEMM) from 16 rows: the
// streaming kernel with 64-row tiles (weights in a register ring, activations
// in LDS passes) where it covers the format, else the LDS-staged GEMM. On the
// fused QKV projection of 2048 tokens ([2048, 2304] x [2304, 3 x 4096]) the
// streaming kernel takes 226 us, the LDS-staged GEMM 421 us. The path knob
// dense_gemm=lds forces the LDS-staged GEMM.
template <int FMT>
int dense_launch(const GemmArgs& g, int64_t tiles, hipStream_t s, const char* what) {
  const bool lds = path_choice(kKnobDenseGemm) == 1;
  if (!lds && stream_fits(g.k, 4, g.group, FMT != kFmtW4A16))
    return stream_launch<FMT, 1>(g, Mode::Dense, tiles, 4, s, what);
  return gemm_launch<FMT, 1>(g, Mode::Dense, tiles, wide_cols_for(tiles * g.outputs, g.n), s, what);
}

int check_schedule_dims(int64_t tokens, int64_t routes, int64_t experts) {
  LK_REQUIRE(experts > 0 && experts + 1 <= kMaxBuckets, "expert-major schedule supports 1..%d experts",
             kMaxBuckets - 1);
  LK_REQUIRE(tokens >= 0 && routes > 0, "invalid route table dimensions");
  LK_REQUIRE(tokens * routes < (1LL << 30), "too many token-routes for one call");
  return LK_OK;
}

template <int MATS>
int launch_fmt(bool mx, const GemmArgs& g, Mode mode, int64_t tiles, bool wide_cols,
                      hipStream_t s, const char* what) {
  if (mx) return gemm_launch<kFmtMxBf16, MATS>(g, mode, tiles, wide_cols, s, what);
  return gemm_launch<kFmtW4A16, MATS>(g, mode, tiles, wide_cols, s, what);
}

template <int MATS>
int stream_fmt(bool mx, const GemmArgs& g, Mode mode, int64_t tiles, int mt, hipStream_t s,
               const char* what) {
  if (mx) return stream_launch<kFmtMxBf16, MATS>(g, mode, tiles, mt, s, what);
  return stream_launch<kFmtW4A16, MATS>(g, mode, tiles, mt, s, what);
}

// Expert-major calls use the streaming kernel: 16-row tiles up to
// kStreamSmallEntries token-routes (decode batches, few rows per expert),
// 64-row tiles above (prefill). The path knob moe_gemm=lds selects the
// LDS-staged kernel instead, moe_gemm=stream16|stream64 forces a tile height.
constexpr int64_t kStreamSmallEntries = 2048;

// Which MFMA form the MXFP4 expert GEMMs take: bf16 MFMA on weights decoded
// by the scaled convert unless the path knob mxfp4_mfma=fp4 asks for the
// scaled fp4 MFMA (raw fp4 weights, activations split into fp8 hi + lo). The
// split keeps bf16 precision but takes two scaled MFMAs per 128-wide k-step,
// the same MFMA time as four bf16 ones, plus two split launches: a 2048-token
// Kimi-Linear layer measured 581 us in the bf16 form against 620 us, and 64
// tokens 145 against 196 us.
bool mxfp4_scaled_mfma() { return path_choice(kKnobMxfp4Mfma) == 1; }

// 16-row tiles -> 1, 64-row tiles -> 4, the LDS-staged kernel -> 0.
int stream_tile_mt(int64_t entries) {
  switch (path_choice(kKnobMoeGemm)) {
    case 1: return 0;
    case 2: return 1;
    case 3: return 4;
    default: return entries <= kStreamSmallEntries ? 1 : 4;
  }
}

// Whether an expert-major W4A16 call of `entries` token-routes sizes the
// paired-activation buffers of its 64-row launches into the workspace (the
// workspace query and the call agree through this; calls whose group is not
// 128 leave them unused).
bool moe_pairs(int64_t entries, bool mx) { return !mx && stream_tile_mt(entries) == 4; }

// Whether an expert-major call of `entries` token-routes sizes its activation
// region for the split SwiGLU of the 16-row launches ([gate | up] rows, twice
// the SwiGLU's width); the workspace query and the call agree through this.
int moe_act_mult(int64_t entries) { return stream_tile_mt(entries) == 1 ? 2 : 1; }

template <int MATS>
int persist_fmt(bool mx, const GemmArgs& g, Mode mode, int64_t tiles_bound, hipStream_t s,
                const char* what, PsForm form, bool launch) {
  if (mx) return persist_launch<kFmtMxBf16, MATS>(g, mode, tiles_bound, s, what, form, launch);
  return persist_launch<kFmtW4A16, MATS>(g, mode, tiles_bound, s, what, form, launch);
}

// W4A16: a power-of-two group (multiple of 32) dividing k; MXFP4: 32.
int check_format(bool mx, int64_t k, int64_t group) {
  if (mx) {
    LK_REQUIRE(k > 0 && k % 32 == 0, "MXFP4 reduction dimension must be divisible by 32");
    return LK_OK;
  }
  return check_pow2_group(k, group);
}

void dense_args(GemmArgs& g, const uint16_t* x, int64_t m, int64_t n, int64_t k,
                       int64_t group) {
  g.a = x;
  g.n = n;
  g.k = k;
  g.group = group;
  g.routes = 1;
  g.dense_rows = static_cast<int>(m);
  g.outputs = 1;
  g.act = kActSwiglu;
}

// Workspace of a dense W4A16 product whose 64-row launches load their rows
// directly: the rows paired in the weight decode's k order and their group
// sums (G = 128, k % 128 == 0, from 16 rows); 0 where that form does not apply.
int64_t dense_pair_bytes(int64_t m, int64_t k, int64_t group) {
  if (m < 16 || group != 128 || k % 128 != 0) return 0;
  return static_cast<int64_t>(align_up(static_cast<size_t>(m * k * 2)) +
                              align_up(static_cast<size_t>(m * (k / 128) * 4)));
}

// The pre-pass of the direct form: pairs x into the workspace and points the
// launch at it.
int dense_pairs(GemmArgs& g, const uint16_t* x, int64_t m, int64_t k, int64_t group,
                void* workspace, int64_t workspace_bytes, hipStream_t s, const char* what) {
  const int64_t need = dense_pair_bytes(m, k, group);
  if (need == 0) return LK_OK;
  LK_REQUIRE(workspace != nullptr && workspace_bytes >= need,
             "%s: workspace too small: %lld < %lld bytes", what, (long long)workspace_bytes,
             (long long)need);
  auto* xp = static_cast<uint16_t*>(workspace);
  auto* neg = reinterpret_cast<float*>(static_cast<char*>(workspace) +
                                       align_up(static_cast<size_t>(m * k * 2)));
  if (int rc = pair_rows_launch(x, xp, neg, m, k, s)) return rc;
  g.a_pair = xp;
  g.a_neg = neg;
  g.a_rows = m;
  return LK_OK;
}

}  // namespace
}  // namespace lk

using namespace lk;

extern "C" {

int lk_moe_schedule_sizes(int64_t tokens, int64_t routes, int64_t experts, int64_t* max_tiles,
                          int64_t* workspace_bytes) {
  if (int rc = check_schedule_dims(tokens, routes, experts)) return rc;
  LK_REQUIRE(max_tiles && workspace_bytes, "null pointer argument");
  const SchedLayout l = sched_layout(tokens * routes, experts);
  *max_tiles = l.max_tiles;
  *workspace_bytes = static_cast<int64_t>(l.total);
  return LK_OK;
}

int lk_moe_schedule(const int64_t* expert_indices, int64_t tokens, int64_t routes,
                    int64_t experts, int64_t shared_expert, int64_t tile_rows, int32_t* offsets,
                    int32_t* perm, int32_t* tiles, int32_t* tile_count, void* workspace,
                    int64_t workspace_bytes, void* stream) {
  const int64_t r_total = routes + (shared_expert >= 0 ? 1 : 0);
  LK_REQUIRE(tile_rows == kSmallTileRows || tile_rows == kTileRows,
             "tile rows must be %d or %d", kSmallTileRows, kTileRows);
  if (int rc = check_schedule_dims(tokens, r_total, experts)) return rc;
  LK_REQUIRE(shared_expert < experts, "shared expert id %lld outside the bank",
             (long long)shared_expert);
  LK_REQUIRE(offsets && perm && tiles && tile_count && workspace, "null pointer argument");
  LK_REQUIRE(routes > 0 || shared_expert >= 0, "empty route table");
  const int64_t entries = tokens * r_total;
  const SchedLayout l = sched_layout(entries, experts);
  LK_REQUIRE(workspace_bytes >= static_cast<int64_t>(l.total),
             "schedule workspace too small: %lld < %lld bytes", (long long)workspace_bytes,
             (long long)l.total);
  if (entries == 0) {  // a fill kernel (no memset node when the call is captured)
    hipStream_t s = as_stream(stream);
    fill_i32_kernel<<<static_cast<unsigned>((experts + 2 + 255) / 256), 256, 0, s>>>(
        offsets, experts + 2, tile_count);
    return check_launch("lk_moe_schedule");
  }
  LK_REQUIRE(expert_indices != nullptr || routes == 0, "null pointer argument");
  const RouteTable rt{expert_indices, routes, r_total, experts, shared_expert};
  return schedule_launch(rt, entries, static_cast<char*>(workspace), l, offsets, perm, tiles,
                         tile_count, static_cast<int>(tile_rows), as_stream(stream));
}

int64_t lk_w4a16_grouped_gemm_workspace(int64_t tokens, int64_t routes, int64_t experts) {
  if (check_schedule_dims(tokens, routes, experts)) return -1;
  return static_cast<int64_t>(moe_layout(tokens * routes, experts, 0, 0).total);
}

static int grouped_gemm_common(bool mx, const uint16_t* x, const int64_t* idx, const uint8_t* p0,
                               const void* s0, const uint8_t* p1, const void* s1, uint16_t* out,
                               int64_t tokens, int64_t routes, int64_t experts, int64_t n,
                               int64_t k, int64_t group, void* workspace,
                               int64_t workspace_bytes, void* stream, bool swiglu,
                               const char* name) {
  LK_REQUIRE(p0 && s0 && out && (!swiglu || (p1 && s1)), "null pointer argument");
  LK_REQUIRE(routes > 0 && experts > 0 && n > 0 && tokens >= 0,
             "%s requires nonzero dimensions", name);
  if (int rc = check_format(mx, k, group)) return rc;
  if (int rc = check_schedule_dims(tokens, routes, experts)) return rc;
  if (tokens == 0) return LK_OK;
  LK_REQUIRE(x && idx && workspace, "null pointer argument");
  const int64_t entries = tokens * routes;
  const MoeLayout l = moe_layout(entries, experts, 0, 0);
  LK_REQUIRE(workspace_bytes >= static_cast<int64_t>(l.total),
             "%s: workspace too small: %lld < %lld bytes", name, (long long)workspace_bytes,
             (long long)l.total);
  char* ws = static_cast<char*>(workspace);
  hipStream_t s = as_stream(stream);
  auto* offsets = reinterpret_cast<int32_t*>(ws + l.offsets);
  auto* perm = reinterpret_cast<int32_t*>(ws + l.perm);
  auto* tiles = reinterpret_cast<int32_t*>(ws + l.tiles);
  auto* count = reinterpret_cast<int32_t*>(ws + l.count);
  int mt = stream_tile_mt(entries);
  if (mt && !stream_fits(k, mt, group, mx)) mt = 0;
  const int tr = mt == 1 ? kSmallTileRows : kTileRows;
  const RouteTable rt{idx, routes, routes, experts, -1};
  if (int rc = schedule_launch(rt, entries, ws, l.sched, offsets, perm, tiles, count, tr, s))
    return rc;
  GemmArgs g{};
  g.a = x;
  g.perm = perm;
  g.tiles = tiles;
  g.tile_count = count;
  g.wp[0] = p0;
  g.ws[0] = s0;
  g.wp[1] = swiglu ? p1 : p0;
  g.ws[1] = swiglu ? s1 : s0;
  g.wp[2] = p0;
  g.ws[2] = s0;
  g.out[0] = g.out[1] = g.out[2] = out;
  g.n = n;
  g.k = k;
  g.group = mx ? 32 : group;
  g.wstride = n * k / 2;
  g.sstride = n * (k / g.group);
  g.routes = routes;
  g.outputs = 1;
  g.act = kActSwiglu;
  const int64_t tiles_bound = max_tiles_for(entries, experts, tr);
  if (mt) {
    if (swiglu) return stream_fmt<2>(mx, g, Mode::GatherScatter, tiles_bound, mt, s, name);
    return stream_fmt<1>(mx, g, Mode::GatherScatter, tiles_bound, mt, s, name);
  }
  const bool wc = wide_cols_for(tiles_bound, n);
  if (swiglu) return launch_fmt<2>(mx, g, Mode::GatherScatter, tiles_bound, wc, s, name);
  return launch_fmt<1>(mx, g, Mode::GatherScatter, tiles_bound, wc, s, name);
}

int lk_w4a16_grouped_gemm(const uint16_t* x, const int64_t* expert_indices,
                          const uint8_t* packed, const uint16_t* scales, uint16_t* out,
                          int64_t tokens, int64_t routes, int64_t experts, int64_t n, int64_t k,
                          int64_t group_size, void* workspace, int64_t workspace_bytes,
                          void* stream) {
  return grouped_gemm_common(false, x, expert_indices, packed, scales, nullptr, nullptr, out,
                             tokens, routes, experts, n, k, group_size, workspace,
                             workspace_bytes, stream, false, "lk_w4a16_grouped_gemm");
}

int lk_w4a16_swiglu_gemm(const uint16_t* x, const int64_t* expert_indices,
                         const uint8_t* w1_packed, const uint16_t* w1_scales,
                         const uint8_t* w3_packed, const uint16_t* w3_scales, uint16_t* out,
                         int64_t tokens, int64_t routes, int64_t experts, int64_t n, int64_t k,
                         int64_t group_size, void* workspace, int64_t workspace_bytes,
                         void* stream) {
  return grouped_gemm_common(false, x, expert_indices, w1_packed, w1_scales, w3_packed,
                             w3_scales, out, tokens, routes, experts, n, k, group_size, workspace,
                             workspace_bytes, stream, true, "lk_w4a16_swiglu_gemm");
}

int lk_mxfp4_grouped_gemm(const uint16_t* x, const int64_t* expert_indices,
                          const uint8_t* packed, const uint8_t* scale, uint16_t* out,
                          int64_t tokens, int64_t routes, int64_t experts, int64_t n, int64_t k,
                          void* workspace, int64_t workspace_bytes, void* stream) {
  return grouped_gemm_common(true, x, expert_indices, packed, scale, nullptr, nullptr, out,
                             tokens, routes, experts, n, k, 32, workspace, workspace_bytes,
                             stream, false, "lk_mxfp4_grouped_gemm");
}

int lk_mxfp4_swiglu_gemm(const uint16_t* x, const int64_t* expert_indices,
                         const uint8_t* w1_packed, const uint8_t* w1_scale,
                         const uint8_t* w3_packed, const uint8_t* w3_scale, uint16_t* out,
                         int64_t tokens, int64_t routes, int64_t experts, int64_t n, int64_t k,
                         void* workspace, int64_t workspace_bytes, void* stream) {
  return grouped_gemm_common(true, x, expert_indices, w1_packed, w1_scale, w3_packed, w3_scale,
                             out, tokens, routes, experts, n, k, 32, workspace, workspace_bytes,
                             stream, true, "lk_mxfp4_swiglu_gemm");
}

int lk_w4a16_dense_gemm(const uint16_t* x, const uint8_t* packed, const uint16_t* scales,
                        uint16_t* y, int64_t m, int64_t n, int64_t k, int64_t group_size,
                        void* stream) {
  LK_REQUIRE(packed && scales && y, "null pointer argument");
  LK_REQUIRE(m >= 0 && n > 0, "invalid dense dimensions m=%lld n=%lld", (long long)m,
             (long long)n);
  if (int rc = check_pow2_group(k, group_size)) return rc;
  if (m == 0) return LK_OK;
  LK_REQUIRE(x != nullptr, "null activation pointer");
  LK_REQUIRE(m < (1LL << 30), "too many rows");
  GemmArgs g{};
  dense_args(g, x, m, n, k, group_size);
  g.wp[0] = g.wp[1] = g.wp[2] = packed;
  g.ws[0] = g.ws[1] = g.ws[2] = scales;
  g.out[0] = g.out[1] = g.out[2] = y;
  const int64_t tiles = (m + kTileRows - 1) / kTileRows;
  return dense_launch<kFmtW4A16>(g, tiles, as_stream(stream), "lk_w4a16_dense_gemm");
}

int lk_mxfp4_gemm(const uint16_t* x, const uint8_t* packed, const uint8_t* scale, uint16_t* y,
                  int64_t m, int64_t n, int64_t k, int act_f16, void* stream) {
  LK_REQUIRE(packed && scale && y, "null pointer argument");
  LK_REQUIRE(m >= 0 && n > 0, "reduction and output dimensions must be nonzero");
  if (int rc = check_format(true, k, 32)) return rc;
  if (m == 0) return LK_OK;
  LK_REQUIRE(x != nullptr, "null activation pointer");
  LK_REQUIRE(m < (1LL << 30), "too many rows");
  GemmArgs g{};
  dense_args(g, x, m, n, k, 32);
  g.a_rows = m;  // bf16 rows load directly (the fp16 form stages them)
  g.wp[0] = g.wp[1] = g.wp[2] = packed;
  g.ws[0] = g.ws[1] = g.ws[2] = scale;
  g.out[0] = g.out[1] = g.out[2] = y;
  const int64_t tiles = (m + kTileRows - 1) / kTileRows;
  if (act_f16)
    return dense_launch<kFmtMxF16>(g, tiles, as_stream(stream), "lk_mxfp4_gemm");
  return dense_launch<kFmtMxBf16>(g, tiles, as_stream(stream), "lk_mxfp4_gemm");
}

int lk_mxfp4_expert_mlp(const uint16_t* x, const uint8_t* w1_packed, const uint8_t* w1_scale,
                        const uint8_t* w3_packed, const uint8_t* w3_scale,
                        const uint8_t* w2_packed, const uint8_t* w2_scale, uint16_t* y,
                        uint16_t* activated, int64_t m, int64_t h, int64_t i, float situ_beta,
                        float situ_linear_beta, void* stream) {
  LK_REQUIRE(w1_packed && w1_scale && w3_packed && w3_scale && w2_packed && w2_scale && y &&
                 activated,
             "null pointer argument");
  LK_REQUIRE(m >= 0 && h > 0 && i > 0, "invalid expert dimensions");
  if (int rc = check_format(true, h, 32)) return rc;
  if (int rc = check_format(true, i, 32)) return rc;
  LK_REQUIRE(situ_beta != 0.f, "SiTU beta must be nonzero");
  if (m == 0) return LK_OK;
  LK_REQUIRE(x != nullptr, "null activation pointer");
  LK_REQUIRE(m < (1LL << 30), "too many rows");
  hipStream_t s = as_stream(stream);
  const int64_t tiles = (m + kTileRows - 1) / kTileRows;
  GemmArgs g{};
  dense_args(g, x, m, i, h, 32);
  g.act = kActSitu;
  g.situ_beta = situ_beta;
  g.situ_linear_beta = situ_linear_beta;
  g.wp[0] = w1_packed;
  g.ws[0] = w1_scale;
  g.wp[1] = w3_packed;
  g.ws[1] = w3_scale;
  g.wp[2] = w1_packed;
  g.ws[2] = w1_scale;
  g.out[0] = g.out[1] = g.out[2] = activated;
  if (int rc = gemm_launch<kFmtMxBf16, 2>(g, Mode::Dense, tiles, false, s, "mxfp4 expert gate/up"))
    return rc;
  GemmArgs d{};
  dense_args(d, activated, m, h, i, 32);
  d.wp[0] = d.wp[1] = d.wp[2] = w2_packed;
  d.ws[0] = d.ws[1] = d.ws[2] = w2_scale;
  d.out[0] = d.out[1] = d.out[2] = y;
  return gemm_launch<kFmtMxBf16, 1>(d, Mode::Dense, tiles, wide_cols_for(tiles, h), s,
                                    "mxfp4 expert down");
}

int lk_w4a16_fused_qkv(const uint16_t* x, const uint8_t* q_packed, const uint16_t* q_scales,
                       const uint8_t* k_packed, const uint16_t* k_scales,
                       const uint8_t* v_packed, const uint16_t* v_scales, uint16_t* q,
                       uint16_t* k_out, uint16_t* v, int64_t m, int64_t n, int64_t k,
                       int64_t group_size, void* stream) {
  LK_REQUIRE(q_packed && q_scales && k_packed && k_scales && v_packed && v_scales && q && k_out &&
                 v,
             "null pointer argument");
  LK_REQUIRE(m >= 0 && n > 0, "invalid QKV dimensions m=%lld n=%lld", (long long)m,
             (long long)n);
  if (int rc = check_pow2_group(k, group_size)) return rc;
  if (m == 0) return LK_OK;
  LK_REQUIRE(x != nullptr, "null activation pointer");
  if (m < 16) {  // decode rows: one K-split GEMV launch over the three projections
    const DenseMats mats{{q_packed, k_packed, v_packed}, {q_scales, k_scales, v_scales},
                         {q, k_out, v}};
    return dense_multi(x, mats, 3, m, n, k, group_size, as_stream(stream), "lk_w4a16_fused_qkv");
  }
  LK_REQUIRE(m < (1LL << 30), "too many rows");
  GemmArgs g{};
  dense_args(g, x, m, n, k, group_size);
  g.wp[0] = q_packed;
  g.wp[1] = k_packed;
  g.wp[2] = v_packed;
  g.ws[0] = q_scales;
  g.ws[1] = k_scales;
  g.ws[2] = v_scales;
  g.out[0] = q;
  g.out[1] = k_out;
  g.out[2] = v;
  g.outputs = 3;
  const int64_t tiles = (m + kTileRows - 1) / kTileRows;
  return dense_launch<kFmtW4A16>(g, tiles, as_stream(stream), "lk_w4a16_fused_qkv");
}

int64_t lk_w4a16_dense_gemm_workspace(int64_t m, int64_t k, int64_t group_size) {
  if (m < 0 || k <= 0 || group_size <= 0) return -1;
  return dense_pair_bytes(m, k, group_size);
}

int lk_w4a16_dense_gemm_ws(const uint16_t* x, const uint8_t* packed, const uint16_t* scales,
                           uint16_t* y, int64_t m, int64_t n, int64_t k, int64_t group_size,
                           void* workspace, int64_t workspace_bytes, void* stream) {
  LK_REQUIRE(packed && scales && y, "null pointer argument");
  LK_REQUIRE(m >= 0 && n > 0, "invalid dense dimensions m=%lld n=%lld", (long long)m,
             (long long)n);
  if (int rc = check_pow2_group(k, group_size)) return rc;
  if (m == 0) return LK_OK;
  LK_REQUIRE(x != nullptr, "null activation pointer");
  LK_REQUIRE(m < (1LL << 30), "too many rows");
  GemmArgs g{};
  dense_args(g, x, m, n, k, group_size);
  g.wp[0] = g.wp[1] = g.wp[2] = packed;
  g.ws[0] = g.ws[1] = g.ws[2] = scales;
  g.out[0] = g.out[1] = g.out[2] = y;
  hipStream_t s = as_stream(stream);
  if (int rc = dense_pairs(g, x, m, k, group_size, workspace, workspace_bytes, s,
                           "lk_w4a16_dense_gemm_ws"))
    return rc;
  const int64_t tiles = (m + kTileRows - 1) / kTileRows;
  return dense_launch<kFmtW4A16>(g, tiles, s, "lk_w4a16_dense_gemm_ws");
}

int lk_w4a16_fused_qkv_ws(const uint16_t* x, const uint8_t* q_packed, const uint16_t* q_scales,
                          const uint8_t* k_packed, const uint16_t* k_scales,
                          const uint8_t* v_packed, const uint16_t* v_scales, uint16_t* q,
                          uint16_t* k_out, uint16_t* v, int64_t m, int64_t n, int64_t k,
                          int64_t group_size, void* workspace, int64_t workspace_bytes,
                          void* stream) {
  LK_REQUIRE(q_packed && q_scales && k_packed && k_scales && v_packed && v_scales && q && k_out &&
                 v,
             "null pointer argument");
  LK_REQUIRE(m >= 0 && n > 0, "invalid QKV dimensions m=%lld n=%lld", (long long)m,
             (long long)n);
  if (int rc = check_pow2_group(k, group_size)) return rc;
  if (m == 0) return LK_OK;
  LK_REQUIRE(x != nullptr, "null activation pointer");
  if (m < 16)  // decode rows: the GEMV path needs no workspace
    return lk_w4a16_fused_qkv(x, q_packed, q_scales, k_packed, k_scales, v_packed, v_scales, q,
                              k_out, v, m, n, k, group_size, stream);
  LK_REQUIRE(m < (1LL << 30), "too many rows");
  GemmArgs g{};
  dense_args(g, x, m, n, k, group_size);
  g.wp[0] = q_packed;
  g.wp[1] = k_packed;
  g.wp[2] = v_packed;
  g.ws[0] = q_scales;
  g.ws[1] = k_scales;
  g.ws[2] = v_scales;
  g.out[0] = q;
  g.out[1] = k_out;
  g.out[2] = v;
  g.outputs = 3;
  hipStream_t s = as_stream(stream);
  if (int rc = dense_pairs(g, x, m, k, group_size, workspace, workspace_bytes, s,
                           "lk_w4a16_fused_qkv_ws"))
    return rc;
  const int64_t tiles = (m + kTileRows - 1) / kTileRows;
  return dense_launch<kFmtW4A16>(g, tiles, s, "lk_w4a16_fused_qkv_ws");
}

int64_t lk_w4a16_moe_forward_workspace(int64_t tokens, int64_t experts, int64_t h, int64_t i,
                                       int64_t top_k) {
  if (tokens < 0 || experts < 2 || h <= 0 || i <= 0 || top_k <= 0) return -1;
  if (check_schedule_dims(tokens, top_k + 1, experts)) return -1;
  const int64_t entries = tokens * (top_k + 1);
  return static_cast<int64_t>(moe_layout(entries, experts, i, h, 0,
                                         moe_pairs(entries, false) ? tokens : 0,
                                         moe_act_mult(entries))
                                  .total);
}

int64_t lk_mxfp4_moe_forward_workspace(int64_t tokens, int64_t experts, int64_t h, int64_t i,
                                       int64_t top_k) {
  if (tokens < 0 || experts < 2 || h <= 0 || i <= 0 || top_k <= 0) return -1;
  if (check_schedule_dims(tokens, top_k + 1, experts)) return -1;
  const int64_t entries = tokens * (top_k + 1);
  return static_cast<int64_t>(
      moe_layout(entries, experts, i, h, tokens * h, 0, moe_act_mult(entries)).total);
}

int lk_mxfp4_split_activations(const uint16_t* x, uint8_t* hi, uint8_t* lo, uint16_t* scales,
                               int64_t rows, int64_t k, void* stream) {
  LK_REQUIRE(rows >= 0 && k > 0 && k % 32 == 0, "fp8 split needs rows >= 0 and k %% 32 == 0");
  if (rows == 0) return LK_OK;
  LK_REQUIRE(x && hi && lo && scales, "null pointer argument");
  return split_launch(x, hi, lo, scales, rows, k, as_stream(stream));
}

// Largest batch whose expert-major block ends in the token-major W2 + combine
// launch instead of the down GEMM and the combine kernel. Measured at the
// Kimi-Linear shape (Zipf routing): 4 tokens 40.96 -> 39.34 us; 6, 8 and 12
// tokens slower (46.96 -> 48.85, 52.32 -> 56.93, 62.88 -> 74.37 us), the
// experts' W2 rows then being read once per route.
constexpr int64_t kW2RowsMaxTokens = 4;

static int moe_forward_common(bool mx, const uint16_t* x, const float* logits, const float* bias,
                              const uint8_t* w1_packed, const void* w1_scales,
                              const uint8_t* w3_packed, const void* w3_scales,
                              const uint8_t* w2_packed, const void* w2_scales, uint16_t* y,
                              int64_t* expert_indices, float* weights, void* workspace,
                              int64_t workspace_bytes, int64_t tokens, int64_t experts,
                              int64_t h, int64_t i, int64_t top_k, float routed_scaling_factor,
                              int renormalize, int64_t group_size, void* stream) {
  LK_REQUIRE(w1_packed && w1_scales && w3_packed && w3_scales && w2_packed && w2_scales && y &&
                 expert_indices && weights,
             "null pointer argument");
  LK_REQUIRE(experts >= 2, "experts (routed + shared) must be at least 2");
  LK_REQUIRE(top_k > 0 && top_k <= 32 && top_k <= experts - 1, "invalid top_k %lld",
             (long long)top_k);
  LK_REQUIRE(h > 0 && i > 0 && tokens >= 0, "invalid dimensions");
  LK_REQUIRE(h % 8 == 0, "hidden size must be a multiple of 8, got %lld", (long long)h);
  if (int rc = check_format(mx, h, group_size)) return rc;
  if (int rc = check_format(mx, i, group_size)) return rc;
  if (int rc = check_schedule_dims(tokens, top_k + 1, experts)) return rc;
  if (tokens == 0) return LK_OK;
  LK_REQUIRE(x && logits && workspace, "null pointer argument");
  const int64_t routes = top_k + 1;
  const int64_t entries = tokens * routes;
  const MoeLayout l = moe_layout(entries, experts, i, h, mx ? tokens * h : 0,
                                 moe_pairs(entries, mx) ? tokens : 0, moe_act_mult(entries));
  LK_REQUIRE(workspace_bytes >= static_cast<int64_t>(l.total),
             "MoE workspace too small: %lld < %lld bytes", (long long)workspace_bytes,
             (long long)l.total);
  hipStream_t s = as_stream(stream);
  char* ws = static_cast<char*>(workspace);
  auto* offsets = reinterpret_cast<int32_t*>(ws + l.offsets);
  auto* perm = reinterpret_cast<int32_t*>(ws + l.perm);
  auto* tiles = reinterpret_cast<int32_t*>(ws + l.tiles);
  auto* count = reinterpret_cast<int32_t*>(ws + l.count);
  auto* mtiles = reinterpret_cast<int32_t*>(ws + l.mtiles);
  int32_t* const mcount = count + 1;
  auto* act = reinterpret_cast<uint16_t*>(ws + l.act);
  auto* eo = reinterpret_cast<uint16_t*>(ws + l.eo);
  const int64_t group = mx ? 32 : group_size;
  int mt = stream_tile_mt(entries);
  if (mt && !(stream_fits(h, mt, group, mx) && stream_fits(i, mt, group, mx))) mt = 0;
  // 64-row tiles load activations directly (32-bit byte offsets)
  if (mt == 4 && (tokens * h * 2 > kMaxDirectBytes || entries * i * 2 > kMaxDirectBytes)) mt = 0;
  const int tr = mt == 1 ? kSmallTileRows : kTileRows;
  // W4A16 G = 128 on 64-row tiles: x and the activations go in paired
  const bool paired = !mx && mt == 4 && group == 128;
  // ...and when the batch takes the router launch (the 64-row tiles route
  // neither in the GEMM nor in the one-launch schedule), that launch also
  // pairs them (route_pair_kernel): one launch instead of two; the path knob
  // of the fused schedules turns it off
  const bool route_pairs = paired && experts - 1 <= 256 &&
                           path_choice(kKnobMoeFusedSchedule) != 1 &&
                           !route_schedule_fits(tokens, experts - 1, top_k);
  const int64_t tb = max_tiles_for(entries, experts, tr);
  // Few tokens (W4A16): the activations go to (token, route) rows and one
  // token-major launch does W2, the combine and the shared expert, instead of
  // the down GEMM and the combine kernel; it reads an expert's W2 once per
  // route that uses it rather than once per call.
  const bool w2_rows = !mx && tokens <= kW2RowsMaxTokens && w2_rows_fits(routes, i);
  // MXFP4 on the scaled fp4 MFMA: x and the activations go in as fp8 hi + lo
  const bool f8 = mx && mt != 0 && h % 128 == 0 && i % 128 == 0 && mxfp4_scaled_mfma();
  SplitBufs xs{}, as{};
  if (f8) {
    xs = split_bufs(ws + l.x_split, tokens * h);
    as = split_bufs(ws + l.act_split, entries * i);
    if (int rc = split_launch(x, xs.hi, xs.lo, xs.sc, tokens, h, s)) return rc;
  }

  GemmArgs g{};
  g.perm = perm;
  g.tiles = tiles;
  g.tile_count = count;
  g.mtiles = mtiles;
  g.mtile_count = mcount;
  g.group = group;
  g.routes = routes;
  g.outputs = 1;
  g.act = kActSwiglu;
  // gate/up + SwiGLU: rows gathered from x, activations written in sorted order
  g.a = x;
  g.a_hi = xs.hi;
  g.a_lo = xs.lo;
  g.a_sc = xs.sc;
  g.a_rows = tokens;
  if (paired) {
    g.a_pair = reinterpret_cast<uint16_t*>(ws + l.x_pair);
    g.a_neg = reinterpret_cast<float*>(ws + l.x_neg);
    if (!route_pairs) {
      if (int rc = pair_rows_launch(x, const_cast<uint16_t*>(g.a_pair),
                                    const_cast<float*>(g.a_neg), tokens, h, s))
        return rc;
    }
  }
  g.wp[0] = w1_packed;
  g.ws[0] = w1_scales;
  g.wp[1] = w3_packed;
  g.ws[1] = w3_scales;
  g.wp[2] = w1_packed;
  g.ws[2] = w1_scales;
  g.out[0] = g.out[1] = g.out[2] = act;
  if (paired) g.out_neg = reinterpret_cast<float*>(ws + l.act_neg);
  g.n = i;
  g.k = h;
  g.wstride = i * h / 2;
  g.sstride = i * (h / group);
  const Mode gu_mode = w2_rows ? Mode::GatherScatter : Mode::Gather;
  // down projection: sorted activation rows, outputs scattered to (token, route) rows
  auto down_args = [&](GemmArgs d) {
    d.a = act;
    d.a_hi = as.hi;
    d.a_lo = as.lo;
    d.a_sc = as.sc;
    d.a_rows = entries;
    if (paired) {  // written paired by the gate/up GEMM, with their group sums
      d.a_pair = act;
      d.a_neg = d.out_neg;
      d.out_neg = nullptr;
    }
    d.wp[0] = d.wp[1] = d.wp[2] = w2_packed;
    d.ws[0] = d.ws[1] = d.ws[2] = w2_scales;
    d.out[0] = d.out[1] = d.out[2] = eo;
    d.n = h;
    d.k = i;
    d.wstride = h * i / 2;
    d.sstride = h * (i / group);
    return d;
  };
  // Decode batches on the persistent kernels take the split SwiGLU (gate and
  // up as separate one-matrix units into [gate | up] rows, the SwiGLU applied
  // by the down GEMM's staging) when both of its launches apply; the results
  // are the fused form's bits (the path knob moe_split_swiglu=off keeps the
  // fused form). The act region holds 2i per row for it (moe_act_mult). At
  // 64 tokens of the Kimi-Linear layer the gate/up launch takes 73.1 us split
  // against 81.4 us fused, at 16 tokens 34.8 against 38.1 us: units of half
  // the bytes shorten the launch's tail, where each block's last units
  // stream alone.
  const bool split =
      mt == 1 && !f8 && !w2_rows && moe_act_mult(entries) == 2 &&
      path_choice(kKnobMoeSplitSwiglu) != 1 &&
      persist_fmt<1>(mx, g, Mode::Gather, tb, s, "", PsForm::SplitGateUp, false) == 0 &&
      persist_fmt<1>(mx, down_args(g), Mode::Scatter, tb, s, "", PsForm::SwiDown, false) == 0;
  // Batches of at most 8 tokens (one per wave) on the persistent 16-row
  // GEMMs: the gate/up GEMM routes and schedules the batch in every block
  // (route_schedule_block) where that launch applies, with no router or
  // schedule launch before it; for the split SwiGLU its block 0 also writes
  // the schedule for the down GEMM. (Two tokens per wave made the prologue of
  // every block longer than the router launch: at 16 tokens 68.0 against
  // 66.3 us per step with the router launch and the ranking below.) The
  // path knob of the one-launch router + schedule turns it off.
  bool gemm_routes = false;
  if ((w2_rows || split) && mt == 1 && tokens <= kStWaves && entries <= kRoutedEntries &&
      route_schedule_fits(tokens, experts - 1, top_k)) {
    GemmArgs probe = g;
    probe.rt_logits = logits;
    probe.rt_tokens = static_cast<int>(tokens);
    probe.rt_routed = static_cast<int>(experts - 1);
    probe.rt_top_k = static_cast<int>(top_k);
    gemm_routes = (w2_rows ? persist_fmt<2>(mx, probe, Mode::GatherScatter, tb, s, "",
                                            PsForm::Plain, false)
                           : persist_fmt<1>(mx, probe, Mode::Gather, tb, s, "",
                                            PsForm::SplitGateUp, false)) == 0;
  }
  // Larger batches on the split SwiGLU (up to kRoutedEntries token-routes):
  // the router launch, then every block of the gate/up GEMM ranks the
  // router's selections itself and block 0 writes the schedule for the down
  // GEMM: no schedule launch. The same path knob turns it off.
  bool gemm_ranks = false;
  if (!gemm_routes && split && mt == 1 && entries <= kRoutedEntries &&
      path_choice(kKnobMoeFusedSchedule) != 1) {
    GemmArgs probe = g;
    probe.rt_from_idx = 1;
    probe.rt_tokens = static_cast<int>(tokens);
    probe.rt_routed = static_cast<int>(experts - 1);
    probe.rt_top_k = static_cast<int>(top_k);
    gemm_ranks =
        persist_fmt<1>(mx, probe, Mode::Gather, tb, s, "", PsForm::SplitGateUp, false) == 0;
  }
  if (gemm_routes) {
    g.rt_logits = logits;
    g.rt_bias = bias;
    g.rt_idx = expert_indices;
    g.rt_w = weights;
    g.rt_tokens = static_cast<int>(tokens);
    g.rt_routed = static_cast<int>(experts - 1);
    g.rt_top_k = static_cast<int>(top_k);
    g.rt_renorm = renormalize;
    g.rt_scaling = routed_scaling_factor;
    if (split) {
      g.rt_perm_out = perm;
      g.rt_tiles_out = tiles;
      g.rt_count_out = count;
    }
  } else if (gemm_ranks) {
    if (int rc = lk_moe_router(logits, bias, expert_indices, weights, tokens, experts - 1, top_k,
                               routed_scaling_factor, renormalize, stream))
      return rc;
    g.rt_from_idx = 1;
    g.rt_idx = expert_indices;
    g.rt_tokens = static_cast<int>(tokens);
    g.rt_routed = static_cast<int>(experts - 1);
    g.rt_top_k = static_cast<int>(top_k);
    g.rt_perm_out = perm;
    g.rt_tiles_out = tiles;
    g.rt_count_out = count;
  } else if (route_schedule_fits(tokens, experts - 1, top_k)) {
    if (int rc = route_schedule_launch(logits, bias, expert_indices, weights, tokens, experts - 1,
                                       top_k, routed_scaling_factor, renormalize, offsets, perm,
                                       tiles, count, tr, mtiles, mcount, s))
      return rc;
  } else {
    if (int rc = route_pairs
                     ? route_pair_launch(logits, bias, expert_indices, weights, tokens, experts - 1,
                                         top_k, routed_scaling_factor, renormalize, x,
                                         const_cast<uint16_t*>(g.a_pair),
                                         const_cast<float*>(g.a_neg), h, s)
                     : lk_moe_router(logits, bias, expert_indices, weights, tokens, experts - 1,
                                     top_k, routed_scaling_factor, renormalize, stream))
      return rc;
    const RouteTable rt{expert_indices, top_k, routes, experts, experts - 1};
    if (int rc = schedule_launch(rt, entries, ws, l.sched, offsets, perm, tiles, count, tr, s,
                                 mtiles, mcount))
      return rc;
  }
  if (int rc = gemm_routes && w2_rows
                   ? persist_fmt<2>(mx, g, Mode::GatherScatter, tb, s, "moe gate/up gemm (routing)",
                                    PsForm::Plain, true)
               : f8 ? stream_launch<kFmtMxF8, 2>(g, Mode::Gather, tb, mt, s, "moe gate/up gemm")
               : split ? persist_fmt<1>(mx, g, Mode::Gather, tb, s, "moe gate/up gemm",
                                        PsForm::SplitGateUp, true)
               : mt    ? stream_fmt<2>(mx, g, gu_mode, tb, mt, s, "moe gate/up gemm")
                       : launch_fmt<2>(mx, g, gu_mode, tb, wide_cols_for(tb, i), s,
                                       "moe gate/up gemm"))
    return rc;
  if (w2_rows)
    return w2_combine_rows(act, expert_indices, top_k, experts - 1, weights, top_k, w2_packed,
                           static_cast<const uint16_t*>(w2_scales), y, tokens, routes, experts,
                           h, i, group, s);
  if (f8) {
    if (int rc = split_launch(act, as.hi, as.lo, as.sc, entries, i, s)) return rc;
  }
  g = down_args(g);
  if (int rc = f8 ? stream_launch<kFmtMxF8, 1>(g, Mode::Scatter, tb, mt, s, "moe down gemm")
               : split ? persist_fmt<1>(mx, g, Mode::Scatter, tb, s, "moe down gemm",
                                        PsForm::SwiDown, true)
               : mt    ? stream_fmt<1>(mx, g, Mode::Scatter, tb, mt, s, "moe down gemm")
                       : launch_fmt<1>(mx, g, Mode::Scatter, tb, wide_cols_for(tb, h), s,
                                       "moe down gemm"))
    return rc;
  const int64_t work = tokens * (h / 8);
  moe_combine_kernel<<<static_cast<unsigned>((work + 255) / 256), 256, 0, s>>>(
      eo, weights, y, tokens, static_cast<int>(top_k), h);
  return check_launch("moe combine");
}

int lk_w4a16_moe_forward(const uint16_t* x, const float* logits, const float* bias,
                         const uint8_t* w1_packed, const uint16_t* w1_scales,
                         const uint8_t* w3_packed, const uint16_t* w3_scales,
                         const uint8_t* w2_packed, const uint16_t* w2_scales, uint16_t* y,
                         int64_t* expert_indices, float* weights, void* workspace,
                         int64_t workspace_bytes, int64_t tokens, int64_t experts, int64_t h,
                         int64_t i, int64_t top_k, float routed_scaling_factor, int renormalize,
                         int64_t group_size, void* stream) {
  return moe_forward_common(false, x, logits, bias, w1_packed, w1_scales, w3_packed, w3_scales,
                            w2_packed, w2_scales, y, expert_indices, weights, workspace,
                            workspace_bytes, tokens, experts, h, i, top_k, routed_scaling_factor,
                            renormalize, group_size, stream);
}

}  // extern "C"

// Device scratch of lk_w4a16_moe_forward_static: one array per GPU, held until
// the process ends. Host code never passes the array's name to a kernel (on
// the host it is a stand-in, not a device address); it uses the address
// hipGetSymbolAddress returns for the current device.
constexpr size_t kStaticScratchBytes = size_t{12} << 20;
static __device__ __align__(256) uint8_t scratch[kStaticScratchBytes];

namespace lk {
namespace {

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxScratchDevices] = {};

// The current device's scratch address, looked up once per device.
int static_scratch(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0 || dev >= kMaxScratchDevices) {
    set_error("static scratch: no usable current device (%s)", hipGetErrorString(e));
    return LK_ERR_HIP;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr) {
      set_error("static scratch: hipGetSymbolAddress failed on device %d (%s)", dev,
                hipGetErrorString(e));
      return LK_ERR_HIP;
    }
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return LK_OK;
}

}  // namespace
}  // namespace lk

extern "C" {

int64_t lk_w4a16_moe_forward_static_capacity(void) {
  return static_cast<int64_t>(kStaticScratchBytes);
}

int lk_w4a16_moe_forward_static(const uint16_t* x, const float* logits, const float* bias,
                                const uint8_t* w1_packed, const uint16_t* w1_scales,
                                const uint8_t* w3_packed, const uint16_t* w3_scales,
                                const uint8_t* w2_packed, const uint16_t* w2_scales, uint16_t* y,
                                int64_t* expert_indices, float* weights, int64_t tokens,
                                int64_t experts, int64_t h, int64_t i, int64_t top_k,
                                float routed_scaling_factor, int renormalize, int64_t group_size,
                                void* stream) {
  const int64_t need = lk_w4a16_moe_forward_workspace(tokens, experts, h, i, top_k);
  LK_REQUIRE(need >= 0, "invalid MoE dimensions (tokens %lld, experts %lld, top_k %lld)",
             (long long)tokens, (long long)experts, (long long)top_k);
  LK_REQUIRE(need <= static_cast<int64_t>(kStaticScratchBytes),
             "lk_w4a16_moe_forward_static: this call needs %lld bytes of scratch, the static "
             "scratch holds %lld; use lk_w4a16_moe_forward with a workspace",
             (long long)need, (long long)kStaticScratchBytes);
  if (tokens == 0) {  // nothing to launch; the usual argument checks still apply
    return lk_w4a16_moe_forward(x, logits, bias, w1_packed, w1_scales, w3_packed, w3_scales,
                                w2_packed, w2_scales, y, expert_indices, weights, nullptr, 0,
                                tokens, experts, h, i, top_k, routed_scaling_factor, renormalize,
                                group_size, stream);
  }
  void* ws = nullptr;
  if (int rc = static_scratch(&ws)) return rc;
  return lk_w4a16_moe_forward(x, logits, bias, w1_packed, w1_scales, w3_packed, w3_scales,
                              w2_packed, w2_scales, y, expert_indices, weights, ws,
                              static_cast<int64_t>(kStaticScratchBytes), tokens, experts, h, i,
                              top_k, routed_scaling_factor, renormalize, group_size, stream);
}

int lk_mxfp4_moe_forward(const uint16_t* x, const float* logits, const float* bias,
                         const uint8_t* w1_packed, const uint8_t* w1_scale,
                         const uint8_t* w3_packed, const uint8_t* w3_scale,
                         const uint8_t* w2_packed, const uint8_t* w2_scale, uint16_t* y,
                         int64_t* expert_indices, float* weights, void* workspace,
                         int64_t workspace_bytes, int64_t tokens, int64_t experts, int64_t h,
                         int64_t i, int64_t top_k, float routed_scaling_factor, int renormalize,
                         void* stream) {
  return moe_forward_common(true, x, logits, bias, w1_packed, w1_scale, w3_packed, w3_scale,
                            w2_packed, w2_scale, y, expert_indices, weights, workspace,
                            workspace_bytes, tokens, experts, h, i, top_k, routed_scaling_factor,
                            renormalize, 32, stream);
}

}  // extern "C"
