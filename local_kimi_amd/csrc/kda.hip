// Kimi Delta Attention decode kernels for gfx950: the recurrent-state step
// (engine/kernels/kda_step.py) and its launch-fused preparation, the three
// width-4 short convolutions and the gates (engine/kernels/kda_prepare.py).
//
// All three are small and memory- or latency-bound at decode: the step reads
// and writes each head's d_k x d_v fp32 state once (2 MB each way for 32
// heads of 128 x 128), the preparation touches a few KB per token.

#include "lk_common.hpp"
#include "lk_kda.h"

namespace lk {
namespace {

// ---------------------------------------------------------------------------
// Recurrence step. Block = (batch * head, tile of 32 value columns), 256
// threads: thread t owns columns c0 + 4 * (t & 7) .. + 3 (one 16-byte load per
// row, eight threads per 128-byte row segment) and key rows
// (t >> 3) + 32 p, p < P. The state tile is loaded once into registers,
// decayed, its prediction S^T k reduced over the 32 row groups (three xor
// shuffles inside a wave, then the four waves through LDS in wave order),
// updated with the delta, reduced again for the output, and stored once.
constexpr int kStepThreads = 256;
constexpr int kStepCols = 32;
constexpr int kStepRowGroups = kStepThreads / (kStepCols / 4);  // 32

// Sums of v[0..3] over the 32 row groups of the block for this thread's
// column group; every thread of the column group gets the same values (fixed
// order: three xor shuffles, then waves 0..3).
__device__ inline void row_group_sum4(float (&v)[4], float (*red)[kStepCols]) {
  const int wave = threadIdx.x / kWave;
  const int lane = threadIdx.x & (kWave - 1);
  const int cg = threadIdx.x & 7;
#pragma unroll
  for (int c = 0; c < 4; ++c) {  // lanes 8 apart hold the same columns
    v[c] += __shfl_xor(v[c], 8);
    v[c] += __shfl_xor(v[c], 16);
    v[c] += __shfl_xor(v[c], 32);
  }
  __syncthreads();  // the previous use of red is over
  if (lane < 8) {
#pragma unroll
    for (int c = 0; c < 4; ++c) red[wave][cg * 4 + c] = v[c];
  }
  __syncthreads();
#pragma unroll
  for (int c = 0; c < 4; ++c)
    v[c] = ((red[0][cg * 4 + c] + red[1][cg * 4 + c]) + red[2][cg * 4 + c]) + red[3][cg * 4 + c];
}

template <int P>
__global__ void __launch_bounds__(kStepThreads)
kda_step_kernel(float* __restrict__ state, const float* __restrict__ q,
                const float* __restrict__ k, const float* __restrict__ v,
                const float* __restrict__ decay, const float* __restrict__ beta,
                float* __restrict__ out, int dk, int dv, float scale) {
  __shared__ float red[kStepThreads / kWave][kStepCols];
  const int64_t bh = blockIdx.y;
  const int cg = threadIdx.x & 7;
  const int rg = threadIdx.x >> 3;
  const int c0 = blockIdx.x * kStepCols + cg * 4;
  float* const s_head = state + bh * dk * dv;
  const float* const kh = k + bh * dk;
  const float* const qh = q + bh * dk;
  const float* const dh = decay + bh * dk;
  bool col_ok[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) col_ok[c] = c0 + c < dv;
  const bool vec = (dv & 3) == 0 && c0 + 3 < dv;

  // the state rows of this thread, decayed; the key and query rows
  float s[P][4], kr[P], qr[P];
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int i = rg + kStepRowGroups * p;
    const bool row_ok = i < dk;
    const int ic = row_ok ? i : 0;
    const float* row = s_head + static_cast<int64_t>(ic) * dv;
    if (vec) {
      const float4 x = *reinterpret_cast<const float4*>(row + c0);
      s[p][0] = x.x;
      s[p][1] = x.y;
      s[p][2] = x.z;
      s[p][3] = x.w;
    } else {
#pragma unroll
      for (int c = 0; c < 4; ++c) s[p][c] = col_ok[c] ? row[c0 + c] : 0.f;
    }
    const float g = row_ok ? expf(dh[ic]) : 0.f;
    kr[p] = row_ok ? kh[ic] : 0.f;
    qr[p] = row_ok ? qh[ic] * scale : 0.f;
#pragma unroll
    for (int c = 0; c < 4; ++c) s[p][c] *= g;
  }
  const float b = beta[bh];
  float vc[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) vc[c] = col_ok[c] ? v[bh * dv + c0 + c] : 0.f;

  // prediction S^T k for the four columns, then the delta
  float delta[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    float part = 0.f;
#pragma unroll
    for (int p = 0; p < P; ++p) part = fmaf(s[p][c], kr[p], part);
    delta[c] = part;
  }
  row_group_sum4(delta, red);
#pragma unroll
  for (int c = 0; c < 4; ++c) delta[c] = vc[c] - delta[c];
  // S += beta * k * delta^T; output S^T (q * scale)
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const float bk = b * kr[p];
#pragma unroll
    for (int c = 0; c < 4; ++c) s[p][c] = fmaf(bk, delta[c], s[p][c]);
  }
  float o[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    float part = 0.f;
#pragma unroll
    for (int p = 0; p < P; ++p) part = fmaf(s[p][c], qr[p], part);
    o[c] = part;
  }
  row_group_sum4(o, red);
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int i = rg + kStepRowGroups * p;
    if (i >= dk) continue;
    float* row = s_head + static_cast<int64_t>(i) * dv;
    if (vec) {
      *reinterpret_cast<float4*>(row + c0) = make_float4(s[p][0], s[p][1], s[p][2], s[p][3]);
    } else {
#pragma unroll
      for (int c = 0; c < 4; ++c)
        if (col_ok[c]) row[c0 + c] = s[p][c];
    }
  }
  if (rg == 0) {
#pragma unroll
    for (int c = 0; c < 4; ++c)
      if (col_ok[c]) out[bh * dv + c0 + c] = o[c];
  }
}

// ---------------------------------------------------------------------------
// storage dtypes of the preparation kernels

__device__ inline float load_value(const void* p, int64_t i, int dtype) {
  if (dtype == LK_DTYPE_F32) return static_cast<const float*>(p)[i];
  const uint16_t b = static_cast<const uint16_t*>(p)[i];
  if (dtype == LK_DTYPE_BF16) return bf16_to_f32(b);
  return static_cast<float>(__builtin_bit_cast(_Float16, b));
}

// one of the first two pointers of an argument triple, without indexing the
// kernel arguments by a per-thread value (which would load the pointer from
// memory before the data it points to)
template <typename T>
__device__ inline T pick2(const T (&v)[3], int i) {
  return i ? v[1] : v[0];
}

template <typename T>
__device__ inline T pick3(const T (&v)[3], int i) {
  return i == 0 ? v[0] : (i == 1 ? v[1] : v[2]);
}

__device__ inline void store_value(void* p, int64_t i, float x, int dtype) {
  if (dtype == LK_DTYPE_F32) {
    static_cast<float*>(p)[i] = x;
  } else if (dtype == LK_DTYPE_BF16) {
    static_cast<uint16_t*>(p)[i] = f32_to_bf16(x);
  } else {
    static_cast<uint16_t*>(p)[i] = __builtin_bit_cast(uint16_t, static_cast<_Float16>(x));
  }
}

// ---------------------------------------------------------------------------
// Short convolutions: one thread per (convolution, batch row, channel); grid
// (channel blocks, batch, 3). The window's products are accumulated in window
// order, as the reference kernel sums them; the state values are stored back
// from their exact fp32 images, so the shifted state is bit-identical to the
// inputs.
constexpr int kConvThreads = 256;

struct ConvArgs {
  const void* in[3];
  void* state[3];
  const void* weight[3];
  void* out[3];
};

__global__ void __launch_bounds__(kConvThreads)
short_conv_kernel(const ConvArgs a, int64_t channels, int vdt, int wdt) {
  const int conv = blockIdx.z;
  const int64_t b = blockIdx.y;
  const int64_t ch = static_cast<int64_t>(blockIdx.x) * kConvThreads + threadIdx.x;
  if (ch >= channels) return;
  const int64_t si = (b * channels + ch) * 4;
  const float s1 = load_value(a.state[conv], si + 1, vdt);
  const float s2 = load_value(a.state[conv], si + 2, vdt);
  const float s3 = load_value(a.state[conv], si + 3, vdt);
  const float token = load_value(a.in[conv], b * channels + ch, vdt);
  const float w0 = load_value(a.weight[conv], ch * 4 + 0, wdt);
  const float w1 = load_value(a.weight[conv], ch * 4 + 1, wdt);
  const float w2 = load_value(a.weight[conv], ch * 4 + 2, wdt);
  const float w3 = load_value(a.weight[conv], ch * 4 + 3, wdt);
  float acc = s1 * w0;
  acc += s2 * w1;
  acc += s3 * w2;
  acc += token * w3;
  store_value(a.out[conv], b * channels + ch, acc / (1.0f + expf(-acc)), vdt);
  store_value(a.state[conv], si + 0, s1, vdt);
  store_value(a.state[conv], si + 1, s2, vdt);
  store_value(a.state[conv], si + 2, s3, vdt);
  store_value(a.state[conv], si + 3, token, vdt);
}

// ---------------------------------------------------------------------------
// Gates: one wave per (row, head). Lane l takes elements l, l + 64, ...; the
// squared norms are summed per lane in element order, then across the wave
// by a fixed butterfly.
constexpr int kGateWaves = 4;

__device__ inline float wave_sum(float v) {
#pragma unroll
  for (int m = 1; m < kWave; m <<= 1) v += __shfl_xor(v, m);
  return v;
}

__device__ inline float softplus_f32(float x) {
  // x above the threshold passes through (torch's and the reference kernel's
  // 20); below it the stable form max(x, 0) + log1p(exp(-|x|))
  return x > 20.0f ? x : fmaxf(x, 0.0f) + log1pf(expf(-fabsf(x)));
}

__global__ void __launch_bounds__(kGateWaves * kWave)
kda_gates_kernel(const void* __restrict__ raw_decay, const float* __restrict__ dt_bias,
                 const float* __restrict__ a_log, const void* __restrict__ raw_beta,
                 const void* __restrict__ q, const void* __restrict__ k,
                 float* __restrict__ decay, float* __restrict__ beta,
                 float* __restrict__ q_out, float* __restrict__ k_out, int64_t programs,
                 int heads, int dim, float eps, int ddt, int bdt, int qdt) {
  const int64_t prog = static_cast<int64_t>(blockIdx.x) * kGateWaves + threadIdx.x / kWave;
  if (prog >= programs) return;  // wave-uniform
  const int lane = threadIdx.x & (kWave - 1);
  const int h = static_cast<int>(prog % heads);
  const int64_t base = prog * dim;
  const float rate = expf(a_log[h]);
  float qs = 0.f, ks = 0.f;
  for (int d = lane; d < dim; d += kWave) {
    const float biased = load_value(raw_decay, base + d, ddt) + dt_bias[h * dim + d];
    decay[base + d] = -rate * softplus_f32(biased);
    const float qv = load_value(q, base + d, qdt);
    const float kv = load_value(k, base + d, qdt);
    qs = fmaf(qv, qv, qs);
    ks = fmaf(kv, kv, ks);
  }
  const float qn = 1.0f / sqrtf(wave_sum(qs) + eps);
  const float kn = 1.0f / sqrtf(wave_sum(ks) + eps);
  for (int d = lane; d < dim; d += kWave) {
    q_out[base + d] = load_value(q, base + d, qdt) * qn;
    k_out[base + d] = load_value(k, base + d, qdt) * kn;
  }
  if (lane == 0) beta[prog] = 1.0f / (1.0f + expf(-load_value(raw_beta, prog, bdt)));
}

// ---------------------------------------------------------------------------
// A whole decode layer in one launch: one block of 1024 threads per (batch,
// head) owns the head's 3 x D convolution channels (so its in-place state
// updates cannot race with another block), computes the convolutions and the
// gates into LDS, and runs the recurrence step on the head's D x D state,
// whose loads are issued first so their latency overlaps the preparation.
// The preparation repeats the separate kernels' arithmetic exactly (the same
// per-channel sums and the same per-lane norm order), so q, k, v, decay and
// beta are bit-identical to fused_short_conv_triple + fused_kda_gates; the
// step reduces its 32 row groups in another order than kda_step_kernel.
constexpr int kLayerThreads = 1024;
constexpr int kLayerMaxDim = 128;
constexpr int kLayerRowGroups = kLayerThreads / (kLayerMaxDim / 4);  // 32
constexpr int kLayerWaves = kLayerThreads / kWave;                    // 16

struct LayerArgs {
  const void* in[3];
  void* conv_state[3];
  const void* conv_weight[3];
  const void* raw_decay;
  const float* dt_bias;
  const float* a_log;
  const void* raw_beta;
  float* state;
  float* out;
};

// storage of compile-time dtype DT (the split kernel's conv loads go out in
// one batch only when no run-time dtype branch sits between them)
template <int DT>
__device__ inline float load_as(const void* p, int64_t i) {
  if constexpr (DT == LK_DTYPE_F32) {
    return static_cast<const float*>(p)[i];
  } else if constexpr (DT == LK_DTYPE_BF16) {
    return bf16_to_f32(static_cast<const uint16_t*>(p)[i]);
  } else {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<const uint16_t*>(p)[i]));
  }
}

// One width-4 convolution channel: the loads (window, token, weights) of
// load(), then apply() (short_conv_kernel's arithmetic) and the shifted
// window into state_out.
template <int VDT, int WDT>
struct ConvChannel {
  float s1, s2, s3, token, w0, w1, w2, w3;
  __device__ inline void load(const void* state_in, const void* in, const void* weight,
                              int64_t si, int64_t xi, int64_t wi) {
    s1 = load_as<VDT>(state_in, si + 1);
    s2 = load_as<VDT>(state_in, si + 2);
    s3 = load_as<VDT>(state_in, si + 3);
    token = load_as<VDT>(in, xi);
    w0 = load_as<WDT>(weight, wi + 0);
    w1 = load_as<WDT>(weight, wi + 1);
    w2 = load_as<WDT>(weight, wi + 2);
    w3 = load_as<WDT>(weight, wi + 3);
  }
  __device__ inline float apply() const {
    float acc = s1 * w0;
    acc += s2 * w1;
    acc += s3 * w2;
    acc += token * w3;
    float y = acc / (1.0f + expf(-acc));
    if constexpr (VDT == LK_DTYPE_BF16) y = round_bf16(y);
    else if constexpr (VDT == LK_DTYPE_F16) y = static_cast<float>(static_cast<_Float16>(y));
    return y;
  }
  // the shifted window, issued at the end of the kernel: a store among the
  // preparation's loads would make every later wait on those loads count it
  __device__ inline void store_shifted(void* state_out, int64_t si) const {
    store_value(state_out, si + 0, s1, VDT);
    store_value(state_out, si + 1, s2, VDT);
    store_value(state_out, si + 2, s3, VDT);
    store_value(state_out, si + 3, token, VDT);
  }
};

template <int VDT, int WDT, bool GATES_AS_VALUES>
__global__ void __launch_bounds__(kLayerThreads)
kda_layer_kernel(const LayerArgs a, int heads, int dim, float eps, float scale, int ddt_arg,
                 int bdt_arg) {
  const int ddt = GATES_AS_VALUES ? VDT : ddt_arg;
  const int bdt = GATES_AS_VALUES ? VDT : bdt_arg;
  __shared__ float qkv[3][kLayerMaxDim];
  __shared__ float gain[kLayerMaxDim];  // exp(decay)
  __shared__ float norm[2];
  __shared__ float beta_s;
  __shared__ float red[kLayerWaves][kLayerMaxDim];
  const int t = threadIdx.x;
  const int64_t bh = blockIdx.x;  // batch * heads + head
  const int64_t b = bh / heads;
  const int h = static_cast<int>(bh - b * heads);
  const int channels = heads * dim;
  const int cg = t & 31, rg = t >> 5;
  const int c0 = cg * 4;
  const bool cols = c0 < dim;  // dim % 4 == 0 (host-checked)
  float* const s_head = a.state + bh * dim * dim;

  // 1. every load of the preparation, before the state rows (loads retire in
  // issue order, so the convolutions and gates wait only for their own
  // inputs): thread t < 3 dim one convolution channel, t < dim the gate
  // inputs of row t, every thread the beta input (no branch around a load)
  const bool conv_live = t < 3 * dim;
  const int tc = conv_live ? t : 0;
  const int conv = tc / dim, j = tc - conv * dim;
  const int64_t ch = static_cast<int64_t>(h) * dim + j;
  const int64_t si = (b * channels + ch) * 4;
  ConvChannel<VDT, WDT> cc;
  cc.load(pick3(a.conv_state, conv), pick3(a.in, conv), pick3(a.conv_weight, conv), si,
          b * channels + ch, ch * 4);
  const bool grow = t < dim;
  const float raw = load_value(a.raw_decay, bh * dim + (grow ? t : 0), ddt);
  const float dtb = a.dt_bias[h * dim + (grow ? t : 0)];
  const float alog = a.a_log[h];
  const float rbeta = load_value(a.raw_beta, bh, bdt);

  // 2. the state rows of this thread (rows rg + 32 p), every load
  // unconditional (rows or columns past the head read its first values and
  // are zeroed)
  float s[4][4];
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const int i = rg + kLayerRowGroups * p;
    const bool ok = cols && i < dim;
    const float4 x = *reinterpret_cast<const float4*>(
        s_head + (ok ? static_cast<int64_t>(i) * dim + c0 : 0));
    s[p][0] = ok ? x.x : 0.f;
    s[p][1] = ok ? x.y : 0.f;
    s[p][2] = ok ? x.z : 0.f;
    s[p][3] = ok ? x.w : 0.f;
  }

  // 3. the three convolutions (as short_conv_kernel; the output rounded to the
  // value dtype, as the reference's gates read their bf16 / fp16 inputs), the
  // decay (as kda_gates_kernel) kept as exp(decay) for the step, and beta
  if (conv_live) qkv[conv][j] = cc.apply();
  if (grow) gain[t] = expf(-expf(alog) * softplus_f32(raw + dtb));
  if (t == 0) beta_s = 1.0f / (1.0f + expf(-rbeta));
  __syncthreads();
  // 4. q and k norms: waves 0 and 1, the gates kernel's per-lane order
  if (t < 2 * kWave) {
    const int which = t / kWave, lane = t & (kWave - 1);
    float acc = 0.f;
    for (int d = lane; d < dim; d += kWave) acc = fmaf(qkv[which][d], qkv[which][d], acc);
    acc = wave_sum(acc);
    if (lane == 0) norm[which] = 1.0f / sqrtf(acc + eps);
  }
  __syncthreads();
  const float rq = norm[0], rk = norm[1], beta = beta_s;

  // 5. the recurrence step
  float kr[4], qr[4];
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const int i = rg + kLayerRowGroups * p;
    const bool row_ok = i < dim;
    const float g = row_ok ? gain[i] : 0.f;
    kr[p] = row_ok ? qkv[1][i] * rk : 0.f;
    qr[p] = row_ok ? (qkv[0][i] * rq) * scale : 0.f;
#pragma unroll
    for (int c = 0; c < 4; ++c) s[p][c] *= g;
  }
  auto reduce = [&](float (&v)[4]) {  // over the 32 row groups, fixed order
#pragma unroll
    for (int c = 0; c < 4; ++c) v[c] += __shfl_xor(v[c], 32);
    const int wave = t / kWave, lane = t & (kWave - 1);
    __syncthreads();
    if (lane < 32) {
#pragma unroll
      for (int c = 0; c < 4; ++c) red[wave][c0 + c] = v[c];
    }
    __syncthreads();
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      float acc = 0.f;
      for (int w = 0; w < kLayerWaves; ++w) acc += red[w][c0 + c];
      v[c] = acc;
    }
  };
  float delta[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    float part = 0.f;
#pragma unroll
    for (int p = 0; p < 4; ++p) part = fmaf(s[p][c], kr[p], part);
    delta[c] = part;
  }
  reduce(delta);
#pragma unroll
  for (int c = 0; c < 4; ++c) delta[c] = (cols ? qkv[2][c0 + c] : 0.f) - delta[c];
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const float bk = beta * kr[p];
#pragma unroll
    for (int c = 0; c < 4; ++c) s[p][c] = fmaf(bk, delta[c], s[p][c]);
  }
  float o[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    float part = 0.f;
#pragma unroll
    for (int p = 0; p < 4; ++p) part = fmaf(s[p][c], qr[p], part);
    o[c] = part;
  }
  reduce(o);
  if (cols) {
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const int i = rg + kLayerRowGroups * p;
      if (i < dim)
        *reinterpret_cast<float4*>(s_head + static_cast<int64_t>(i) * dim + c0) =
            make_float4(s[p][0], s[p][1], s[p][2], s[p][3]);
    }
    if (rg == 0)
      *reinterpret_cast<float4*>(a.out + bh * dim + c0) = make_float4(o[0], o[1], o[2], o[3]);
  }
  // the shifted windows, in place: each channel is read and written by one
  // thread of this block only
  if (conv_live) cc.store_shifted(pick3(a.conv_state, conv), si);
}

// A decode layer over several blocks per head: block (b, h, y) owns value
// columns [16 y, 16 y + 16) of the head's D x D state (128 threads: column
// group cg = lane / 16 of 4 columns, row group rg = 16 * wave + lane % 16 of
// rows rg + 32 p), so 256 blocks cover 32 heads of 128 and every CU streams a
// slice of the state. Every block of a head needs all of q and k (the norms,
// and every row's k and q in the step), so each block computes the q and k
// convolutions itself, and the v convolutions of its own columns. The
// convolution states are read from one buffer and the shifted states written
// to another (the caller alternates them from call to call), so no block can
// read a state that another block already shifted: block y = 0 writes the q
// and k states, each block the v states of its columns. The arithmetic of
// every convolution, gate and norm is kda_layer_kernel's, so q, k, v, decay
// and beta are bit-identical with it; the step's sums run over the rows in
// another grouping, and the output is S^T q + beta (k . q) delta of the
// decayed state S (one reduction pass instead of two). The blocks of a 128-byte state line (two column
// blocks) are dispatched to one XCD when the item count allows, so the line
// is fetched into one L2 once.
constexpr int kSplitThreads = 128;
constexpr int kSplitCols = 16;
constexpr int kSplitRowGroups = 32;

struct SplitArgs {
  const void* in[3];
  const void* conv_in[3];
  void* conv_out[3];
  const void* conv_weight[3];
  const void* raw_decay;
  const float* dt_bias;
  const float* a_log;
  const void* raw_beta;
  float* state;
  float* out;
};


// GATES_AS_VALUES: the raw decay and beta are stored in the value dtype (the
// common case), fixed at compile time so that no dtype branch splits the
// preparation's loads; otherwise ddt and bdt are taken at run time.
template <int VDT, int WDT, bool GATES_AS_VALUES>
__global__ void __launch_bounds__(kSplitThreads)
kda_layer_split_kernel(const SplitArgs a, int heads, int dim, int vs, int64_t items, int paired,
                       float eps, float scale, int ddt_arg, int bdt_arg) {
  const int ddt = GATES_AS_VALUES ? VDT : ddt_arg;
  const int bdt = GATES_AS_VALUES ? VDT : bdt_arg;
  __shared__ float qk[2][kLayerMaxDim];
  __shared__ float vcol[kSplitCols];
  __shared__ float gain[kLayerMaxDim];
  __shared__ float norm[2];
  __shared__ float beta_s;
  __shared__ float red[2][4][9];
  // item = (batch * heads + head) * vs + column block; with `paired`, the
  // two column blocks of a 128-byte line sit 8 blocks apart (one XCD)
  const int64_t lin = blockIdx.x;
  const int64_t item = paired ? 2 * ((lin >> 4) * 8 + (lin & 7)) + ((lin >> 3) & 1) : lin;
  if (item >= items) return;  // block-uniform
  const int64_t bh = item / vs;
  const int y = static_cast<int>(item - bh * vs);
  const int64_t b = bh / heads;
  const int h = static_cast<int>(bh - b * heads);
  const int channels = heads * dim;
  const int t = threadIdx.x;
  const int wave = t / kWave, lane = t & (kWave - 1);
  const int cg = lane >> 4, rg = wave * 16 + (lane & 15);
  const int c0 = y * kSplitCols + cg * 4;
  const bool cols = c0 < dim;  // dim % 4 == 0 (host-checked)
  float* const s_head = a.state + bh * dim * dim;

  // 1. every load of the preparation in one batch: the q and k convolution
  // channels of the head (thread t takes channels t and t + 128 of the 2 * dim),
  // the v channel of this block's column t, the gate inputs of row t. They go
  // out before the state rows: loads retire in issue order, so the
  // preparation below waits only for its own inputs and runs while the
  // state (the bulk of the bytes, from HBM) is still arriving.
  ConvChannel<VDT, WDT> cc[3];
  int conv_of[2], j_of[2];
  bool live[3];
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int u = t + kSplitThreads * q;
    live[q] = u < 2 * dim;
    const int uc = live[q] ? u : 0;
    conv_of[q] = uc >= dim ? 1 : 0;
    j_of[q] = uc - conv_of[q] * dim;
    const int64_t ch = static_cast<int64_t>(h) * dim + j_of[q];
    cc[q].load(pick2(a.conv_in, conv_of[q]), pick2(a.in, conv_of[q]),
               pick2(a.conv_weight, conv_of[q]),
               (b * channels + ch) * 4, b * channels + ch, ch * 4);
  }
  const int vj = y * kSplitCols + t;
  live[2] = t < kSplitCols && vj < dim;
  const int64_t vch = static_cast<int64_t>(h) * dim + (live[2] ? vj : 0);
  cc[2].load(a.conv_in[2], a.in[2], a.conv_weight[2], (b * channels + vch) * 4, b * channels + vch,
             vch * 4);
  const bool grow = t < dim;
  const float raw = load_value(a.raw_decay, bh * dim + (grow ? t : 0), ddt);
  const float dtb = a.dt_bias[h * dim + (grow ? t : 0)];
  const float alog = a.a_log[h];
  const float rbeta_all = load_value(a.raw_beta, bh, bdt);  // every thread: no branch
  const float rbeta = t == 0 ? rbeta_all : 0.f;
  // 2. this thread's state rows, every load unconditional (rows or columns
  // past the head read its first four values and are zeroed): the wait for
  // a preparation input then counts only the loads issued after it
  float s[4][4];
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const int i = rg + kSplitRowGroups * p;
    const bool ok = cols && i < dim;
    const float4 x = *reinterpret_cast<const float4*>(
        s_head + (ok ? static_cast<int64_t>(i) * dim + c0 : 0));
    s[p][0] = ok ? x.x : 0.f;
    s[p][1] = ok ? x.y : 0.f;
    s[p][2] = ok ? x.z : 0.f;
    s[p][3] = ok ? x.w : 0.f;
  }
#pragma unroll
  for (int q = 0; q < 2; ++q)
    if (live[q]) qk[conv_of[q]][j_of[q]] = cc[q].apply();
  if (live[2]) vcol[t] = cc[2].apply();
  // 3. exp(decay) of every row, beta
  if (grow) gain[t] = expf(-expf(alog) * softplus_f32(raw + dtb));
  if (t == 0) beta_s = 1.0f / (1.0f + expf(-rbeta));
  __syncthreads();
  // 4. q and k norms: wave 0 and wave 1, the gates kernel's per-lane order
  {
    float acc = 0.f;
    for (int d = lane; d < dim; d += kWave) acc = fmaf(qk[wave][d], qk[wave][d], acc);
    acc = wave_sum(acc);
    if (lane == 0) norm[wave] = 1.0f / sqrtf(acc + eps);
  }
  __syncthreads();
  const float rq = norm[0], rk = norm[1], beta = beta_s;

  // 5. the recurrence step on this block's columns
  float kr[4], qr[4];
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const int i = rg + kSplitRowGroups * p;
    const bool row_ok = i < dim;
    const float g = row_ok ? gain[i] : 0.f;
    kr[p] = row_ok ? qk[1][i] * rk : 0.f;
    qr[p] = row_ok ? (qk[0][i] * rq) * scale : 0.f;
#pragma unroll
    for (int c = 0; c < 4; ++c) s[p][c] *= g;
  }
  // One pass of sums over the 32 row groups (the 16 lanes of a DPP row, then
  // the 2 waves) gives S^T k and S^T q of the decayed state S and k . q; the
  // output needs no second pass over the updated state:
  //   o = (S + beta k delta^T)^T q = S^T q + beta (k . q) delta.
  float sum[9];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    float pk = 0.f, pq = 0.f;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      pk = fmaf(s[p][c], kr[p], pk);
      pq = fmaf(s[p][c], qr[p], pq);
    }
    sum[c] = pk;
    sum[4 + c] = pq;
  }
  sum[8] = 0.f;
#pragma unroll
  for (int p = 0; p < 4; ++p) sum[8] = fmaf(kr[p], qr[p], sum[8]);
#pragma unroll
  for (int c = 0; c < 9; ++c) {
    float x = sum[c];
    x += dpp_f32<kQuadXor1>(x);
    x += dpp_f32<kQuadXor2>(x);
    x += dpp_f32<kRowHalfMirror>(x);
    x += dpp_f32<kRowMirror>(x);
    sum[c] = x;
  }
  if ((lane & 15) == 0) {
#pragma unroll
    for (int c = 0; c < 9; ++c) red[wave][cg][c] = sum[c];
  }
  __syncthreads();
  float delta[4], o[4];
  const float bkq = beta * (red[0][cg][8] + red[1][cg][8]);
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const float sk = red[0][cg][c] + red[1][cg][c];
    const float sq = red[0][cg][4 + c] + red[1][cg][4 + c];
    delta[c] = (cols ? vcol[cg * 4 + c] : 0.f) - sk;
    o[c] = fmaf(bkq, delta[c], sq);
  }
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const float bk = beta * kr[p];
#pragma unroll
    for (int c = 0; c < 4; ++c) s[p][c] = fmaf(bk, delta[c], s[p][c]);
  }
  if (cols) {
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const int i = rg + kSplitRowGroups * p;
      if (i < dim)
        *reinterpret_cast<float4*>(s_head + static_cast<int64_t>(i) * dim + c0) =
            make_float4(s[p][0], s[p][1], s[p][2], s[p][3]);
    }
    if (rg == 0)
      *reinterpret_cast<float4*>(a.out + bh * dim + c0) = make_float4(o[0], o[1], o[2], o[3]);
  }
  // the shifted conv windows into the second state set: q and k channels
  // from column block 0 of a head, each block its own v columns
  if (y == 0) {
#pragma unroll
    for (int q = 0; q < 2; ++q)
      if (live[q])
        cc[q].store_shifted(pick2(a.conv_out, conv_of[q]),
                            (b * channels + static_cast<int64_t>(h) * dim + j_of[q]) * 4);
  }
  if (live[2]) cc[2].store_shifted(a.conv_out[2], (b * channels + vch) * 4);
}

bool valid_dtype(int d) { return d == LK_DTYPE_F32 || d == LK_DTYPE_F16 || d == LK_DTYPE_BF16; }

}  // namespace
}  // namespace lk

using namespace lk;

extern "C" {

int lk_kda_decode_step(float* state, const float* q, const float* k, const float* v,
                       const float* decay, const float* beta, float* out, int64_t batch,
                       int64_t heads, int64_t d_k, int64_t d_v, float scale, void* stream) {
  LK_REQUIRE(batch > 0 && heads > 0 && d_k > 0 && d_v > 0, "KDA decode dimensions must be nonzero");
  LK_REQUIRE(d_k <= 256, "KDA decode step supports d_k up to 256, got %lld", (long long)d_k);
  LK_REQUIRE(batch * heads <= 65535, "at most 65535 batch x heads per call");
  LK_REQUIRE(d_v <= (int64_t{1} << 20), "d_v too large");
  LK_REQUIRE(state && q && k && v && decay && beta && out, "null pointer argument");
  LK_REQUIRE(reinterpret_cast<uintptr_t>(state) % 16 == 0, "state must be 16-byte aligned");
  dim3 grid(static_cast<unsigned>((d_v + kStepCols - 1) / kStepCols),
            static_cast<unsigned>(batch * heads));
  hipStream_t s = as_stream(stream);
  const int dk = static_cast<int>(d_k), dv = static_cast<int>(d_v);
  if (d_k <= 128)
    kda_step_kernel<4><<<grid, kStepThreads, 0, s>>>(state, q, k, v, decay, beta, out, dk, dv,
                                                      scale);
  else
    kda_step_kernel<8><<<grid, kStepThreads, 0, s>>>(state, q, k, v, decay, beta, out, dk, dv,
                                                      scale);
  return check_launch("lk_kda_decode_step");
}

int lk_kda_short_conv_triple(const void* q_in, const void* k_in, const void* v_in,
                             void* q_state, void* k_state, void* v_state, const void* q_weight,
                             const void* k_weight, const void* v_weight, void* q_out,
                             void* k_out, void* v_out, int64_t batch, int64_t channels,
                             int value_dtype, int weight_dtype, void* stream) {
  LK_REQUIRE(batch > 0 && channels > 0, "fused short convolution requires nonempty input");
  LK_REQUIRE(batch <= 65535, "at most 65535 batch rows per call");
  LK_REQUIRE(valid_dtype(value_dtype) && valid_dtype(weight_dtype), "unknown dtype code");
  LK_REQUIRE(q_in && k_in && v_in && q_state && k_state && v_state && q_weight && k_weight &&
                 v_weight && q_out && k_out && v_out,
             "null pointer argument");
  ConvArgs a{{q_in, k_in, v_in}, {q_state, k_state, v_state}, {q_weight, k_weight, v_weight},
             {q_out, k_out, v_out}};
  dim3 grid(static_cast<unsigned>((channels + kConvThreads - 1) / kConvThreads),
            static_cast<unsigned>(batch), 3);
  short_conv_kernel<<<grid, kConvThreads, 0, as_stream(stream)>>>(a, channels, value_dtype,
                                                                  weight_dtype);
  return check_launch("lk_kda_short_conv_triple");
}

int lk_kda_gates(const void* raw_decay, const float* dt_bias, const float* a_log,
                 const void* raw_beta, const void* q, const void* k, float* decay, float* beta,
                 float* q_out, float* k_out, int64_t rows, int64_t heads, int64_t head_dim,
                 float eps, int decay_dtype, int beta_dtype, int qk_dtype, void* stream) {
  LK_REQUIRE(heads > 0 && head_dim > 0 && head_dim <= 1024,
             "num_heads and head_dim must be positive, with head_dim at most 1024");
  LK_REQUIRE(eps > 0, "eps must be positive");
  LK_REQUIRE(rows > 0, "KDA gate inputs must have nonempty batch and sequence dimensions");
  LK_REQUIRE(valid_dtype(decay_dtype) && valid_dtype(beta_dtype) && valid_dtype(qk_dtype),
             "unknown dtype code");
  LK_REQUIRE(raw_decay && dt_bias && a_log && raw_beta && q && k && decay && beta && q_out &&
                 k_out,
             "null pointer argument");
  const int64_t programs = rows * heads;
  const int64_t blocks = (programs + kGateWaves - 1) / kGateWaves;
  LK_REQUIRE(blocks < (int64_t{1} << 31), "too many rows");
  kda_gates_kernel<<<static_cast<unsigned>(blocks), kGateWaves * kWave, 0, as_stream(stream)>>>(
      raw_decay, dt_bias, a_log, raw_beta, q, k, decay, beta, q_out, k_out, programs,
      static_cast<int>(heads), static_cast<int>(head_dim), eps, decay_dtype, beta_dtype,
      qk_dtype);
  return check_launch("lk_kda_gates");
}

int lk_kda_decode_layer(const void* q_in, const void* k_in, const void* v_in, void* q_state,
                        void* k_state, void* v_state, const void* q_weight, const void* k_weight,
                        const void* v_weight, const void* raw_decay, const float* dt_bias,
                        const float* a_log, const void* raw_beta, float* state, float* out,
                        int64_t batch, int64_t heads, int64_t head_dim, float eps, float scale,
                        int value_dtype, int weight_dtype, int decay_dtype, int beta_dtype,
                        void* stream) {
  LK_REQUIRE(batch > 0 && heads > 0, "KDA decode dimensions must be nonzero");
  LK_REQUIRE(head_dim > 0 && head_dim <= kLayerMaxDim && head_dim % 4 == 0,
             "one-launch KDA layer takes head_dim a multiple of 4 up to %d, got %lld",
             kLayerMaxDim, (long long)head_dim);
  LK_REQUIRE(eps > 0, "eps must be positive");
  LK_REQUIRE(batch * heads < (int64_t{1} << 31), "too many heads");
  LK_REQUIRE(heads * head_dim < (int64_t{1} << 31), "too many channels");
  LK_REQUIRE(valid_dtype(value_dtype) && valid_dtype(weight_dtype) && valid_dtype(decay_dtype) &&
                 valid_dtype(beta_dtype),
             "unknown dtype code");
  LK_REQUIRE(q_in && k_in && v_in && q_state && k_state && v_state && q_weight && k_weight &&
                 v_weight && raw_decay && dt_bias && a_log && raw_beta && state && out,
             "null pointer argument");
  LK_REQUIRE(reinterpret_cast<uintptr_t>(state) % 16 == 0 && reinterpret_cast<uintptr_t>(out) % 16 == 0,
             "state and out must be 16-byte aligned");
  LayerArgs a{{q_in, k_in, v_in}, {q_state, k_state, v_state}, {q_weight, k_weight, v_weight},
              raw_decay, dt_bias, a_log, raw_beta, state, out};
  const dim3 grid(static_cast<unsigned>(batch * heads));
  const int nh = static_cast<int>(heads), nd = static_cast<int>(head_dim);
  hipStream_t s = as_stream(stream);
  const bool gates_as_values = decay_dtype == value_dtype && beta_dtype == value_dtype;
#define LK_KDA_LAYER(V, W)                                                                  \
  do {                                                                                      \
    if (gates_as_values)                                                                    \
      kda_layer_kernel<V, W, true><<<grid, kLayerThreads, 0, s>>>(a, nh, nd, eps, scale,    \
                                                                  decay_dtype, beta_dtype); \
    else                                                                                    \
      kda_layer_kernel<V, W, false><<<grid, kLayerThreads, 0, s>>>(a, nh, nd, eps, scale,   \
                                                                   decay_dtype, beta_dtype); \
  } while (0)
#define LK_KDA_LAYER_W(V)                                                  \
  do {                                                                     \
    if (weight_dtype == LK_DTYPE_F32) LK_KDA_LAYER(V, LK_DTYPE_F32);       \
    else if (weight_dtype == LK_DTYPE_F16) LK_KDA_LAYER(V, LK_DTYPE_F16);  \
    else LK_KDA_LAYER(V, LK_DTYPE_BF16);                                   \
  } while (0)
  if (value_dtype == LK_DTYPE_F32) LK_KDA_LAYER_W(LK_DTYPE_F32);
  else if (value_dtype == LK_DTYPE_F16) LK_KDA_LAYER_W(LK_DTYPE_F16);
  else LK_KDA_LAYER_W(LK_DTYPE_BF16);
#undef LK_KDA_LAYER_W
#undef LK_KDA_LAYER
  return check_launch("lk_kda_decode_layer");
}

int lk_kda_decode_layer_split(const void* q_in, const void* k_in, const void* v_in,
                              const void* q_state, const void* k_state, const void* v_state,
                              void* q_state_out, void* k_state_out, void* v_state_out,
                              const void* q_weight, const void* k_weight, const void* v_weight,
                              const void* raw_decay, const float* dt_bias, const float* a_log,
                              const void* raw_beta, float* state, float* out, int64_t batch,
                              int64_t heads, int64_t head_dim, float eps, float scale,
                              int value_dtype, int weight_dtype, int decay_dtype, int beta_dtype,
                              void* stream) {
  LK_REQUIRE(batch > 0 && heads > 0, "KDA decode dimensions must be nonzero");
  LK_REQUIRE(head_dim > 0 && head_dim <= kLayerMaxDim && head_dim % 4 == 0,
             "one-launch KDA layer takes head_dim a multiple of 4 up to %d, got %lld",
             kLayerMaxDim, (long long)head_dim);
  LK_REQUIRE(eps > 0, "eps must be positive");
  LK_REQUIRE(heads * head_dim < (int64_t{1} << 31), "too many channels");
  LK_REQUIRE(valid_dtype(value_dtype) && valid_dtype(weight_dtype) && valid_dtype(decay_dtype) &&
                 valid_dtype(beta_dtype),
             "unknown dtype code");
  LK_REQUIRE(q_in && k_in && v_in && q_state && k_state && v_state && q_state_out &&
                 k_state_out && v_state_out && q_weight && k_weight && v_weight && raw_decay &&
                 dt_bias && a_log && raw_beta && state && out,
             "null pointer argument");
  LK_REQUIRE(q_state_out != q_state && k_state_out != k_state && v_state_out != v_state,
             "the split KDA layer writes the shifted convolution states to other buffers");
  LK_REQUIRE(reinterpret_cast<uintptr_t>(state) % 16 == 0 && reinterpret_cast<uintptr_t>(out) % 16 == 0,
             "state and out must be 16-byte aligned");
  const int64_t vs = (head_dim + kSplitCols - 1) / kSplitCols;
  const int64_t items = batch * heads * vs;
  LK_REQUIRE(items < (int64_t{1} << 31), "too many heads");
  const int paired = (vs % 2 == 0 && items % 16 == 0) ? 1 : 0;
  SplitArgs a{{q_in, k_in, v_in}, {q_state, k_state, v_state},
              {q_state_out, k_state_out, v_state_out}, {q_weight, k_weight, v_weight},
              raw_decay, dt_bias, a_log, raw_beta, state, out};
  const dim3 grid(static_cast<unsigned>(items));
  const int nh = static_cast<int>(heads), nd = static_cast<int>(head_dim),
            nvs = static_cast<int>(vs);
  hipStream_t s = as_stream(stream);
  const bool gates_as_values = decay_dtype == value_dtype && beta_dtype == value_dtype;
#define LK_KDA_SPLIT(V, W)                                                                   \
  do {                                                                                       \
    if (gates_as_values)                                                                     \
      kda_layer_split_kernel<V, W, true><<<grid, kSplitThreads, 0, s>>>(                     \
          a, nh, nd, nvs, items, paired, eps, scale, decay_dtype, beta_dtype);               \
    else                                                                                     \
      kda_layer_split_kernel<V, W, false><<<grid, kSplitThreads, 0, s>>>(                    \
          a, nh, nd, nvs, items, paired, eps, scale, decay_dtype, beta_dtype);               \
  } while (0)
#define LK_KDA_SPLIT_W(V)                                             \
  do {                                                                \
    if (weight_dtype == LK_DTYPE_F32) LK_KDA_SPLIT(V, LK_DTYPE_F32);  \
    else if (weight_dtype == LK_DTYPE_F16) LK_KDA_SPLIT(V, LK_DTYPE_F16); \
    else LK_KDA_SPLIT(V, LK_DTYPE_BF16);                              \
  } while (0)
  if (value_dtype == LK_DTYPE_F32) LK_KDA_SPLIT_W(LK_DTYPE_F32);
  else if (value_dtype == LK_DTYPE_F16) LK_KDA_SPLIT_W(LK_DTYPE_F16);
  else LK_KDA_SPLIT_W(LK_DTYPE_BF16);
#undef LK_KDA_SPLIT_W
#undef LK_KDA_SPLIT
  return check_launch("lk_kda_decode_layer_split");
}

}  // extern "C"
