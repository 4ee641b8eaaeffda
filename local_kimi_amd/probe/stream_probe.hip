// Measurement probes for the memory-system floors the decode kernels are held
// against (no reference counterpart; bench.py --workload stream_floor):
//
//  * a streaming read of up to kProbeRegions regions, each read once with
//    16-byte non-temporal loads (the weight loads of the decode kernels), so
//    one launch over the 27 weight matrices of a batch-1 MoE layer (9 experts
//    x gate, up, down) measures what reading that layer can cost at best;
//  * an empty kernel, whose back-to-back launches give the per-launch floor.
//
// The read kernel folds what it loads into one word per thread and stores it
// only if it equals a value no input produces in practice, so the loads stay
// live without adding write traffic.
//
// This file builds into its own library (liblkprobe.so), apart from the
// product library, so it keeps its own error state.

#include <stdarg.h>
#include <stdio.h>

#include "lk_common.hpp"
#include "lk_probe.h"

namespace lk {

static thread_local char g_probe_error[256] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_probe_error, sizeof(g_probe_error), fmt, ap);
  va_end(ap);
}

int fail_arg(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_probe_error, sizeof(g_probe_error), fmt, ap);
  va_end(ap);
  return LK_ERR_ARGUMENT;
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: kernel launch failed: %s", what, hipGetErrorString(e));
    return LK_ERR_HIP;
  }
  return LK_OK;
}

namespace {

constexpr int kProbeRegions = 32;
constexpr int kProbeThreads = 256;
constexpr int kProbeUnits = 8;  // 16-byte loads per thread per block
constexpr int64_t kProbeBlockBytes = int64_t{kProbeThreads} * kProbeUnits * 16;

struct RegionList {
  const uint8_t* base[kProbeRegions];
  int64_t bytes[kProbeRegions];
  int64_t first_block[kProbeRegions + 1];  // prefix of blocks per region
  int count;
};

__global__ void __launch_bounds__(kProbeThreads)
stream_read_kernel(const RegionList list, uint32_t* __restrict__ sink) {
  const int64_t b = blockIdx.x;
  int r = 0;
  while (r + 1 < list.count && list.first_block[r + 1] <= b) ++r;
  const int64_t start = (b - list.first_block[r]) * kProbeBlockBytes;
  const int64_t units = list.bytes[r] / 16;
  const uint8_t* base = list.base[r];
  uint4 v[kProbeUnits];
#pragma unroll
  for (int u = 0; u < kProbeUnits; ++u) {
    const int64_t unit = start / 16 + u * kProbeThreads + threadIdx.x;
    v[u] = load_stream_u4(base + (unit < units ? unit : units - 1) * 16);
  }
  uint32_t acc = 0;
#pragma unroll
  for (int u = 0; u < kProbeUnits; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  if (acc == 0x9E3779B9u) sink[threadIdx.x] = acc;
}

__global__ void empty_kernel() {}

}  // namespace
}  // namespace lk

using namespace lk;

extern "C" {

int lk_probe_stream_read(const void* const* regions, const int64_t* bytes, int count,
                         uint32_t* sink, void* stream) {
  LK_REQUIRE(regions && bytes && sink, "null pointer argument");
  LK_REQUIRE(count > 0 && count <= kProbeRegions, "1..%d regions per probe, got %d",
             kProbeRegions, count);
  RegionList list{};
  list.count = count;
  list.first_block[0] = 0;
  for (int r = 0; r < count; ++r) {
    LK_REQUIRE(regions[r] != nullptr, "null region %d", r);
    LK_REQUIRE(bytes[r] >= 16 && bytes[r] % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(regions[r]) % 16 == 0,
               "region %d must be 16-byte aligned and a positive multiple of 16 bytes", r);
    list.base[r] = static_cast<const uint8_t*>(regions[r]);
    list.bytes[r] = bytes[r];
    list.first_block[r + 1] =
        list.first_block[r] + (bytes[r] + kProbeBlockBytes - 1) / kProbeBlockBytes;
  }
  const int64_t blocks = list.first_block[count];
  LK_REQUIRE(blocks < (int64_t{1} << 31), "probe regions too large");
  stream_read_kernel<<<static_cast<unsigned>(blocks), kProbeThreads, 0, as_stream(stream)>>>(
      list, sink);
  return check_launch("lk_probe_stream_read");
}

int lk_probe_empty(void* stream) {
  empty_kernel<<<1, kWave, 0, as_stream(stream)>>>();
  return check_launch("lk_probe_empty");
}

const char* lk_probe_last_error(void) { return lk::g_probe_error; }

}  // extern "C"
