// Measurement probes (no counterpart in the reference): read-only HBM streaming kernels that set
// the practical ceiling the decode kernels are measured against.
//
//   imq_probe_read      one launch reads one buffer (16-byte non-temporal loads, four per lane in
//                       flight, grid-stride) -- the per-launch ceiling of a linear's weight read;
//   imq_probe_read_seq  one persistent launch reads a list of buffers in order, every workgroup
//                       taking its share of each buffer in turn -- the same bytes with no launch
//                       boundary between buffers.
// Both fold the loaded words into a value that is stored only if it equals an impossible key, so
// the loads cannot be removed and nothing is written.
#include "imq_common.h"

namespace {

#ifndef IMQ_PROBE_UNROLL
#define IMQ_PROBE_UNROLL 4
#endif
#ifndef IMQ_PROBE_GRID_PER_CU
#define IMQ_PROBE_GRID_PER_CU 8
#endif
constexpr int kProbeThreads = 256;
constexpr int kProbeUnroll = IMQ_PROBE_UNROLL;
constexpr uint32_t kNeverKey = 0x9e3779b9u;

IMQ_DEV uint32_t read_span(const u32x4_t* __restrict__ p, int64_t n16, int64_t first, int64_t stride) {
  uint32_t acc = 0;
  for (int64_t i = first; i < n16; i += stride) {
    u32x4_t v[kProbeUnroll];
#pragma unroll
    for (int u = 0; u < kProbeUnroll; ++u) {
      const int64_t j = i + (int64_t)u * kProbeThreads;
      v[u] = j < n16 ? __builtin_nontemporal_load(p + j) : u32x4_t{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int u = 0; u < kProbeUnroll; ++u) acc ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
  }
  return acc;
}

__global__ __launch_bounds__(kProbeThreads) void probe_read_kernel(const u32x4_t* __restrict__ p, int64_t n16,
                                                                   uint32_t* __restrict__ sink) {
  const int64_t first = (int64_t)blockIdx.x * kProbeThreads * kProbeUnroll + threadIdx.x;
  const int64_t stride = (int64_t)gridDim.x * kProbeThreads * kProbeUnroll;
  const uint32_t acc = read_span(p, n16, first, stride);
  if (acc == kNeverKey) sink[blockIdx.x * kProbeThreads + threadIdx.x] = acc;
}

__global__ __launch_bounds__(kProbeThreads) void probe_read_seq_kernel(const uint64_t* __restrict__ ptrs,
                                                                       const int64_t* __restrict__ n16s, int nbuf,
                                                                       uint32_t* __restrict__ sink) {
  const int64_t first = (int64_t)blockIdx.x * kProbeThreads * kProbeUnroll + threadIdx.x;
  const int64_t stride = (int64_t)gridDim.x * kProbeThreads * kProbeUnroll;
  uint32_t acc = 0;
  for (int b = 0; b < nbuf; ++b) acc ^= read_span((const u32x4_t*)ptrs[b], n16s[b], first, stride);
  if (acc == kNeverKey) sink[blockIdx.x * kProbeThreads + threadIdx.x] = acc;
}

int probe_grid(int64_t n16, int cus) {
  const int64_t per_block = (int64_t)kProbeThreads * kProbeUnroll;
  int64_t g = (n16 + per_block - 1) / per_block;
  const int64_t cap = (int64_t)cus * IMQ_PROBE_GRID_PER_CU;
  return (int)(g < cap ? (g > 0 ? g : 1) : cap);
}

}  // namespace

extern "C" int64_t imq_probe_sink_bytes(void) {
  return (int64_t)probe_grid(INT64_MAX / 2, device_info().cus) * kProbeThreads * 4;
}

extern "C" int imq_probe_read(const void* buf, int64_t bytes, void* sink, int64_t sink_bytes, void* stream) {
  if (!buf || !sink || bytes < 16 || (bytes & 15) || ((uintptr_t)buf & 15) || ((uintptr_t)sink & 3))
    return IMQ_ERR_INVALID;
  const int64_t n16 = bytes / 16;
  const int grid = probe_grid(n16, device_info().cus);
  if (sink_bytes < (int64_t)grid * kProbeThreads * 4) return IMQ_ERR_INVALID;
  probe_read_kernel<<<dim3((unsigned)grid), dim3(kProbeThreads), 0, (hipStream_t)stream>>>(
      (const u32x4_t*)buf, n16, (uint32_t*)sink);
  IMQ_LAUNCH_CHECK();
  return IMQ_OK;
}

extern "C" int imq_probe_read_seq(const void* ptrs, const void* n16s, int nbuf, int64_t max_n16, void* sink,
                                  int64_t sink_bytes, void* stream) {
  if (!ptrs || !n16s || !sink || nbuf <= 0 || max_n16 <= 0 || ((uintptr_t)sink & 3)) return IMQ_ERR_INVALID;
  const int grid = probe_grid(max_n16, device_info().cus);
  if (sink_bytes < (int64_t)grid * kProbeThreads * 4) return IMQ_ERR_INVALID;
  probe_read_seq_kernel<<<dim3((unsigned)grid), dim3(kProbeThreads), 0, (hipStream_t)stream>>>(
      (const uint64_t*)ptrs, (const int64_t*)n16s, nbuf, (uint32_t*)sink);
  IMQ_LAUNCH_CHECK();
  return IMQ_OK;
}
