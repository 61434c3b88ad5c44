// Measurement probes (no counterpart in the reference): the hardware ceilings the hot-path
// kernels are measured against, each a kernel of its own so the figures are reproduced by
// committed code.
//
//   imq_probe_stream  read-only stream over a list of buffers in one launch. The buffers'
//                     16-byte words are cut into chunks of 256 x U words (U loads per lane);
//                     workgroup g reads chunks g, g + grid, g + 2 grid, ... of the buffers taken
//                     in order, so one launch over one linear's buffers is the per-launch ceiling
//                     of its weight read, and one launch over every linear of a pass is the same
//                     bytes with no launch boundary. Software-pipelined: the next chunk's U loads
//                     are issued before the current chunk's are consumed (2 U loads per lane in
//                     flight), every load unconditional (addresses clamped into the buffer), so
//                     no buffer boundary drains the stream.
//   imq_probe_copy    device copy with U 16-byte loads, then U non-temporal stores, per lane.
//   imq_probe_empty   an empty kernel (the launch cost of a chain of dependent kernels).
//   imq_probe_mfma    independent bf16 MFMA chains on register operands (the MFMA issue peak).
// The read-only kernels fold what they load into a value stored only if it equals an impossible
// key, so the loads cannot be removed and nothing is written.
#include "imq_common.h"

namespace {

constexpr int kProbeThreads = 256;
constexpr uint32_t kNeverKey = 0x9e3779b9u;
constexpr int kMaxWgPerCu = 32;

// Chunk loads are buffer loads: one SGPR resource per chunk (base = the chunk's first word,
// num_records = the chunk's in-bounds bytes), a per-lane offset of 16 * lane and the load index in
// the scalar offset. No VALU per load, and the hardware range check returns zeros past the
// buffer instead of needing clamped addresses.
IMQ_DEV __amdgpu_buffer_rsrc_t chunk_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

template <bool NT>
IMQ_DEV u32x4_t probe_load(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, NT ? 2 : 0));
}

// Uniform (per-workgroup) walker over the concatenated chunk sequence of the buffer list. Chunk
// indices are 32-bit (a chunk is at least 4 KiB, so 2^32 chunks cover 16 TiB): the compares stay
// scalar, with no VGPR temporaries that could alias a load still in flight.
template <int U>
struct ChunkWalker {
  static constexpr uint32_t CH = (uint32_t)kProbeThreads * U;
  const uint64_t* ptrs;
  const int64_t* n16s;
  int nbuf;
  int b;
  uint32_t base;  // global chunk index of buffer b's first chunk
  uint32_t end;   // global chunk index one past buffer b's last chunk
  int64_t n16;    // 16-byte words of buffer b

  IMQ_DEV void init(const uint64_t* p, const int64_t* n, int nb) {
    ptrs = p;
    n16s = n;
    nbuf = nb;
    b = 0;
    base = 0;
    n16 = n16s[0];
    end = (uint32_t)((n16 + CH - 1) / CH);
  }
  // Position of global chunk g (g never decreases between calls): base pointer, first word and
  // word count of its buffer. False past the last buffer, leaving p / off / lim unchanged.
  // Buffers of zero words hold no chunk and are skipped.
  IMQ_DEV bool locate(uint32_t g, const u32x4_t*& p, int64_t& off, int64_t& lim) {
    while (g >= end) {
      if (++b >= nbuf) return false;
      base = end;
      n16 = n16s[b];
      end = base + (uint32_t)((n16 + CH - 1) / CH);
    }
    p = (const u32x4_t*)ptrs[b];
    off = (int64_t)(g - base) * CH;
    lim = n16;
    return true;
  }
};

// The chunk's U loads: word off + 256 u + lane of p, for words below lim (zeros past it).
template <int U, bool NT>
IMQ_DEV void issue_chunk(u32x4_t (&v)[U], const u32x4_t* p, int64_t off, int64_t lim, uint32_t voff) {
  const int64_t left = lim - off;
  const uint32_t bytes = (uint32_t)(left < (int64_t)kProbeThreads * U ? left : (int64_t)kProbeThreads * U) * 16u;
  const __amdgpu_buffer_rsrc_t r = chunk_rsrc(p + off, bytes);
#pragma unroll
  for (int u = 0; u < U; ++u) v[u] = probe_load<NT>(r, voff, (uint32_t)u * kProbeThreads * 16u);
}

template <int U>
IMQ_DEV uint32_t fold_chunk(const u32x4_t (&v)[U]) {
  uint32_t a = 0;
#pragma unroll
  for (int u = 0; u < U; ++u) a ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
  return a;
}

template <int U, bool NT>
__global__ __launch_bounds__(kProbeThreads) void probe_stream_kernel(const uint64_t* __restrict__ ptrs,
                                                                     const int64_t* __restrict__ n16s, int nbuf,
                                                                     uint32_t* __restrict__ sink) {
  const int tid = threadIdx.x;
  const uint32_t G = gridDim.x;
  ChunkWalker<U> w;
  w.init(ptrs, n16s, nbuf);
  uint32_t g = blockIdx.x;
  const uint32_t voff = (uint32_t)tid * 16u;
  const u32x4_t* p;
  int64_t off, lim;
  if (!w.locate(g, p, off, lim)) return;
  u32x4_t a[U], c[U];
  issue_chunk<U, NT>(a, p, off, lim, voff);
  uint32_t acc = 0;
  // Each half issues the next chunk's loads, then consumes the previous chunk. Past the end the
  // loads are issued anyway (locate leaves p / off / lim at the last chunk: in bounds, cached) and
  // never consumed, so no fold follows a branch and one load set stays in flight while the other
  // is folded.
  for (;;) {
    g += G;
    const bool m1 = w.locate(g, p, off, lim);
    issue_chunk<U, NT>(c, p, off, lim, voff);
    __builtin_amdgcn_sched_barrier(0);
    acc ^= fold_chunk<U>(a);
    __builtin_amdgcn_sched_barrier(0);
    if (!m1) break;
    g += G;
    const bool m2 = w.locate(g, p, off, lim);
    issue_chunk<U, NT>(a, p, off, lim, voff);
    __builtin_amdgcn_sched_barrier(0);
    acc ^= fold_chunk<U>(c);
    __builtin_amdgcn_sched_barrier(0);
    if (!m2) break;
  }
  if (acc == kNeverKey) sink[(int64_t)blockIdx.x * kProbeThreads + tid] = acc;
}

template <int U>
__global__ __launch_bounds__(kProbeThreads) void probe_copy_kernel(u32x4_t* __restrict__ dst,
                                                                   const u32x4_t* __restrict__ src, int64_t n16) {
  constexpr int64_t CH = (int64_t)kProbeThreads * U;
  const int tid = threadIdx.x;
  for (int64_t c = blockIdx.x; c * CH < n16; c += gridDim.x) {
    u32x4_t v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      int64_t j = c * CH + (int64_t)u * kProbeThreads + tid;
      j = j < n16 ? j : n16 - 1;
      v[u] = __builtin_nontemporal_load(src + j);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t j = c * CH + (int64_t)u * kProbeThreads + tid;
      if (j < n16) __builtin_nontemporal_store(v[u], dst + j);
    }
  }
}

__global__ void probe_empty_kernel() {}

// Four independent accumulator chains per wave on loop-invariant register operands.
template <int KIND>
__global__ __launch_bounds__(kProbeThreads) void probe_mfma_kernel(int64_t iters, float* __restrict__ sink) {
  const uint32_t t = threadIdx.x;
  u32x4_t ra = {0x3f803f80u ^ t, 0x3f813f80u, 0x3f803f82u, 0x3f833f80u};
  u32x4_t rb = {0x3f803f80u, 0x3f803f84u ^ (t << 1), 0x3f853f80u, 0x3f803f80u};
  const bf16x8_t a = __builtin_bit_cast(bf16x8_t, ra);
  const bf16x8_t b = __builtin_bit_cast(bf16x8_t, rb);
  float s = 0.f;
  if constexpr (KIND == 0) {
    f32x16_t c0 = {}, c1 = {}, c2 = {}, c3 = {};
    for (int64_t i = 0; i < iters; ++i) {
      c0 = mfma32x32x16(a, b, c0);
      c1 = mfma32x32x16(a, b, c1);
      c2 = mfma32x32x16(a, b, c2);
      c3 = mfma32x32x16(a, b, c3);
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) s += c0[r] + c1[r] + c2[r] + c3[r];
  } else {
    f32x4_t c0 = {}, c1 = {}, c2 = {}, c3 = {};
    for (int64_t i = 0; i < iters; ++i) {
      c0 = mfma16x16x32(a, b, c0);
      c1 = mfma16x16x32(a, b, c1);
      c2 = mfma16x16x32(a, b, c2);
      c3 = mfma16x16x32(a, b, c3);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) s += c0[r] + c1[r] + c2[r] + c3[r];
  }
  if (s == 1234.5f) sink[(int64_t)blockIdx.x * kProbeThreads + t] = s;
}

template <int U, bool NT>
void launch_stream(int grid, const uint64_t* ptrs, const int64_t* n16s, int nbuf, uint32_t* sink, hipStream_t st) {
  probe_stream_kernel<U, NT><<<dim3((unsigned)grid), dim3(kProbeThreads), 0, st>>>(ptrs, n16s, nbuf, sink);
}

}  // namespace

extern "C" int64_t imq_probe_sink_bytes(void) {
  return (int64_t)device_info().cus * kMaxWgPerCu * kProbeThreads * 4;
}

extern "C" int imq_probe_stream(const void* ptrs, const void* n16s, int nbuf, int64_t total_n16, int loads_per_lane,
                                int wg_per_cu, int nontemporal, void* sink, int64_t sink_bytes, void* stream) {
  if (!ptrs || !n16s || !sink || nbuf <= 0 || total_n16 <= 0 || wg_per_cu < 1 || wg_per_cu > kMaxWgPerCu ||
      ((uintptr_t)sink & 3))
    return IMQ_ERR_INVALID;
  const int U = loads_per_lane;
  if (U != 1 && U != 2 && U != 4 && U != 8 && U != 16) return IMQ_ERR_INVALID;
  // the chunk count of the concatenated list is at least ceil(total / chunk), so no workgroup of
  // this grid starts past the end
  const int64_t chunks = imq_cdiv(total_n16, (int64_t)kProbeThreads * U);
  if (chunks >= ((int64_t)1 << 31)) return IMQ_ERR_UNSUPPORTED;
  const int64_t cap = (int64_t)device_info().cus * wg_per_cu;
  const int grid = (int)(chunks < cap ? chunks : cap);
  if (sink_bytes < (int64_t)grid * kProbeThreads * 4) return IMQ_ERR_INVALID;
  const uint64_t* p = (const uint64_t*)ptrs;
  const int64_t* n = (const int64_t*)n16s;
  uint32_t* s = (uint32_t*)sink;
  hipStream_t st = (hipStream_t)stream;
  const bool nt = nontemporal != 0;
  switch (U) {
    case 1: nt ? launch_stream<1, true>(grid, p, n, nbuf, s, st) : launch_stream<1, false>(grid, p, n, nbuf, s, st); break;
    case 2: nt ? launch_stream<2, true>(grid, p, n, nbuf, s, st) : launch_stream<2, false>(grid, p, n, nbuf, s, st); break;
    case 4: nt ? launch_stream<4, true>(grid, p, n, nbuf, s, st) : launch_stream<4, false>(grid, p, n, nbuf, s, st); break;
    case 8: nt ? launch_stream<8, true>(grid, p, n, nbuf, s, st) : launch_stream<8, false>(grid, p, n, nbuf, s, st); break;
    default: nt ? launch_stream<16, true>(grid, p, n, nbuf, s, st) : launch_stream<16, false>(grid, p, n, nbuf, s, st); break;
  }
  IMQ_LAUNCH_CHECK();
  return IMQ_OK;
}

extern "C" int imq_probe_copy(void* dst, const void* src, int64_t bytes, int loads_per_lane, int wg_per_cu,
                              void* stream) {
  if (!dst || !src || bytes < 16 || (bytes & 15) || ((uintptr_t)dst & 15) || ((uintptr_t)src & 15) ||
      wg_per_cu < 1 || wg_per_cu > kMaxWgPerCu)
    return IMQ_ERR_INVALID;
  const int64_t n16 = bytes / 16;
  const int U = loads_per_lane;
  if (U != 2 && U != 4 && U != 8) return IMQ_ERR_INVALID;
  const int64_t chunks = imq_cdiv(n16, (int64_t)kProbeThreads * U);
  const int64_t cap = (int64_t)device_info().cus * wg_per_cu;
  const dim3 grid((unsigned)(chunks < cap ? chunks : cap));
  hipStream_t st = (hipStream_t)stream;
  if (U == 2) probe_copy_kernel<2><<<grid, dim3(kProbeThreads), 0, st>>>((u32x4_t*)dst, (const u32x4_t*)src, n16);
  else if (U == 4) probe_copy_kernel<4><<<grid, dim3(kProbeThreads), 0, st>>>((u32x4_t*)dst, (const u32x4_t*)src, n16);
  else probe_copy_kernel<8><<<grid, dim3(kProbeThreads), 0, st>>>((u32x4_t*)dst, (const u32x4_t*)src, n16);
  IMQ_LAUNCH_CHECK();
  return IMQ_OK;
}

extern "C" int imq_probe_empty(int grid, void* stream) {
  if (grid < 1 || grid > 65536) return IMQ_ERR_INVALID;
  probe_empty_kernel<<<dim3((unsigned)grid), dim3(64), 0, (hipStream_t)stream>>>();
  IMQ_LAUNCH_CHECK();
  return IMQ_OK;
}

extern "C" int imq_probe_mfma(int kind, int64_t iters, int wg_per_cu, void* sink, int64_t sink_bytes,
                              void* stream) {
  if ((kind != 0 && kind != 1) || iters < 1 || wg_per_cu < 1 || wg_per_cu > kMaxWgPerCu || !sink ||
      ((uintptr_t)sink & 3))
    return IMQ_ERR_INVALID;
  const int grid = device_info().cus * wg_per_cu;
  if (sink_bytes < (int64_t)grid * kProbeThreads * 4) return IMQ_ERR_INVALID;
  hipStream_t st = (hipStream_t)stream;
  if (kind == 0) probe_mfma_kernel<0><<<dim3((unsigned)grid), dim3(kProbeThreads), 0, st>>>(iters, (float*)sink);
  else probe_mfma_kernel<1><<<dim3((unsigned)grid), dim3(kProbeThreads), 0, st>>>(iters, (float*)sink);
  IMQ_LAUNCH_CHECK();
  return IMQ_OK;
}
