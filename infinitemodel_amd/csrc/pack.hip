// RTN packers on the GPU, bit-identical to the CPU packers the cache compiler and the load-time
// quantizer share (shard_compile.py:50-94 pack_linear_int2 / pack_linear_int4, 170-178
// pack_linear_int8; worker_quant.py:1588-1608, 1921-1944, 511-536). They quantize a weight
// already resident on the device instead of round-tripping it through the host.
//
// Group-wise asymmetric (int4 / int2), per group of G columns of a row, K zero-padded to a
// multiple of G before the min / max (the pad takes part in them):
//   scale = clamp((max - min) / qmax, 1e-8), zero = clamp(rint(-min / scale), 0, qmax),
//   q = clamp(rint(w / scale + zero), 0, qmax),
// in fp32 with IEEE division and round-half-even, the divide and the add rounded separately;
// scale and zero are stored in W's dtype (round to nearest even). Clamps are written as compares
// so that, as in torch, a -0.0 zero point (min exactly 0) keeps its sign.
// Per-row symmetric (int8), in W's own dtype: scale = max(dt(amax|w| / 127), dt(1e-8)),
// q = clamp(rint(dt(w / scale)), -127, 127) -- the quotient is rounded to dt before rint.
#include <algorithm>

#include "imq_common.h"

namespace {

template <int DT>
IMQ_DEV float load_w(const void* p, int64_t idx) { return load_as_f32<DT>(p, idx); }

// One wave per (row, group) item, grid-strided; a lane holds EPL = G / 64 consecutive columns.
template <int BITS, int DT, int EPL>
__global__ __launch_bounds__(256) void pack_g_kernel(const void* __restrict__ W, int64_t sw, int64_t N,
                                                     int64_t in_f, int ng, uint8_t* __restrict__ q, int64_t sq,
                                                     void* __restrict__ sc, void* __restrict__ zr, int64_t ssn) {
  constexpr int G = 64 * EPL;
  constexpr float QMAX = (float)((1 << BITS) - 1);
  constexpr int CPB = 8 / BITS;                        // codes per byte
  __shared__ uint8_t codes[4][G];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t items = N * ng;
  for (int64_t it = (int64_t)blockIdx.x * 4 + wave; it < items; it += (int64_t)gridDim.x * 4) {
    const int64_t n = it / ng;
    const int g = (int)(it - n * ng);
    const int64_t k0 = (int64_t)g * G + lane * EPL;
    float v[EPL];
    float lo = 0.f, hi = 0.f;
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
      v[e] = (k0 + e < in_f) ? load_w<DT>(W, n * sw + k0 + e) : 0.f;
      lo = e == 0 ? v[e] : fminf(lo, v[e]);
      hi = e == 0 ? v[e] : fmaxf(hi, v[e]);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      lo = fminf(lo, __shfl_xor(lo, off, 64));
      hi = fmaxf(hi, __shfl_xor(hi, off, 64));
    }
    float s = (hi - lo) / QMAX;
    s = s < 1e-8f ? 1e-8f : s;
    float z = rintf(-lo / s);
    z = z < 0.f ? 0.f : z;
    z = z > QMAX ? QMAX : z;
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
      float t = rintf(v[e] / s + z);
      t = t < 0.f ? 0.f : t;
      t = t > QMAX ? QMAX : t;
      codes[wave][lane * EPL + e] = (uint8_t)(int)t;
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");   // codes visible to the wave's lanes
    constexpr int NB = G / CPB;                               // packed bytes of the group
    for (int b = lane; b < NB; b += 64) {
      uint32_t byte = 0;
#pragma unroll
      for (int j = 0; j < CPB; ++j) byte |= (uint32_t)codes[wave][b * CPB + j] << (BITS * j);
      q[n * sq + (int64_t)g * NB + b] = (uint8_t)byte;
    }
    if (lane == 0) {
      store_from_f32<DT>(sc, n * ssn + g, s);
      store_from_f32<DT>(zr, n * ssn + g, z);
    }
    __builtin_amdgcn_wave_barrier();                          // codes reused by the next item
  }
}

// One wave per row: |w| max over the row, then the codes.
template <int DT>
__global__ __launch_bounds__(256) void pack_w8_kernel(const void* __restrict__ W, int64_t sw, int64_t N,
                                                      int64_t K, int8_t* __restrict__ q, int64_t sq,
                                                      void* __restrict__ sc, int64_t ssn) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  for (int64_t n = (int64_t)blockIdx.x * 4 + wave; n < N; n += (int64_t)gridDim.x * 4) {
    float amax = 0.f;
    for (int64_t k = lane; k < K; k += 64) amax = fmaxf(amax, fabsf(load_w<DT>(W, n * sw + k)));
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 64));
    float s = round_to<DT>(amax / 127.f);
    const float smin = round_to<DT>(1e-8f);
    s = s < smin ? smin : s;
    for (int64_t k = lane; k < K; k += 64) {
      float t = rintf(round_to<DT>(load_w<DT>(W, n * sw + k) / s));
      t = t < -127.f ? -127.f : t;                   // NaN (0 / 0 at an fp16 zero row) stays NaN
      t = t > 127.f ? 127.f : t;
      q[n * sq + k] = (int8_t)(t == t ? (int)t : 0);  // and converts to 0, as the host cast does
    }
    if (lane == 0) store_from_f32<DT>(sc, n * ssn, s);
  }
}

bool dt_ok(int d) { return d == IMQ_DT_BF16 || d == IMQ_DT_FP16 || d == IMQ_DT_FP32; }

unsigned grid_for(int64_t items) {
  const int64_t b = (items + 3) / 4;
  return (unsigned)(b < 65536 ? (b > 0 ? b : 1) : 65536);
}

template <int BITS, int DT>
int launch_g(const void* W, int64_t sw, int64_t N, int64_t in_f, int64_t G, uint8_t* q, int64_t sq, void* sc,
             void* zr, int64_t ssn, hipStream_t st) {
  const int ng = (int)((in_f + G - 1) / G);
  const unsigned grid = grid_for(N * ng);
  switch (G) {
    case 64: pack_g_kernel<BITS, DT, 1><<<grid, 256, 0, st>>>(W, sw, N, in_f, ng, q, sq, sc, zr, ssn); break;
    case 128: pack_g_kernel<BITS, DT, 2><<<grid, 256, 0, st>>>(W, sw, N, in_f, ng, q, sq, sc, zr, ssn); break;
    case 256: pack_g_kernel<BITS, DT, 4><<<grid, 256, 0, st>>>(W, sw, N, in_f, ng, q, sq, sc, zr, ssn); break;
    default: return IMQ_ERR_UNSUPPORTED;
  }
  IMQ_LAUNCH_CHECK();
  return IMQ_OK;
}

template <int BITS>
int pack_g(const void* W, int64_t sw, int wdt, int64_t N, int64_t in_f, int64_t G, void* q, int64_t sq, void* sc,
           void* zr, int64_t ssn, void* stream) {
  if (!W || !q || !sc || !zr || !dt_ok(wdt)) return IMQ_ERR_INVALID;
  if (N < 0 || in_f <= 0 || G <= 0 || sw < in_f) return IMQ_ERR_INVALID;
  const int64_t ng = (in_f + G - 1) / G;
  if (sq < ng * G * BITS / 8 || ssn < ng) return IMQ_ERR_INVALID;
  if (G != 64 && G != 128 && G != 256) return IMQ_ERR_UNSUPPORTED;
  if (N == 0) return IMQ_OK;
  if (ng > 0x7fffffff) return IMQ_ERR_UNSUPPORTED;
  hipStream_t st = (hipStream_t)stream;
  uint8_t* qb = (uint8_t*)q;
  switch (wdt) {
    case IMQ_DT_BF16: return launch_g<BITS, IMQ_DT_BF16>(W, sw, N, in_f, G, qb, sq, sc, zr, ssn, st);
    case IMQ_DT_FP16: return launch_g<BITS, IMQ_DT_FP16>(W, sw, N, in_f, G, qb, sq, sc, zr, ssn, st);
    case IMQ_DT_FP32: return launch_g<BITS, IMQ_DT_FP32>(W, sw, N, in_f, G, qb, sq, sc, zr, ssn, st);
  }
  return IMQ_ERR_INVALID;
}

// Line-tiled layout of packed weight rows (int4 / int2 codes alike: it moves bytes): in 16-row tile
// t, the 2 KiB block of line-step l (bytes [128 l, 128 l + 128) of each row) lies at 2048 (KL t + l)
// (KL = row bytes / 128); its half h holds rows 8 h .. 8 h + 7 of the tile, and its 16-byte slot s
// (0..63) piece 4 (((s >> 3) & 1) ^ h) + (s >> 4) of row 8 h + (s & 7).
IMQ_DEV void tiled_slot_src(int h, int s, int& r, int& piece) {
  r = 8 * h + (s & 7);
  piece = 4 * (((s >> 3) & 1) ^ h) + (s >> 4);
}

// One thread per 16-byte piece of the tiled array (tile) or of the row array (untile); the write
// side is the contiguous one. Pieces are 64-bit indexed.
__global__ __launch_bounds__(256) void line_tile_kernel(const uint8_t* __restrict__ src, int64_t srs, int64_t KL,
                                                        int64_t pieces, uint8_t* __restrict__ dst) {
  for (int64_t i = blockIdx.x * 256ll + threadIdx.x; i < pieces; i += (int64_t)gridDim.x * 256) {
    const int s = (int)(i & 63), h = (int)((i >> 6) & 1);
    const int64_t blk = i >> 7, t = blk / KL, l = blk - t * KL;
    int r, piece;
    tiled_slot_src(h, s, r, piece);
    const u32x4_t v = *(const u32x4_t*)(src + (16 * t + r) * srs + 128 * l + 16 * piece);
    *(u32x4_t*)(dst + 16 * i) = v;
  }
}

__global__ __launch_bounds__(256) void line_untile_kernel(const uint8_t* __restrict__ src, int64_t KL, int64_t pieces,
                                                          uint8_t* __restrict__ dst, int64_t drs) {
  for (int64_t i = blockIdx.x * 256ll + threadIdx.x; i < pieces; i += (int64_t)gridDim.x * 256) {
    // row-order piece i: row n, line-step l, piece p (8 per line)
    const int p = (int)(i & 7);
    const int64_t rl = i >> 3, n = rl / KL, l = rl - n * KL;
    const int r = (int)(n & 15), h = r >> 3;
    const int s = (r & 7) + 8 * ((p >> 2) ^ h) + 16 * (p & 3);
    const int64_t j = (((n >> 4) * KL + l) * 2 + h) * 64 + s;
    *(u32x4_t*)(dst + n * drs + 128 * l + 16 * p) = *(const u32x4_t*)(src + 16 * j);
  }
}

int tile_args_ok(const void* a, const void* b, int64_t rs, int64_t N, int64_t row_bytes) {
  if (!a || !b || N < 0 || row_bytes <= 0 || N % 16 != 0 || row_bytes % 128 != 0 || rs < row_bytes)
    return IMQ_ERR_INVALID;
  if (((uintptr_t)a & 15) || ((uintptr_t)b & 15) || (rs & 15)) return IMQ_ERR_ALIGN;
  return IMQ_OK;
}

}  // namespace

extern "C" int imq_line_tile(const void* q_rows, int64_t q_row_stride, int64_t N, int64_t row_bytes, void* q_tiled,
                             void* stream) {
  const int rc = tile_args_ok(q_rows, q_tiled, q_row_stride, N, row_bytes);
  if (rc != IMQ_OK || N == 0) return rc;
  const int64_t pieces = N * (row_bytes / 16);
  const unsigned grid = (unsigned)std::min<int64_t>((pieces + 255) / 256, 65536);
  line_tile_kernel<<<grid, 256, 0, (hipStream_t)stream>>>((const uint8_t*)q_rows, q_row_stride, row_bytes / 128, pieces,
                                                           (uint8_t*)q_tiled);
  IMQ_LAUNCH_CHECK();
  return IMQ_OK;
}

extern "C" int imq_line_untile(const void* q_tiled, int64_t N, int64_t row_bytes, void* q_rows, int64_t q_row_stride,
                               void* stream) {
  const int rc = tile_args_ok(q_tiled, q_rows, q_row_stride, N, row_bytes);
  if (rc != IMQ_OK || N == 0) return rc;
  const int64_t pieces = N * (row_bytes / 16);
  const unsigned grid = (unsigned)std::min<int64_t>((pieces + 255) / 256, 65536);
  line_untile_kernel<<<grid, 256, 0, (hipStream_t)stream>>>((const uint8_t*)q_tiled, row_bytes / 128, pieces,
                                                             (uint8_t*)q_rows, q_row_stride);
  IMQ_LAUNCH_CHECK();
  return IMQ_OK;
}

extern "C" int imq_pack_w4(const void* W, int64_t w_row_stride, int w_dtype, int64_t N, int64_t in_features,
                           int64_t group_size, void* qweight, int64_t q_row_stride, void* scale, void* zero,
                           int64_t sz_row_stride, void* stream) {
  return pack_g<4>(W, w_row_stride, w_dtype, N, in_features, group_size, qweight, q_row_stride, scale, zero,
                   sz_row_stride, stream);
}

extern "C" int imq_pack_w2(const void* W, int64_t w_row_stride, int w_dtype, int64_t N, int64_t in_features,
                           int64_t group_size, void* qweight, int64_t q_row_stride, void* scale, void* zero,
                           int64_t sz_row_stride, void* stream) {
  return pack_g<2>(W, w_row_stride, w_dtype, N, in_features, group_size, qweight, q_row_stride, scale, zero,
                   sz_row_stride, stream);
}

extern "C" int imq_pack_w8(const void* W, int64_t w_row_stride, int w_dtype, int64_t N, int64_t K, void* qweight,
                           int64_t q_row_stride, void* scale, int64_t s_stride_n, void* stream) {
  if (!W || !qweight || !scale || !dt_ok(w_dtype)) return IMQ_ERR_INVALID;
  if (N < 0 || K <= 0 || w_row_stride < K || q_row_stride < K || s_stride_n < 1) return IMQ_ERR_INVALID;
  if (N == 0) return IMQ_OK;
  hipStream_t st = (hipStream_t)stream;
  const unsigned grid = grid_for(N);
  int8_t* qb = (int8_t*)qweight;
  switch (w_dtype) {
    case IMQ_DT_BF16: pack_w8_kernel<IMQ_DT_BF16><<<grid, 256, 0, st>>>(W, w_row_stride, N, K, qb, q_row_stride, scale, s_stride_n); break;
    case IMQ_DT_FP16: pack_w8_kernel<IMQ_DT_FP16><<<grid, 256, 0, st>>>(W, w_row_stride, N, K, qb, q_row_stride, scale, s_stride_n); break;
    case IMQ_DT_FP32: pack_w8_kernel<IMQ_DT_FP32><<<grid, 256, 0, st>>>(W, w_row_stride, N, K, qb, q_row_stride, scale, s_stride_n); break;
  }
  IMQ_LAUNCH_CHECK();
  return IMQ_OK;
}
