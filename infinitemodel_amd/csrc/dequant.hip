// Bit-exact reference dequant kernels (int4 g-wise, int2 g-wise, int8 per-row).
//
// These reproduce `_dequant(dtype)` of the reference modules exactly, rounding after every
// elementwise op in the output dtype (worker_quant.py:638-648, 1652-1664, 439). They serve the
// module's `_dequant` on the GPU (the naive path and the self-checks) and are the unit the
// bit-exact parity tests pin. HBM-bound: each thread reads one packed word, writes 8 values.
#include "imq_common.h"

namespace {

template <int BITS, int SDT, int ZDT, int ODT>
__global__ __launch_bounds__(256) void dequant_g_kernel(
    const uint8_t* __restrict__ q, int64_t sq, const void* __restrict__ sc, int64_t ssn, int64_t ssg,
    const void* __restrict__ zr, int64_t szn, int64_t szg, int64_t N, int64_t in_f, int64_t G,
    void* __restrict__ out, int64_t so, int64_t chunks_per_row) {
  constexpr int CODES_PER_BYTE = 8 / BITS;
  constexpr int BYTES_PER_CHUNK = 8 / CODES_PER_BYTE;   // 8 codes per thread
  const int64_t total = N * chunks_per_row;
  for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total;
       t += (int64_t)gridDim.x * blockDim.x) {
    const int64_t n = t / chunks_per_row;
    const int64_t c = t - n * chunks_per_row;
    const int64_t k0 = c * 8;
    const uint8_t* qp = q + n * sq + c * BYTES_PER_CHUNK;
    uint32_t bits = 0;
#pragma unroll
    for (int b = 0; b < BYTES_PER_CHUNK; ++b) bits |= (uint32_t)qp[b] << (8 * b);
    // All 8 codes of a chunk share one group when G % 8 == 0 (always true: G is a multiple
    // of the 8-code chunk for every format this library accepts; checked on the host).
    const int64_t g = k0 / G;
    const float z = round_to<ODT>(load_as_f32<ZDT>(zr, n * szn + g * szg));
    const float s = round_to<ODT>(load_as_f32<SDT>(sc, n * ssn + g * ssg));
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int64_t k = k0 + i;
      if (k < in_f) {
        const float code = (float)((bits >> (BITS * i)) & ((1u << BITS) - 1u));
        const float d = round_to<ODT>(code - z);
        const float w = round_to<ODT>(d * s);
        store_from_f32<ODT>(out, n * so + k, w);
      }
    }
  }
}

template <int SDT, int ODT>
__global__ __launch_bounds__(256) void dequant_w8_kernel(const int8_t* __restrict__ q, int64_t sq,
                                                         const void* __restrict__ sc, int64_t ssn,
                                                         int64_t N, int64_t K, void* __restrict__ out,
                                                         int64_t so) {
  const int64_t total = N * K;
  for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total;
       t += (int64_t)gridDim.x * blockDim.x) {
    const int64_t n = t / K;
    const int64_t k = t - n * K;
    const float s = load_as_f32<SDT>(sc, n * ssn);
    // q.to(x_dtype) is exact for |q| <= 127; one fp32 product, one rounding to the result dtype.
    store_from_f32<ODT>(out, n * so + k, round_to<ODT>((float)q[n * sq + k] * s));
  }
}

template <int BITS, int SDT, int ZDT, int ODT>
int launch_g(const void* q, int64_t sq, const void* sc, int64_t ssn, int64_t ssg, const void* zr,
             int64_t szn, int64_t szg, int64_t N, int64_t in_f, int64_t G, void* out, int64_t so,
             hipStream_t st) {
  const int64_t kpad_chunks = imq_cdiv(in_f, 8);
  const int64_t total = N * kpad_chunks;
  if (total == 0) return IMQ_OK;
  const int64_t blocks = imq_cdiv(total, 256) < 65536 ? imq_cdiv(total, 256) : 65536;
  dequant_g_kernel<BITS, SDT, ZDT, ODT><<<dim3((unsigned)blocks), dim3(256), 0, st>>>(
      (const uint8_t*)q, sq, sc, ssn, ssg, zr, szn, szg, N, in_f, G, out, so, kpad_chunks);
  IMQ_LAUNCH_CHECK();
  return IMQ_OK;
}

template <int BITS, int SDT, int ZDT>
int dispatch_out(int odt, const void* q, int64_t sq, const void* sc, int64_t ssn, int64_t ssg,
                 const void* zr, int64_t szn, int64_t szg, int64_t N, int64_t in_f, int64_t G,
                 void* out, int64_t so, hipStream_t st) {
  switch (odt) {
    case IMQ_DT_BF16: return launch_g<BITS, SDT, ZDT, IMQ_DT_BF16>(q, sq, sc, ssn, ssg, zr, szn, szg, N, in_f, G, out, so, st);
    case IMQ_DT_FP16: return launch_g<BITS, SDT, ZDT, IMQ_DT_FP16>(q, sq, sc, ssn, ssg, zr, szn, szg, N, in_f, G, out, so, st);
    case IMQ_DT_FP32: return launch_g<BITS, SDT, ZDT, IMQ_DT_FP32>(q, sq, sc, ssn, ssg, zr, szn, szg, N, in_f, G, out, so, st);
  }
  return IMQ_ERR_INVALID;
}

template <int BITS, int SDT>
int dispatch_z(int zdt, int odt, const void* q, int64_t sq, const void* sc, int64_t ssn, int64_t ssg,
               const void* zr, int64_t szn, int64_t szg, int64_t N, int64_t in_f, int64_t G, void* out,
               int64_t so, hipStream_t st) {
  switch (zdt) {
    case IMQ_DT_BF16: return dispatch_out<BITS, SDT, IMQ_DT_BF16>(odt, q, sq, sc, ssn, ssg, zr, szn, szg, N, in_f, G, out, so, st);
    case IMQ_DT_FP16: return dispatch_out<BITS, SDT, IMQ_DT_FP16>(odt, q, sq, sc, ssn, ssg, zr, szn, szg, N, in_f, G, out, so, st);
    case IMQ_DT_FP32: return dispatch_out<BITS, SDT, IMQ_DT_FP32>(odt, q, sq, sc, ssn, ssg, zr, szn, szg, N, in_f, G, out, so, st);
  }
  return IMQ_ERR_INVALID;
}

template <int BITS>
int dequant_g(const void* q, int64_t sq, const void* sc, int64_t ssn, int64_t ssg, int sdt,
              const void* zr, int64_t szn, int64_t szg, int zdt, int64_t N, int64_t in_f, int64_t G,
              void* out, int64_t so, int odt, void* stream) {
  if (!q || !sc || !zr || !out || N < 0 || in_f < 0 || G <= 0 || (G % 8) != 0) return IMQ_ERR_INVALID;
  if (sq < (imq_cdiv(in_f, G) * G * BITS) / 8) return IMQ_ERR_INVALID;
  hipStream_t st = (hipStream_t)stream;
  switch (sdt) {
    case IMQ_DT_BF16: return dispatch_z<BITS, IMQ_DT_BF16>(zdt, odt, q, sq, sc, ssn, ssg, zr, szn, szg, N, in_f, G, out, so, st);
    case IMQ_DT_FP16: return dispatch_z<BITS, IMQ_DT_FP16>(zdt, odt, q, sq, sc, ssn, ssg, zr, szn, szg, N, in_f, G, out, so, st);
    case IMQ_DT_FP32: return dispatch_z<BITS, IMQ_DT_FP32>(zdt, odt, q, sq, sc, ssn, ssg, zr, szn, szg, N, in_f, G, out, so, st);
  }
  return IMQ_ERR_INVALID;
}

template <int SDT>
int dequant8_out(int odt, const void* q, int64_t sq, const void* sc, int64_t ssn, int64_t N, int64_t K,
                 void* out, int64_t so, hipStream_t st) {
  const int64_t total = N * K;
  if (total == 0) return IMQ_OK;
  const int64_t blocks = imq_cdiv(total, 256) < 65536 ? imq_cdiv(total, 256) : 65536;
  switch (odt) {
    case IMQ_DT_BF16:
      dequant_w8_kernel<SDT, IMQ_DT_BF16><<<dim3((unsigned)blocks), dim3(256), 0, st>>>((const int8_t*)q, sq, sc, ssn, N, K, out, so);
      break;
    case IMQ_DT_FP16:
      dequant_w8_kernel<SDT, IMQ_DT_FP16><<<dim3((unsigned)blocks), dim3(256), 0, st>>>((const int8_t*)q, sq, sc, ssn, N, K, out, so);
      break;
    case IMQ_DT_FP32:
      dequant_w8_kernel<SDT, IMQ_DT_FP32><<<dim3((unsigned)blocks), dim3(256), 0, st>>>((const int8_t*)q, sq, sc, ssn, N, K, out, so);
      break;
    default:
      return IMQ_ERR_INVALID;
  }
  IMQ_LAUNCH_CHECK();
  return IMQ_OK;
}

}  // namespace

extern "C" int imq_dequant_w4(const void* qweight, int64_t q_row_stride, const void* scale,
                              int64_t s_stride_n, int64_t s_stride_g, int s_dtype, const void* zero,
                              int64_t z_stride_n, int64_t z_stride_g, int z_dtype, int64_t N,
                              int64_t in_features, int64_t group_size, void* out, int64_t out_row_stride,
                              int out_dtype, void* stream) {
  return dequant_g<4>(qweight, q_row_stride, scale, s_stride_n, s_stride_g, s_dtype, zero, z_stride_n,
                      z_stride_g, z_dtype, N, in_features, group_size, out, out_row_stride, out_dtype,
                      stream);
}

extern "C" int imq_dequant_w2(const void* qweight, int64_t q_row_stride, const void* scale,
                              int64_t s_stride_n, int64_t s_stride_g, int s_dtype, const void* zero,
                              int64_t z_stride_n, int64_t z_stride_g, int z_dtype, int64_t N,
                              int64_t in_features, int64_t group_size, void* out, int64_t out_row_stride,
                              int out_dtype, void* stream) {
  return dequant_g<2>(qweight, q_row_stride, scale, s_stride_n, s_stride_g, s_dtype, zero, z_stride_n,
                      z_stride_g, z_dtype, N, in_features, group_size, out, out_row_stride, out_dtype,
                      stream);
}

extern "C" int imq_dequant_w8(const void* qweight, int64_t q_row_stride, const void* scale,
                              int64_t s_stride_n, int s_dtype, int64_t N, int64_t K, void* out,
                              int64_t out_row_stride, int out_dtype, void* stream) {
  if (!qweight || !scale || !out || N < 0 || K < 0 || q_row_stride < K) return IMQ_ERR_INVALID;
  hipStream_t st = (hipStream_t)stream;
  switch (s_dtype) {
    case IMQ_DT_BF16: return dequant8_out<IMQ_DT_BF16>(out_dtype, qweight, q_row_stride, scale, s_stride_n, N, K, out, out_row_stride, st);
    case IMQ_DT_FP16: return dequant8_out<IMQ_DT_FP16>(out_dtype, qweight, q_row_stride, scale, s_stride_n, N, K, out, out_row_stride, st);
    case IMQ_DT_FP32: return dequant8_out<IMQ_DT_FP32>(out_dtype, qweight, q_row_stride, scale, s_stride_n, N, K, out, out_row_stride, st);
  }
  return IMQ_ERR_INVALID;
}
