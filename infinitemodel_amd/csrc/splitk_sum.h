// Ordered sum of split-K fp32 partials into bf16 rows, shared by the prefill GEMM launchers:
// y[m, n] = bf16((..((0 + part[0][m][n]) + part[1][m][n]) + ...) * scale[n]), the splits added in
// index order (deterministic), the per-row int8 scale applied after the sum.
#pragma once
#include "imq_common.h"

namespace imq {
namespace {

// S splits (compile time): each thread issues all S 16-byte partial loads of its 4 columns before
// adding any, then stores the 4 bf16 results as one 8-byte store. Needs N % 4 == 0, sym % 4 == 0, an
// 8-byte aligned y and a 16-byte aligned part.
template <int BITS, int SDT, int S>
__global__ __launch_bounds__(256) void splitk_sum_kernel(const float* __restrict__ part, int M, int N,
                                                         const void* __restrict__ sc, int64_t ssn,
                                                         uint16_t* __restrict__ y, int64_t sym) {
  const int64_t n4 = N / 4;
  const int64_t total = (int64_t)M * n4;
  const size_t plane = (size_t)M * N;
  for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total; t += (int64_t)gridDim.x * blockDim.x) {
    const int m = (int)(t / n4);
    const int n = 4 * (int)(t - (int64_t)m * n4);
    const float* src = part + (size_t)m * N + n;
    f32x4_t p[S];
#pragma unroll
    for (int sp = 0; sp < S; ++sp) p[sp] = *(const f32x4_t*)(src + sp * plane);
    float v[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int sp = 0; sp < S; ++sp)
#pragma unroll
      for (int q = 0; q < 4; ++q) v[q] += p[sp][q];
    if constexpr (BITS == 8) {
#pragma unroll
      for (int q = 0; q < 4; ++q) v[q] *= load_as_f32<SDT>(sc, (int64_t)(n + q) * ssn);
    }
    uint32_t o[2] = {cvt_pk_bf16(v[0], v[1]), cvt_pk_bf16(v[2], v[3])};
    *(uint2*)(y + (int64_t)m * sym + n) = make_uint2(o[0], o[1]);
  }
}

// Any layout, any split count: 4 columns per thread, element by element.
template <int BITS, int SDT>
__global__ __launch_bounds__(256) void splitk_sum_any_kernel(const float* __restrict__ part, int splits, int M,
                                                             int N, const void* __restrict__ sc, int64_t ssn,
                                                             uint16_t* __restrict__ y, int64_t sym) {
  const int64_t n4 = (N + 3) / 4;
  const int64_t total = (int64_t)M * n4;
  for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total; t += (int64_t)gridDim.x * blockDim.x) {
    const int m = (int)(t / n4);
    const int n = 4 * (int)(t - (int64_t)m * n4);
    float v[4] = {0.f, 0.f, 0.f, 0.f};
    for (int sp = 0; sp < splits; ++sp) {
      const float* src = part + ((size_t)sp * M + m) * N + n;
#pragma unroll
      for (int q = 0; q < 4; ++q)
        if (n + q < N) v[q] += src[q];
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      if (n + q >= N) break;
      float o = v[q];
      if constexpr (BITS == 8) o *= load_as_f32<SDT>(sc, (int64_t)(n + q) * ssn);
      y[(int64_t)m * sym + n + q] = (uint16_t)cvt_pk_bf16(o, 0.f);
    }
  }
}

// Launches the ordered sum of `splits` partial planes [splits][M][N] on stream st.
template <int BITS, int SDT>
int splitk_sum(const float* part, int splits, int M, int N, const void* sc, int64_t ssn, uint16_t* y, int64_t sym,
               hipStream_t st) {
  const bool vec = N % 4 == 0 && sym % 4 == 0 && ((uintptr_t)y & 7) == 0 && ((uintptr_t)part & 15) == 0;
  const int64_t total = (int64_t)M * ((N + 3) / 4);
  const int64_t blocks = imq_cdiv(total, 256) < 8192 ? imq_cdiv(total, 256) : 8192;
  const dim3 g((unsigned)blocks), b(256);
  if (vec) {
    switch (splits) {
#define IMQ_SUM(S) \
  case S: splitk_sum_kernel<BITS, SDT, S><<<g, b, 0, st>>>(part, M, N, sc, ssn, y, sym); break;
      IMQ_SUM(2) IMQ_SUM(3) IMQ_SUM(4) IMQ_SUM(5) IMQ_SUM(6) IMQ_SUM(7) IMQ_SUM(8)
#undef IMQ_SUM
      default: splitk_sum_any_kernel<BITS, SDT><<<g, b, 0, st>>>(part, splits, M, N, sc, ssn, y, sym);
    }
  } else {
    splitk_sum_any_kernel<BITS, SDT><<<g, b, 0, st>>>(part, splits, M, N, sc, ssn, y, sym);
  }
  IMQ_LAUNCH_CHECK();
  return IMQ_OK;
}

}  // namespace
}  // namespace imq
