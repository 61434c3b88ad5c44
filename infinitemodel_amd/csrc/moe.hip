// Fused int4 MoE expert kernels for gfx950.
//
// imq_moe_rows_w4  : per (token, slot) row GEMV against the row's expert -- the contract of the
//                    reference's `_mk` grouped kernel (worker_quant.py:1419-1450), without its
//                    split-K atomics (fixed-order wave reduction, deterministic).
// imq_moe_experts_w4: one MoE layer's experts forward, the semantics of the transformers eager
//                    experts loop the reference self-checks against (modeling_olmoe.py:301-325)
//                    in the reference's fused form (worker_quant.py:2167-2191):
//                      gate_up rows -> silu(gate) * up -> down rows -> weighted combine,
//                    with fp32 intermediates (the eager path rounds each stage to bf16; only h,
//                    the down projection's activation, is rounded to bf16 here).
#include "imq_common.h"

namespace {

constexpr int64_t kAlign = 256;
int64_t align_up(int64_t v, int64_t a) { return (v + a - 1) / a * a; }

// One wave per (row b, output channel n). Lane l handles 8-code words l, l+64, ...
// Output fp32 (OUT_F32) or bf16. x row for b is x + (b / xdiv) * sxm.
template <int SDT, bool OUT_F32>
__global__ __launch_bounds__(256) void moe_rows_kernel(
    const uint16_t* __restrict__ x, int64_t sxm, int64_t xdiv, int64_t B, int64_t Kpad,
    const int32_t* __restrict__ eid, int64_t E, const uint8_t* __restrict__ q, int64_t sqe, int64_t sqn,
    const void* __restrict__ sc, int64_t sse, int64_t ssn, int64_t ssg, const void* __restrict__ zr,
    int64_t sze, int64_t szn, int64_t szg, int64_t N, int64_t G, void* __restrict__ y, int64_t sym) {
  const int lane = threadIdx.x & 63;
  const int64_t n = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int64_t b = blockIdx.y;
  if (n >= N || b >= B) return;
  int64_t e = eid[b];
  if (e < 0 || e >= E) e = 0;   // out-of-range ids are rejected on the host; keep loads in bounds
  const uint8_t* qr = q + e * sqe + n * sqn;
  const uint16_t* xr = x + (b / xdiv) * sxm;
  float acc = 0.f;
  const int64_t words = Kpad / 8;
  for (int64_t wd = lane; wd < words; wd += 64) {
    const uint32_t w = *(const uint32_t*)(qr + wd * 4);
    const u32x4_t xv = *(const u32x4_t*)(xr + wd * 8);
    const int64_t g = (wd * 8) / G;
    const float s = load_as_bf16_f32<SDT>(sc, e * sse + n * ssn + g * ssg);
    const float z = load_as_bf16_f32<SDT>(zr, e * sze + n * szn + g * szg);
    float dq = 0.f, xsum = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float xi = __uint_as_float(i & 1 ? (xv[i >> 1] & 0xffff0000u) : (xv[i >> 1] << 16));
      dq = fmaf(xi, (float)((w >> (4 * i)) & 0xFu), dq);
      xsum += xi;
    }
    acc = fmaf(s, dq - z * xsum, acc);
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
  if (lane == 0) {
    if constexpr (OUT_F32) ((float*)y)[b * sym + n] = acc;
    else ((uint16_t*)y)[b * sym + n] = (uint16_t)f32_to_bf16_bits(acc);
  }
}

// h[b][i] = bf16(silu(g) * u), g = gu[b][i], u = gu[b][I + i]; zero for I <= i < I_pad.
__global__ __launch_bounds__(256) void swiglu_kernel(const float* __restrict__ gu, int64_t B, int64_t I,
                                                     int64_t I_pad, uint16_t* __restrict__ h) {
  const int64_t total = B * I_pad;
  for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total;
       t += (int64_t)gridDim.x * blockDim.x) {
    const int64_t b = t / I_pad;
    const int64_t i = t - b * I_pad;
    float v = 0.f;
    if (i < I) {
      const float g = gu[b * 2 * I + i];
      const float u = gu[b * 2 * I + I + i];
      v = g / (1.f + __expf(-g)) * u;
    }
    h[t] = (uint16_t)f32_to_bf16_bits(v);
  }
}

// out[t][n] = bf16(sum_j w[t][j] * z[t*k + j][n]), j in slot order (fixed).
__global__ __launch_bounds__(256) void combine_kernel(const float* __restrict__ z, const uint16_t* __restrict__ w,
                                                      int64_t T, int64_t k, int64_t H,
                                                      uint16_t* __restrict__ out, int64_t so) {
  const int64_t total = T * H;
  for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total;
       t += (int64_t)gridDim.x * blockDim.x) {
    const int64_t tok = t / H;
    const int64_t n = t - tok * H;
    float acc = 0.f;
    for (int64_t j = 0; j < k; ++j) acc = fmaf(bf16_bits_to_f32(w[tok * k + j]), z[(tok * k + j) * H + n], acc);
    out[tok * so + n] = (uint16_t)f32_to_bf16_bits(acc);
  }
}

template <bool OUT_F32>
int launch_rows(const uint16_t* x, int64_t sxm, int64_t xdiv, int64_t B, int64_t Kpad, const int32_t* eid,
                int64_t E, const uint8_t* q, int64_t sqe, int64_t sqn, const void* sc, int64_t sse, int64_t ssn,
                int64_t ssg, const void* zr, int64_t sze, int64_t szn, int64_t szg, int sdt, int64_t N, int64_t G,
                void* y, int64_t sym, hipStream_t st) {
  if (B == 0 || N == 0) return IMQ_OK;
  if (B > 65535) return IMQ_ERR_UNSUPPORTED;
  dim3 grid((unsigned)imq_cdiv(N, 4), (unsigned)B);
  switch (sdt) {
    case IMQ_DT_BF16:
      moe_rows_kernel<IMQ_DT_BF16, OUT_F32><<<grid, dim3(256), 0, st>>>(x, sxm, xdiv, B, Kpad, eid, E, q, sqe, sqn, sc, sse, ssn, ssg, zr, sze, szn, szg, N, G, y, sym);
      break;
    case IMQ_DT_FP16:
      moe_rows_kernel<IMQ_DT_FP16, OUT_F32><<<grid, dim3(256), 0, st>>>(x, sxm, xdiv, B, Kpad, eid, E, q, sqe, sqn, sc, sse, ssn, ssg, zr, sze, szn, szg, N, G, y, sym);
      break;
    case IMQ_DT_FP32:
      moe_rows_kernel<IMQ_DT_FP32, OUT_F32><<<grid, dim3(256), 0, st>>>(x, sxm, xdiv, B, Kpad, eid, E, q, sqe, sqn, sc, sse, ssn, ssg, zr, sze, szn, szg, N, G, y, sym);
      break;
    default:
      return IMQ_ERR_INVALID;
  }
  IMQ_LAUNCH_CHECK();
  return IMQ_OK;
}

bool aligned(const void* p, int a) { return ((uintptr_t)p % a) == 0; }

}  // namespace

extern "C" int imq_moe_rows_w4(const void* x, int64_t x_row_stride, int64_t B, int64_t K_pad,
                               const int32_t* eid, int64_t E, const void* qweight, int64_t q_stride_e,
                               int64_t q_row_stride, const void* scale, int64_t s_stride_e, int64_t s_stride_n,
                               int64_t s_stride_g, const void* zero, int64_t z_stride_e, int64_t z_stride_n,
                               int64_t z_stride_g, int sz_dtype, int64_t N, int64_t group_size, void* y,
                               int64_t y_row_stride, void* stream) {
  if (!x || !eid || !qweight || !scale || !zero || !y) return IMQ_ERR_INVALID;
  if (B < 0 || N < 0 || E <= 0 || K_pad <= 0 || group_size <= 0 || K_pad % group_size || group_size % 8)
    return IMQ_ERR_INVALID;
  if (q_row_stride < K_pad / 2 || x_row_stride < K_pad || y_row_stride < N) return IMQ_ERR_INVALID;
  if (!aligned(qweight, 4) || (q_row_stride % 4) || (q_stride_e % 4) || !aligned(x, 16) || (x_row_stride % 8))
    return IMQ_ERR_ALIGN;
  return launch_rows<false>((const uint16_t*)x, x_row_stride, 1, B, K_pad, eid, E, (const uint8_t*)qweight,
                            q_stride_e, q_row_stride, scale, s_stride_e, s_stride_n, s_stride_g, zero,
                            z_stride_e, z_stride_n, z_stride_g, sz_dtype, N, group_size, y, y_row_stride,
                            (hipStream_t)stream);
}

extern "C" int64_t imq_moe_workspace_bytes(int64_t T, int64_t top_k, int64_t E, int64_t H, int64_t I,
                                           int64_t group_size) {
  (void)E;
  if (T < 0 || top_k <= 0 || H <= 0 || I <= 0 || group_size <= 0) return -1;
  const int64_t B = T * top_k;
  const int64_t I_pad = imq_cdiv(I, group_size) * group_size;
  return align_up(B * 2 * I * 4, kAlign) + align_up(B * I_pad * 2, kAlign) + align_up(B * H * 4, kAlign);
}

extern "C" int imq_moe_experts_w4(const void* hidden, int64_t h_row_stride, int64_t T, int64_t H, int64_t top_k,
                                  const int32_t* topk_idx, const void* topk_w, int64_t E, const void* gu_q,
                                  int64_t gu_q_stride_e, int64_t gu_q_row_stride, const void* gu_s, const void* gu_z,
                                  int64_t gu_sz_stride_e, int64_t gu_sz_stride_n, int64_t I, const void* dn_q,
                                  int64_t dn_q_stride_e, int64_t dn_q_row_stride, const void* dn_s, const void* dn_z,
                                  int64_t dn_sz_stride_e, int64_t dn_sz_stride_n, int sz_dtype, int64_t group_size,
                                  void* out, int64_t out_row_stride, void* workspace, int64_t workspace_bytes,
                                  void* stream) {
  if (!hidden || !topk_idx || !topk_w || !gu_q || !gu_s || !gu_z || !dn_q || !dn_s || !dn_z || !out)
    return IMQ_ERR_INVALID;
  if (T < 0 || H <= 0 || top_k <= 0 || E <= 0 || I <= 0 || group_size <= 0 || group_size % 8) return IMQ_ERR_INVALID;
  if (T == 0) return IMQ_OK;
  const int64_t G = group_size;
  const int64_t H_pad = imq_cdiv(H, G) * G;
  const int64_t I_pad = imq_cdiv(I, G) * G;
  const int64_t need = imq_moe_workspace_bytes(T, top_k, E, H, I, G);
  if (!workspace || workspace_bytes < need) return IMQ_ERR_INVALID;
  if (h_row_stride < H_pad || out_row_stride < H) return IMQ_ERR_INVALID;
  if (!aligned(gu_q, 4) || !aligned(dn_q, 4) || (gu_q_row_stride % 4) || (dn_q_row_stride % 4) ||
      (gu_q_stride_e % 4) || (dn_q_stride_e % 4) || !aligned(hidden, 16) || (h_row_stride % 8) ||
      !aligned(workspace, 256))
    return IMQ_ERR_ALIGN;
  hipStream_t st = (hipStream_t)stream;
  const int64_t B = T * top_k;
  char* ws = (char*)workspace;
  float* gu = (float*)ws;
  uint16_t* h = (uint16_t*)(ws + align_up(B * 2 * I * 4, kAlign));
  float* z = (float*)(ws + align_up(B * 2 * I * 4, kAlign) + align_up(B * I_pad * 2, kAlign));
  const int64_t ng1 = H_pad / G, ng2 = I_pad / G;
  (void)ng1;
  (void)ng2;
  int rc = launch_rows<true>((const uint16_t*)hidden, h_row_stride, top_k, B, H_pad, topk_idx, E,
                             (const uint8_t*)gu_q, gu_q_stride_e, gu_q_row_stride, gu_s, gu_sz_stride_e,
                             gu_sz_stride_n, 1, gu_z, gu_sz_stride_e, gu_sz_stride_n, 1, sz_dtype, 2 * I, G, gu,
                             2 * I, st);
  if (rc != IMQ_OK) return rc;
  {
    const int64_t total = B * I_pad;
    const int64_t blocks = imq_cdiv(total, 256) < 4096 ? imq_cdiv(total, 256) : 4096;
    swiglu_kernel<<<dim3((unsigned)blocks), dim3(256), 0, st>>>(gu, B, I, I_pad, h);
    IMQ_LAUNCH_CHECK();
  }
  rc = launch_rows<true>(h, I_pad, 1, B, I_pad, topk_idx, E, (const uint8_t*)dn_q, dn_q_stride_e, dn_q_row_stride,
                         dn_s, dn_sz_stride_e, dn_sz_stride_n, 1, dn_z, dn_sz_stride_e, dn_sz_stride_n, 1, sz_dtype,
                         H, G, z, H, st);
  if (rc != IMQ_OK) return rc;
  {
    const int64_t total = T * H;
    const int64_t blocks = imq_cdiv(total, 256) < 4096 ? imq_cdiv(total, 256) : 4096;
    combine_kernel<<<dim3((unsigned)blocks), dim3(256), 0, st>>>(z, (const uint16_t*)topk_w, T, top_k, H,
                                                               (uint16_t*)out, out_row_stride);
    IMQ_LAUNCH_CHECK();
  }
  return IMQ_OK;
}
