// GPTQ int2 solver on gfx950: the column-by-column quantization of the reference's calibrated
// int2 packer (gptq_pack.py:78-189) after its Cholesky stage, emitting the same crumb format as
// the RTN int2 packer (qweight [out][in_pad / 4], crumb i of byte j = column 4 j + i, group
// scale / zero on the asymmetric 0..3 grid).
//
// The host loop walks blocks of `blocksize` columns:
//   gptq_block_kernel   one thread per output row (rows are independent inside a block): the
//                       block's columns of W staged in LDS, the parameters of every group starting
//                       in the block found from those block-start values (the reference reads W,
//                       not the in-block copy), then column by column: q = clamp(rint(w / s + z),
//                       0, 3), dq = (q - z) s, err = (w - dq) / Hinv[c][c], the rest of the block's
//                       columns updated by err Hinv[c][j]; crumbs packed four to a byte as they
//                       come, dq and err written out;
//   gptq_update_kernel  W[:, i2:] -= Err1 @ Hinv[i1:i2, i2:], each product summed over K in order.
// All arithmetic is float32 with every operation rounded on its own -- no FMA contraction in
// this file -- and sums in a fixed left-to-right order, so the result is reproducible bit for bit
// by a restatement with the same order. |x|^2.4 (the group search's error norm) is gptq_pow24,
// x^2 x^0.4 with x^0.4 range-reduced (atanh series for the logarithm, Taylor polynomial for 2^f).
#include "imq_common.h"

#pragma clang fp contract(off)

namespace {

constexpr int kGptqRows = 64;           // rows (threads) per workgroup of the block kernel
constexpr int kGptqMaxBlock = 128;      // columns per block
constexpr int kGptqMaxCand = 64;        // shrink candidates int(maxshrink * grid)

__device__ __forceinline__ float gptq_pow24(float a) {
  if (!(a >= 0x1p-50f)) return 0.f;     // the result would be below 2^-120
  const int bits = __float_as_int(a);
  int e = ((bits >> 23) & 0xFF) - 127;
  float m = __int_as_float((bits & 0x7FFFFF) | 0x3F800000);
  if (m > (float)1.4142135623730951) {
    m = m * 0.5f;
    e = e + 1;
  }
  const float t = (m - 1.f) / (m + 1.f);
  const float t2 = t * t;
  float p = (float)(1.0 / 9.0);
  p = p * t2 + (float)(1.0 / 7.0);
  p = p * t2 + (float)(1.0 / 5.0);
  p = p * t2 + (float)(1.0 / 3.0);
  p = p * t2 + 1.f;
  const float ln_m = (t + t) * p;
  const float log2a = (float)e + ln_m * (float)1.4426950408889634;
  const float y = (float)0.4 * log2a;
  const float n = rintf(y);
  const float u = (y - n) * (float)0.6931471805599453;
  float q = (float)(1.0 / 5040.0);
  q = q * u + (float)(1.0 / 720.0);
  q = q * u + (float)(1.0 / 120.0);
  q = q * u + (float)(1.0 / 24.0);
  q = q * u + (float)(1.0 / 6.0);
  q = q * u + 0.5f;
  q = q * u + 1.f;
  q = q * u + 1.f;
  const int ni = (int)n;                       // within [-20, 52] for these inputs
  return (a * a) * (q * __int_as_float((ni + 127) << 23));
}

__device__ __forceinline__ float clamp03(float x) { return fminf(fmaxf(x, 0.f), 3.f); }

struct GptqShrink {
  float pf3[kGptqMaxCand];              // fp32(p / 3), p = 1 - k / grid
  float pf[kGptqMaxCand];               // fp32(p)
  int nk;
};

// The group search of one row over cols values at v[0], v[stride], ... (gptq_pack.py:78-100).
__device__ void gptq_find_params(const float* v, int stride, int cols, const GptqShrink& sh, float* s_out,
                                 float* z_out) {
  float xmin = 0.f, xmax = 0.f;
  for (int c = 0; c < cols; ++c) {
    const float w = v[c * stride];
    xmin = fminf(xmin, w);
    xmax = fmaxf(xmax, w);
  }
  const float span = xmax - xmin;
  float best_err = __int_as_float(0x7F800000), best_s = 1.f, best_z = 0.f;
  for (int k = 0; k < sh.nk; ++k) {
    const float s1 = fmaxf(span * sh.pf3[k], 1e-8f);
    const float z1 = clamp03(rintf((-xmin * sh.pf[k]) / s1));
    float err = 0.f;
    for (int c = 0; c < cols; ++c) {
      const float w = v[c * stride];
      const float q = clamp03(rintf(w / s1 + z1));
      const float dq = (q - z1) * s1;
      err = err + gptq_pow24(fabsf(dq - w));
    }
    if (err < best_err) {
      best_err = err;
      best_s = s1;
      best_z = z1;
    }
  }
  *s_out = best_s;
  *z_out = best_z;
}

struct GptqBlockArgs {
  const float* W;                       // [out][ldw], the block's columns at their block-start values
  int64_t ldw;
  int out, in_f, i1, count, G, in_pad;
  const float* Hinv;                    // [in_f][ldh], upper factor
  int64_t ldh;
  uint8_t* q;                           // [out][ldq] crumbs
  int64_t ldq;
  float* scale;                         // [out][ldsz]
  float* zero;
  int64_t ldsz;
  float* dq;                            // [out][lddq] or null
  int64_t lddq;
  float* err;                           // [out][kGptqMaxBlock] this block's errors
  GptqShrink sh;
};

__global__ __launch_bounds__(kGptqRows) void gptq_block_kernel(GptqBlockArgs a) {
  __shared__ float W1[kGptqMaxBlock * kGptqRows];      // [column j][row]
  __shared__ float SG[kGptqMaxBlock / 4 * kGptqRows];  // [group of the block][row] scale, zero
  __shared__ float ZG[kGptqMaxBlock / 4 * kGptqRows];
  const int tid = threadIdx.x;
  const int r = blockIdx.x * kGptqRows + tid;
  const bool live = r < a.out;
  const int rr = live ? r : a.out - 1;
  const float* wrow = a.W + (int64_t)rr * a.ldw + a.i1;
  for (int j = 0; j < a.count; ++j) W1[j * kGptqRows + tid] = wrow[j];
  // parameters of the groups starting in this block, from the block-start values
  const int ngb = (a.count + a.G - 1) / a.G;
  for (int gi = 0; gi < ngb; ++gi) {
    const int c0 = gi * a.G;
    const int cols = a.count - c0 < a.G ? a.count - c0 : a.G;
    float sgi, zgi;
    gptq_find_params(W1 + c0 * kGptqRows + tid, kGptqRows, cols, a.sh, &sgi, &zgi);
    SG[gi * kGptqRows + tid] = sgi;
    ZG[gi * kGptqRows + tid] = zgi;
    const int g = (a.i1 + c0) / a.G;
    if (live) {
      a.scale[(int64_t)r * a.ldsz + g] = sgi;
      a.zero[(int64_t)r * a.ldsz + g] = zgi;
    }
  }
  uint32_t crumbs = 0;
  for (int i = 0; i < a.count; ++i) {
    const int col = a.i1 + i;
    const int gi = i / a.G;
    const float s = SG[gi * kGptqRows + tid], z = ZG[gi * kGptqRows + tid];
    const float w = W1[i * kGptqRows + tid];
    const float q = clamp03(rintf(w / s + z));
    const float dqv = (q - z) * s;
    const float* hrow = a.Hinv + (int64_t)col * a.ldh + a.i1;
    const float e = (w - dqv) / hrow[i];
    for (int j = i + 1; j < a.count; ++j) W1[j * kGptqRows + tid] = W1[j * kGptqRows + tid] - e * hrow[j];
    crumbs |= (uint32_t)q << (2 * (col & 3));
    if (live) {
      if ((col & 3) == 3) {
        a.q[(int64_t)r * a.ldq + (col >> 2)] = (uint8_t)crumbs;
        crumbs = 0;
      }
      if (a.dq != nullptr) a.dq[(int64_t)r * a.lddq + col] = dqv;
      a.err[(int64_t)r * kGptqMaxBlock + i] = e;
    }
  }
  // the last block: padded tail columns take the last group's rounded zero point
  if (a.i1 + a.count == a.in_f && live) {
    const uint32_t qt = (uint32_t)clamp03(rintf(ZG[(ngb - 1) * kGptqRows + tid]));   // the last group
    for (int col = a.in_f; col < a.in_pad; ++col) {
      crumbs |= qt << (2 * (col & 3));
      if ((col & 3) == 3) {
        a.q[(int64_t)r * a.ldq + (col >> 2)] = (uint8_t)crumbs;
        crumbs = 0;
      }
    }
  }
}

// W[r][c] -= sum_k err[r][k] * Hinv[i1 + k][c] for c in [c0, in_f): 64 x 64 tiles, 4 x 4 outputs
// per thread, the sum over k in order.
struct GptqUpdateArgs {
  float* W;
  int64_t ldw;
  int out, in_f, i1, count, c0;
  const float* Hinv;
  int64_t ldh;
  const float* err;
};

__global__ __launch_bounds__(256) void gptq_update_kernel(GptqUpdateArgs a) {
  __shared__ float Es[kGptqMaxBlock * 64];   // [k][row]
  __shared__ float Hs[kGptqMaxBlock * 64];   // [k][col]
  const int tid = threadIdx.x;
  const int rt = blockIdx.y * 64, ct = a.c0 + blockIdx.x * 64;
  for (int idx = tid; idx < a.count * 64; idx += 256) {
    const int k = idx / 64, x = idx - k * 64;
    const int row = rt + x < a.out ? rt + x : a.out - 1;
    const int col = ct + x < a.in_f ? ct + x : a.in_f - 1;
    Es[k * 64 + x] = a.err[(int64_t)row * kGptqMaxBlock + k];
    Hs[k * 64 + x] = a.Hinv[(int64_t)(a.i1 + k) * a.ldh + col];
  }
  __syncthreads();
  const int tr = (tid >> 4) * 4, tc = (tid & 15) * 4;
  float acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = 0.f;
  for (int k = 0; k < a.count; ++k) {
    float ev[4], hv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) ev[i] = Es[k * 64 + tr + i];
#pragma unroll
    for (int j = 0; j < 4; ++j) hv[j] = Hs[k * 64 + tc + j];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = acc[i][j] + ev[i] * hv[j];
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = rt + tr + i;
    if (row >= a.out) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int col = ct + tc + j;
      if (col < a.in_f) a.W[(int64_t)row * a.ldw + col] = a.W[(int64_t)row * a.ldw + col] - acc[i][j];
    }
  }
}

// The group search alone, one thread per row (the reference's _find_params as a call).
struct GptqParamsArgs {
  const float* Wg;
  int64_t ldw;
  int rows, cols;
  float* scale;
  float* zero;
  GptqShrink sh;
};

__global__ __launch_bounds__(256) void gptq_params_kernel(GptqParamsArgs a) {
  const int r = blockIdx.x * 256 + threadIdx.x;
  if (r >= a.rows) return;
  float s, z;
  gptq_find_params(a.Wg + (int64_t)r * a.ldw, 1, a.cols, a.sh, &s, &z);
  a.scale[r] = s;
  a.zero[r] = z;
}

int make_shrink(int grid, double maxshrink, GptqShrink* sh) {
  if (grid <= 0 || !(maxshrink > 0.0)) return IMQ_ERR_INVALID;
  const int nk = (int)(maxshrink * grid);           // int(maxshrink * grid) in double, as Python computes it
  if (nk < 1 || nk > kGptqMaxCand) return IMQ_ERR_UNSUPPORTED;
  sh->nk = nk;
  for (int k = 0; k < nk; ++k) {
    const double p = 1.0 - (double)k / grid;
    sh->pf3[k] = (float)(p / 3.0);
    sh->pf[k] = (float)p;
  }
  return IMQ_OK;
}

}  // namespace

extern "C" int64_t imq_gptq_int2_workspace_bytes(int64_t out, int64_t blocksize) {
  if (out <= 0 || blocksize <= 0 || blocksize > kGptqMaxBlock) return -1;
  return out * kGptqMaxBlock * 4;
}

extern "C" int imq_gptq_int2_params(const float* Wg, int64_t ldw, int64_t rows, int64_t cols, int grid,
                                    double maxshrink, float* scale, float* zero, void* stream) {
  if (!Wg || !scale || !zero || rows <= 0 || cols <= 0 || ldw < cols || rows > 0x7fffffff || cols > 0x7fffffff)
    return IMQ_ERR_INVALID;
  GptqParamsArgs a{Wg, ldw, (int)rows, (int)cols, scale, zero, {}};
  const int rc = make_shrink(grid, maxshrink, &a.sh);
  if (rc != IMQ_OK) return rc;
  gptq_params_kernel<<<dim3((unsigned)((rows + 255) / 256)), dim3(256), 0, (hipStream_t)stream>>>(a);
  IMQ_LAUNCH_CHECK();
  return IMQ_OK;
}

extern "C" int imq_gptq_int2_solve(float* W, int64_t ldw, int64_t out, int64_t in_f, const float* Hinv, int64_t ldh,
                                   int64_t group_size, int grid, double maxshrink, int64_t blocksize,
                                   uint8_t* qweight, int64_t ldq, float* scale, float* zero, int64_t ldsz, float* dq,
                                   int64_t lddq, void* workspace, int64_t workspace_bytes, void* stream) {
  if (!W || !Hinv || !qweight || !scale || !zero || out <= 0 || in_f <= 0) return IMQ_ERR_INVALID;
  const int64_t G = group_size;
  if (G <= 0 || G % 4 || blocksize <= 0 || blocksize > kGptqMaxBlock || blocksize % G) return IMQ_ERR_INVALID;
  const int64_t ng = (in_f + G - 1) / G, in_pad = ng * G;
  if (ldw < in_f || ldh < in_f || ldq < in_pad / 4 || ldsz < ng || (dq && lddq < in_f)) return IMQ_ERR_INVALID;
  if (out > 0x7fffffff || in_pad > 0x7fffffff) return IMQ_ERR_UNSUPPORTED;
  // the update kernel's grid.y is the 64-row tile count: refuse before anything is written
  if ((out + 63) / 64 > 65535) return IMQ_ERR_UNSUPPORTED;
  const int64_t need = imq_gptq_int2_workspace_bytes(out, blocksize);
  if (!workspace || workspace_bytes < need || ((uintptr_t)workspace & 15)) return IMQ_ERR_INVALID;
  GptqShrink sh;
  int rc = make_shrink(grid, maxshrink, &sh);
  if (rc != IMQ_OK) return rc;
  hipStream_t st = (hipStream_t)stream;
  float* err = (float*)workspace;
  for (int64_t i1 = 0; i1 < in_f; i1 += blocksize) {
    const int64_t i2 = i1 + blocksize < in_f ? i1 + blocksize : in_f;
    GptqBlockArgs b{W, ldw, (int)out, (int)in_f, (int)i1, (int)(i2 - i1), (int)G, (int)in_pad, Hinv, ldh,
                    qweight, ldq, scale, zero, ldsz, dq, lddq, err, sh};
    gptq_block_kernel<<<dim3((unsigned)((out + kGptqRows - 1) / kGptqRows)), dim3(kGptqRows), 0, st>>>(b);
    IMQ_LAUNCH_CHECK();
    if (i2 < in_f) {
      GptqUpdateArgs u{W, ldw, (int)out, (int)in_f, (int)i1, (int)(i2 - i1), (int)i2, Hinv, ldh, err};
      const int64_t gx = (in_f - i2 + 63) / 64, gy = (out + 63) / 64;
      gptq_update_kernel<<<dim3((unsigned)gx, (unsigned)gy), dim3(256), 0, st>>>(u);
      IMQ_LAUNCH_CHECK();
    }
  }
  return IMQ_OK;
}
