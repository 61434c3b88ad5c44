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
// imq_moe_experts_w4_ex: the same with the kernel layout's K_pad of each projection given
//                    explicitly (rows padded past in_features with zero codes and zero scales),
//                    optional per-expert row biases and a choice of activation: SiLU-GLU over
//                    [gate | up] halves, or gpt-oss's clamped GLU over interleaved gate / up rows
//                    (worker_quant.py:2280-2314: gate = y[::2] <= limit, up = y[1::2] in
//                    [-limit, limit], h = (up + 1) * gate * sigmoid(alpha * gate), biases added
//                    to both projections' outputs).
#include "imq_common.h"

namespace imq {
int moe_gemm_bm();
int moe_gemm_bn();
int moe_gemm_w4(int mode, const uint16_t* x, int64_t sxm, int64_t xrows, int64_t K, const uint8_t* q, int64_t sqe,
                int64_t sqn, const void* sc, const void* zr, int64_t sse, int64_t ssn, int sdt, int64_t N, int64_t I,
                const int32_t* mtl, const int32_t* nmt, int64_t max_mt, const int32_t* off, const int32_t* perm, int k,
                const void* bias, int64_t sbe, int bdt, float alpha, float limit, uint16_t* h, int64_t hs,
                float* yr, hipStream_t st, bool check_only = false);
int moe_rb(int mode, int ib, const uint16_t* x, int64_t sxm, int64_t xrows, int64_t K, int64_t xk, const uint8_t* q,
           int64_t sqe, int64_t sqn, const void* sc, const void* zr, int64_t sse, int64_t ssn, int sdt, int64_t N,
           int64_t I, const int32_t* mtl, const int32_t* nmt, int64_t max_mt, const int32_t* off,
           const int32_t* perm, int k, const void* bias, int64_t sbe, int bdt, float alpha, float limit,
           uint16_t* h, int64_t hs, float* yr, bool yr_bf16, const float* rs, int rs_stride, int rs_groups,
           float* hrs, int hrs_stride, hipStream_t st, bool check_only);
bool moe_rb_folded();
}  // namespace imq
using imq::moe_gemm_bm;
using imq::moe_gemm_bn;
using imq::moe_gemm_w4;
using imq::moe_rb;
using imq::moe_rb_folded;

namespace {

constexpr int64_t kAlign = 256;
int64_t align_up(int64_t v, int64_t a) { return (v + a - 1) / a * a; }

// The routed experts' ids as the caller holds them: int32, or int64 as torch's top-k returns
// them (the reference's MoE op reads those directly), so no conversion launch precedes a layer.
struct Ids {
  const void* p;
  int is64;
  IMQ_HOST_DEV int at(int64_t i) const {
    return is64 ? (int)((const int64_t*)p)[i] : ((const int32_t*)p)[i];
  }
};

// One wave per (row b, output channel n). Lane l handles 8-code words l, l+64, ...
// Output fp32 (OUT_F32) or bf16. x row for b is x + (b / xdiv) * sxm; its columns >= xk (a
// multiple of 8) are never read but taken as zero, as the reference's zero-padded activation
// (the read is clamped into the row, the value replaced by zeros).
template <int SDT, bool OUT_F32>
__global__ __launch_bounds__(256) void moe_rows_kernel(
    const uint16_t* __restrict__ x, int64_t sxm, int64_t xdiv, int64_t xk, int64_t B, int64_t Kpad,
    Ids eid, int64_t E, const uint8_t* __restrict__ q, int64_t sqe, int64_t sqn,
    const void* __restrict__ sc, int64_t sse, int64_t ssn, int64_t ssg, const void* __restrict__ zr,
    int64_t sze, int64_t szn, int64_t szg, int64_t N, int64_t G, void* __restrict__ y, int64_t sym) {
  const int lane = threadIdx.x & 63;
  const int64_t n = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int64_t b = blockIdx.y;
  if (n >= N || b >= B) return;
  int64_t e = eid.at(b);
  if (e < 0 || e >= E) e = 0;   // out-of-range ids are rejected on the host; keep loads in bounds
  const uint8_t* qr = q + e * sqe + n * sqn;
  const uint16_t* xr = x + (b / xdiv) * sxm;
  float acc = 0.f;
  const int64_t words = Kpad / 8;
  for (int64_t wd = lane; wd < words; wd += 64) {
    const uint32_t w = *(const uint32_t*)(qr + wd * 4);
    const bool xin = wd * 8 < xk;
    u32x4_t xv = *(const u32x4_t*)(xr + (xin ? wd * 8 : xk - 8));
    if (!xin) xv = u32x4_t{0u, 0u, 0u, 0u};
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

// Element i of a per-expert bias row in the bias dtype.
IMQ_DEV float load_bias(const void* p, int dt, int64_t i) {
  if (dt == IMQ_DT_FP32) return ((const float*)p)[i];
  if (dt == IMQ_DT_FP16) return f16_bits_to_f32(((const uint16_t*)p)[i]);
  return bf16_bits_to_f32(((const uint16_t*)p)[i]);
}

// gpt-oss's clamped GLU: gate <= limit, up in [-limit, limit] (comparisons, so NaN propagates as
// in torch's clamp), h = (up + 1) * gate * sigmoid(alpha * gate).
IMQ_DEV float gptoss_glu(float g, float u, float alpha, float limit) {
  g = g > limit ? limit : g;
  u = u > limit ? limit : (u < -limit ? -limit : u);
  return (u + 1.f) * (g / (1.f + __expf(-alpha * g)));
}

// h[b][i] (row stride hs) = bf16(act(gate, up)) for i < I, zero for I <= i < hk. ACT 0: gate =
// gu[b][i], up = gu[b][I + i]; ACT 1: gate = gu[b][2i], up = gu[b][2i + 1]. The row bias of the
// routed expert eid[b] (stride sbe, dtype bdt) is added to gu first when given.
template <int ACT>
__global__ __launch_bounds__(256) void swiglu_kernel(const float* __restrict__ gu, int64_t B, int64_t I, int64_t hk,
                                                     int64_t hs, Ids eid, int64_t E,
                                                     const void* __restrict__ bias, int64_t sbe, int bdt,
                                                     float alpha, float limit, uint16_t* __restrict__ h) {
  const int64_t total = B * hk;
  for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total;
       t += (int64_t)gridDim.x * blockDim.x) {
    const int64_t b = t / hk;
    const int64_t i = t - b * hk;
    float v = 0.f;
    if (i < I) {
      const int64_t ig = ACT == 0 ? i : 2 * i, iu = ACT == 0 ? I + i : 2 * i + 1;
      float g = gu[b * 2 * I + ig];
      float u = gu[b * 2 * I + iu];
      if (bias) {
        int64_t e = eid.at(b);
        e = (e >= 0 && e < E) ? e : 0;
        g += load_bias(bias, bdt, e * sbe + ig);
        u += load_bias(bias, bdt, e * sbe + iu);
      }
      if constexpr (ACT == 0) v = g / (1.f + __expf(-g)) * u;
      else v = gptoss_glu(g, u, alpha, limit);
    }
    h[b * hs + i] = (uint16_t)f32_to_bf16_bits(v);
  }
}

// out[t][n] = bf16(sum_j w[t][j] * (z[t*k + j][n] + bias[e(t, j)][n])), j in slot order (fixed).
__global__ __launch_bounds__(256) void combine_kernel(const float* __restrict__ z, const uint16_t* __restrict__ w,
                                                      int64_t T, int64_t k, int64_t H, Ids eid,
                                                      int64_t E, const void* __restrict__ bias, int64_t sbe, int bdt,
                                                      uint16_t* __restrict__ out, int64_t so) {
  const int64_t total = T * H;
  for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total;
       t += (int64_t)gridDim.x * blockDim.x) {
    const int64_t tok = t / H;
    const int64_t n = t - tok * H;
    float acc = 0.f;
    for (int64_t j = 0; j < k; ++j) {
      float v = z[(tok * k + j) * H + n];
      if (bias) {
        int64_t e = eid.at(tok * k + j);
        e = (e >= 0 && e < E) ? e : 0;
        v += load_bias(bias, bdt, e * sbe + n);
      }
      acc = fmaf(bf16_bits_to_f32(w[tok * k + j]), v, acc);
    }
    out[tok * so + n] = (uint16_t)f32_to_bf16_bits(acc);
  }
}


// ---------------------------------------------------------------------------------------------
// Token-sorted grouped path (G == 128, K of both projections a multiple of 256 and at most 4096,
// I % 32 == 0, H % 64 == 0, unit group strides):
//   moe_sort_kernel    counting sort of the T*k routed rows by expert -> off[E+1], perm[B] (sorted
//                      position -> routed row t*k + j) and the ascending list of hit experts
//                      hit[0 .. hit[E]) -- the work list of the grouped kernels
//   moe_line_kernel    workgroups over the (hit expert, row block) work list. A block's
//                      weights (NTL tiles of 16 rows) are loaded once into registers in the decode
//                      line kernel's full-line layout and reused for all of the expert's tokens, 16
//                      per MFMA pass. MODE 0 is gate_up: NTL/2 tiles of gate rows and the matching
//                      up rows, SwiGLU in the epilogue, bf16 h in sorted order. MODE 2 is gpt-oss's
//                      gate_up: NTL tiles of interleaved (gate, up) row pairs, its clamped GLU in
//                      the epilogue. MODE 1 is down: NTL tiles of H, fp32 rows written in routed
//                      order. Row biases, when given, are added to the sums in the epilogue.
//   moe_combine_kernel out[t] = bf16(sum_j w[t, j] * yr[t*k + j]), slot order.
constexpr int kMoeLine = 256;

// mtl (optional): the grouped GEMM's row blocks, mtl[0] = their number, then from mtl[2] one pair
// per block: (expert | rows of the block << 16, first sorted row), bm sorted rows per block -- at
// most ceil(B / bm) + (hit experts) blocks.
// Workgroups past the first (rs != nullptr): rs[t][g] = the fp32 sum of row t of x over columns
// [128 g, 128 g + 128), g < ng, columns at or past xk (even) read as zero -- one wave per (row,
// group), a fixed-order wave reduction; they run beside the sort in the same launch.
__global__ __launch_bounds__(1024) void moe_sort_kernel(Ids idx, int B, int E,
                                                        int32_t* __restrict__ off, int32_t* __restrict__ perm,
                                                        int32_t* __restrict__ hit, int32_t* __restrict__ mtl,
                                                        int bm, const uint16_t* __restrict__ x = nullptr,
                                                        int64_t sxm = 0, int64_t T = 0, int ng = 0,
                                                        float* __restrict__ rs = nullptr, int xk = 0) {
  extern __shared__ int32_t cnt[];     // [E]: counts, then scatter cursors
  const int tid = threadIdx.x, nt = blockDim.x;
  if (blockIdx.x > 0) {
    const int64_t wid = (int64_t)(blockIdx.x - 1) * (nt >> 6) + (tid >> 6);
    const int lane = tid & 63;
    if (rs == nullptr || wid >= T * ng) return;
    const int64_t t = wid / ng;
    const int g = (int)(wid - t * ng);
    const int col = 128 * g + 2 * lane;            // columns at or past xk count as zero
    const bool in = col < xk;
    uint32_t v = *(const uint32_t*)(x + t * sxm + (in ? col : xk - 2));
    v = in ? v : 0u;
    float sum = __uint_as_float(v << 16) + __uint_as_float(v & 0xffff0000u);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o, 64);
    if (lane == 0) rs[t * ng + g] = sum;
    return;
  }
  for (int e = tid; e < E; e += nt) cnt[e] = 0;
  __syncthreads();
  int ec[4];                           // the first 4 of this thread's ids stay in registers
  for (int b = tid, i = 0; b < B; b += nt, ++i) {
    int e = idx.at(b);
    e = (e >= 0 && e < E) ? e : 0;   // ids outside [0, E) are clamped, so every access stays in bounds
    if (i < 4) ec[i] = e;
    atomicAdd(&cnt[e], 1);
  }
  __syncthreads();
  if (tid < 64) {
    // wave 0: lane l owns experts [l*per, l*per + per); exclusive scans of the row counts and of
    // the hit flags give the sorted offsets and the ascending list of hit experts
    const int per = (E + 63) / 64;
    const int e0 = tid * per, e1 = (e0 + per < E) ? e0 + per : E;
    int rows = 0, hits = 0, blks = 0;
    for (int e = e0; e < e1; ++e) {
      rows += cnt[e];
      hits += cnt[e] > 0;
      blks += (cnt[e] + bm - 1) / bm;
    }
    int rs = rows, hs = hits, bs = blks;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int r = __shfl_up(rs, d, 64), h = __shfl_up(hs, d, 64), b = __shfl_up(bs, d, 64);
      if (tid >= d) {
        rs += r;
        hs += h;
        bs += b;
      }
    }
    int run = rs - rows, hrun = hs - hits, brun = bs - blks;
    for (int e = e0; e < e1; ++e) {
      const int c = cnt[e];
      off[e] = run;
      if (c > 0) hit[hrun++] = e;
      if (mtl != nullptr)
        for (int r0 = 0; r0 < c; r0 += bm, ++brun) {
          mtl[2 + 2 * brun] = e | ((c - r0 < bm ? c - r0 : bm) << 16);   // E <= 16384, bm <= 128
          mtl[3 + 2 * brun] = run + r0;
        }
      cnt[e] = run;
      run += c;
    }
    if (tid == 63) {
      off[E] = rs;
      hit[E] = hs;                        // number of hit experts
      if (mtl != nullptr) mtl[0] = bs;
    }
  }
  __syncthreads();
  for (int b = tid, i = 0; b < B; b += nt, ++i) {
    int e = i < 4 ? ec[i] : idx.at(b);
    e = (e >= 0 && e < E) ? e : 0;
    perm[atomicAdd(&cnt[e], 1)] = b;
  }
}

struct MoeLineArgs {
  const uint16_t* x;     // MODE 0 / 2: hidden [T, >= Kpad]; MODE 1: h [B, >= Kpad] in sorted order
  int64_t sxm;
  int Kpad;
  int k;                 // top_k: MODE 0 / 2 read hidden row perm[p] / k
  const int32_t* off;
  const int32_t* perm;
  const int32_t* hit;    // [E + 1]: ascending hit experts, hit[E] = their number
  const uint8_t* q;
  int64_t sqe, sqn;
  const void* sc;
  const void* zr;
  int64_t sse, ssn;      // scale and zero share strides (expert, row); groups are unit-strided
  int E;
  int NB;                // row blocks (NTL * 16 rows) per expert
  int I;                 // MODE 0: intermediate size (up rows start at I)
  void* out;             // MODE 0 / 2: h bf16 [B, >= I] sorted order; MODE 1: fp32 [B, H] routed order
  int64_t som;
  const void* bias;      // per-expert row bias [E][rows] (expert stride sbe, dtype bdt), or null
  int64_t sbe;
  int bdt;
  float alpha, limit;    // MODE 2 activation
  int xk;                // valid x columns (a multiple of 8): columns past them read as zero
  // direct decode form (no sort): an item is (routed row b, row block), expert idx[b], one row
  Ids idx;
  int nrows;             // routed rows B
  int direct;
};

IMQ_DEV float moe_row_swap8(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x128, 0xf, 0xf, false));
}

// Raw buffer resources and loads of the token-sorted line kernel (offsets below 2^31, checked
// by the launcher); nt: the weight stream's non-temporal hint.
IMQ_DEV __amdgpu_buffer_rsrc_t moe_rsrc(const void* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, 0x7fffffff, 0x00020000);
}
IMQ_DEV u32x4_t moe_bload(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, 0));
}
IMQ_DEV u32x4_t moe_bload_nt(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, 2));
}

// XCL: activation rows shorter than K (a.xk < a.Kpad), columns past xk read as zero. xk is a
// multiple of 32 (H % 64 == 0 and I % 32 == 0 on this path): a lane's 32 columns of one
// (line-step, half) lie all below xk or all past it, and past it the lane reads its row's first
// 32 columns and zeroes them -- one address per 32 columns, the rest immediate offsets.
template <int S2, int NTL, int SDT, int MODE, int XCL>
__global__ __launch_bounds__(512) void moe_line_kernel(MoeLineArgs a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  constexpr int VB = (SDT == IMQ_DT_FP32) ? 4 : 2;
  constexpr int DPR = S2 * VB / 2;                   // scale dwords per row per wave
  constexpr int HALF = NTL / 2;                      // MODE 0: gate tiles (= up tiles) per block
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int W = blockDim.x >> 6;
  const int c = lane & 15, ar = lane >> 4;
  const bool lo8 = c < 8;
  const int KL = a.Kpad / kMoeLine;
  const int ls0 = wave * S2;
  // The sort's outputs are read through the scalar cache: the item's expert, its row range and
  // the routed rows of its first pass are uniform over the workgroup, and scalar loads count on
  // lgkmcnt, so no wait for them queues behind the weight stream on the in-order vmcnt.
  using cint32 = const __attribute__((address_space(4))) int32_t;
  cint32* const chit = (cint32*)a.hit;
  cint32* const coff = (cint32*)a.off;
  cint32* const cperm = (cint32*)a.perm;
  // (hit expert, row block) work items, or (routed row, row block) in the direct form
  const int items = a.direct ? a.nrows * a.NB : chit[a.E] * a.NB;

  uint32_t* szl = (uint32_t*)smem + wave * (2 * NTL * 16 * DPR);
  float* red = (float*)(smem + (size_t)W * (2 * NTL * 16 * DPR) * 4);   // [W][NTL][16][16]
  float* bst = red + W * NTL * 256;                                     // [NTL * 16] row biases
  int* prow = (int*)(bst + NTL * 16);                                   // [16] first pass's routed rows
  for (int item = blockIdx.x; item < items; item += gridDim.x) {
  const int ib = item / a.NB;
  const int blk = item - ib * a.NB;
  int e, beg, end;
  if (a.direct) {
    beg = ib;
    end = beg + 1;
    e = a.idx.at(beg);
    e = (e >= 0 && e < a.E) ? e : 0;   // ids outside [0, E) are clamped, as in the sort
  } else {
    e = chit[ib];
    beg = coff[e];
    end = coff[e + 1];
  }
  auto perm_at = [&](int p) -> int { return a.direct ? p : a.perm[p]; };

  auto rbase = [&](int t) -> int {
    if constexpr (MODE == 0) return (t < HALF) ? 16 * HALF * blk + 16 * t : a.I + 16 * HALF * blk + 16 * (t - HALF);
    else return 16 * NTL * blk + 16 * t;
  };
  // ---- the item's row biases (one per row of the block), issued first: the epilogue reads them
  // from LDS instead of waiting on a load after the reduction ----
  // (unconditional: a load under a branch ends in a full wait where the paths join; without a
  // bias the weights' first word is read and ignored. The aligned dword holding a 2-byte element
  // lies in the element's page.)
  const bool has_bias = a.bias != nullptr;
  uint32_t bw;        // the raw dword; converted where it is stored, after the activation loads
  bool bhi;
  {
    const int br = rbase((threadIdx.x >> 4) & (NTL - 1)) + (threadIdx.x & 15);
    const int bsz = a.bdt == IMQ_DT_FP32 ? 4 : 2;
    const char* bb = has_bias ? (const char*)a.bias : (const char*)a.q;
    const int64_t boff = has_bias ? ((int64_t)e * a.sbe + br) * bsz : 0;
    const int mis = (int)(((uintptr_t)bb + (uintptr_t)boff) & 3);   // 0, or 2 for the upper half
    bw = *(const uint32_t*)(bb + boff - mis);
    bhi = mis != 0;
  }
  // ---- scale / zero words of this wave's groups for the 4 tiles -> wave LDS ----
  constexpr int ZN = 2 * NTL * 16 * DPR;
  constexpr int ZU = (ZN + 63) / 64;
  const int ngd = a.Kpad / 128 * VB / 4;
  const unsigned char* sbase = (const unsigned char*)a.sc + (int64_t)e * a.sse * VB;
  const unsigned char* zbase = (const unsigned char*)a.zr + (int64_t)e * a.sse * VB;
  uint32_t zv[ZU];
#pragma unroll
  for (int u = 0; u < ZU; ++u) {
    int d = lane + 64 * u;
    d = d < ZN ? d : ZN - 1;
    const int arr = d / (NTL * 16 * DPR);
    const int rem = d - arr * (NTL * 16 * DPR);
    const int t = rem / (16 * DPR);
    const int rem2 = rem - t * (16 * DPR);
    const int r = rem2 / DPR, dw = rem2 - r * DPR;
    int gd = ls0 * (VB / 2) + dw;
    gd = gd < ngd ? gd : ngd - 1;
    const int64_t ro = (int64_t)(rbase(t) + r) * a.ssn * VB + 4 * gd;
    zv[u] = *(const uint32_t*)((arr ? zbase : sbase) + ro);
  }
  // ---- weights: per tile and line-step one full-line load for rows 0-7 and one for rows 8-15 ----
  // buffer loads from the expert's first row: a lane's offsets (row c & 7 or 8 + (c & 7), its 16
  // bytes of the line) are fixed, the tile's rows and the line-step are scalar offsets
  const __amdgpu_buffer_rsrc_t qrs = moe_rsrc(a.q + (int64_t)e * a.sqe);
  const uint32_t qv0 = (uint32_t)((c & 7) * (int)a.sqn + 16 * ar + (lo8 ? 0 : 64));
  const uint32_t qv1 = (uint32_t)((8 + (c & 7)) * (int)a.sqn + 16 * ar + (lo8 ? 64 : 0));
  u32x4_t wb[NTL][2 * S2];
#pragma unroll
  for (int t = 0; t < NTL; ++t) {
#pragma unroll
    for (int i = 0; i < S2; ++i) {
      int l = ls0 + i;
      l = l < KL ? l : KL - 1;
      const uint32_t so = (uint32_t)(rbase(t) * (int)a.sqn + 128 * l);
      wb[t][2 * i] = moe_bload_nt(qrs, qv0, so);
      wb[t][2 * i + 1] = moe_bload_nt(qrs, qv1, so);
    }
  }
  // ---- activations of the first pass, issued behind the weights so both arrive in one wait ----
  // Routed rows of the first pass, sorted positions beg .. beg + 15, with one scalar load (perm's
  // workspace slot holds spare entries past its B); lane i < 16 of sp holds row i and a lane
  // picks its row with a cross-lane read. Placed after the weight loads, so that its wait (and
  // that for beg) does not hold them back.
  int sp = beg + (lane & 15);
  if (!a.direct) {
    typedef int32_t v16i __attribute__((ext_vector_type(16), aligned(4)));
    const v16i pv = *(const __attribute__((address_space(4))) v16i*)(cperm + beg);   // one s_load_dwordx16
#pragma unroll
    for (int i = 0; i < 16; ++i) asm("v_writelane_b32 %0, %1, %2" : "+v"(sp) : "s"(pv[i]), "n"(i));
  }
  auto pick16 = [&](int i) -> int { return __shfl(sp, i, 64); };
  // the lane's activation row as a byte offset into x (the launcher keeps x below 2^31 bytes)
  const __amdgpu_buffer_rsrc_t xrs = moe_rsrc(a.x);
  auto xrow_of = [&](int p0, bool first) -> uint32_t {
    const int nrow = (end - p0) < 16 ? end - p0 : 16;
    const int cc = c < nrow ? c : nrow - 1;           // A row of this lane (rows >= nrow repeat the last)
    if constexpr (MODE != 1) {
      const int rid = first ? pick16(cc) : perm_at(p0 + cc);
      return (uint32_t)((rid / a.k) * (int)a.sxm * 2);   // gate_up: gather hidden rows
    } else {
      return (uint32_t)((p0 + cc) * (int)a.sxm * 2);
    }
  };
  auto xcol = [&](int i, int h, int kk) -> int {
    int l = ls0 + i;
    l = l < KL ? l : KL - 1;
    return kMoeLine * l + 128 * h + 32 * ar + 8 * kk;
  };
  u32x4_t X[S2][2][4];
  // zo: 0, opaque to the compiler, so that the column offsets are computed where the loads are
  // issued (per item, per pass) rather than hoisted out of the loops and held in registers
  auto load_x = [&](uint32_t xo, int zo) {
#pragma unroll
    for (int i = 0; i < S2; ++i)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        int cb = xcol(i, h, 0) + zo;                   // the lane's 32 columns [cb, cb + 32)
        if constexpr (XCL != 0) cb = xcol(i, h, 0) < a.xk ? cb : zo;
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) X[i][h][kk] = moe_bload(xrs, xo + 2 * (uint32_t)(cb + 8 * kk), 0);
      }
  };
  {
    int zo = 0;
    asm volatile("" : "+v"(zo));
    load_x(xrow_of(beg, true), zo);
  }
#pragma unroll
  for (int u = 0; u < ZU; ++u) {
    const int d = lane + 64 * u;
    if (d < ZN) szl[d] = zv[u];
  }
  if (threadIdx.x < 16) prow[threadIdx.x] = sp;        // for the epilogue (read after its barrier)
  if (has_bias && threadIdx.x < 16 * NTL) {
    const uint32_t hb = bhi ? (bw >> 16) : (bw & 0xffffu);
    bst[threadIdx.x] = a.bdt == IMQ_DT_FP32 ? __uint_as_float(bw) : a.bdt == IMQ_DT_FP16 ? f16_bits_to_f32(hb) : bf16_bits_to_f32(hb);
  }
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   // wave-private LDS, in-order

  auto val = [&](int t, int arr, int row, int g) -> float {   // group g of row `row` of tile t
    const uint32_t* p = szl + ((arr * NTL + t) * 16 + row) * DPR;
    if constexpr (VB == 4) return round_bf16_hw(__uint_as_float(p[g]));
    else return raw_to_bf16_f32<SDT>((g & 1) ? (p[g >> 1] >> 16) : (p[g >> 1] & 0xffffu));
  };
  // scale and -(128 + z) * scale of tile t, line-step i: read from the staged words at use (held
  // in registers for all tiles they would crowd out the activation loads)
  auto szpair = [&](int t, int i, float& s0, float& s1, float& cz0, float& cz1) {
    const bool v = ls0 + i < KL;
    const float r0 = val(t, 0, c, 2 * i), r1 = val(t, 0, c ^ 8, 2 * i + 1);   // read, then select
    s0 = v ? r0 : 0.f;
    s1 = v ? r1 : 0.f;
    cz0 = -(128.f + val(t, 1, c, 2 * i)) * s0;
    cz1 = -(128.f + val(t, 1, c ^ 8, 2 * i + 1)) * s1;
  };

  const uint32_t magic = magic_bf16_128x2();
  const bf16x8_t ones = __builtin_bit_cast(bf16x8_t, u32x4_t{0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u});
  for (int p0 = beg; p0 < end; p0 += 16) {
    if constexpr (S2 > 1) {
      // keep the unpack inside the token loop: hoisting the unpacked operands of all tiles out of
      // it would exceed the register budget beyond one line-step per wave
#pragma unroll
      for (int t = 0; t < NTL; ++t)
#pragma unroll
        for (int i = 0; i < 2 * S2; ++i) asm volatile("" : "+v"(wb[t][i]));
    }
    const int nrow = (end - p0) < 16 ? end - p0 : 16;
    if (p0 != beg) {
      int zo = 0;
      asm volatile("" : "+v"(zo));
      load_x(xrow_of(p0, false), zo);
    }
    f32x4_t y0[NTL], y1[NTL];
#pragma unroll
    for (int t = 0; t < NTL; ++t) {
      y0[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      y1[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int i = 0; i < S2; ++i) {
      bf16x8_t A[2][4];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
          u32x4_t v = X[i][h][kk];
          if constexpr (XCL != 0) {
            if (!(xcol(i, h, 0) < a.xk)) v = u32x4_t{0u, 0u, 0u, 0u};
          }
          A[h][kk] = __builtin_bit_cast(bf16x8_t, permute_x8(v));
        }
      }
      // group row sums straight into the D layout (row m = 4*ar + r of every lane): MFMAs against
      // a B of ones, in place of per-lane sums and cross-lane shuffles
      f32x4_t xs0 = {0.f, 0.f, 0.f, 0.f}, xs1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        xs0 = mfma16x16x32(A[0][kk], ones, xs0);
        xs1 = mfma16x16x32(A[1][kk], ones, xs1);
      }
#pragma unroll
      for (int t = 0; t < NTL; ++t) {
        const u32x4_t w0 = wb[t][2 * i], w1 = wb[t][2 * i + 1];
        u32x4_t gA, gB;
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          gA[d] = lo8 ? w0[d] : w1[d];
          gB[d] = lo8 ? w1[d] : w0[d];
        }
        f32x4_t acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
          acc0 = mfma16x16x32(A[0][kk], unpack_nib8_bf16(gA[kk], magic), acc0);
          acc1 = mfma16x16x32(A[1][kk], unpack_nib8_bf16(gB[kk], magic), acc1);
        }
        float s0, s1, cz0, cz1;
        szpair(t, i, s0, s1, cz0, cz1);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          y0[t][r] = fmaf(cz0, xs0[r], y0[t][r]);
          y1[t][r] = fmaf(cz1, xs1[r], y1[t][r]);
          y0[t][r] = fmaf(s0, acc0[r], y0[t][r]);
          y1[t][r] = fmaf(s1, acc1[r], y1[t][r]);
        }
      }
    }
    // wave partials -> LDS [wave][tile][m][n]; the B-group columns hold row c ^ 8
#pragma unroll
    for (int t = 0; t < NTL; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        red[((wave * NTL + t) * 16 + 4 * ar + r) * 16 + c] = y0[t][r] + moe_row_swap8(y1[t][r]);
    lds_barrier();
    for (int o = threadIdx.x; o < 16 * 16 * NTL; o += blockDim.x) {
      const int m = o / (16 * NTL), j = o - m * (16 * NTL);
      if (m < nrow) {
        if constexpr (MODE == 0) {
          if (j < 16 * HALF) {
            const int t = j >> 4, n = j & 15;
            float g = 0.f, u = 0.f;
            for (int w = 0; w < W; ++w) {
              g += red[((w * NTL + t) * 16 + m) * 16 + n];
              u += red[((w * NTL + t + HALF) * 16 + m) * 16 + n];
            }
            if (has_bias) {
              g += bst[j];
              u += bst[16 * HALF + j];
            }
            const float hv = g / (1.f + __expf(-g)) * u;
            ((uint16_t*)a.out)[(int64_t)(p0 + m) * a.som + 16 * HALF * blk + j] = (uint16_t)f32_to_bf16_bits(hv);
          }
        } else if constexpr (MODE == 2) {
          if (j < 8 * NTL) {                     // h column 8*NTL*blk + j from rows 2j (gate), 2j + 1 (up)
            const int rg = 2 * j, ru = 2 * j + 1;
            float g = 0.f, u = 0.f;
            for (int w = 0; w < W; ++w) {
              g += red[((w * NTL + (rg >> 4)) * 16 + m) * 16 + (rg & 15)];
              u += red[((w * NTL + (ru >> 4)) * 16 + m) * 16 + (ru & 15)];
            }
            if (has_bias) {
              g += bst[rg];
              u += bst[ru];
            }
            const float hv = gptoss_glu(g, u, a.alpha, a.limit);
            ((uint16_t*)a.out)[(int64_t)(p0 + m) * a.som + 8 * NTL * blk + j] = (uint16_t)f32_to_bf16_bits(hv);
          }
        } else {
          const int t = j >> 4, n = j & 15;
          float v = 0.f;
          for (int w = 0; w < W; ++w) v += red[((w * NTL + t) * 16 + m) * 16 + n];
          if (has_bias) v += bst[j];
          const int orow = p0 == beg ? prow[m] : perm_at(p0 + m);
          ((float*)a.out)[(int64_t)orow * a.som + 16 * NTL * blk + j] = v;
        }
      }
    }
    lds_barrier();                                     // red is rewritten by the next pass
  }
  }
}

// out[t][n .. n+7] = bf16(sum_j w[t][j] * yr[t*k + j][n .. n+7]) for bf16 rows yr (the register-B
// grouped down's output), slot order, fp32 sums; H % 8 == 0. 16-byte loads, 8 slots in flight.
__global__ __launch_bounds__(256) void moe_combine_bf16_kernel(const uint16_t* __restrict__ yr,
                                                               const uint16_t* __restrict__ w, int64_t T, int64_t k,
                                                               int64_t H, uint16_t* __restrict__ out, int64_t so) {
  const int64_t H8 = H / 8;
  const int64_t total = T * H8;
  for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total;
       t += (int64_t)gridDim.x * blockDim.x) {
    const int64_t tok = t / H8;
    const int64_t n = 8 * (t - tok * H8);
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int64_t j0 = 0; j0 < k; j0 += 8) {
      u32x4_t v[8];
      float wj[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int64_t jj = j0 + j < k ? j0 + j : k - 1;
        v[j] = *(const u32x4_t*)(yr + (tok * k + jj) * H + n);
        wj[j] = bf16_bits_to_f32(w[tok * k + jj]);
      }
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (j0 + j < k)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            acc[2 * q] = fmaf(wj[j], __uint_as_float(v[j][q] << 16), acc[2 * q]);
            acc[2 * q + 1] = fmaf(wj[j], __uint_as_float(v[j][q] & 0xffff0000u), acc[2 * q + 1]);
          }
    }
    u32x4_t o;
#pragma unroll
    for (int q = 0; q < 4; ++q) o[q] = cvt_pk_bf16(acc[2 * q], acc[2 * q + 1]);
    *(u32x4_t*)(out + tok * so + n) = o;
  }
}

// out[t][n .. n+3] = bf16(sum_j w[t][j] * yr[t*k + j][n .. n+3]), slot order, fp32 sums; H % 4 == 0.
__global__ __launch_bounds__(256) void moe_combine_kernel(const float* __restrict__ yr, const uint16_t* __restrict__ w,
                                                          int64_t T, int64_t k, int64_t H,
                                                          uint16_t* __restrict__ out, int64_t so) {
  // 4 columns per thread; the slots' loads go out 8 at a time before their sums (slot order kept)
  const int64_t H4 = H / 4;
  const int64_t total = T * H4;
  for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total;
       t += (int64_t)gridDim.x * blockDim.x) {
    const int64_t tok = t / H4;
    const int64_t n = 4 * (t - tok * H4);
    f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
    for (int64_t j0 = 0; j0 < k; j0 += 8) {
      f32x4_t v[8];
      float wj[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int64_t jj = j0 + j < k ? j0 + j : k - 1;
        v[j] = *(const f32x4_t*)(yr + (tok * k + jj) * H + n);
        wj[j] = bf16_bits_to_f32(w[tok * k + jj]);
      }
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (j0 + j < k)
#pragma unroll
          for (int q = 0; q < 4; ++q) acc[q] = fmaf(wj[j], v[j][q], acc[q]);
    }
    u32x2_t o;
    o[0] = cvt_pk_bf16(acc[0], acc[1]);
    o[1] = cvt_pk_bf16(acc[2], acc[3]);
    *(u32x2_t*)(out + tok * so + n) = o;
  }
}

// zero h's pad columns [I, hk) of rows with stride hs (down reads K = hk)
__global__ __launch_bounds__(256) void moe_zero_pad_kernel(uint16_t* __restrict__ h, int64_t B, int64_t I,
                                                           int64_t hk, int64_t hs) {
  const int64_t wpad = hk - I;
  const int64_t total = B * wpad;
  for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total;
       t += (int64_t)gridDim.x * blockDim.x) {
    const int64_t b = t / wpad;
    h[b * hs + I + (t - b * wpad)] = 0;
  }
}


// ---------------------------------------------------------------------------------------------
// Decode form on the dense line kernel's structure (routed rows B with 4 B <= E, about one row
// per hit expert): two launches, no sort and no combine launch.
//   moe_gu_line_kernel  workgroup (routed row b, unit u) streams 16-row tiles of expert idx[b]'s
//                       gate_up rows against hidden[b / k]: waves split K in S2 line-steps of
//                       256 codes with every load issued up front (two full-line loads per
//                       line-step, MFMA 16x16x32 with the +128 bias fold). ACT 0 pairs gate tile
//                       u with up tile u + I/16 (two wave groups) and writes 16 h columns; ACT 1
//                       (gpt-oss) takes 16 interleaved rows and writes 8. Row biases and the
//                       activation run in the epilogue.
//   moe_dn_line_kernel  workgroup (token t, 16 output rows) with one wave group per routed slot
//                       j streaming expert idx[t k + j]'s down rows against h[t k + j]; or
//                       (PAIR, when 16-row tiles would leave CUs idle) workgroup (t, 8 output
//                       rows) with one wave group per slot pair (2p, 2p + 1): one 16-row MFMA
//                       tile holds the 8 rows of both slots' experts, A rows 0 and 1 their h
//                       rows. Each partial is scaled by w[t, j] (the down bias added once per
//                       slot), and the fixed-order cross-wave LDS reduction is the weighted
//                       combine: out[t] = bf16(sum_j w[t, j] (down_j + b_j)).
// ---------------------------------------------------------------------------------------------
constexpr int kDLine = 256;   // int4 codes per line-step (128 bytes of a row, 2 groups of 128)

struct MoeDecArgs {
  const uint16_t* x;       // gu: hidden (row b / k); dn: h (row b)
  int64_t sxm;
  int xk;                  // valid x columns (a multiple of 8): columns past them read as zero
  int Kpad;                // kernel K (a multiple of 256)
  int k;                   // top_k
  Ids idx;                 // [B] expert of each routed row
  const uint16_t* topk_w;  // [B] routing weights, bf16 (dn)
  int E;
  const uint8_t* q;
  int64_t sqe, sqn;
  const void* sc;
  const void* zr;
  int64_t sse, ssn;        // scale and zero share strides (expert, row); unit group stride
  int I;                   // gu: intermediate size
  int NR;                  // gu: units per routed row; dn: row tiles per token (set by dec_dn)
  int Wk;                  // waves per tile (gu) or per routed slot (dn)
  const void* bias;        // per-expert row bias [E][rows] or null
  int64_t sbe;
  int bdt;
  float alpha, limit;      // gpt-oss activation
  uint16_t* out;           // gu: h [B][som]; dn: out [T][som]
  int64_t som;
};

// LDS of one wave: staged activation row(s) (two in the paired form), their group sums, the
// scale / zero words of the 16 weight rows.
IMQ_HOST_DEV inline int dec_wave_lds(int S2, int vb, bool pair) {
  const int nx = pair ? 2 : 1;
  return nx * (S2 * kDLine + 8) * 2 + nx * 2 * S2 * 4 + 2 * 16 * (S2 * vb / 2) * 4;
}

// One wave's share of a 16-row tile (line-steps [ls0, ls0 + S2)): returns the wave's partial dot
// for column c in lanes with ar == 0.
//   PAIR false: rows rbase.. rbase+15 of expert e against the activation row xrow (the MFMA's A
//               rows all hold it; D row 0 is used).
//   PAIR true:  rows rbase.. rbase+7 of expert e (columns 0-7) against xrow and the same rows of
//               expert e2 (columns 8-15) against xrow2: A row 1 holds xrow2, so D row 0 gives
//               columns 0-7 and D row 1 columns 8-15 -- two routed slots share one 16-row MFMA.
template <int S2, int SDT, bool XCL, bool PAIR>
IMQ_DEV float dec_tile_partial(const MoeDecArgs& a, int e, int rbase, const uint16_t* xrow, int ls0, int KL,
                               unsigned char* wl, int lane, int e2, const uint16_t* xrow2) {
  constexpr int VB = (SDT == IMQ_DT_FP32) ? 4 : 2;
  constexpr int DPR = S2 * VB / 2;                   // scale dwords per row per array
  const int c = lane & 15, ar = lane >> 4;
  const bool lo8 = c < 8;
  constexpr int NX = PAIR ? 2 : 1;
  const int xrowl = S2 * kDLine + 8;
  uint16_t* xw = (uint16_t*)wl;                      // [NX][xrowl], unpack order
  float* xs = (float*)(wl + NX * xrowl * 2);         // [NX][2 * S2] group sums
  uint32_t* szl = (uint32_t*)(xs + NX * 2 * S2);     // [2 arrays][16 rows][DPR]

  // 1) x: 32*S2 blocks of 8 of this wave's K range (of each activation row)
  constexpr int XB = 32 * S2;
  constexpr int XU = XB / 64;
  u32x4_t xv[NX][XU];
#pragma unroll
  for (int h = 0; h < NX; ++h)
#pragma unroll
    for (int u = 0; u < XU; ++u) {
      const uint16_t* xr = h ? xrow2 : xrow;
      const int bidx = lane + 64 * u;
      const int col = ls0 * kDLine + 8 * bidx;
      if constexpr (XCL) {
        const bool in = col < a.xk;
        xv[h][u] = *(const u32x4_t*)(xr + (in ? col : a.xk - 8));
        if (!in) xv[h][u] = u32x4_t{0u, 0u, 0u, 0u};
      } else {
        xv[h][u] = *(const u32x4_t*)(xr + (col < a.Kpad ? col : a.Kpad - 8));
      }
    }
  // 2) scale / zero words of groups [2*ls0, 2*ls0 + 2*S2) of the 16 rows
  constexpr int ZU = (32 * DPR + 63) / 64;
  const int ngd = a.Kpad / 128 * VB / 4;
  uint32_t zv[ZU];
#pragma unroll
  for (int u = 0; u < ZU; ++u) {
    int d = lane + 64 * u;
    d = d < 32 * DPR ? d : 32 * DPR - 1;
    const int arr = d / (16 * DPR);
    const int rem = d - arr * (16 * DPR);
    const int r = rem / DPR;
    const int dw = rem - r * DPR;
    int gd = ls0 * (VB / 2) + dw;
    gd = gd < ngd ? gd : ngd - 1;
    const bool second = PAIR && r >= 8;             // rows 8-15: expert e2's rows rbase..
    const int64_t el = (int64_t)(second ? e2 : e) * a.sse + (int64_t)(rbase + (second ? r - 8 : r)) * a.ssn;
    zv[u] = *(const uint32_t*)((const unsigned char*)(arr ? a.zr : a.sc) + el * VB + 4 * gd);
  }
  // 3) weights: per line-step one full-line load for rows 0-7 and one for rows 8-15
  const uint8_t* qt = a.q + (int64_t)e * a.sqe + (int64_t)rbase * a.sqn;
  const uint8_t* qt2 = PAIR ? a.q + (int64_t)e2 * a.sqe + (int64_t)rbase * a.sqn : qt + 8 * a.sqn;
  const uint8_t* q0 = qt + (int64_t)(c & 7) * a.sqn + 16 * ar + (lo8 ? 0 : 64);
  const uint8_t* q1 = qt2 + (int64_t)(c & 7) * a.sqn + 16 * ar + (lo8 ? 64 : 0);
  u32x4_t wb[2 * S2];
#pragma unroll
  for (int i = 0; i < S2; ++i) {
    int l = ls0 + i;
    l = l < KL ? l : KL - 1;
    wb[2 * i] = __builtin_nontemporal_load((const u32x4_t*)(q0 + 128 * l));
    wb[2 * i + 1] = __builtin_nontemporal_load((const u32x4_t*)(q1 + 128 * l));
  }
  // 4) stage x (unpack order) with its per-group sums, and the scale / zero words
#pragma unroll
  for (int h = 0; h < NX; ++h)
#pragma unroll
    for (int u = 0; u < XU; ++u) {
      const int bidx = lane + 64 * u;
      const float sum = row_sum16(bf16x8_sum(xv[h][u]));
      *(u32x4_t*)(xw + h * xrowl + 8 * bidx) = permute_x8(xv[h][u]);
      if ((bidx & 15) == 0) xs[h * 2 * S2 + (bidx >> 4)] = sum;
    }
#pragma unroll
  for (int u = 0; u < ZU; ++u) {
    const int d = lane + 64 * u;
    if (d < 32 * DPR) szl[d] = zv[u];
  }
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   // wave-private LDS, in-order

  const uint32_t magic = magic_bf16_128x2();
  // A row 1: PAIR the second activation row; else the line-step's second group (128 codes on), so
  // each full-line load feeds its MFMAs as loaded (the line kernel's M = 1 form)
  const uint16_t* xa = xw + ((PAIR && c == 1) ? xrowl : 0) + ((!PAIR && c == 1) ? 128 : 0) + 32 * ar;
  // group sums of the activation each lane's column meets: y0 columns 0-7 / 8-15 are expert e / e2,
  // y1 (read across the row swap) the other way round
  const float* xs0p = xs + ((PAIR && !lo8) ? 2 * S2 : 0);
  const float* xs1p = xs + ((PAIR && lo8) ? 2 * S2 : 0);
  const uint32_t* sc_c = szl + c * DPR;
  const uint32_t* sc_x = szl + (c ^ 8) * DPR;
  const uint32_t* zr_c = szl + 16 * DPR + c * DPR;
  const uint32_t* zr_x = szl + 16 * DPR + (c ^ 8) * DPR;
  auto val = [&](const uint32_t* p, int g) -> float {
    if constexpr (VB == 4) return round_bf16_hw(__uint_as_float(p[g]));
    else return raw_to_bf16_f32<SDT>((g & 1) ? (p[g >> 1] >> 16) : (p[g >> 1] & 0xffffu));
  };
  float y0 = 0.f, y1 = 0.f;
#pragma unroll
  for (int i = 0; i < S2; ++i) {
    const bool v = ls0 + i < KL;
    const float xs0 = xs0p[2 * i], xs1 = xs1p[2 * i + 1];
    float s0 = val(sc_c, 2 * i), s1 = val(sc_x, 2 * i + 1);   // read, then select
    s0 = v ? s0 : 0.f;
    s1 = v ? s1 : 0.f;
    const float cz0 = -(128.f + val(zr_c, 2 * i)) * s0;
    const float cz1 = -(128.f + val(zr_x, 2 * i + 1)) * s1;
    const u32x4_t w0 = wb[2 * i], w1 = wb[2 * i + 1];
    if constexpr (!PAIR) {
      // column c < 8 of load L0 is row c's group 2l (D row 0), c >= 8 row c ^ 8's group 2l+1 (D
      // row 1); load L1 the other way round
      bf16x8_t A[4];
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) A[kk] = *(const bf16x8_t*)(xa + i * kDLine + 8 * kk);
      f32x4_t a0 = {0.f, 0.f, 0.f, 0.f}, a1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        a0 = mfma16x16x32(A[kk], unpack_nib8_bf16(w0[kk], magic), a0);
        a1 = mfma16x16x32(A[kk], unpack_nib8_bf16(w1[kk], magic), a1);
      }
      y0 = fmaf(cz0, xs0, y0);
      y1 = fmaf(cz1, xs1, y1);
      y0 = fmaf(s0, lo8 ? a0[0] : a1[0], y0);   // row c, group 2l
      y1 = fmaf(s1, lo8 ? a1[1] : a0[1], y1);   // row c ^ 8, group 2l+1
      continue;
    }
    bf16x8_t A0[4], A1[4];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      A0[kk] = *(const bf16x8_t*)(xa + i * kDLine + 8 * kk);
      A1[kk] = *(const bf16x8_t*)(xa + i * kDLine + 128 + 8 * kk);
    }
    u32x4_t gA, gB;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      gA[d] = lo8 ? w0[d] : w1[d];
      gB[d] = lo8 ? w1[d] : w0[d];
    }
    f32x4_t acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      acc0 = mfma16x16x32(A0[kk], unpack_nib8_bf16(gA[kk], magic), acc0);
      acc1 = mfma16x16x32(A1[kk], unpack_nib8_bf16(gB[kk], magic), acc1);
    }
    y0 = fmaf(cz0, xs0, y0);
    y1 = fmaf(cz1, xs1, y1);
    // D row 0 (xrow) in lanes ar == 0; PAIR: row 1 (xrow2) for expert e2's columns
    y0 = fmaf(s0, (PAIR && !lo8) ? acc0[1] : acc0[0], y0);
    y1 = fmaf(s1, (PAIR && lo8) ? acc1[1] : acc1[0], y1);
  }
  return y0 + moe_row_swap8(y1);
}

template <int S2, int SDT, int ACT, bool XCL>
__global__ __launch_bounds__(1024) void moe_gu_line_kernel(MoeDecArgs a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  constexpr int VB = (SDT == IMQ_DT_FP32) ? 4 : 2;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int W = blockDim.x >> 6;
  const int wbytes = dec_wave_lds(S2, VB, false);
  // grid (unit, slot, token): routed row b = token k + slot with k = gridDim.y, no division
  const int b = blockIdx.z * gridDim.y + blockIdx.y, u = blockIdx.x;
  const int tile = (ACT == 0 && wave >= a.Wk) ? 1 : 0;   // SiLU-GLU: gate waves, then up waves
  const int wk = wave - tile * a.Wk;
  const int rbase = ACT == 0 ? (tile == 0 ? 16 * u : a.I + 16 * u) : 16 * u;
  const uint16_t* xrow = a.x + (int64_t)blockIdx.z * a.sxm;
  int e = a.idx.at(b);
  e = (e >= 0 && e < a.E) ? e : 0;   // ids outside [0, E) are clamped, as in the sort
  const float v = dec_tile_partial<S2, SDT, XCL, false>(a, e, rbase, xrow, wk * S2, a.Kpad / kDLine,
                                                        smem + (size_t)wave * wbytes, lane, e, xrow);
  float* red = (float*)(smem + (size_t)W * wbytes);  // [W][16]
  if ((lane >> 4) == 0) red[wave * 16 + (lane & 15)] = v;
  lds_barrier();
  auto bias_at = [&](int row) -> float {
    return a.bias != nullptr ? load_bias(a.bias, a.bdt, (int64_t)e * a.sbe + row) : 0.f;
  };
  const int n = threadIdx.x;
  if constexpr (ACT == 0) {
    if (n < 16) {
      float g = 0.f, up = 0.f;
      for (int w = 0; w < a.Wk; ++w) {
        g += red[w * 16 + n];
        up += red[(a.Wk + w) * 16 + n];
      }
      g += bias_at(16 * u + n);
      up += bias_at(a.I + 16 * u + n);
      a.out[(int64_t)b * a.som + 16 * u + n] = (uint16_t)f32_to_bf16_bits(g / (1.f + __expf(-g)) * up);
    }
  } else {
    if (n < 8) {
      float g = 0.f, up = 0.f;
      for (int w = 0; w < a.Wk; ++w) {
        g += red[w * 16 + 2 * n];
        up += red[w * 16 + 2 * n + 1];
      }
      g += bias_at(16 * u + 2 * n);
      up += bias_at(16 * u + 2 * n + 1);
      a.out[(int64_t)b * a.som + 8 * u + n] = (uint16_t)f32_to_bf16_bits(gptoss_glu(g, up, a.alpha, a.limit));
    }
  }
}

template <int S2, int SDT, bool XCL, bool PAIR>
__global__ __launch_bounds__(1024) void moe_dn_line_kernel(MoeDecArgs a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  constexpr int VB = (SDT == IMQ_DT_FP32) ? 4 : 2;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int W = blockDim.x >> 6;
  constexpr int ROWS = PAIR ? 8 : 16;               // output rows per workgroup
  const int wbytes = dec_wave_lds(S2, VB, PAIR);
  const int t = blockIdx.y, rt = blockIdx.x;                       // grid (row tile, token)
  const int grp = wave / a.Wk, wk = wave - grp * a.Wk;            // group: slot pair or slot
  const int j = PAIR ? 2 * grp : grp;
  const bool has2 = PAIR && j + 1 < a.k;                           // odd k: the last pair is one slot
  const int b = t * a.k + j, b2 = has2 ? b + 1 : b;
  int e = a.idx.at(b), e2 = a.idx.at(b2);
  e = (e >= 0 && e < a.E) ? e : 0;
  e2 = (e2 >= 0 && e2 < a.E) ? e2 : 0;
  float v = dec_tile_partial<S2, SDT, XCL, PAIR>(a, e, ROWS * rt, a.x + (int64_t)b * a.sxm, wk * S2,
                                                 a.Kpad / kDLine, smem + (size_t)wave * wbytes, lane, e2,
                                                 a.x + (int64_t)b2 * a.sxm);
  const int c = lane & 15;
  const bool hi = PAIR && c >= 8;                                  // PAIR columns 8-15: slot b2
  const int row = PAIR ? 8 * rt + (c & 7) : 16 * rt + c;
  if (wk == 0 && a.bias != nullptr) v += load_bias(a.bias, a.bdt, (int64_t)(hi ? e2 : e) * a.sbe + row);
  v *= hi ? (has2 ? bf16_bits_to_f32(a.topk_w[b2]) : 0.f) : bf16_bits_to_f32(a.topk_w[b]);
  float* red = (float*)(smem + (size_t)W * wbytes);  // [W][16]
  if ((lane >> 4) == 0) red[wave * 16 + c] = v;
  lds_barrier();
  const int n = threadIdx.x;
  if (n < ROWS) {
    float sum = 0.f;
    for (int w = 0; w < W; ++w) sum += PAIR ? red[w * 16 + n] + red[w * 16 + 8 + n] : red[w * 16 + n];
    a.out[(int64_t)t * a.som + ROWS * rt + n] = (uint16_t)f32_to_bf16_bits(sum);
  }
}

template <class KERN>
int dec_launch(KERN kern, dim3 grid, int W, size_t lds, hipStream_t st, const MoeDecArgs& a) {
  if (lds > 65536) {
    hipError_t err = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (err != hipSuccess) return (int)err;
  }
  kern<<<grid, dim3(64 * W), lds, st>>>(a);
  IMQ_LAUNCH_CHECK();
  return IMQ_OK;
}

// S2 line-steps per wave (2, or 4 when K needs more waves than the workgroup has room for):
// Wk waves per tile or slot, at most 16 waves per workgroup in all.
bool dec_shape(int64_t Kpad, int groups, int* S2, int* Wk) {
  if (Kpad % kDLine) return false;
  const int64_t KL = Kpad / kDLine;
  for (int s = 2; s <= 4; s += 2) {
    const int64_t w = (KL + s - 1) / s;
    if (w * groups <= 16) {
      *S2 = s;
      *Wk = (int)w;
      return true;
    }
  }
  return false;
}

template <int SDT>
int dec_gu(const MoeDecArgs& a0, int act, int64_t B, int max_lds, hipStream_t st) {
  MoeDecArgs a = a0;
  int S2, Wk;
  const int groups = act == IMQ_ACT_GPTOSS ? 1 : 2;
  if (!dec_shape(a.Kpad, groups, &S2, &Wk)) return IMQ_ERR_UNSUPPORTED;
  a.Wk = Wk;
  a.NR = act == IMQ_ACT_GPTOSS ? 2 * a.I / 16 : a.I / 16;
  const int W = groups * Wk;
  const size_t lds = (size_t)W * dec_wave_lds(S2, SDT == IMQ_DT_FP32 ? 4 : 2, false) + (size_t)W * 16 * 4;
  const int64_t T = B / a.k;
  if (lds > (size_t)max_lds || a.NR > 0x7fffffff || a.k > 65535 || T > 65535 || T * a.k != B)
    return IMQ_ERR_UNSUPPORTED;
  const dim3 grid((unsigned)a.NR, (unsigned)a.k, (unsigned)T);
  const bool xcl = a.xk < a.Kpad;
#define IMQ_GU(S, A, X) dec_launch(moe_gu_line_kernel<S, SDT, A, X>, grid, W, lds, st, a)
  if (act == IMQ_ACT_GPTOSS) {
    if (S2 == 2) return xcl ? IMQ_GU(2, 1, true) : IMQ_GU(2, 1, false);
    return xcl ? IMQ_GU(4, 1, true) : IMQ_GU(4, 1, false);
  }
  if (S2 == 2) return xcl ? IMQ_GU(2, 0, true) : IMQ_GU(2, 0, false);
  return xcl ? IMQ_GU(4, 0, true) : IMQ_GU(4, 0, false);
#undef IMQ_GU
}

// Slot pairs (8 output rows per workgroup) while the T * H / 8 workgroups fit the CUs in one
// round -- measured on MI355X: OLMoE T=1 (H 2048: 256 workgroups) 1741 -> 1823 GB/s, gpt-oss T=1
// (H 2880: 360) 2631 -> 2543 -- else one slot per wave group and 16 rows per workgroup.
// Returns true when the pair form is taken; `groups` gets the wave groups per workgroup.
inline bool dec_dn_pairs(int64_t T, int64_t H, int k, int* groups) {
  const bool pair = H % 8 == 0 && T * (H / 8) <= device_info().cus;
  *groups = pair ? (k + 1) / 2 : k;
  return pair;
}

template <int SDT>
int dec_dn(const MoeDecArgs& a0, int64_t T, int64_t H, int max_lds, hipStream_t st) {
  MoeDecArgs a = a0;
  int S2, Wk, groups;
  const bool pair = dec_dn_pairs(T, H, a.k, &groups);
  if (!pair && H % 16 != 0) return IMQ_ERR_UNSUPPORTED;
  if (!dec_shape(a.Kpad, groups, &S2, &Wk)) return IMQ_ERR_UNSUPPORTED;
  a.Wk = Wk;
  a.NR = (int)(pair ? H / 8 : H / 16);
  const int W = groups * Wk;
  const size_t lds = (size_t)W * dec_wave_lds(S2, SDT == IMQ_DT_FP32 ? 4 : 2, pair) + (size_t)W * 16 * 4;
  if (lds > (size_t)max_lds || T > 65535) return IMQ_ERR_UNSUPPORTED;
  const dim3 grid((unsigned)a.NR, (unsigned)T);
  const bool xcl = a.xk < a.Kpad;
#define IMQ_DN(S, X, P) dec_launch(moe_dn_line_kernel<S, SDT, X, P>, grid, W, lds, st, a)
  if (pair) {
    if (S2 == 2) return xcl ? IMQ_DN(2, true, true) : IMQ_DN(2, false, true);
    return xcl ? IMQ_DN(4, true, true) : IMQ_DN(4, false, true);
  }
  if (S2 == 2) return xcl ? IMQ_DN(2, true, false) : IMQ_DN(2, false, false);
  return xcl ? IMQ_DN(4, true, false) : IMQ_DN(4, false, false);
#undef IMQ_DN
}

template <int S2, int NTL, int SDT, int MODE, int XCL>
int moe_line_launch(const MoeLineArgs& a, int W, int grid, hipStream_t st) {
  const size_t lds = (size_t)W * 2 * NTL * 16 * (S2 * ((SDT == IMQ_DT_FP32) ? 4 : 2) / 2) * 4 +
                     (size_t)W * NTL * 256 * 4 + (size_t)NTL * 16 * 4 + 16 * 4;
  auto kern = moe_line_kernel<S2, NTL, SDT, MODE, XCL>;
  if (lds > 65536) {
    hipError_t err = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (err != hipSuccess) return (int)err;
  }
  kern<<<dim3((unsigned)grid), dim3(64 * W), lds, st>>>(a);
  IMQ_LAUNCH_CHECK();
  return IMQ_OK;
}

// Line-steps per wave S2 (2 when K spans at least two, else 1) and waves W = ceil(KL / S2) <= 8,
// i.e. K <= 4096; deeper line-steps would exceed the register budget.
bool moe_line_shape(int64_t Kpad, int* S2, int* W) {
  if (Kpad % kMoeLine) return false;
  const int64_t KL = Kpad / kMoeLine;
  const int s = KL >= 2 ? 2 : 1;
  if ((KL + s - 1) / s > 8) return false;
  *S2 = s;
  *W = (int)((KL + s - 1) / s);
  return true;
}

// One workgroup per possible (expert, row block) item; those past the device-side work list
// exit after reading its length. Measured on MI355X at the OLMoE shape against persistent grids
// of 2-4 workgroups per CU and 32-row blocks: 64-row blocks with two line-steps per wave were
// fastest at T = 1, 16 and 256.
template <int NTL, int SDT, int MODE>
int moe_line_go(MoeLineArgs a, int rows, int64_t maxhit, int S2, int W, hipStream_t st) {
  a.NB = rows / (16 * NTL);
  // at most min(E, routed rows) experts are hit: no workgroups for items that cannot exist
  const int64_t items = (maxhit < a.E ? maxhit : (int64_t)a.E) * a.NB;
  if (items > 0x7fffffff) return IMQ_ERR_UNSUPPORTED;
  // the kernel's 32-bit buffer offsets: into one expert's rows, and into the activation rows
  // (hidden rows for gate_up, sorted h rows for down)
  const int64_t xrows = MODE == 1 ? (int64_t)a.nrows : (int64_t)a.nrows / a.k;
  if ((int64_t)rows * a.sqn > 0x7fffffff || (xrows * a.sxm + a.Kpad) * 2 > 0x7fffffff) return IMQ_ERR_UNSUPPORTED;
  if (a.xk < a.Kpad) {
    if (a.xk % 32) return IMQ_ERR_UNSUPPORTED;      // not produced by this path (H % 64, I % 32)
    if (S2 == 1) return moe_line_launch<1, NTL, SDT, MODE, 1>(a, W, (int)items, st);
    return moe_line_launch<2, NTL, SDT, MODE, 1>(a, W, (int)items, st);
  }
  if (S2 == 1) return moe_line_launch<1, NTL, SDT, MODE, 0>(a, W, (int)items, st);
  return moe_line_launch<2, NTL, SDT, MODE, 0>(a, W, (int)items, st);
}

template <int SDT, int MODE>
int moe_line_dispatch(MoeLineArgs a, int rows, int64_t maxhit, hipStream_t st) {
  int S2, W;
  if (!moe_line_shape(a.Kpad, &S2, &W)) return IMQ_ERR_UNSUPPORTED;
  const int KL = a.Kpad / kMoeLine;
  if (a.direct && KL <= 8) {
    // decode rows of a short K: 32-row blocks, and one line-step per wave below 8 line-steps,
    // so a hit expert's rows spread over twice the workgroups, several of them per CU (measured
    // on MI355X: OLMoE T=1 1189 -> 1258 GB/s; at gpt-oss's 12 line-steps 64-row blocks stay
    // faster)
    if (KL < 8) {
      S2 = 1;
      W = KL;
    }
    return moe_line_go<2, SDT, MODE>(a, rows, maxhit, S2, W, st);
  }
  return moe_line_go<4, SDT, MODE>(a, rows, maxhit, S2, W, st);
}

template <int MODE>
int moe_line_sdt(const MoeLineArgs& a, int rows, int64_t maxhit, int sdt, hipStream_t st) {
  switch (sdt) {
    case IMQ_DT_BF16: return moe_line_dispatch<IMQ_DT_BF16, MODE>(a, rows, maxhit, st);
    case IMQ_DT_FP16: return moe_line_dispatch<IMQ_DT_FP16, MODE>(a, rows, maxhit, st);
    case IMQ_DT_FP32: return moe_line_dispatch<IMQ_DT_FP32, MODE>(a, rows, maxhit, st);
  }
  return IMQ_ERR_INVALID;
}

template <bool OUT_F32>
int launch_rows(const uint16_t* x, int64_t sxm, int64_t xdiv, int64_t xk, int64_t B, int64_t Kpad, Ids eid,
                int64_t E, const uint8_t* q, int64_t sqe, int64_t sqn, const void* sc, int64_t sse, int64_t ssn,
                int64_t ssg, const void* zr, int64_t sze, int64_t szn, int64_t szg, int sdt, int64_t N, int64_t G,
                void* y, int64_t sym, hipStream_t st) {
  if (B == 0 || N == 0) return IMQ_OK;
  if (B > 65535) return IMQ_ERR_UNSUPPORTED;
  dim3 grid((unsigned)imq_cdiv(N, 4), (unsigned)B);
  switch (sdt) {
    case IMQ_DT_BF16:
      moe_rows_kernel<IMQ_DT_BF16, OUT_F32><<<grid, dim3(256), 0, st>>>(x, sxm, xdiv, xk, B, Kpad, eid, E, q, sqe, sqn, sc, sse, ssn, ssg, zr, sze, szn, szg, N, G, y, sym);
      break;
    case IMQ_DT_FP16:
      moe_rows_kernel<IMQ_DT_FP16, OUT_F32><<<grid, dim3(256), 0, st>>>(x, sxm, xdiv, xk, B, Kpad, eid, E, q, sqe, sqn, sc, sse, ssn, ssg, zr, sze, szn, szg, N, G, y, sym);
      break;
    case IMQ_DT_FP32:
      moe_rows_kernel<IMQ_DT_FP32, OUT_F32><<<grid, dim3(256), 0, st>>>(x, sxm, xdiv, xk, B, Kpad, eid, E, q, sqe, sqn, sc, sse, ssn, ssg, zr, sze, szn, szg, N, G, y, sym);
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
  return launch_rows<false>((const uint16_t*)x, x_row_stride, 1, K_pad, B, K_pad, Ids{eid, 0}, E, (const uint8_t*)qweight,
                            q_stride_e, q_row_stride, scale, s_stride_e, s_stride_n, s_stride_g, zero,
                            z_stride_e, z_stride_n, z_stride_g, sz_dtype, N, group_size, y, y_row_stride,
                            (hipStream_t)stream);
}

namespace {
// Workspace layout: [gu fp32 B x 2I][h bf16 B x hw][z fp32 B x H][off int32 E+1][perm int32 B+64]
// [hit int32 E+1], each 256-byte aligned; hw = I_pad rounded up to a multiple of 256, the widest
// down K_pad a kernel layout may use. The token-sorted path uses h, z, off, perm and hit; the
// per-row path gu, h and z.
struct MoeWs {
  int64_t gu, h, z, off, perm, hit, rsx, rsh, total, hw;
};

MoeWs moe_ws(int64_t T, int64_t top_k, int64_t E, int64_t H, int64_t I, int64_t G) {
  const int64_t B = T * top_k;
  const int64_t I_pad = imq_cdiv(I, G) * G;
  MoeWs w;
  w.hw = imq_cdiv(I_pad, 256) * 256;
  w.gu = 0;
  w.h = w.gu + align_up(B * 2 * I * 4, kAlign);
  w.z = w.h + align_up(B * w.hw * 2, kAlign);
  w.off = w.z + align_up(B * H * 4, kAlign);
  w.perm = w.off + align_up((E + 1) * 4, kAlign);
  w.hit = w.perm + align_up((B + 64) * 4, kAlign);   // 64 spare entries: the kernels' scalar reads
  // the register-B grouped GEMM's row group sums (groups of 128): hidden rows, then h rows
  w.rsx = w.hit + align_up((E + 1) * 4, kAlign);
  w.rsh = w.rsx + align_up(T * imq_cdiv(H, 128) * 4, kAlign);
  w.total = w.rsh + align_up(B * imq_cdiv(I, 128) * 4, kAlign);
  return w;
}
}  // namespace

extern "C" int64_t imq_moe_workspace_bytes(int64_t T, int64_t top_k, int64_t E, int64_t H, int64_t I,
                                           int64_t group_size) {
  if (T < 0 || top_k <= 0 || E <= 0 || H <= 0 || I <= 0 || group_size <= 0) return -1;
  return moe_ws(T, top_k, E, H, I, group_size).total;
}

namespace {
struct MoeCall {
  const uint16_t* hidden;
  int64_t hs, T, H, k;
  Ids idx;
  const uint16_t* topk_w;
  int64_t E;
  const uint8_t* gq;
  int64_t gqe, gqn, gK;
  const void *gs, *gz;
  int64_t gse, gsn, I;
  const uint8_t* dq;
  int64_t dqe, dqn, dK;
  const void *ds, *dz;
  int64_t dse, dsn;
  int sdt;
  int64_t G;
  const void* gb;
  int64_t gbe;
  const void* db;
  int64_t dbe;
  int bdt, act;
  float alpha, limit;
  uint16_t* out;
  int64_t os;
  int64_t xk;            // valid hidden columns: gu_K_pad for padded rows, else H (H % 8 == 0)
};

// Grouped GEMM path for many routed rows per expert (prefill): the sort also lists the row
// blocks of each hit expert; gate_up and down then run as grouped GEMMs over those blocks --
// the register-B kernel's MoE forms where they apply (int4 groups of 128, K a multiple of 128 up
// to 5120, I a multiple of 128 or the gpt-oss layout), else the LDS-dequant GEMM's -- the
// activation in gate_up's epilogue, the row bias and the scatter to routed order in down's; the
// combine is moe_combine_kernel's. It pays once an expert's rows times K is large enough to
// amortize the per-block costs; measured on MI355X (us per layer, line kernels -> register-B
// GEMM; rows per expert = B / E):
//   OLMoE (K 2048)   T=64 (8 rows) 81 -> 84, T=128 (16) 101 -> 88, T=256 (32) 146 -> 94,
//                    T=512 (64) 256 -> 147, T=1024 (128) 400 -> 230
//   gpt-oss (K 3072) T=64 (8 rows) 191 -> 223, T=128 (16) 241 -> 228, T=256 (32) 370 -> 234
// so the register-B forms run from (B / E) * gate_up K >= 32768 (16 rows at K 2048); the
// LDS-dequant GEMM, slower at these sizes, from 81920 (its crossover with the line kernels).
#ifndef IMQ_MOE_RB_WORK
#define IMQ_MOE_RB_WORK 32768
#endif
#ifndef IMQ_MOE_GEMM_WORK
#define IMQ_MOE_GEMM_WORK 81920
#endif
#ifndef IMQ_MOE_RB_WORK_WIDE
#define IMQ_MOE_RB_WORK_WIDE 8192
#endif
constexpr int64_t kMoeRbWork = IMQ_MOE_RB_WORK;
// gate_up K past 2048 (line kernel workgroups of more than 4 waves, one resident per CU at their
// register count): the register-B forms take over at a quarter of the work (measured, gpt-oss-20b
// K 3072: T=32 2237 -> 2393 GB/s, T=64 2105 -> 2420; OLMoE K 2048 keeps the line kernels to
// T=64, 2829 against 2398)
constexpr int64_t kMoeRbWorkWide = IMQ_MOE_RB_WORK_WIDE;
constexpr int64_t kRbKStep = 64;   // the register-B kernel's K step (RB_BK)
constexpr int64_t kMoeGemmWork = IMQ_MOE_GEMM_WORK;
int moe_gemm(const MoeCall& c, char* ws, const MoeWs& L, bool line_ok, hipStream_t st) {
  const int64_t B = c.T * c.k;
  const int64_t hits = c.E < B ? c.E : B;
  int32_t* off = (int32_t*)(ws + L.off);
  int32_t* perm = (int32_t*)(ws + L.perm);
  int32_t* hit = (int32_t*)(ws + L.hit);
  int32_t* mtl = (int32_t*)(ws + L.gu);
  uint16_t* h = (uint16_t*)(ws + L.h);
  float* yr = (float*)(ws + L.z);
  const int gmode = c.act == IMQ_ACT_GPTOSS ? 2 : 1;
  const int ib = 2;
  // the register-B form (weights dequantized into MFMA operands) where it takes both
  // projections, else the LDS-dequant GEMM; the block size of the sort's list follows the form
  bool rb = true;
  int bm = 32 * ib;
  int64_t max_mt = imq_cdiv(B, bm) + hits;
  // the folded form's row group sums: hidden rows (a launch of their own), h rows (gate_up's epilogue)
  float* rsx = (float*)(ws + L.rsx);
  float* rsh = (float*)(ws + L.rsh);
  const int ngx = (int)imq_cdiv(c.H, 128), ngh = (int)imq_cdiv(c.I, 128);
  // the register-B form skips down's K steps past I when I is a multiple of the 64-column K
  // step; otherwise h's columns past I are zeroed after gate_up
  const int64_t dxk = c.I % kRbKStep == 0 ? c.I : c.dK;
  auto gate_up = [&](bool check) {
    if (rb)
      return moe_rb(gmode, ib, c.hidden, c.hs, c.T, c.gK, c.xk, c.gq, c.gqe, c.gqn, c.gs, c.gz, c.gse, c.gsn, c.sdt,
                    2 * c.I, c.I, mtl + 2, mtl, max_mt, off, perm, (int)c.k, c.gb, c.gbe, c.bdt, c.alpha, c.limit, h,
                    L.hw, nullptr, false, rsx, ngx, ngx, rsh, ngh, st, check);
    return moe_gemm_w4(gmode, c.hidden, c.hs, c.T, c.gK, c.gq, c.gqe, c.gqn, c.gs, c.gz, c.gse, c.gsn, c.sdt,
                       2 * c.I, c.I, mtl + 2, mtl, max_mt, off, perm, (int)c.k, c.gb, c.gbe, c.bdt, c.alpha, c.limit,
                       h, L.hw, nullptr, st, check);
  };
  auto down = [&](bool check) {
    if (rb)
      return moe_rb(3, ib, h, L.hw, B, c.dK, dxk, c.dq, c.dqe, c.dqn, c.ds, c.dz, c.dse, c.dsn, c.sdt, c.H, 0, mtl + 2,
                    mtl, max_mt, off, perm, (int)c.k, c.db, c.dbe, c.bdt, 0.f, 0.f, nullptr, 0, yr, true, rsh, ngh,
                    ngh, nullptr, 0, st, check);
    return moe_gemm_w4(3, h, L.hw, B, c.dK, c.dq, c.dqe, c.dqn, c.ds, c.dz, c.dse, c.dsn, c.sdt, c.H, 0, mtl + 2, mtl,
                       max_mt, off, perm, (int)c.k, c.db, c.dbe, c.bdt, 0.f, 0.f, nullptr, 0, yr, st, check);
  };
  // both projections are validated before anything is launched
  if (gate_up(true) != IMQ_OK || down(true) != IMQ_OK) {
    // the LDS-dequant GEMM only above its own crossover, while the line kernels take the shape
    if (line_ok && B * c.gK < kMoeGemmWork * c.E) return IMQ_ERR_UNSUPPORTED;
    if (c.xk != c.gK) return IMQ_ERR_UNSUPPORTED;   // the LDS-dequant GEMM reads K columns per row
    rb = false;
    bm = moe_gemm_bm();
    max_mt = imq_cdiv(B, bm) + hits;
    int rc = gate_up(true);
    if (rc == IMQ_OK) rc = down(true);
    if (rc != IMQ_OK) return rc;
  }
  if ((2 + 2 * max_mt) * 4 > L.h - L.gu) return IMQ_ERR_UNSUPPORTED;   // the list lives in gu's room
  int rc;
  // the sort, and beside it (folded form) the hidden rows' group sums: 16 (row, group) waves per
  // extra workgroup
  const bool sums = rb && moe_rb_folded();
  const int64_t rs_blocks = sums ? imq_cdiv(c.T * ngx, 16) : 0;
  if (rs_blocks > 0x7ffffffe) return IMQ_ERR_UNSUPPORTED;
  moe_sort_kernel<<<dim3((unsigned)(1 + rs_blocks)), dim3(1024), (size_t)c.E * 4, st>>>(
      c.idx, (int)B, (int)c.E, off, perm, hit, mtl, bm, c.hidden, c.hs, c.T, ngx, sums ? rsx : nullptr, (int)c.xk);
  IMQ_LAUNCH_CHECK();
  rc = gate_up(false);
  if (rc != IMQ_OK) return rc;
  if (c.dK > c.I && (!rb || dxk > c.I)) {   // h's columns past I that down's K steps read: zero them
    const int64_t total = B * (c.dK - c.I);
    const int64_t blocks = imq_cdiv(total, 256) < 4096 ? imq_cdiv(total, 256) : 4096;
    moe_zero_pad_kernel<<<dim3((unsigned)blocks), dim3(256), 0, st>>>(h, B, c.I, c.dK, L.hw);
    IMQ_LAUNCH_CHECK();
  }
  rc = down(false);
  if (rc != IMQ_OK) return rc;
  const int64_t total = c.T * (c.H / 4);
  const int64_t blocks = imq_cdiv(total, 256) < 4096 ? imq_cdiv(total, 256) : 4096;
  if (rb) {
    const int64_t t8 = c.T * (c.H / 8);
    const int64_t b8 = imq_cdiv(t8, 256) < 4096 ? imq_cdiv(t8, 256) : 4096;
    moe_combine_bf16_kernel<<<dim3((unsigned)b8), dim3(256), 0, st>>>((const uint16_t*)yr, c.topk_w, c.T, c.k, c.H,
                                                                       c.out, c.os);
  } else {
    moe_combine_kernel<<<dim3((unsigned)blocks), dim3(256), 0, st>>>(yr, c.topk_w, c.T, c.k, c.H, c.out, c.os);
  }
  IMQ_LAUNCH_CHECK();
  return IMQ_OK;
}

// Token-sorted grouped path; IMQ_ERR_UNSUPPORTED when the shape or layout does not qualify.
int moe_sorted(const MoeCall& c, char* ws, const MoeWs& L, hipStream_t st) {
  const int64_t B = c.T * c.k;
  const int vb = c.sdt == IMQ_DT_FP32 ? 4 : 2;
  // (K padded to a multiple of the line, 256, is the line kernels' condition -- moe_line_shape /
  // dec_shape; the grouped GEMMs take K_pad multiples of 128)
  if (c.G != 128 || c.I % 32 || c.H % 64) return IMQ_ERR_UNSUPPORTED;
  if (!aligned(c.out, 16) || (c.os % 8)) return IMQ_ERR_UNSUPPORTED;
  if (c.E > 16384 || B > 0x7fffffff || c.T * c.hs > 0x7fffffffLL * 8) return IMQ_ERR_UNSUPPORTED;
  if (!aligned(c.gq, 16) || !aligned(c.dq, 16) || (c.gqn % 16) || (c.dqn % 16) || (c.gqe % 16) || (c.dqe % 16))
    return IMQ_ERR_UNSUPPORTED;
  // the line kernels read scale / zero pairs as 4-byte words and take K up to 4096; the grouped
  // GEMMs read them element-wise and take any K
  const bool sz_words = aligned(c.gs, 4) && aligned(c.gz, 4) && aligned(c.ds, 4) && aligned(c.dz, 4) &&
                        (c.gsn * vb) % 4 == 0 && (c.dsn * vb) % 4 == 0 && (c.gse * vb) % 4 == 0 &&
                        (c.dse * vb) % 4 == 0;
  int s2, w, gw = 0;
  const bool line_ok = sz_words && moe_line_shape(c.gK, &s2, &gw) && moe_line_shape(c.dK, &s2, &w);
  int32_t* off = (int32_t*)(ws + L.off);
  int32_t* perm = (int32_t*)(ws + L.perm);
  int32_t* hit = (int32_t*)(ws + L.hit);
  uint16_t* h = (uint16_t*)(ws + L.h);
  float* yr = (float*)(ws + L.z);
  // Decode: with few routed rows per expert there is little weight reuse to win by grouping, and
  // the sort and combine launches plus the item's dependent loads dominate; rows then run
  // directly (routed order, one row per item, expert idx[b]) up to 1.25 routed rows per expert
  // (1.75 where gate_up's K takes more than 4 waves and the token-sorted kernel runs one
  // workgroup per CU): measured crossovers on MI355X at the OLMoE and gpt-oss-20b shapes.
  const bool direct = B * 4 <= c.E * (gw > 4 ? 7 : 5);
  if (direct && line_ok && c.I % 16 == 0 && c.H % 16 == 0) {
    // two line-kernel launches: gate_up with the activation, down with the weighted combine
    MoeDecArgs gu{c.hidden, c.hs, (int)c.xk, (int)c.gK, (int)c.k, c.idx, c.topk_w, (int)c.E, c.gq, c.gqe, c.gqn,
                  c.gs, c.gz, c.gse, c.gsn, (int)c.I, 0, 0, c.gb, c.gbe, c.bdt, c.alpha, c.limit, h, L.hw};
    MoeDecArgs dn{h, L.hw, (int)c.I, (int)c.dK, (int)c.k, c.idx, c.topk_w, (int)c.E, c.dq, c.dqe, c.dqn,
                  c.ds, c.dz, c.dse, c.dsn, (int)c.I, 0, 0, c.db, c.dbe, c.bdt, 0.f, 0.f, c.out, c.os};
    int gs, gwk, dshape, dwk;
    const int groups = c.act == IMQ_ACT_GPTOSS ? 1 : 2;
    int dgroups;
    const bool dpair = dec_dn_pairs(c.T, c.H, (int)c.k, &dgroups);
    const int vb = c.sdt == IMQ_DT_FP32 ? 4 : 2;
    // both launches' shapes and LDS are checked before the first is issued, so a down that
    // would decline never follows a gate_up already in flight
    if (dec_shape(c.gK, groups, &gs, &gwk) && dec_shape(c.dK, dgroups, &dshape, &dwk) &&
        (size_t)groups * gwk * (dec_wave_lds(gs, vb, false) + 64) <= 65536 &&
        (size_t)dgroups * dwk * (dec_wave_lds(dshape, vb, dpair) + 64) <= 65536 && (dpair || c.H % 16 == 0)) {
      int rc = IMQ_ERR_UNSUPPORTED;
      switch (c.sdt) {
        case IMQ_DT_BF16: rc = dec_gu<IMQ_DT_BF16>(gu, c.act, B, 65536, st); break;
        case IMQ_DT_FP16: rc = dec_gu<IMQ_DT_FP16>(gu, c.act, B, 65536, st); break;
        case IMQ_DT_FP32: rc = dec_gu<IMQ_DT_FP32>(gu, c.act, B, 65536, st); break;
      }
      if (rc == IMQ_OK) {
        switch (c.sdt) {
          case IMQ_DT_BF16: return dec_dn<IMQ_DT_BF16>(dn, c.T, c.H, 65536, st);
          case IMQ_DT_FP16: return dec_dn<IMQ_DT_FP16>(dn, c.T, c.H, 65536, st);
          case IMQ_DT_FP32: return dec_dn<IMQ_DT_FP32>(dn, c.T, c.H, 65536, st);
        }
      }
      if (rc != IMQ_ERR_UNSUPPORTED) return rc;
    }
  }
  const bool gemm_shape = c.act == IMQ_ACT_GPTOSS || c.I % (moe_gemm_bn() / 2) == 0;
  const int64_t rb_work = gw > 4 ? kMoeRbWorkWide : kMoeRbWork;
  if (!direct && (!line_ok || B * c.gK >= rb_work * c.E) && gemm_shape) {
    const int rc = moe_gemm(c, ws, L, line_ok, st);
    if (rc != IMQ_ERR_UNSUPPORTED) return rc;
  }
  if (!line_ok) return IMQ_ERR_UNSUPPORTED;
  if (!direct) {
    moe_sort_kernel<<<dim3(1), dim3(1024), (size_t)c.E * 4, st>>>(c.idx, (int)B, (int)c.E, off, perm, hit, nullptr,
                                                                   1);
    IMQ_LAUNCH_CHECK();
  }
  MoeLineArgs g{c.hidden, c.hs, (int)c.gK, (int)c.k, off, perm, hit, c.gq, c.gqe, c.gqn, c.gs, c.gz, c.gse, c.gsn,
                (int)c.E, 0, (int)c.I, h, L.hw, c.gb, c.gbe, c.bdt, c.alpha, c.limit, (int)c.xk,
                c.idx, (int)B, direct ? 1 : 0};
  int rc = c.act == IMQ_ACT_GPTOSS ? moe_line_sdt<2>(g, (int)(2 * c.I), B, c.sdt, st)
                                   : moe_line_sdt<0>(g, (int)(2 * c.I), B, c.sdt, st);
  if (rc != IMQ_OK) return rc;
  // h's columns past I read as zero when I % 8 == 0; otherwise the partial last 8 is zeroed here
  const int64_t hxk = c.I % 8 == 0 ? c.I : c.dK;
  if (hxk > c.I) {
    const int64_t total = B * (c.dK - c.I);
    const int64_t blocks = imq_cdiv(total, 256) < 4096 ? imq_cdiv(total, 256) : 4096;
    moe_zero_pad_kernel<<<dim3((unsigned)blocks), dim3(256), 0, st>>>(h, B, c.I, c.dK, L.hw);
    IMQ_LAUNCH_CHECK();
  }
  MoeLineArgs d{h, L.hw, (int)c.dK, (int)c.k, off, perm, hit, c.dq, c.dqe, c.dqn, c.ds, c.dz, c.dse, c.dsn,
                (int)c.E, 0, 0, yr, c.H, c.db, c.dbe, c.bdt, 0.f, 0.f, (int)hxk, c.idx, (int)B, direct ? 1 : 0};
  rc = moe_line_sdt<1>(d, (int)c.H, B, c.sdt, st);
  if (rc != IMQ_OK) return rc;
  const int64_t total = c.T * (c.H / 4);
  const int64_t blocks = imq_cdiv(total, 256) < 4096 ? imq_cdiv(total, 256) : 4096;
  moe_combine_kernel<<<dim3((unsigned)blocks), dim3(256), 0, st>>>(yr, c.topk_w, c.T, c.k, c.H, c.out, c.os);
  IMQ_LAUNCH_CHECK();
  return IMQ_OK;
}

// Per-row path for every other shape: gate_up rows, activation, down rows, combine.
int moe_per_row(const MoeCall& c, char* ws, const MoeWs& L, hipStream_t st) {
  const int64_t B = c.T * c.k;
  float* gu = (float*)(ws + L.gu);
  uint16_t* h = (uint16_t*)(ws + L.h);
  float* z = (float*)(ws + L.z);
  int rc = launch_rows<true>(c.hidden, c.hs, c.k, c.xk, B, c.gK, c.idx, c.E, c.gq, c.gqe, c.gqn, c.gs, c.gse, c.gsn, 1,
                             c.gz, c.gse, c.gsn, 1, c.sdt, 2 * c.I, c.G, gu, 2 * c.I, st);
  if (rc != IMQ_OK) return rc;
  {
    const int64_t total = B * c.dK;
    const int64_t blocks = imq_cdiv(total, 256) < 4096 ? imq_cdiv(total, 256) : 4096;
    if (c.act == IMQ_ACT_GPTOSS)
      swiglu_kernel<1><<<dim3((unsigned)blocks), dim3(256), 0, st>>>(gu, B, c.I, c.dK, L.hw, c.idx, c.E, c.gb, c.gbe,
                                                                   c.bdt, c.alpha, c.limit, h);
    else
      swiglu_kernel<0><<<dim3((unsigned)blocks), dim3(256), 0, st>>>(gu, B, c.I, c.dK, L.hw, c.idx, c.E, c.gb, c.gbe,
                                                                   c.bdt, c.alpha, c.limit, h);
    IMQ_LAUNCH_CHECK();
  }
  rc = launch_rows<true>(h, L.hw, 1, c.dK, B, c.dK, c.idx, c.E, c.dq, c.dqe, c.dqn, c.ds, c.dse, c.dsn, 1, c.dz, c.dse,
                         c.dsn, 1, c.sdt, c.H, c.G, z, c.H, st);
  if (rc != IMQ_OK) return rc;
  const int64_t total = c.T * c.H;
  const int64_t blocks = imq_cdiv(total, 256) < 4096 ? imq_cdiv(total, 256) : 4096;
  combine_kernel<<<dim3((unsigned)blocks), dim3(256), 0, st>>>(z, c.topk_w, c.T, c.k, c.H, c.idx, c.E, c.db, c.dbe,
                                                             c.bdt, c.out, c.os);
  IMQ_LAUNCH_CHECK();
  return IMQ_OK;
}
}  // namespace

extern "C" int imq_moe_experts_w4_ex(
    const void* hidden, int64_t h_row_stride, int64_t T, int64_t H, int64_t top_k, const void* topk_idx,
    int idx_dtype, const void* topk_w, int64_t E, const void* gu_q, int64_t gu_q_stride_e, int64_t gu_q_row_stride, int64_t gu_K_pad,
    const void* gu_s, const void* gu_z, int64_t gu_sz_stride_e, int64_t gu_sz_stride_n, int64_t I, const void* dn_q,
    int64_t dn_q_stride_e, int64_t dn_q_row_stride, int64_t dn_K_pad, const void* dn_s, const void* dn_z,
    int64_t dn_sz_stride_e, int64_t dn_sz_stride_n, int sz_dtype, int64_t group_size, const void* gu_bias,
    int64_t gu_bias_stride_e, const void* dn_bias, int64_t dn_bias_stride_e, int bias_dtype, int act, float alpha,
    float limit, void* out, int64_t out_row_stride, void* workspace, int64_t workspace_bytes, void* stream) {
  if (!hidden || !topk_idx || !topk_w || !gu_q || !gu_s || !gu_z || !dn_q || !dn_s || !dn_z || !out)
    return IMQ_ERR_INVALID;
  if (T < 0 || H <= 0 || top_k <= 0 || E <= 0 || I <= 0 || group_size <= 0 || group_size % 8) return IMQ_ERR_INVALID;
  if (idx_dtype != IMQ_DT_I32 && idx_dtype != IMQ_DT_I64) return IMQ_ERR_INVALID;
  if (sz_dtype != IMQ_DT_BF16 && sz_dtype != IMQ_DT_FP16 && sz_dtype != IMQ_DT_FP32) return IMQ_ERR_INVALID;
  if (act != IMQ_ACT_SILU_GLU && act != IMQ_ACT_GPTOSS) return IMQ_ERR_INVALID;
  if ((gu_bias || dn_bias) && bias_dtype != IMQ_DT_BF16 && bias_dtype != IMQ_DT_FP16 && bias_dtype != IMQ_DT_FP32)
    return IMQ_ERR_INVALID;
  if (gu_bias && gu_bias_stride_e < 2 * I) return IMQ_ERR_INVALID;
  if (dn_bias && dn_bias_stride_e < H) return IMQ_ERR_INVALID;
  const int64_t G = group_size;
  const MoeWs L = moe_ws(T, top_k, E, H, I, G);
  // kernel K_pads: multiples of the group covering in_features; down's fits the workspace's h rows
  if (gu_K_pad < H || gu_K_pad % G || dn_K_pad < I || dn_K_pad % G || dn_K_pad > L.hw) return IMQ_ERR_INVALID;
  if (gu_q_row_stride < gu_K_pad / 2 || dn_q_row_stride < dn_K_pad / 2) return IMQ_ERR_INVALID;
  if (gu_sz_stride_n < gu_K_pad / G || dn_sz_stride_n < dn_K_pad / G) return IMQ_ERR_INVALID;
  if (T == 0) return IMQ_OK;
  if (!workspace || workspace_bytes < L.total) return IMQ_ERR_INVALID;
  // hidden rows either cover gu_K_pad (zero past H), or just H with H % 8 == 0: the kernels then
  // clamp their reads to the first H columns
  if (out_row_stride < H || h_row_stride < H || (h_row_stride < gu_K_pad && H % 8 != 0)) return IMQ_ERR_INVALID;
  if (!aligned(gu_q, 4) || !aligned(dn_q, 4) || (gu_q_row_stride % 4) || (dn_q_row_stride % 4) ||
      (gu_q_stride_e % 4) || (dn_q_stride_e % 4) || !aligned(hidden, 16) || (h_row_stride % 8) ||
      !aligned(workspace, 256))
    return IMQ_ERR_ALIGN;
  const MoeCall c{(const uint16_t*)hidden, h_row_stride, T, H, top_k, Ids{topk_idx, idx_dtype == IMQ_DT_I64},
                  (const uint16_t*)topk_w, E,
                  (const uint8_t*)gu_q, gu_q_stride_e, gu_q_row_stride, gu_K_pad, gu_s, gu_z, gu_sz_stride_e,
                  gu_sz_stride_n, I, (const uint8_t*)dn_q, dn_q_stride_e, dn_q_row_stride, dn_K_pad, dn_s, dn_z,
                  dn_sz_stride_e, dn_sz_stride_n, sz_dtype, G, gu_bias, gu_bias_stride_e, dn_bias, dn_bias_stride_e,
                  bias_dtype, act, alpha, limit, (uint16_t*)out, out_row_stride,
                  h_row_stride >= gu_K_pad ? gu_K_pad : H};
  hipStream_t st = (hipStream_t)stream;
  char* ws = (char*)workspace;
  const int rs = moe_sorted(c, ws, L, st);
  if (rs != IMQ_ERR_UNSUPPORTED) return rs;
  return moe_per_row(c, ws, L, st);
}

extern "C" int imq_moe_experts_w4(const void* hidden, int64_t h_row_stride, int64_t T, int64_t H, int64_t top_k,
                                  const int32_t* topk_idx, const void* topk_w, int64_t E, const void* gu_q,
                                  int64_t gu_q_stride_e, int64_t gu_q_row_stride, const void* gu_s, const void* gu_z,
                                  int64_t gu_sz_stride_e, int64_t gu_sz_stride_n, int64_t I, const void* dn_q,
                                  int64_t dn_q_stride_e, int64_t dn_q_row_stride, const void* dn_s, const void* dn_z,
                                  int64_t dn_sz_stride_e, int64_t dn_sz_stride_n, int sz_dtype, int64_t group_size,
                                  void* out, int64_t out_row_stride, void* workspace, int64_t workspace_bytes,
                                  void* stream) {
  if (group_size <= 0) return IMQ_ERR_INVALID;
  const int64_t H_pad = imq_cdiv(H, group_size) * group_size;
  const int64_t I_pad = imq_cdiv(I, group_size) * group_size;
  return imq_moe_experts_w4_ex(hidden, h_row_stride, T, H, top_k, topk_idx, IMQ_DT_I32, topk_w, E, gu_q, gu_q_stride_e,
                               gu_q_row_stride, H_pad, gu_s, gu_z, gu_sz_stride_e, gu_sz_stride_n, I, dn_q,
                               dn_q_stride_e, dn_q_row_stride, I_pad, dn_s, dn_z, dn_sz_stride_e, dn_sz_stride_n,
                               sz_dtype, group_size, nullptr, 0, nullptr, 0, IMQ_DT_BF16, IMQ_ACT_SILU_GLU, 0.f, 0.f,
                               out, out_row_stride, workspace, workspace_bytes, stream);
}
