// Decode-regime (M <= 16) fused dequant GEMV kernels for gfx950: the int4 / int2 / int8 line
// kernels (M <= 4), the wave-split and K-split kernels (4 < M <= 16) and the skinny kernels below
// (the shapes those decline). The line, split and int8 skinny kernels also read weights in the
// line-tiled layout (line_bases; the imq_linear_w*_tiled entry points).
//
// w4 skinny kernel
// ----------------
// Tile = 16 output rows (n) x all of K; a workgroup of W waves owns one tile at a time and
// splits its K range across the waves; the tile loop is grid-strided.
//
// Per K-step (128 codes = 64 bytes of a packed row) every lane (j = lane/16, n = lane%16) does
// ONE 16-byte load of row n (codes 32j..32j+31 of the step), so a wave reads 16 rows x 64
// contiguous bytes per load instruction. The 32 codes are turned into four MFMA B operands
// with one v_and_or_b32 per code pair: (code | 0x4300) is exactly the bf16 value 128 + code.
// Four v_mfma_f32_16x16x32_bf16 accumulate  acc[m][n] = sum_k x[m][k] * (128 + q[n][k])  over
// the step; the zero point and scale are folded in per step (all 128 codes share one group
// because G % 128 == 0):
//     y[m][n] += s * acc[m][n] - s * (128 + z) * xsum[m]
// with xsum[m] = sum of x[m][k] over the step. That is sum_k x * (q - z) * s exactly in fp32,
// i.e. the unrounded-weight GEMV of the reference's split-K kernel (worker_quant.py:1176-1177).
// s and z are first rounded to bf16 like _dequant(torch.bfloat16) (worker_quant.py:646-647).
//
// Activations are staged once per workgroup in LDS, pre-permuted into the element order the
// unpacked weight operands use ([x0,x4,x1,x5,x2,x6,x3,x7] per 8), together with per-step
// row sums. Rows m >= M are never read (their MFMA A lanes are zero). When M*K does not fit
// in LDS, K is processed in chunks that are restaged per tile.
//
// Partial sums of the W waves are reduced through LDS in a fixed order: deterministic, no
// atomics, no memset, a single launch per linear.
#include "imq_common.h"

namespace imq {

struct SkinnyArgs {
  const uint16_t* x;
  int64_t sxm;
  int M;
  int Kpad;
  const uint8_t* q;
  int64_t sqn;
  const void* sc;
  int64_t ssn, ssg;
  const void* zr;
  int64_t szn, szg;
  int N;
  int G;
  uint16_t* y;
  int64_t sym;
  int chunk_steps;   // K-steps staged in LDS at once
  const int8_t* q8;  // int8 weights (the int8 kernel; q is unused there)
  float* part;       // split-K partials [splits][M][N] fp32 (the K-split kernel)
  int tiled;         // weights in the line-tiled layout (int4 line / K-split / wave-split, int2 line /
                     // K-split, int8 line / skinny)
};

constexpr int kStep = 128;          // codes per K-step
constexpr int kXPad = 8;            // bf16 elements of padding per LDS activation row

// Raw 16/32-bit scale/zero word -> fp32 value rounded to bf16 (conversion deferred to use, so the
// loads of a whole unit can be issued back to back).
template <int DT>
IMQ_DEV uint32_t load_raw(const void* p, int64_t idx) {
  if constexpr (DT == IMQ_DT_FP32) return ((const uint32_t*)p)[idx];
  else return ((const uint16_t*)p)[idx];
}

// Load exactly NW dwords (NW in {2, 4, 8, 16}) from an address aligned to min(4*NW, 16) bytes.
template <int NW>
IMQ_DEV void load_strip(const unsigned char* p, uint32_t* out) {
  static_assert(NW == 2 || NW == 4 || NW == 8 || NW == 16, "strip of 8, 16, 32 or 64 bytes");
  if constexpr (NW == 2) {
    const u32x2_t t = *(const u32x2_t*)p;
    out[0] = t[0];
    out[1] = t[1];
  } else {
#pragma unroll
    for (int v = 0; v < NW; v += 4) {
      const u32x4_t t = *(const u32x4_t*)(p + 4 * v);
#pragma unroll
      for (int e = 0; e < 4; ++e) out[v + e] = t[e];
    }
  }
}

// x resident in LDS (M * K_pad fits). One workgroup = one 16-row tile; its W waves split K,
// wave w owning steps [(r*W + w)*S, +S) of round r. Each wave issues all S loads of a round
// back to back (S*1 KB per wave in flight), then consumes them; latency is hidden by the many
// resident waves/workgroups, not by in-wave double buffering. Steps past K and rows past N are
// clamped to valid addresses (zero scale / never stored), so every load is unconditional.
//
// STRIP: with one group per step (G == 128), contiguous per-row scale/zero storage and K-steps a
// multiple of S, a wave's S scales of a row are S adjacent values: they are fetched with one
// vector load per row (all four lanes of a row load the same strip) instead of S scattered
// 2-byte loads, which would cost a cache-line lookup per row per step in the texture path.
template <int S, int MC, int SDT, int ZDT, bool STRIP, int MAXW>
__global__ __launch_bounds__(64 * MAXW) void w4_skinny_kernel(SkinnyArgs a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // uniform -> SGPR
  const int W = blockDim.x >> 6;
  const int nl = lane & 15;
  const int jl = lane >> 4;
  constexpr int RC = (MC < 4) ? MC : 4;
  constexpr int SZB = (SDT == IMQ_DT_FP32) ? 4 : 2;
  constexpr int ZZB = (ZDT == IMQ_DT_FP32) ? 4 : 2;

  const int KS = a.Kpad / kStep;
  const int R = (KS + W * S - 1) / (W * S);
  const int xls = KS * kStep + kXPad;
  uint16_t* xl = (uint16_t*)smem;                                    // [M][xls]
  float* xs = (float*)(smem + (size_t)a.M * xls * 2);                // [KS][16]
  float* red = xs + (size_t)KS * 16;                                 // [2][W][256]
  const int gsh = 31 - __builtin_clz(a.G / kStep);                   // steps per group = 2^gsh
  const int NT = (a.N + 15) / 16;
  int tile = blockIdx.x;          // the grid never exceeds the tile count

  const uint8_t* qrow;
  const unsigned char* srow;
  const unsigned char* zrow;
  auto set_tile = [&](int t) {
    int row = t * 16 + nl;
    row = row < a.N ? row : a.N - 1;
    qrow = a.q + (int64_t)row * a.sqn + 16 * jl;
    srow = (const unsigned char*)a.sc + (int64_t)row * a.ssn * SZB;
    zrow = (const unsigned char*)a.zr + (int64_t)row * a.szn * ZZB;
  };
  set_tile(tile);
  const int64_t ssg_b = a.ssg * SZB, szg_b = a.szg * ZZB;

  u32x4_t wv[S];
  uint32_t sr[S], zr[S];
  // strip words: S values of SZB bytes = S*SZB/4 dwords
  constexpr int SW = STRIP ? (S * SZB + 3) / 4 : 1;
  constexpr int ZW = STRIP ? (S * ZZB + 3) / 4 : 1;
  uint32_t sst[SW], zst[ZW];
  auto load_round = [&](int rnd) {
    const int sbase = (rnd * W + wave) * S;
#pragma unroll
    for (int i = 0; i < S; ++i) {
      int s = sbase + i;
      s = s < KS ? s : KS - 1;
      wv[i] = __builtin_nontemporal_load((const u32x4_t*)(qrow + (int64_t)s * 64));
      if constexpr (!STRIP) {
        const int64_t g = s >> gsh;
        sr[i] = load_raw<SDT>(srow + g * ssg_b, 0);
        zr[i] = load_raw<ZDT>(zrow + g * szg_b, 0);
      }
    }
    if constexpr (STRIP) {
      // exactly S values (S*SZB bytes, naturally aligned: the host checks 16-byte row and
      // base alignment and S*SZB is 8, 16 or 32) -- never past the row end
      const int64_t g0 = sbase < KS ? sbase : 0;     // whole strip past K: any valid strip
      load_strip<SW>(srow + g0 * SZB, sst);
      load_strip<ZW>(zrow + g0 * ZZB, zst);
    }
  };
  // raw 16/32-bit scale and zero word of step i of the current round
  auto s_raw = [&](int i) -> uint32_t {
    if constexpr (!STRIP) return sr[i];
    else if constexpr (SZB == 4) return sst[i];
    else return (i & 1) ? (sst[i >> 1] >> 16) : (sst[i >> 1] & 0xffffu);
  };
  auto z_raw = [&](int i) -> uint32_t {
    if constexpr (!STRIP) return zr[i];
    else if constexpr (ZZB == 4) return zst[i];
    else return (i & 1) ? (zst[i >> 1] >> 16) : (zst[i >> 1] & 0xffffu);
  };

  // ---- stage x (permuted) and per-step row sums --------------------------------------------
  // Loads complete in issue order, so the x loads are issued *before* the first weight round:
  // the staging then finishes under the weight latency and compute consumes the weights as
  // they arrive. Up to XB 16-byte blocks per thread are held in registers across the weight
  // issue; any remainder (large M) is staged afterwards.
  constexpr int XB = 4;
  const int nblk = KS * (kStep / 8);
  const int xtotal = a.M * nblk;
  u32x4_t xv[XB];
#pragma unroll
  for (int u = 0; u < XB; ++u) {
    int idx = threadIdx.x + u * blockDim.x;
    idx = idx < xtotal ? idx : xtotal - 1;
    const int m = idx / nblk;
    const int b = idx - m * nblk;
    xv[u] = *(const u32x4_t*)(a.x + (int64_t)m * a.sxm + 8 * b);
  }
  load_round(0);
  for (int idx = threadIdx.x; idx < 16 * KS; idx += blockDim.x) xs[idx] = 0.f;
  lds_barrier();
  auto stage_block = [&](int idx, const u32x4_t& v) {
    const int m = idx / nblk;
    const int b = idx - m * nblk;
    *(u32x4_t*)(xl + m * xls + 8 * b) = permute_x8(v);
    // the 16 blocks of one step are 16 consecutive idx (nblk is a multiple of 16, and idx
    // groups of 16 lie entirely inside or outside [0, xtotal))
    const float sum = row_sum16(bf16x8_sum(v));
    if ((b & 15) == 0) xs[(b >> 4) * 16 + m] = sum;
  };
#pragma unroll
  for (int u = 0; u < XB; ++u) {
    const int idx = threadIdx.x + u * blockDim.x;
    if (idx < xtotal) stage_block(idx, xv[u]);
  }
  for (int idx = threadIdx.x + XB * blockDim.x; idx < xtotal; idx += blockDim.x)
    stage_block(idx, *(const u32x4_t*)(a.x + (int64_t)(idx / nblk) * a.sxm + 8 * (idx % nblk)));
  lds_barrier();

  // A rows m >= M read row M-1: they only feed D rows that are never stored.
  const uint16_t* xlane = xl + (nl < a.M ? nl : a.M - 1) * xls + 32 * jl;
  const float* xslane = xs + 4 * jl;
  const uint32_t magic = magic_bf16_128x2();
  float yacc[4] = {0.f, 0.f, 0.f, 0.f};
  int buf = 0;

  for (;;) {
  for (int rnd = 0; rnd < R; ++rnd) {
    if (rnd > 0) load_round(rnd);
    // steps in pairs: two independent MFMA chains interleaved (ILP across the MFMA latency).
    // Everything the corrections need (row sums from LDS, scale terms) is read *before* the
    // MFMAs are issued, so no LDS return can land in a register an in-flight MFMA still reads.
#pragma unroll
    for (int i = 0; i < S; i += 2) {
      const int s0a = (rnd * W + wave) * S + i;
      const int s0b = s0a + 1;
      const bool va = s0a < KS, vb = s0b < KS;
      const int sa = va ? s0a : KS - 1;
      const int sb = vb ? s0b : KS - 1;
      const f32x4_t xsa = *(const f32x4_t*)(xslane + sa * 16);
      const f32x4_t xsb = *(const f32x4_t*)(xslane + sb * 16);
      bf16x8_t aa[4], ab[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        aa[k] = *(const bf16x8_t*)(xlane + sa * kStep + 8 * k);
        ab[k] = *(const bf16x8_t*)(xlane + sb * kStep + 8 * k);
      }
      const float sca = va ? raw_to_bf16_f32<SDT>(s_raw(i)) : 0.f;
      const float scb = vb ? raw_to_bf16_f32<SDT>(s_raw(i + 1)) : 0.f;
      const float cza = -(128.f + raw_to_bf16_f32<ZDT>(z_raw(i))) * sca;
      const float czb = -(128.f + raw_to_bf16_f32<ZDT>(z_raw(i + 1))) * scb;
      f32x4_t acca = {0.f, 0.f, 0.f, 0.f}, accb = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        acca = mfma16x16x32(aa[k], unpack_nib8_bf16(wv[i][k], magic), acca);
        accb = mfma16x16x32(ab[k], unpack_nib8_bf16(wv[i + 1][k], magic), accb);
      }
#pragma unroll
      for (int q = 0; q < RC; ++q) {
        yacc[q] = fmaf(cza, xsa[q], yacc[q]);
        yacc[q] = fmaf(czb, xsb[q], yacc[q]);
        yacc[q] = fmaf(sca, acca[q], yacc[q]);
        yacc[q] = fmaf(scb, accb[q], yacc[q]);
      }
    }
  }

  // cross-wave reduction in a fixed order; the buffer alternates between tiles, so one barrier
  // per tile suffices (a buffer is rewritten only after the next tile's barrier)
  float* rb = red + buf * (W * 256);
#pragma unroll
  for (int q = 0; q < 4; ++q) rb[wave * 256 + (4 * jl + q) * 16 + nl] = yacc[q];
  lds_barrier();
  const int n0 = tile * 16;
  // next tile's first round before the reduction, to overlap its latency
  const int next = tile + gridDim.x;
  if (next < NT) {
    set_tile(next);
    load_round(0);
  }
  for (int e = threadIdx.x; e < 16 * a.M; e += blockDim.x) {
    const int m = e >> 4;
    const int n = e & 15;
    float sum = 0.f;
    for (int w = 0; w < W; ++w) sum += rb[w * 256 + e];
    if (n0 + n < a.N) a.y[(int64_t)m * a.sym + n0 + n] = (uint16_t)f32_to_bf16_bits(sum);
  }
  if (next >= NT) break;
  tile = next;
  buf ^= 1;
#pragma unroll
  for (int q = 0; q < 4; ++q) yacc[q] = 0.f;
  }
}

// x too large for LDS (large M * K_pad): K is staged in chunks, restaged per tile.
template <int W, int MC, int SDT, int ZDT>
__global__ __launch_bounds__(64 * W) void w4_skinny_chunked_kernel(SkinnyArgs a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int nl = lane & 15;          // row within tile (B/D column), also A row m
  const int jl = lane >> 4;          // K quarter of the step (A/B), D row group
  constexpr int RC = (MC < 4) ? MC : 4;   // D registers that can hold a real row

  const int KS = a.Kpad / kStep;
  const int cs_max = a.chunk_steps;
  const int nchunks = (KS + cs_max - 1) / cs_max;
  const int xls = cs_max * kStep + kXPad;           // LDS row stride (elements)

  uint16_t* xl = (uint16_t*)smem;                                    // [M][xls]
  float* xs = (float*)(smem + (size_t)a.M * xls * 2);                // [cs_max][16]
  float* red = xs + (size_t)cs_max * 16;                             // [2][W][16][16]

  const int NT = (a.N + 15) / 16;
  const int gpd = a.G / kStep;       // K-steps per group

  auto stage = [&](int c0, int c1) {
    const int nblk = (c1 - c0) * (kStep / 8);
    for (int idx = threadIdx.x; idx < a.M * nblk; idx += 64 * W) {
      const int m = idx / nblk;
      const int b = idx - m * nblk;
      const u32x4_t v = *(const u32x4_t*)(a.x + (int64_t)m * a.sxm + (int64_t)c0 * kStep + 8 * b);
      *(u32x4_t*)(xl + m * xls + 8 * b) = permute_x8(v);
    }
    __syncthreads();
    const int cs = c1 - c0;
    for (int idx = threadIdx.x; idx < 16 * cs; idx += 64 * W) {
      const int st = idx >> 4;
      const int m = idx & 15;
      float sum = 0.f;
      if (m < a.M) {
        const uint16_t* p = xl + m * xls + st * kStep;
        for (int e = 0; e < kStep; e += 8) {
          const u32x4_t v = *(const u32x4_t*)(p + e);
#pragma unroll
          for (int d = 0; d < 4; ++d) {
            sum += __uint_as_float(v[d] << 16);
            sum += __uint_as_float(v[d] & 0xffff0000u);
          }
        }
      }
      xs[st * 16 + m] = sum;
    }
    __syncthreads();
  };

  if (nchunks == 1) stage(0, KS);

  int buf = 0;
  for (int tile = blockIdx.x; tile < NT; tile += gridDim.x) {
    const int n0 = tile * 16;
    const int row = n0 + nl;
    const bool row_ok = row < a.N;
    const uint8_t* qrow = a.q + (int64_t)(row_ok ? row : 0) * a.sqn;
    float yacc[4] = {0.f, 0.f, 0.f, 0.f};

    for (int c = 0; c < nchunks; ++c) {
      const int c0 = c * cs_max;
      const int c1 = (c0 + cs_max < KS) ? c0 + cs_max : KS;
      if (nchunks > 1) stage(c0, c1);
      const int spw = (c1 - c0 + W - 1) / W;
      const int s_beg = c0 + wave * spw;
      const int s_end = (s_beg + spw < c1) ? s_beg + spw : c1;

      constexpr int U = 4;
      for (int sb = s_beg; sb < s_end; sb += U) {
        u32x4_t wv[U];
        float sv[U], zv[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int s = sb + u;
          if (s < s_end && row_ok) {
            wv[u] = __builtin_nontemporal_load((const u32x4_t*)(qrow + (int64_t)s * 64 + 16 * jl));
            const int g = s / gpd;
            sv[u] = load_as_bf16_f32<SDT>(a.sc, (int64_t)row * a.ssn + (int64_t)g * a.ssg);
            zv[u] = load_as_bf16_f32<ZDT>(a.zr, (int64_t)row * a.szn + (int64_t)g * a.szg);
          } else {
            wv[u] = u32x4_t{0u, 0u, 0u, 0u};
            sv[u] = 0.f;
            zv[u] = 0.f;
          }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int s = sb + u;
          if (s < s_end) {
            const int sl = s - c0;
            const uint16_t* xa = xl + nl * xls + sl * kStep + 32 * jl;
            f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              bf16x8_t av;
              if (nl < a.M) {
                av = *(const bf16x8_t*)(xa + 8 * i);
              } else {
                av = __builtin_bit_cast(bf16x8_t, u32x4_t{0u, 0u, 0u, 0u});
              }
              acc = mfma16x16x32(av, unpack_nib8_bf16(wv[u][i], magic_bf16_128x2()), acc);
            }
            const f32x4_t xsum = *(const f32x4_t*)(xs + sl * 16 + 4 * jl);
            const float sc = sv[u];
            const float cz = -(128.f + zv[u]) * sc;
#pragma unroll
            for (int r = 0; r < RC; ++r) {
              yacc[r] = fmaf(sc, acc[r], yacc[r]);
              yacc[r] = fmaf(cz, xsum[r], yacc[r]);
            }
          }
        }
      }
      if (nchunks > 1) __syncthreads();   // before the next chunk overwrites the staged x
    }

    // Cross-wave reduction, fixed order.
    float* rb = red + buf * (W * 256);
#pragma unroll
    for (int r = 0; r < 4; ++r) rb[wave * 256 + (4 * jl + r) * 16 + nl] = yacc[r];
    __syncthreads();
    for (int t = threadIdx.x; t < 16 * a.M; t += 64 * W) {
      const int m = t >> 4;
      const int n = t & 15;
      float sum = 0.f;
#pragma unroll
      for (int w = 0; w < W; ++w) sum += rb[w * 256 + t];
      if (n0 + n < a.N) a.y[(int64_t)m * a.sym + n0 + n] = (uint16_t)f32_to_bf16_bits(sum);
    }
    buf ^= 1;
  }
}


// ---------------------------------------------------------------------------------------------
// int4 line kernel: the decode path for M <= 4, G == 128.
//
// One workgroup = one tile of 16 output rows; its W waves split K into line-steps of 256 codes
// (128 bytes of every packed row), wave w owning line-steps [w*S2, w*S2 + S2). Per line-step a
// wave issues two 16-byte loads per lane whose 64 lanes cover FULL 128-byte lines: load L0 reads
// rows 0-7, load L1 rows 8-15. Lane (c = lane % 16, a = lane / 16) of L0 reads row c & 7 at byte
// 16a (group 2l, columns c < 8) or 64 + 16a (group 2l+1, columns c >= 8); L1 mirrors it for rows
// 8-15. Selecting per lane then gives every lane the codes of ONE group of ONE row:
//   operand A-group (group 2l): c < 8 ? L0 : L1  -> row c
//   operand B-group (group 2l+1): c < 8 ? L1 : L0  -> row c ^ 8
// Each group feeds four v_mfma_f32_16x16x32_bf16 (weights = B operand, column = row) with the
// (code | 0x4300) = 128 + code unpack; the zero point and the +128 bias fold into one correction
// per group, y += s*acc - s*(128 + z)*sum(x), so every MFMA stays inside one group. The B-group
// accumulators hold row c ^ 8 in column c and are swapped back with one DPP row rotate.
//
// Issue order per wave: its x range, its scale/zero words (16 rows x S2 dwords per array, one
// dword per lane), then the weights; x and scale/zero are staged in wave-private LDS, so no
// workgroup barrier precedes the compute, which consumes line-steps as their loads land. The
// wave partials meet in LDS once at the end (fixed order, deterministic).
// ---------------------------------------------------------------------------------------------
constexpr int kLine = 256;
#ifndef IMQ_LINE_PAIRED
#define IMQ_LINE_PAIRED 1
#endif
#ifndef IMQ_LINE_PAIRED4
#define IMQ_LINE_PAIRED4 1
#endif

// lane c of each 16-lane row receives the value of lane c ^ 8 (DPP row_ror:8)
IMQ_DEV float row_swap8(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x128, 0xf, 0xf, false));
}

// Per-lane addresses of a 16-row tile's two full-line loads (rows 0-7 and rows 8-15 of the tile
// at qt) for line-step 0, and the byte stride between line-steps. Row layout: lane (c, ar) reads
// row c & 7 (+ 8 in the second load) at bytes 16 ar of the 128-byte line, + 64 (the line's second
// group) for c >= 8 in the first load and c < 8 in the second; rows past N read the last row.
// Line-tiled layout (a.tiled; N a multiple of 16, dense rows): those same pieces are stored in lane
// order, one 1 KiB half per load of the tile's 2 KiB line-step block, so lane l reads bytes 16 l
// and each 16-lane quarter of a load covers two whole 128-byte lines instead of eight partial ones.
template <class T>
IMQ_DEV void line_bases(const SkinnyArgs& a, const T* qt, int lane, int rlast, const T*& q0, const T*& q1,
                        int& lstride) {
  if (a.tiled) {
    q0 = qt + 16 * lane;
    q1 = q0 + 1024;
    lstride = 2048;
    return;
  }
  const int c = lane & 15, ar = lane >> 4;
  const int rr0 = (c & 7) < rlast ? (c & 7) : rlast;
  const int rr1 = 8 + (c & 7) < rlast ? 8 + (c & 7) : rlast;
  q0 = qt + rr0 * (int)a.sqn + 16 * ar + (c < 8 ? 0 : 64);
  q1 = qt + rr1 * (int)a.sqn + 16 * ar + (c < 8 ? 64 : 0);
  lstride = 128;
}

// LDS bytes of one wave's staging area / of a whole workgroup
IMQ_HOST_DEV inline int line_wave_lds(int M, int S2, int vb) {
  return M * (S2 * kLine + 8) * 2 + 2 * S2 * 16 * 4 + 2 * 16 * S2 * vb / 2 * 4;
}

template <int S2, int MC, int SDT, int MAXW>
__global__ __launch_bounds__(64 * MAXW) void w4_line_kernel(SkinnyArgs a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  constexpr int VB = (SDT == IMQ_DT_FP32) ? 4 : 2;   // bytes per scale / zero value
  constexpr int DPR = S2 * VB / 2;                   // dwords per row per array (2*S2 values)
  constexpr int RC = MC < 4 ? MC : 4;                 // D registers that can hold a real row
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int W = blockDim.x >> 6;
  const int c = lane & 15, ar = lane >> 4;
  const bool lo8 = c < 8;
  const int M = MC <= 2 ? MC : a.M;                 // MC 1 and 2 launch exactly that M
  const int KL = a.Kpad / kLine;
  const int ls0 = wave * S2;
  const int row0 = blockIdx.x * 16;
  const int rlast = a.N - 1 - row0;                  // last valid row within the tile

  const int xrow = S2 * kLine + 8;
  const int wbytes = line_wave_lds(M, S2, VB);
  unsigned char* wl = smem + (size_t)wave * wbytes;
  uint16_t* xw = (uint16_t*)wl;
  float* xs = (float*)(wl + M * xrow * 2);
  uint32_t* szl = (uint32_t*)(xs + 2 * S2 * 16);
  float* red = (float*)(smem + (size_t)W * wbytes);

  // 1) x: M rows x 32*S2 16-byte blocks of this wave's K range (clamped into the row)
  constexpr int XB = 32 * S2;
  constexpr int XU = (MC * XB + 63) / 64;
  const int xtot = M * XB;
  const uint16_t* xbase = a.x + (int64_t)ls0 * kLine;
  const int xlim = a.Kpad - ls0 * kLine - 8;         // last valid block start in the range
  u32x4_t xv[XU];
#pragma unroll
  for (int u = 0; u < XU; ++u) {
    int idx = lane + 64 * u;
    idx = idx < xtot ? idx : xtot - 1;
    const int m = idx / XB, b = idx - m * XB;
    int kb = 8 * b;
    kb = kb < xlim ? kb : xlim;
    xv[u] = *(const u32x4_t*)(xbase + m * (int)a.sxm + kb);
  }
  // 2) scale / zero words of groups [2*ls0, 2*ls0 + 2*S2): 2 arrays x 16 rows x DPR dwords
  constexpr int ZU = (32 * DPR + 63) / 64;
  const int ngd = a.Kpad / 128 * VB / 4;             // dwords per row holding real groups
  const unsigned char* sbase = (const unsigned char*)a.sc + (int64_t)row0 * a.ssn * VB;
  const unsigned char* zbase = (const unsigned char*)a.zr + (int64_t)row0 * a.szn * VB;
  uint32_t zv[ZU];
#pragma unroll
  for (int u = 0; u < ZU; ++u) {
    int d = lane + 64 * u;
    d = d < 32 * DPR ? d : 32 * DPR - 1;
    const int arr = d / (16 * DPR);
    const int rem = d - arr * (16 * DPR);
    int r = rem / DPR;
    const int dw = rem - r * DPR;
    r = r < rlast ? r : rlast;
    int gd = ls0 * (VB / 2) + dw;                    // dword index within the row (VB/2 per line-step)
    gd = gd < ngd ? gd : ngd - 1;
    const unsigned char* p = arr ? zbase + r * (int)a.szn * VB : sbase + r * (int)a.ssn * VB;
    zv[u] = *(const uint32_t*)(p + 4 * gd);
  }
  // 3) weights: per line-step one full-line load for rows 0-7 and one for rows 8-15
  const uint8_t* qt = a.q + (int64_t)row0 * a.sqn;
  const uint8_t* q0;
  const uint8_t* q1;
  int lst;
  line_bases(a, qt, lane, rlast, q0, q1, lst);
  u32x4_t wb[2 * S2];
#pragma unroll
  for (int i = 0; i < S2; ++i) {
    int l = ls0 + i;
    l = l < KL ? l : KL - 1;
    wb[2 * i] = __builtin_nontemporal_load((const u32x4_t*)(q0 + lst * l));
    wb[2 * i + 1] = __builtin_nontemporal_load((const u32x4_t*)(q1 + lst * l));
  }
  // 4) stage x (permuted to the unpack order) with its per-group sums, and scale/zero
#pragma unroll
  for (int u = 0; u < XU; ++u) {
    const int idx = lane + 64 * u;
    const bool ok = idx < xtot;
    const int m = (ok ? idx : 0) / XB, b = (ok ? idx : 0) - m * XB;
    float sum = bf16x8_sum(xv[u]);
    // the 16 blocks of one group are 16 consecutive idx (XB is a multiple of 16)
    sum = row_sum16(sum);
    if (ok) {
      *(u32x4_t*)(xw + m * xrow + 8 * b) = permute_x8(xv[u]);
      if ((b & 15) == 0) xs[(b >> 4) * 16 + m] = sum;
    }
  }
#pragma unroll
  for (int u = 0; u < ZU; ++u) {
    const int d = lane + 64 * u;
    if (d < 32 * DPR) szl[d] = zv[u];
  }
  // LDS is written and read by this wave only; its LDS operations execute in order
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");

  const uint32_t magic = magic_bf16_128x2();
  // PAIRED (M <= 2): A lane row m < M reads activation row m in group 2l, M <= m < 2M row m - M
  // in group 2l+1 (128 codes on), other rows repeat row 0 of group 2l (their D rows are unused)
  constexpr bool PAIRED = MC <= 2 && IMQ_LINE_PAIRED;
  // PAIRED4 (M 3..4): A rows 0-3 hold group 2l of activation rows 0-3, rows 4-7 group 2l+1 (rows
  // past M repeat row M - 1, their D rows are dropped), so D rows 0-3 (lanes 0-15) accumulate
  // group 2l and D rows 4-7 (lanes 16-31, hB) group 2l+1; A rows 8-15 are unused
  constexpr bool PAIRED4 = MC == 4 && IMQ_LINE_PAIRED4;
  const bool hB = ar == 1;
  const uint16_t* xa = PAIRED ? xw + (c < 2 * M ? c % M : 0) * xrow + 32 * ar + (c >= M && c < 2 * M ? 128 : 0)
                     : PAIRED4 ? xw + ((c & 3) < M ? (c & 3) : M - 1) * xrow + 32 * ar + ((c & 4) ? 128 : 0)
                               : xw + (c < M ? c : M - 1) * xrow + 32 * ar;
  const uint32_t* sc_c = szl + c * DPR;
  const uint32_t* sc_x = szl + (c ^ 8) * DPR;
  const uint32_t* zr_c = szl + 16 * DPR + c * DPR;
  const uint32_t* zr_x = szl + 16 * DPR + (c ^ 8) * DPR;
  auto val = [&](const uint32_t* p, int g) -> float {   // group g (0 .. 2*S2) of a staged row
    if constexpr (VB == 4) return round_bf16_hw(__uint_as_float(p[g]));
    else return raw_to_bf16_f32<SDT>((g & 1) ? (p[g >> 1] >> 16) : (p[g >> 1] & 0xffffu));
  };
  float y0[4] = {0.f, 0.f, 0.f, 0.f}, y1[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < S2; ++i) {
    const bool v = ls0 + i < KL;
    // PAIRED4 lanes read the sums of their own group's rows 0-3 (xs1 unused)
    const f32x4_t xs0 = PAIRED4 ? *(const f32x4_t*)(xs + (2 * i + (hB ? 1 : 0)) * 16)
                                : *(const f32x4_t*)(xs + (2 * i) * 16 + 4 * ar);
    const f32x4_t xs1 = PAIRED4 ? xs0 : *(const f32x4_t*)(xs + (2 * i + 1) * 16 + 4 * ar);
    bf16x8_t A0[4], A1[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      A0[k] = *(const bf16x8_t*)(xa + i * kLine + 8 * k);
      if constexpr (!PAIRED && !PAIRED4) A1[k] = *(const bf16x8_t*)(xa + i * kLine + 128 + 8 * k);
    }
    // read unconditionally (the staged strip covers every i), then select: a conditional read
    // becomes a branch with an LDS round trip inside each line-step
    float s0 = val(sc_c, 2 * i), s1 = val(sc_x, 2 * i + 1);
    s0 = v ? s0 : 0.f;
    s1 = v ? s1 : 0.f;
    const float cz0 = -(128.f + val(zr_c, 2 * i)) * s0;
    const float cz1 = -(128.f + val(zr_x, 2 * i + 1)) * s1;
    const u32x4_t w0 = wb[2 * i], w1 = wb[2 * i + 1];
    if constexpr (PAIRED) {
      // A rows [0, M) hold group 2l, rows [M, 2M) group 2l+1, so each full-line load feeds its
      // MFMAs as loaded: column c < 8 of load L0 (row c, group 2l) meets D rows [0, M), column
      // c >= 8 (row c ^ 8, group 2l+1) D rows [M, 2M); L1 the other way round
      f32x4_t a0 = {0.f, 0.f, 0.f, 0.f}, a1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        a0 = mfma16x16x32(A0[k], unpack_nib8_bf16(w0[k], magic), a0);
        a1 = mfma16x16x32(A0[k], unpack_nib8_bf16(w1[k], magic), a1);
      }
#pragma unroll
      for (int r = 0; r < RC; ++r) {
        const float accA = lo8 ? a0[r] : a1[r];            // row c, group 2l
        const float accB = lo8 ? a1[MC + r] : a0[MC + r];  // row c ^ 8, group 2l+1
        y0[r] = fmaf(cz0, xs0[r], y0[r]);
        y1[r] = fmaf(cz1, xs1[r], y1[r]);
        y0[r] = fmaf(s0, accA, y0[r]);
        y1[r] = fmaf(s1, accB, y1[r]);
      }
    } else if constexpr (PAIRED4) {
      // lanes 0-15: D rows 0-3 of column c < 8 of L0 / c >= 8 of L1 are group 2l of row c; lanes
      // 16-31: D rows 4-7 of column c >= 8 of L0 / c < 8 of L1 are group 2l+1 of row c ^ 8
      f32x4_t a0 = {0.f, 0.f, 0.f, 0.f}, a1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        a0 = mfma16x16x32(A0[k], unpack_nib8_bf16(w0[k], magic), a0);
        a1 = mfma16x16x32(A0[k], unpack_nib8_bf16(w1[k], magic), a1);
      }
      const bool pick0 = lo8 != hB;
      const float sl = hB ? s1 : s0, czl = hB ? cz1 : cz0;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        y0[r] = fmaf(czl, xs0[r], y0[r]);
        y0[r] = fmaf(sl, pick0 ? a0[r] : a1[r], y0[r]);
      }
    } else {
      u32x4_t gA, gB;
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        gA[d] = lo8 ? w0[d] : w1[d];
        gB[d] = lo8 ? w1[d] : w0[d];
      }
      f32x4_t acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        acc0 = mfma16x16x32(A0[k], unpack_nib8_bf16(gA[k], magic), acc0);
        acc1 = mfma16x16x32(A1[k], unpack_nib8_bf16(gB[k], magic), acc1);
      }
#pragma unroll
      for (int r = 0; r < RC; ++r) {
        y0[r] = fmaf(cz0, xs0[r], y0[r]);
        y1[r] = fmaf(cz1, xs1[r], y1[r]);
        y0[r] = fmaf(s0, acc0[r], y0[r]);
        y1[r] = fmaf(s1, acc1[r], y1[r]);
      }
    }
  }
  // D row m = 4*ar + r; rows m < M <= 4 live in lanes ar == 0 (PAIRED4: their group 2l+1 parts
  // in lanes 16-31, brought over by a lane-xor-16 swizzle)
  float* rb = red + wave * (RC * 16);
#pragma unroll
  for (int r = 0; r < RC; ++r) {
    float v;
    if constexpr (PAIRED4)
      v = y0[r] + __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(row_swap8(y0[r])), 0x401F));
    else
      v = y0[r] + row_swap8(y1[r]);
    if (ar == 0) rb[r * 16 + c] = v;
  }
  lds_barrier();
  for (int e = threadIdx.x; e < 16 * M; e += blockDim.x) {
    const int m = e >> 4, n = e & 15;
    float sum = 0.f;
    for (int w = 0; w < W; ++w) sum += red[w * (RC * 16) + m * 16 + n];
    if (n <= rlast) a.y[(int64_t)m * a.sym + row0 + n] = (uint16_t)f32_to_bf16_bits(sum);
  }
}

// ---------------------------------------------------------------------------------------------
// int4 decode kernel for 4 < M <= 16 (G = 128): K split across workgroups.
//
// At M = 16 the activations of a whole row (M * K_pad * 2 bytes: 128 KB at K = 4096, 448 KB at
// K = 14336) no longer fit a workgroup's LDS next to enough waves, and a 16-row tile per
// workgroup would restage them once per 16 weight rows (4x the weight bytes through L2). Here a
// workgroup owns NW row tiles (16 * NW rows) and one split of S2 line-steps (S2 * 256 codes):
//   * its activations chunk x[0:M, split] (M x S2*256 bf16) is staged once in LDS, permuted to
//     the unpack order with per-group row sums, and shared by the NW waves;
//   * wave w streams rows [16 w, 16 w + 16) of the tile over the split exactly like the line
//     kernel (two full-line loads per line-step, MFMA 16x16x32 with the +128 bias fold), so every
//     packed byte is read once;
//   * D registers hold all 16 activation rows (m = 4 * (lane / 16) + r), and each wave writes its
//     fp32 partial y[m, n] of this split to part[split][m][n]; no cross-wave reduction.
// splitk_rows_reduce_kernel then sums the splits in order (deterministic) into bf16 y.
// ---------------------------------------------------------------------------------------------
IMQ_HOST_DEV inline int ksplit_lds(int M, int S2, int NW, int vb) {
  return M * (S2 * kLine + 8) * 2 + 2 * S2 * 16 * 4 + NW * 2 * 16 * (S2 * vb / 2) * 4;
}

template <int S2, int MC, int SDT, int NW>
__global__ __launch_bounds__(64 * NW) void w4_ksplit_kernel(SkinnyArgs a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  constexpr int VB = (SDT == IMQ_DT_FP32) ? 4 : 2;   // bytes per scale / zero value
  constexpr int DPR = S2 * VB / 2;                   // dwords per row per array (2*S2 values)
  constexpr int NT = 64 * NW;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int c = lane & 15, ar = lane >> 4;
  const bool lo8 = c < 8;
  const int M = a.M;
  const int KL = a.Kpad / kLine;
  const int RB = (a.N + 16 * NW - 1) / (16 * NW);
  const int split = blockIdx.x / RB;
  const int rb = blockIdx.x - split * RB;
  const int ls0 = split * S2;                        // first line-step of this split
  const int row0 = (rb * NW + wave) * 16;
  const bool tile_ok = row0 < a.N;                   // a partial last row block has idle waves
  const int rowa = tile_ok ? row0 : 0;               // addressing base (any valid rows when idle)
  const int rlast = a.N - 1 - rowa;                  // last valid row within the tile

  const int xrow = S2 * kLine + 8;
  uint16_t* xw = (uint16_t*)smem;                                  // [M][xrow] permuted x
  float* xs = (float*)(smem + (size_t)M * xrow * 2);               // [2*S2 groups][16 rows]
  uint32_t* szl = (uint32_t*)(xs + 2 * S2 * 16) + wave * (2 * 16 * DPR);   // this wave's s/z

  // 1) x chunk: M rows x 32*S2 16-byte blocks, spread over the workgroup (clamped into the row)
  constexpr int XB = 32 * S2;
  constexpr int XU = (MC * XB + NT - 1) / NT;
  const int xtot = M * XB;
  const uint16_t* xbase = a.x + (int64_t)ls0 * kLine;
  const int xlim = a.Kpad - ls0 * kLine - 8;         // last valid block start in the split
  u32x4_t xv[XU];
#pragma unroll
  for (int u = 0; u < XU; ++u) {
    int idx = threadIdx.x + NT * u;
    idx = idx < xtot ? idx : xtot - 1;
    const int m = idx / XB, b = idx - m * XB;
    int kb = 8 * b;
    kb = kb < xlim ? kb : xlim;
    xv[u] = *(const u32x4_t*)(xbase + m * (int)a.sxm + kb);
  }
  // 2) scale / zero words of groups [2*ls0, 2*ls0 + 2*S2) of this wave's 16 rows
  constexpr int ZU = (32 * DPR + 63) / 64;
  const int ngd = a.Kpad / 128 * VB / 4;             // dwords per row holding real groups
  const unsigned char* sbase = (const unsigned char*)a.sc + (int64_t)rowa * a.ssn * VB;
  const unsigned char* zbase = (const unsigned char*)a.zr + (int64_t)rowa * a.szn * VB;
  uint32_t zv[ZU];
#pragma unroll
  for (int u = 0; u < ZU; ++u) {
    int d = lane + 64 * u;
    d = d < 32 * DPR ? d : 32 * DPR - 1;
    const int arr = d / (16 * DPR);
    const int rem = d - arr * (16 * DPR);
    int r = rem / DPR;
    const int dw = rem - r * DPR;
    r = r < rlast ? r : rlast;
    int gd = ls0 * (VB / 2) + dw;
    gd = gd < ngd ? gd : ngd - 1;
    const unsigned char* p = arr ? zbase + r * (int)a.szn * VB : sbase + r * (int)a.ssn * VB;
    zv[u] = *(const uint32_t*)(p + 4 * gd);
  }
  // 3) weights: per line-step one full-line load for rows 0-7 and one for rows 8-15
  const uint8_t* qt = a.q + (int64_t)rowa * a.sqn;
  const uint8_t* q0;
  const uint8_t* q1;
  int lst;
  line_bases(a, qt, lane, rlast, q0, q1, lst);
  u32x4_t wb[2 * S2];
#pragma unroll
  for (int i = 0; i < S2; ++i) {
    int l = ls0 + i;
    l = l < KL ? l : KL - 1;
    wb[2 * i] = __builtin_nontemporal_load((const u32x4_t*)(q0 + lst * l));
    wb[2 * i + 1] = __builtin_nontemporal_load((const u32x4_t*)(q1 + lst * l));
  }
  // 4) stage x (permuted) with per-group row sums, and this wave's scale / zero words
#pragma unroll
  for (int u = 0; u < XU; ++u) {
    const int idx = threadIdx.x + NT * u;
    const bool ok = idx < xtot;
    const int m = (ok ? idx : 0) / XB, b = (ok ? idx : 0) - m * XB;
    float sum = bf16x8_sum(xv[u]);
    // the 16 blocks of one group are 16 consecutive idx (XB and NT are multiples of 16)
    sum = row_sum16(sum);
    if (ok) {
      *(u32x4_t*)(xw + m * xrow + 8 * b) = permute_x8(xv[u]);
      if ((b & 15) == 0) xs[(b >> 4) * 16 + m] = sum;
    }
  }
#pragma unroll
  for (int u = 0; u < ZU; ++u) {
    const int d = lane + 64 * u;
    if (d < 32 * DPR) szl[d] = zv[u];
  }
  lds_barrier();   // x and its sums are shared by the waves; weights stay in flight

  const uint32_t magic = magic_bf16_128x2();
  const uint16_t* xa = xw + (c < M ? c : M - 1) * xrow + 32 * ar;   // A rows m >= M repeat M-1
  const uint32_t* sc_c = szl + c * DPR;
  const uint32_t* sc_x = szl + (c ^ 8) * DPR;
  const uint32_t* zr_c = szl + 16 * DPR + c * DPR;
  const uint32_t* zr_x = szl + 16 * DPR + (c ^ 8) * DPR;
  auto val = [&](const uint32_t* p, int g) -> float {   // group g (0 .. 2*S2) of a staged row
    if constexpr (VB == 4) return round_bf16_hw(__uint_as_float(p[g]));
    else return raw_to_bf16_f32<SDT>((g & 1) ? (p[g >> 1] >> 16) : (p[g >> 1] & 0xffffu));
  };
  float y0[4] = {0.f, 0.f, 0.f, 0.f}, y1[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < S2; ++i) {
    const bool v = ls0 + i < KL;
    const f32x4_t xs0 = *(const f32x4_t*)(xs + (2 * i) * 16 + 4 * ar);
    const f32x4_t xs1 = *(const f32x4_t*)(xs + (2 * i + 1) * 16 + 4 * ar);
    bf16x8_t A0[4], A1[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      A0[k] = *(const bf16x8_t*)(xa + i * kLine + 8 * k);
      A1[k] = *(const bf16x8_t*)(xa + i * kLine + 128 + 8 * k);
    }
    float s0 = val(sc_c, 2 * i), s1 = val(sc_x, 2 * i + 1);   // read, then select
    s0 = v ? s0 : 0.f;
    s1 = v ? s1 : 0.f;
    const float cz0 = -(128.f + val(zr_c, 2 * i)) * s0;
    const float cz1 = -(128.f + val(zr_x, 2 * i + 1)) * s1;
    const u32x4_t w0 = wb[2 * i], w1 = wb[2 * i + 1];
    u32x4_t gA, gB;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      gA[d] = lo8 ? w0[d] : w1[d];
      gB[d] = lo8 ? w1[d] : w0[d];
    }
    f32x4_t acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      acc0 = mfma16x16x32(A0[k], unpack_nib8_bf16(gA[k], magic), acc0);
      acc1 = mfma16x16x32(A1[k], unpack_nib8_bf16(gB[k], magic), acc1);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      y0[r] = fmaf(cz0, xs0[r], y0[r]);
      y1[r] = fmaf(cz1, xs1[r], y1[r]);
      y0[r] = fmaf(s0, acc0[r], y0[r]);
      y1[r] = fmaf(s1, acc1[r], y1[r]);
    }
  }
  // lane (c, ar) holds rows m = 4*ar + r of output column row0 + c (group 2i+1 of row c came
  // from lane c ^ 8)
  float* pbase = a.part + (size_t)split * M * a.N + row0 + c;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const float v = y0[r] + row_swap8(y1[r]);
    const int m = 4 * ar + r;
    if (tile_ok && m < M && c <= rlast) pbase[(size_t)m * a.N] = v;
  }
}

// y[m, n] = bf16(sum over splits s of part[s][m][n]), summed in split order; 4 columns per thread
// (N % 4 == 0: one 16-byte load per split). The loads of up to 16 splits are issued before any is
// consumed: the partials were just written by another kernel and sit in the memory-side cache.
__global__ __launch_bounds__(256) void splitk_rows_reduce_kernel(const float* __restrict__ part, int splits,
                                                                 int M, int N, uint16_t* __restrict__ y,
                                                                 int64_t sym) {
  const int n4 = N / 4;
  const int t = blockIdx.x * 256 + threadIdx.x;
  if (t >= M * n4) return;
  const int m = t / n4;
  const int n = 4 * (t - m * n4);
  const size_t sstride = (size_t)M * N;
  const float* src = part + (size_t)m * N + n;
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
  for (int s0 = 0; s0 < splits; s0 += 16) {
    f32x4_t v[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int sp = s0 + j < splits ? s0 + j : splits - 1;
      v[j] = *(const f32x4_t*)(src + sp * sstride);
    }
#pragma unroll
    for (int j = 0; j < 16; ++j)
      if (s0 + j < splits) acc += v[j];
  }
  u32x2_t o;
  o[0] = cvt_pk_bf16(acc[0], acc[1]);
  o[1] = cvt_pk_bf16(acc[2], acc[3]);
  *(u32x2_t*)(y + (int64_t)m * sym + n) = o;
}

// ---------------------------------------------------------------------------------------------
// int4 decode kernel for 4 < M <= 16 (G = 128) with K split across the waves of one workgroup.
//
// Wave w of the NW waves owns line-steps [w R, w R + R) of every row (K_pad = NW R 256). Its slice
// of the activations is read once, one full row per load, arranged through wave-private LDS
// (unpack order, per-group row sums) and kept in registers as the 16 A-operand rows (zero beyond
// M) with the group sums in the D layout; it serves every row tile the workgroup streams (a
// persistent grid over the N / 16 tiles, one workgroup per CU). Per tile a wave reads 16 rows x
// R line-steps of packed weights with two full-line loads per line-step, PD tiles ahead, plus one
// scale and one zero dword (two groups) per line-step and row. The per-group math is the K-split
// kernel's: B = 128 + code, y += s acc - s (128 + z) sum(x). The waves' 16 x 16 fp32 partials meet
// in LDS (double-buffered, one barrier per tile) and are summed in wave order (deterministic).
// The bf16 results wait in LDS and are stored after the last tile (or every kWsYB tiles): a store
// in flight would make each tile's wait for its weights drain every outstanding load (loads and
// stores share one counter). No workspace and no second launch: no partial leaves the workgroup.
// ---------------------------------------------------------------------------------------------
constexpr int kWsYB = 8;   // tiles of bf16 results held in LDS between stores

IMQ_HOST_DEV inline int wsplit_lds(int R, int NW) {
  return NW * (16 * (R * kLine + 8) * 2 + 2 * R * 16 * 4) + 2 * NW * 256 * 4 + kWsYB * 256 * 2;
}

// TL: weights in the line-tiled layout (a separate instantiation: the address selection sits in
// the per-tile prefetch of the persistent loop)
template <int R, int SDT, int NW, int PD, bool TL>
__global__ __launch_bounds__(64 * NW) void w4_wsplit_kernel(SkinnyArgs a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  constexpr int XROW = R * kLine + 8;                // staged row stride (bf16 elements)
  constexpr int CPR = R * 32;                        // 16-byte chunks per row of the slice
  constexpr int XU = 16 * CPR / 64;                  // row loads per lane (all 16 rows)
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int c = lane & 15, ar = lane >> 4;
  const bool lo8 = c < 8;
  const int M = a.M;
  const int T = (a.N + 15) / 16;
  const int ls0 = wave * R;                          // first line-step of this wave
  uint16_t* xw = (uint16_t*)(smem + (size_t)wave * (16 * XROW * 2 + 2 * R * 16 * 4));
  float* xsum = (float*)(xw + 16 * XROW);            // [2 R groups][16 rows]
  float (*red)[NW][256] = (float (*)[NW][256])(smem + (size_t)NW * (16 * XROW * 2 + 2 * R * 16 * 4));
  uint16_t (*ybuf)[256] = (uint16_t (*)[256])((unsigned char*)red + 2 * NW * 256 * 4);

  // 1) the activation slice, one row (or two) per load: chunk ch of row m is x[m, 256 ls0 + 8 ch).
  //    Every load is unconditional (rows past M read row M - 1 and are not staged): a load under a
  //    branch makes the compiler wait for all outstanding loads where the paths join.
  u32x4_t xv[XU];
#pragma unroll
  for (int u = 0; u < XU; ++u) {
    const int idx = 64 * u + lane;
    const int m = idx / CPR, ch = idx - m * CPR;
    xv[u] = *(const u32x4_t*)(a.x + (int64_t)(m < M ? m : M - 1) * a.sxm + ls0 * kLine + 8 * ch);
  }

  // 2) per tile: weights (two full-line loads per line-step) and scale / zero dwords of row c
  struct Tile {
    u32x4_t w[2 * R];
    uint32_t sw[R * (SDT == IMQ_DT_FP32 ? 2 : 1)], zw[R * (SDT == IMQ_DT_FP32 ? 2 : 1)];
  };
  // A tile past the workgroup's last (t > tlast: the prefetch runs PD tiles ahead) loads one
  // 16-byte word of the operands for every lane and row -- a single request per load, no branch.
  auto load_tile = [&](int t, Tile& tl, int tlast) {
    const bool live = t <= tlast;
    const int row0 = t * 16;
    const int rlast = a.N - 1 - row0;
    const uint8_t* q0;
    const uint8_t* q1;
    int ist;
    if constexpr (TL) {   // line-tiled: lane l reads bytes 16 l of each half of the 2 KiB block
      const int64_t qo = (int64_t)row0 * a.sqn + ls0 * 2048 + 16 * lane;
      q0 = a.q + (live ? qo : 0);
      q1 = a.q + (live ? qo + 1024 : 0);
      ist = live ? 2048 : 0;
    } else {
      const int rr0 = (c & 7) < rlast ? (c & 7) : rlast;
      const int rr1 = 8 + (c & 7) < rlast ? 8 + (c & 7) : rlast;
      const int64_t qo = (int64_t)row0 * a.sqn + ls0 * 128 + 16 * ar;
      q0 = a.q + (live ? qo + rr0 * a.sqn + (lo8 ? 0 : 64) : 0);
      q1 = a.q + (live ? qo + rr1 * a.sqn + (lo8 ? 64 : 0) : 0);
      ist = live ? 128 : 0;
    }
#pragma unroll
    for (int i = 0; i < R; ++i) {
      tl.w[2 * i] = __builtin_nontemporal_load((const u32x4_t*)(q0 + ist * i));
      tl.w[2 * i + 1] = __builtin_nontemporal_load((const u32x4_t*)(q1 + ist * i));
    }
    const int rc = live ? row0 + (c < rlast ? c : rlast) : 0;
    const int g0 = live ? 2 * ls0 : 0;
    if constexpr (SDT == IMQ_DT_FP32) {
      const uint32_t* sp = (const uint32_t*)a.sc + (int64_t)rc * a.ssn + g0;
      const uint32_t* zp = (const uint32_t*)a.zr + (int64_t)rc * a.szn + g0;
#pragma unroll
      for (int j = 0; j < 2 * R; ++j) {
        tl.sw[j] = sp[j];
        tl.zw[j] = zp[j];
      }
    } else {
      const uint32_t* sp = (const uint32_t*)((const uint16_t*)a.sc + (int64_t)rc * a.ssn + g0);
      const uint32_t* zp = (const uint32_t*)((const uint16_t*)a.zr + (int64_t)rc * a.szn + g0);
#pragma unroll
      for (int j = 0; j < R; ++j) {
        tl.sw[j] = sp[j];
        tl.zw[j] = zp[j];
      }
    }
  };
  // scale / zero of group 2 i (row c) and 2 i + 1 (row c ^ 8, from lane c ^ 8)
  auto sz = [&](const Tile& tl, int i, float& s0, float& s1, float& z0, float& z1) {
    if constexpr (SDT == IMQ_DT_FP32) {
      s0 = round_bf16_hw(__uint_as_float(tl.sw[2 * i]));
      z0 = round_bf16_hw(__uint_as_float(tl.zw[2 * i]));
      s1 = round_bf16_hw(__uint_as_float(dpp_row_ror<8>(tl.sw[2 * i + 1])));
      z1 = round_bf16_hw(__uint_as_float(dpp_row_ror<8>(tl.zw[2 * i + 1])));
    } else {
      const uint32_t sx = dpp_row_ror<8>(tl.sw[i]), zx = dpp_row_ror<8>(tl.zw[i]);
      s0 = raw_to_bf16_f32<SDT>(tl.sw[i] & 0xffffu);
      z0 = raw_to_bf16_f32<SDT>(tl.zw[i] & 0xffffu);
      s1 = raw_to_bf16_f32<SDT>(sx >> 16);
      z1 = raw_to_bf16_f32<SDT>(zx >> 16);
    }
  };
  // the first PD tiles' loads, in flight while the activations are arranged
  const int G = gridDim.x;
  const int tlast = blockIdx.x + (T - 1 - (int)blockIdx.x) / G * G;
  Tile ring[PD + 1];
  int t = blockIdx.x;
#pragma unroll
  for (int j = 0; j < PD; ++j) load_tile(t + j * G, ring[j], tlast);

  // 3) stage the slice permuted to the unpack order with per-group row sums (16 consecutive lanes
  //    hold one group of one row), then read the A operands and the sums in the D layout
#pragma unroll
  for (int u = 0; u < XU; ++u) {
    const int idx = 64 * u + lane;
    const int m = idx / CPR, ch = idx - m * CPR;
    float sum = bf16x8_sum(xv[u]);
    sum = row_sum16(sum);
    if (m < M) {
      *(u32x4_t*)(xw + m * XROW + 8 * ch) = permute_x8(xv[u]);
      if ((ch & 15) == 0) xsum[(ch >> 4) * 16 + m] = sum;
    }
  }
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   // wave-private: the wave's own writes first
  bf16x8_t A0[R][4], A1[R][4];
  f32x4_t xs0[R], xs1[R];
  {
    const uint16_t* xa = xw + (c < M ? c : 0) * XROW + 32 * ar;
#pragma unroll
    for (int i = 0; i < R; ++i) {
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        A0[i][k] = *(const bf16x8_t*)(xa + i * kLine + 8 * k);
        A1[i][k] = *(const bf16x8_t*)(xa + i * kLine + 128 + 8 * k);
        if (c >= M) {
          A0[i][k] = bf16x8_t{};
          A1[i][k] = bf16x8_t{};
        }
      }
      xs0[i] = *(const f32x4_t*)(xsum + (2 * i) * 16 + 4 * ar);
      xs1[i] = *(const f32x4_t*)(xsum + (2 * i + 1) * 16 + 4 * ar);
    }
  }

  const uint32_t magic = magic_bf16_128x2();
  auto compute = [&](const Tile& tl, int buf, int slot) {
    float y0[4] = {0.f, 0.f, 0.f, 0.f}, y1[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < R; ++i) {
      float s0, s1, z0, z1;
      sz(tl, i, s0, s1, z0, z1);
      const float cz0 = -(128.f + z0) * s0;
      const float cz1 = -(128.f + z1) * s1;
      const u32x4_t w0 = tl.w[2 * i], w1 = tl.w[2 * i + 1];
      u32x4_t gA, gB;
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        gA[d] = lo8 ? w0[d] : w1[d];
        gB[d] = lo8 ? w1[d] : w0[d];
      }
      f32x4_t acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        acc0 = mfma16x16x32(A0[i][k], unpack_nib8_bf16(gA[k], magic), acc0);
        acc1 = mfma16x16x32(A1[i][k], unpack_nib8_bf16(gB[k], magic), acc1);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        y0[r] = fmaf(cz0, xs0[i][r], y0[r]);
        y1[r] = fmaf(cz1, xs1[i][r], y1[r]);
        y0[r] = fmaf(s0, acc0[r], y0[r]);
        y1[r] = fmaf(s1, acc1[r], y1[r]);
      }
    }
    float* rw = red[buf][wave];
#pragma unroll
    for (int r = 0; r < 4; ++r) rw[(4 * ar + r) * 16 + c] = y0[r] + row_swap8(y1[r]);
    lds_barrier();
    const int e = threadIdx.x;
    if (e < 256) {
      float sum = 0.f;
#pragma unroll
      for (int w = 0; w < NW; ++w) sum += red[buf][w][e];
      ybuf[slot][e] = (uint16_t)f32_to_bf16_bits(sum);
    }
  };
  // thread e < 256 stores its own buffered results (element (e / 16, e % 16) of each tile)
  auto flush = [&](int k0, int k1) {
    const int e = threadIdx.x;
    const int m = e >> 4, col = e & 15;
    if (e < 256 && m < M) {
      for (int k = k0; k < k1; ++k) {
        const int row = (blockIdx.x + k * G) * 16 + col;
        if (row < a.N) a.y[(int64_t)m * a.sym + row] = ybuf[k % kWsYB][e];
      }
    }
  };

  // 4) tile loop, PD tiles of loads ahead of the one computed, in a ring of PD + 1 register sets
  int buf = 0, k = 0, kf = 0;
  for (; t < T; t += (PD + 1) * G) {
#pragma unroll
    for (int j = 0; j <= PD; ++j) {
      const int tj = t + j * G;
      if (tj >= T) break;
      load_tile(tj + PD * G, ring[(j + PD) % (PD + 1)], tlast);
      compute(ring[j], buf, k % kWsYB);
      buf ^= 1;
      ++k;
      if (k - kf == kWsYB || tj + G >= T) {
        flush(kf, k);
        kf = k;
      }
    }
  }
}

// ---------------------------------------------------------------------------------------------
// int2 decode kernel (M <= 16). A K-step is one 64-code group: 16 bytes of each packed row.
// Lane (row nl, quarter jl) works on dword jl = codes [16*jl, 16*jl+16) of each step, which
// feeds two v_mfma_f32_16x16x32_bf16: MFMA h takes codes {4h..4h+3} and {4h+8..4h+11} of each
// lane, so every MFMA's 32 K positions lie inside one group and the group's scale/zero apply to
// its result exactly (y += s*acc - s*(128+z)*sum(x)). The codes arrive as 16-byte loads of four
// whole steps (a 64-byte line per row) redistributed by a cross-lane 4x4 transpose. Activations
// are staged in LDS in the matching order (permute_x16); K is staged in chunks when M * K_pad
// does not fit.
// ---------------------------------------------------------------------------------------------
constexpr int kStep2 = 64;

// Two 16-byte blocks lo (elements 0..7), hi (8..15) -> [0,8,1,9,2,10,3,11 | 4,12,5,13,6,14,7,15].
IMQ_DEV void permute_x16(const u32x4_t& lo, const u32x4_t& hi, u32x4_t& o0, u32x4_t& o1) {
  o0[0] = perm_b32(hi[0], lo[0], 0x05040100u);
  o0[1] = perm_b32(hi[0], lo[0], 0x07060302u);
  o0[2] = perm_b32(hi[1], lo[1], 0x05040100u);
  o0[3] = perm_b32(hi[1], lo[1], 0x07060302u);
  o1[0] = perm_b32(hi[2], lo[2], 0x05040100u);
  o1[1] = perm_b32(hi[2], lo[2], 0x07060302u);
  o1[2] = perm_b32(hi[3], lo[3], 0x05040100u);
  o1[3] = perm_b32(hi[3], lo[3], 0x07060302u);
}

// 4x4 transpose of dwords across the four 16-lane rows: on entry register k of lane row j holds
// element (k, j); on exit it holds element (j, k). Two v_permlane32_swap (registers k < 2, rows
// 2-3 <-> registers k+2, rows 0-1) then two v_permlane16_swap (even registers, odd rows <->
// odd registers, even rows).
IMQ_DEV void transpose4_lanerows(uint32_t (&d)[4]) {
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const auto r = __builtin_amdgcn_permlane32_swap(d[k], d[k + 2], false, false);
    d[k] = r[0];
    d[k + 2] = r[1];
  }
#pragma unroll
  for (int k = 0; k < 4; k += 2) {
    const auto r = __builtin_amdgcn_permlane16_swap(d[k], d[k + 1], false, false);
    d[k] = r[0];
    d[k + 1] = r[1];
  }
}

// 16 crumbs of one dword -> the 8 bf16 (128 + code) of MFMA half h, in the order
// [c(4h), c(4h+8), c(4h+1), c(4h+9), c(4h+2), c(4h+10), c(4h+3), c(4h+11)].
IMQ_DEV bf16x8_t unpack_crumb8_bf16(uint32_t w, int h, uint32_t magic) {
  u32x4_t r;
#pragma unroll
  for (int k = 0; k < 4; ++k) r[k] = ((w >> (2 * (4 * h + k))) & 0x00030003u) | magic;
  return __builtin_bit_cast(bf16x8_t, r);
}

template <int S, int MC, int SDT, int ZDT, bool STRIP, int MAXW>
__global__ __launch_bounds__(64 * MAXW) void w2_skinny_kernel(SkinnyArgs a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int W = blockDim.x >> 6;
  const int nl = lane & 15;
  const int jl = lane >> 4;
  constexpr int RC = (MC < 4) ? MC : 4;
  constexpr int SZB = (SDT == IMQ_DT_FP32) ? 4 : 2;
  constexpr int ZZB = (ZDT == IMQ_DT_FP32) ? 4 : 2;
  constexpr int SW = STRIP ? (S * SZB + 3) / 4 : 1;
  constexpr int ZW = STRIP ? (S * ZZB + 3) / 4 : 1;

  const int KS = a.Kpad / kStep2;
  const int CS = a.chunk_steps;                      // steps staged per chunk: KS, or a multiple of S
  const int nchunks = (KS + CS - 1) / CS;
  const int xls = CS * kStep2 + kXPad;
  uint16_t* xl = (uint16_t*)smem;                                    // [M][xls]
  float* xs = (float*)(smem + (size_t)a.M * xls * 2);                // [CS][16]
  float* red = xs + (size_t)CS * 16;                                 // [2][W][256]
  const int gsh = 31 - __builtin_clz(a.G / kStep2);                  // steps per group = 2^gsh
  const int NT = (a.N + 15) / 16;
  const int64_t ssg_b = a.ssg * SZB, szg_b = a.szg * ZZB;

  // stage steps [c0, c1): each thread handles 16-element pairs; four consecutive pairs make a
  // step, whose row sum is reduced across those four lanes
  auto stage = [&](int c0, int c1) {
    for (int idx = threadIdx.x; idx < 16 * CS; idx += blockDim.x) xs[idx] = 0.f;
    lds_barrier();
    const int npair = (c1 - c0) * 4;
    const int total = a.M * npair;                   // a multiple of 4
    for (int base = 0; base < total; base += blockDim.x) {
      const int idx = base + threadIdx.x;
      const bool valid = idx < total;
      const int id = valid ? idx : total - 1;
      const int m = id / npair;
      const int pr = id - m * npair;
      const uint16_t* src = a.x + (int64_t)m * a.sxm + (int64_t)c0 * kStep2 + 16 * pr;
      const u32x4_t lo = *(const u32x4_t*)src;
      const u32x4_t hi = *(const u32x4_t*)(src + 8);
      float sum = bf16x8_sum(lo) + bf16x8_sum(hi);
      sum = quad_sum4(sum);
      if (valid) {
        u32x4_t o0, o1;
        permute_x16(lo, hi, o0, o1);
        *(u32x4_t*)(xl + m * xls + 16 * pr) = o0;
        *(u32x4_t*)(xl + m * xls + 16 * pr + 8) = o1;
        if ((pr & 3) == 0) xs[(pr >> 2) * 16 + m] = sum;
      }
    }
    lds_barrier();
  };

  const uint32_t magic = magic_bf16_128x2();
  const uint16_t* xlane = xl + (nl < a.M ? nl : a.M - 1) * xls + 16 * jl;
  const float* xslane = xs + 4 * jl;
  int buf = 0;
  bool staged = false;

  for (int tile = blockIdx.x; tile < NT; tile += gridDim.x) {
    int row = tile * 16 + nl;
    row = row < a.N ? row : a.N - 1;
    const uint8_t* qrow = a.q + (int64_t)row * a.sqn + 16 * jl;
    const unsigned char* srow = (const unsigned char*)a.sc + (int64_t)row * a.ssn * SZB;
    const unsigned char* zrow = (const unsigned char*)a.zr + (int64_t)row * a.szn * ZZB;
    float yacc[4] = {0.f, 0.f, 0.f, 0.f};

    for (int c = 0; c < nchunks; ++c) {
      const int c0 = c * CS;
      const int c1 = (c0 + CS < KS) ? c0 + CS : KS;
      if (nchunks > 1 || !staged) {
        stage(c0, c1);
        staged = true;
      }
      const int R = (c1 - c0 + W * S - 1) / (W * S);
      for (int rnd = 0; rnd < R; ++rnd) {
        const int sbase = c0 + (rnd * W + wave) * S;
        uint32_t wv[S];
        uint32_t sr[S], zr[S];
        uint32_t sst[SW], zst[ZW];
        // 16-byte loads: lane row jl reads step (sb4 + jl) whole (the four lane rows of a tile
        // row cover one 64-byte line); a 4x4 transpose across the lane rows then hands lane row
        // jl the dword jl of each of the four steps
#pragma unroll
        for (int t = 0; t < S / 4; ++t) {
          int sb4 = sbase + 4 * t;
          sb4 = sb4 <= c1 - 4 ? sb4 : c1 - 4;
          const u32x4_t v = __builtin_nontemporal_load((const u32x4_t*)(qrow + (int64_t)sb4 * 16));
#pragma unroll
          for (int k = 0; k < 4; ++k) wv[4 * t + k] = v[k];
        }
        if constexpr (STRIP) {
          const int64_t g0 = sbase < c1 ? sbase : c0;     // a strip past the chunk: any valid one
          load_strip<SW>(srow + g0 * SZB, sst);
          load_strip<ZW>(zrow + g0 * ZZB, zst);
        } else {
#pragma unroll
          for (int i = 0; i < S; ++i) {
            int st = sbase + i;
            st = st < c1 ? st : c1 - 1;
            const int64_t g = st >> gsh;
            sr[i] = load_raw<SDT>(srow + g * ssg_b, 0);
            zr[i] = load_raw<ZDT>(zrow + g * szg_b, 0);
          }
        }
#pragma unroll
        for (int t = 0; t < S / 4; ++t) {
          uint32_t d[4] = {wv[4 * t], wv[4 * t + 1], wv[4 * t + 2], wv[4 * t + 3]};
          transpose4_lanerows(d);
#pragma unroll
          for (int k = 0; k < 4; ++k) wv[4 * t + k] = d[k];
        }
        auto s_raw = [&](int i) -> uint32_t {
          if constexpr (!STRIP) return sr[i];
          else if constexpr (SZB == 4) return sst[i];
          else return (i & 1) ? (sst[i >> 1] >> 16) : (sst[i >> 1] & 0xffffu);
        };
        auto z_raw = [&](int i) -> uint32_t {
          if constexpr (!STRIP) return zr[i];
          else if constexpr (ZZB == 4) return zst[i];
          else return (i & 1) ? (zst[i >> 1] >> 16) : (zst[i >> 1] & 0xffffu);
        };
#pragma unroll
        for (int i = 0; i < S; i += 2) {
          const int s0a = sbase + i, s0b = s0a + 1;
          const bool va = s0a < c1, vb = s0b < c1;
          const int la = (va ? s0a : c1 - 1) - c0;
          const int lb = (vb ? s0b : c1 - 1) - c0;
          const f32x4_t xsa = *(const f32x4_t*)(xslane + la * 16);
          const f32x4_t xsb = *(const f32x4_t*)(xslane + lb * 16);
          const bf16x8_t a0 = *(const bf16x8_t*)(xlane + la * kStep2);
          const bf16x8_t a1 = *(const bf16x8_t*)(xlane + la * kStep2 + 8);
          const bf16x8_t b0 = *(const bf16x8_t*)(xlane + lb * kStep2);
          const bf16x8_t b1 = *(const bf16x8_t*)(xlane + lb * kStep2 + 8);
          const float sca = va ? raw_to_bf16_f32<SDT>(s_raw(i)) : 0.f;
          const float scb = vb ? raw_to_bf16_f32<SDT>(s_raw(i + 1)) : 0.f;
          const float cza = -(128.f + raw_to_bf16_f32<ZDT>(z_raw(i))) * sca;
          const float czb = -(128.f + raw_to_bf16_f32<ZDT>(z_raw(i + 1))) * scb;
          f32x4_t acca = {0.f, 0.f, 0.f, 0.f}, accb = {0.f, 0.f, 0.f, 0.f};
          acca = mfma16x16x32(a0, unpack_crumb8_bf16(wv[i], 0, magic), acca);
          accb = mfma16x16x32(b0, unpack_crumb8_bf16(wv[i + 1], 0, magic), accb);
          acca = mfma16x16x32(a1, unpack_crumb8_bf16(wv[i], 1, magic), acca);
          accb = mfma16x16x32(b1, unpack_crumb8_bf16(wv[i + 1], 1, magic), accb);
#pragma unroll
          for (int q = 0; q < RC; ++q) {
            yacc[q] = fmaf(cza, xsa[q], yacc[q]);
            yacc[q] = fmaf(czb, xsb[q], yacc[q]);
            yacc[q] = fmaf(sca, acca[q], yacc[q]);
            yacc[q] = fmaf(scb, accb[q], yacc[q]);
          }
        }
      }
      if (nchunks > 1) lds_barrier();      // every wave is done with this chunk before restaging
    }

    // cross-wave reduction in a fixed order; the buffer alternates between tiles
    float* rb = red + buf * (W * 256);
#pragma unroll
    for (int q = 0; q < 4; ++q) rb[wave * 256 + (4 * jl + q) * 16 + nl] = yacc[q];
    lds_barrier();
    const int n0 = tile * 16;
    for (int e = threadIdx.x; e < 16 * a.M; e += blockDim.x) {
      const int m = e >> 4;
      const int n = e & 15;
      float sum = 0.f;
      for (int w = 0; w < W; ++w) sum += rb[w * 256 + e];
      if (n0 + n < a.N) a.y[(int64_t)m * a.sym + n0 + n] = (uint16_t)f32_to_bf16_bits(sum);
    }
    buf ^= 1;
  }
}

// ---------------------------------------------------------------------------------------------
// int2 decode line kernel (M <= 4, G = 64): the int4 line kernel's structure for 2-bit codes.
// A line-step is 128 bytes of a row = 512 codes = 8 groups. One workgroup owns a 16-row tile and
// all of K; W waves split K in S2 line-steps each and issue all of their loads up front:
//   * two 16-byte loads per line-step, each covering 8 rows x a whole 128-byte line: lane (c, ar)
//     gets group ar of row c (gA) and group 4 + ar of row c ^ 8 (gB), one group per dword set;
//   * a 4x4 cross-lane transpose (transpose4_lanerows) turns that into dword ar of each of the
//     four groups, so each MFMA pair's 64 K positions lie inside one group and the group's scale
//     and zero apply to its accumulator exactly: y += s*acc - s*(128 + z)*sum(x);
//   * activations of the wave's K range are staged in the wave's LDS (permute_x16 order) with
//     per-group row sums; scale / zero words of the 16 rows likewise.
// Rows c ^ 8 of gB are folded back with a row swap, partials reduce across waves in LDS.
// ---------------------------------------------------------------------------------------------
constexpr int kLine2 = 512;   // codes per int2 line-step (128 bytes of a row, 8 groups of 64)

// Scale / zero of a wave's 16 rows over NGW groups, staged in LDS as float pairs
// (s, -(128 + z) * s) with the bf16 rounding of s and z applied once per (row, group) instead of
// in every lane that uses them; groups past K_pad are staged as (0, 0). Row stride 2 * NGW + 2
// floats spreads the 16 rows over the LDS banks.
IMQ_HOST_DEV constexpr int sz2_row(int ngw) { return 2 * ngw + 2; }
IMQ_HOST_DEV constexpr int sz2_bytes(int ngw) { return 16 * sz2_row(ngw) * 4; }

template <int SDT, int NGW>
struct SzPairs {
  static constexpr int VB = SDT == IMQ_DT_FP32 ? 4 : 2;
  static constexpr int GPD = 4 / VB;                 // groups per dword
  static constexpr int DPR = NGW / GPD;              // dwords per row
  static constexpr int ZU = (16 * DPR + 63) / 64;    // dword pairs per lane
  uint32_t sv[ZU], zv[ZU];

  // rows [0, 16) of the tile (clamped to rlast), dwords gd0 .. gd0 + DPR (clamped below ngd)
  IMQ_DEV void load(int lane, const unsigned char* sbase, const unsigned char* zbase, int ssnb, int sznb,
                    int rlast, int gd0, int ngd) {
#pragma unroll
    for (int u = 0; u < ZU; ++u) {
      int d = lane + 64 * u;
      d = d < 16 * DPR ? d : 16 * DPR - 1;
      int r = d / DPR;
      const int dw = d - r * DPR;
      r = r < rlast ? r : rlast;
      int gd = gd0 + dw;
      gd = gd < ngd ? gd : ngd - 1;
      sv[u] = *(const uint32_t*)(sbase + r * ssnb + 4 * gd);
      zv[u] = *(const uint32_t*)(zbase + r * sznb + 4 * gd);
    }
  }
  // local groups >= gvalid lie past K_pad
  IMQ_DEV void store(int lane, float* szf, int gvalid) const {
#pragma unroll
    for (int u = 0; u < ZU; ++u) {
      const int d = lane + 64 * u;
      if (d < 16 * DPR) {
        const int r = d / DPR;
        const int dw = d - r * DPR;
#pragma unroll
        for (int e = 0; e < GPD; ++e) {
          const int g = dw * GPD + e;
          float sc, zr;
          if constexpr (VB == 4) {
            sc = round_bf16_hw(__uint_as_float(sv[u]));
            zr = round_bf16_hw(__uint_as_float(zv[u]));
          } else {
            sc = raw_to_bf16_f32<SDT>(e ? (sv[u] >> 16) : (sv[u] & 0xffffu));
            zr = raw_to_bf16_f32<SDT>(e ? (zv[u] >> 16) : (zv[u] & 0xffffu));
          }
          sc = g < gvalid ? sc : 0.f;
          f32x2_t v;
          v[0] = sc;
          v[1] = -(128.f + zr) * sc;
          *(f32x2_t*)(szf + r * sz2_row(NGW) + 2 * g) = v;
        }
      }
    }
  }
};

IMQ_HOST_DEV inline int line2_wave_lds(int M, int S2) {
  return M * (S2 * kLine2 + 8) * 2 + S2 * 8 * 16 * 4 + sz2_bytes(S2 * 8);
}

template <int S2, int MC, int SDT, int MAXW>
__global__ __launch_bounds__(64 * MAXW) void w2_line_kernel(SkinnyArgs a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  constexpr int VB = (SDT == IMQ_DT_FP32) ? 4 : 2;   // bytes per scale / zero value
  constexpr int GPL = 8;                              // groups per line-step
  constexpr int NGW = S2 * GPL;                       // groups of the wave's K range
  constexpr int RC = MC < 4 ? MC : 4;                 // D registers that can hold a real row
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int W = blockDim.x >> 6;
  const int c = lane & 15, ar = lane >> 4;
  const bool lo8 = c < 8;
  const int M = MC <= 2 ? MC : a.M;                 // MC 1 and 2 launch exactly that M
  const int KL = a.Kpad / kLine2;
  const int ls0 = wave * S2;
  const int row0 = blockIdx.x * 16;
  const int rlast = a.N - 1 - row0;

  const int xrow = S2 * kLine2 + 8;
  const int wbytes = line2_wave_lds(M, S2);
  unsigned char* wl = smem + (size_t)wave * wbytes;
  uint16_t* xw = (uint16_t*)wl;                       // [M][xrow], permute_x16 order
  float* xs = (float*)(wl + M * xrow * 2);           // [S2 * 8 groups][16 rows]
  float* szf = xs + NGW * 16;                         // [16 rows][sz2_row(NGW)]: (s, cz) pairs
  float* red = (float*)(smem + (size_t)W * wbytes);

  // 1) x: M rows x S2*32 pairs of 16 elements (two 16-byte loads each), clamped into the row
  constexpr int XP = 32 * S2;
  constexpr int XU = (MC * XP + 63) / 64;
  const int xtot = M * XP;
  const uint16_t* xbase = a.x + (int64_t)ls0 * kLine2;
  const int plim = a.Kpad - ls0 * kLine2 - 16;       // last valid pair start in the range
  u32x4_t xlo[XU], xhi[XU];
#pragma unroll
  for (int u = 0; u < XU; ++u) {
    int idx = lane + 64 * u;
    idx = idx < xtot ? idx : xtot - 1;
    const int m = idx / XP, p = idx - m * XP;
    int kb = 16 * p;
    kb = kb < plim ? kb : plim;
    const uint16_t* src = xbase + m * (int)a.sxm + kb;
    xlo[u] = *(const u32x4_t*)src;
    xhi[u] = *(const u32x4_t*)(src + 8);
  }
  // 2) scale / zero words of groups [8*ls0, 8*ls0 + 8*S2) of the 16 rows
  SzPairs<SDT, NGW> szp;
  szp.load(lane, (const unsigned char*)a.sc + (int64_t)row0 * a.ssn * VB,
           (const unsigned char*)a.zr + (int64_t)row0 * a.szn * VB, (int)a.ssn * VB, (int)a.szn * VB, rlast,
           ls0 * (GPL * VB / 4), a.Kpad / 64 * VB / 4);
  // 3) weights: per line-step one full-line load for rows 0-7 and one for rows 8-15
  const uint8_t* qt = a.q + (int64_t)row0 * a.sqn;
  const uint8_t* q0;
  const uint8_t* q1;
  int lst;
  line_bases(a, qt, lane, rlast, q0, q1, lst);
  u32x4_t wb[2 * S2];
#pragma unroll
  for (int i = 0; i < S2; ++i) {
    int l = ls0 + i;
    l = l < KL ? l : KL - 1;
    wb[2 * i] = __builtin_nontemporal_load((const u32x4_t*)(q0 + lst * l));
    wb[2 * i + 1] = __builtin_nontemporal_load((const u32x4_t*)(q1 + lst * l));
  }
  // 4) stage x (permute_x16 per pair) with per-group sums, and scale / zero words
#pragma unroll
  for (int u = 0; u < XU; ++u) {
    const int idx = lane + 64 * u;
    const bool ok = idx < xtot;
    const int m = (ok ? idx : 0) / XP, p = (ok ? idx : 0) - m * XP;
    float sum = bf16x8_sum(xlo[u]) + bf16x8_sum(xhi[u]);
    // the 4 pairs of one group are 4 consecutive idx (XP is a multiple of 4)
    sum = quad_sum4(sum);
    if (ok) {
      u32x4_t o0, o1;
      permute_x16(xlo[u], xhi[u], o0, o1);
      *(u32x4_t*)(xw + m * xrow + 16 * p) = o0;
      *(u32x4_t*)(xw + m * xrow + 16 * p + 8) = o1;
      if ((p & 3) == 0) xs[(p >> 2) * 16 + m] = sum;
    }
  }
  szp.store(lane, szf, (KL - ls0) * GPL);
  // LDS is written and read by this wave only; its LDS operations execute in order
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");

  const uint32_t magic = magic_bf16_128x2();
  const uint16_t* xa = xw + (c < M ? c : M - 1) * xrow + 16 * ar;
  const float* sz_c = szf + c * sz2_row(NGW);
  const float* sz_x = szf + (c ^ 8) * sz2_row(NGW);
  auto xsum = [&](int g) -> f32x4_t {                   // sums of D rows 4*ar .. 4*ar + RC - 1
    f32x4_t v = {0.f, 0.f, 0.f, 0.f};
    const float* p = xs + g * 16 + 4 * ar;
    if constexpr (RC == 1) v[0] = p[0];
    else if constexpr (RC == 2) {
      const f32x2_t t = *(const f32x2_t*)p;
      v[0] = t[0];
      v[1] = t[1];
    } else v = *(const f32x4_t*)p;
    return v;
  };
  float y0[4] = {0.f, 0.f, 0.f, 0.f}, y1[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < S2; ++i) {
    const u32x4_t w0 = wb[2 * i], w1 = wb[2 * i + 1];
    uint32_t dA[4], dB[4];
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      dA[d] = lo8 ? w0[d] : w1[d];
      dB[d] = lo8 ? w1[d] : w0[d];
    }
    transpose4_lanerows(dA);      // dA[k]: dword ar of group k of row c
    transpose4_lanerows(dB);      // dB[k]: dword ar of group 4 + k of row c ^ 8
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int gA = GPL * i + k, gB = GPL * i + 4 + k;
      const f32x4_t xsA = xsum(gA), xsB = xsum(gB);
      const bf16x8_t a0 = *(const bf16x8_t*)(xa + 64 * gA);
      const bf16x8_t a1 = *(const bf16x8_t*)(xa + 64 * gA + 8);
      const bf16x8_t b0 = *(const bf16x8_t*)(xa + 64 * gB);
      const bf16x8_t b1 = *(const bf16x8_t*)(xa + 64 * gB + 8);
      const f32x2_t pA = *(const f32x2_t*)(sz_c + 2 * gA);   // (s, -(128 + z) * s)
      const f32x2_t pB = *(const f32x2_t*)(sz_x + 2 * gB);
      const float sA = pA[0], czA = pA[1], sB = pB[0], czB = pB[1];
      f32x4_t accA = {0.f, 0.f, 0.f, 0.f}, accB = {0.f, 0.f, 0.f, 0.f};
      accA = mfma16x16x32(a0, unpack_crumb8_bf16(dA[k], 0, magic), accA);
      accB = mfma16x16x32(b0, unpack_crumb8_bf16(dB[k], 0, magic), accB);
      accA = mfma16x16x32(a1, unpack_crumb8_bf16(dA[k], 1, magic), accA);
      accB = mfma16x16x32(b1, unpack_crumb8_bf16(dB[k], 1, magic), accB);
#pragma unroll
      for (int r = 0; r < RC; ++r) {
        y0[r] = fmaf(czA, xsA[r], y0[r]);
        y1[r] = fmaf(czB, xsB[r], y1[r]);
        y0[r] = fmaf(sA, accA[r], y0[r]);
        y1[r] = fmaf(sB, accB[r], y1[r]);
      }
    }
  }
  // D row m = 4*ar + r; rows m < M <= 4 live in lanes ar == 0
  float* rb = red + wave * (RC * 16);
#pragma unroll
  for (int r = 0; r < RC; ++r) {
    const float vv = y0[r] + row_swap8(y1[r]);
    if (ar == 0) rb[r * 16 + c] = vv;
  }
  lds_barrier();
  for (int e = threadIdx.x; e < 16 * M; e += blockDim.x) {
    const int m = e >> 4, n = e & 15;
    float sum = 0.f;
    for (int w = 0; w < W; ++w) sum += red[w * (RC * 16) + m * 16 + n];
    if (n <= rlast) a.y[(int64_t)m * a.sym + row0 + n] = (uint16_t)f32_to_bf16_bits(sum);
  }
}

// ---------------------------------------------------------------------------------------------
// int2 decode kernel for 4 < M <= 16 (G = 64): the int4 K-split structure with the int2 line-step
// of the int2 line kernel. A workgroup owns NW row tiles and one split of S2 line-steps (S2 * 512
// codes); the activation chunk x[0:M, split] is staged once in LDS (permute_x16 order, per-group
// row sums) and shared by the waves; wave w streams rows [16 w, 16 w + 16) of the tile over the
// split with two full-line loads per line-step and the cross-lane group transpose; the fp32
// partials go to part[split][m][n] and splitk_rows_reduce_kernel sums the splits in order.
// ---------------------------------------------------------------------------------------------
IMQ_HOST_DEV inline int ksplit2_lds(int M, int S2, int NW) {
  return M * (S2 * kLine2 + 8) * 2 + S2 * 8 * 16 * 4 + NW * sz2_bytes(S2 * 8);
}

// At most 168 VGPRs (three waves per SIMD): three 4-wave workgroups share a CU, so one
// workgroup's weight loads are in flight while another computes (the unbounded kernel takes 165-170
// registers and fit one 8-wave or two 4-wave workgroups per CU; 128 spills).
#ifndef IMQ_W2KS_WPE
#define IMQ_W2KS_WPE 3
#endif
#ifndef IMQ_W2KS_PIPE
#define IMQ_W2KS_PIPE 0
#endif
template <int S2, int MC, int SDT, int NW>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(IMQ_W2KS_WPE))) void w2_ksplit_kernel(SkinnyArgs a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  constexpr int VB = (SDT == IMQ_DT_FP32) ? 4 : 2;
  constexpr int GPL = 8;                              // groups per line-step
  constexpr int NGW = S2 * GPL;                       // groups of the split
  constexpr int NT = 64 * NW;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int c = lane & 15, ar = lane >> 4;
  const bool lo8 = c < 8;
  const int M = a.M;
  const int KL = a.Kpad / kLine2;
  const int RB = (a.N + 16 * NW - 1) / (16 * NW);
  const int split = blockIdx.x / RB;
  const int rb = blockIdx.x - split * RB;
  const int ls0 = split * S2;
  const int row0 = (rb * NW + wave) * 16;
  const bool tile_ok = row0 < a.N;
  const int rowa = tile_ok ? row0 : 0;
  const int rlast = a.N - 1 - rowa;

  const int xrow = S2 * kLine2 + 8;
  uint16_t* xw = (uint16_t*)smem;                                      // [M][xrow]
  float* xs = (float*)(smem + (size_t)M * xrow * 2);                   // [S2 * 8 groups][16 rows]
  float* szf = xs + NGW * 16 + wave * (16 * sz2_row(NGW));             // this wave's (s, cz) pairs

  // 1) x chunk: M rows x S2*32 pairs of 16 elements over the workgroup (clamped into the row)
  constexpr int XP = 32 * S2;
  constexpr int XU = (MC * XP + NT - 1) / NT;
  const int xtot = M * XP;
  const uint16_t* xbase = a.x + (int64_t)ls0 * kLine2;
  const int plim = a.Kpad - ls0 * kLine2 - 16;
  u32x4_t xlo[XU], xhi[XU];
#pragma unroll
  for (int u = 0; u < XU; ++u) {
    int idx = threadIdx.x + NT * u;
    idx = idx < xtot ? idx : xtot - 1;
    const int m = idx / XP, p = idx - m * XP;
    int kb = 16 * p;
    kb = kb < plim ? kb : plim;
    const uint16_t* src = xbase + m * (int)a.sxm + kb;
    xlo[u] = *(const u32x4_t*)src;
    xhi[u] = *(const u32x4_t*)(src + 8);
  }
  // 2) scale / zero words of this wave's 16 rows for groups [8*ls0, 8*ls0 + 8*S2)
  SzPairs<SDT, NGW> szp;
  szp.load(lane, (const unsigned char*)a.sc + (int64_t)rowa * a.ssn * VB,
           (const unsigned char*)a.zr + (int64_t)rowa * a.szn * VB, (int)a.ssn * VB, (int)a.szn * VB, rlast,
           ls0 * (GPL * VB / 4), a.Kpad / 64 * VB / 4);
  // 3) weights: per line-step one full-line load for rows 0-7 and one for rows 8-15
  const uint8_t* qt = a.q + (int64_t)rowa * a.sqn;
  const uint8_t* q0;
  const uint8_t* q1;
  int lst;
  line_bases(a, qt, lane, rlast, q0, q1, lst);
  u32x4_t wb[2 * S2];
#pragma unroll
  for (int i = 0; i < S2; ++i) {
    int l = ls0 + i;
    l = l < KL ? l : KL - 1;
    wb[2 * i] = __builtin_nontemporal_load((const u32x4_t*)(q0 + lst * l));
    wb[2 * i + 1] = __builtin_nontemporal_load((const u32x4_t*)(q1 + lst * l));
  }
  // 4) stage x (permute_x16 per pair) with per-group sums, and this wave's scale / zero words
#pragma unroll
  for (int u = 0; u < XU; ++u) {
    const int idx = threadIdx.x + NT * u;
    const bool ok = idx < xtot;
    const int m = (ok ? idx : 0) / XP, p = (ok ? idx : 0) - m * XP;
    float sum = bf16x8_sum(xlo[u]) + bf16x8_sum(xhi[u]);
    // the 4 pairs of one group are 4 consecutive idx (XP and NT are multiples of 4)
    sum = quad_sum4(sum);
    if (ok) {
      u32x4_t o0, o1;
      permute_x16(xlo[u], xhi[u], o0, o1);
      *(u32x4_t*)(xw + m * xrow + 16 * p) = o0;
      *(u32x4_t*)(xw + m * xrow + 16 * p + 8) = o1;
      if ((p & 3) == 0) xs[(p >> 2) * 16 + m] = sum;
    }
  }
  szp.store(lane, szf, (KL - ls0) * GPL);
  lds_barrier();   // x and its sums are shared by the waves; weights stay in flight

  const uint32_t magic = magic_bf16_128x2();
  const uint16_t* xa = xw + (c < M ? c : M - 1) * xrow + 16 * ar;
  const float* sz_c = szf + c * sz2_row(NGW);
  const float* sz_x = szf + (c ^ 8) * sz2_row(NGW);
  float y0[4] = {0.f, 0.f, 0.f, 0.f}, y1[4] = {0.f, 0.f, 0.f, 0.f};
#if IMQ_W2KS_PIPE
  // Software-pipelined over the S2 * 4 group pairs t: the MFMAs of pair t are issued, then the
  // LDS operands of pair t + 1 are read, and only then is pair t - 1's scale applied to its
  // sums (a scheduling barrier keeps that order) -- so two pairs of sums are live instead of all
  // of them and the fma epilogue runs under the next MFMAs.
  constexpr int TT = S2 * 4;
  struct Ops {
    f32x4_t xsA, xsB;
    bf16x8_t a0, a1, b0, b1;
    f32x2_t pA, pB;
  };
  auto load_ops = [&](int t, Ops& o) {
    const int gA = GPL * (t >> 2) + (t & 3), gB = gA + 4;
    o.xsA = *(const f32x4_t*)(xs + gA * 16 + 4 * ar);
    o.xsB = *(const f32x4_t*)(xs + gB * 16 + 4 * ar);
    o.a0 = *(const bf16x8_t*)(xa + 64 * gA);
    o.a1 = *(const bf16x8_t*)(xa + 64 * gA + 8);
    o.b0 = *(const bf16x8_t*)(xa + 64 * gB);
    o.b1 = *(const bf16x8_t*)(xa + 64 * gB + 8);
    o.pA = *(const f32x2_t*)(sz_c + 2 * gA);   // (s, -(128 + z) * s)
    o.pB = *(const f32x2_t*)(sz_x + 2 * gB);
  };
  Ops op[2];
  f32x4_t acA[2], acB[2];
  uint32_t dA[4], dB[4];
  float sAp = 0.f, sBp = 0.f;
  load_ops(0, op[0]);
#pragma unroll
  for (int t = 0; t < TT; ++t) {
    const int cur = t & 1, k = t & 3;
    if (k == 0) {
      const u32x4_t w0 = wb[2 * (t >> 2)], w1 = wb[2 * (t >> 2) + 1];
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        dA[d] = lo8 ? w0[d] : w1[d];
        dB[d] = lo8 ? w1[d] : w0[d];
      }
      transpose4_lanerows(dA);    // dA[k]: dword ar of group k of row c
      transpose4_lanerows(dB);    // dB[k]: dword ar of group 4 + k of row c ^ 8
    }
    const f32x4_t z4 = {0.f, 0.f, 0.f, 0.f};
    acA[cur] = mfma16x16x32(op[cur].a0, unpack_crumb8_bf16(dA[k], 0, magic), z4);
    acB[cur] = mfma16x16x32(op[cur].b0, unpack_crumb8_bf16(dB[k], 0, magic), z4);
    acA[cur] = mfma16x16x32(op[cur].a1, unpack_crumb8_bf16(dA[k], 1, magic), acA[cur]);
    acB[cur] = mfma16x16x32(op[cur].b1, unpack_crumb8_bf16(dB[k], 1, magic), acB[cur]);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      y0[r] = fmaf(op[cur].pA[1], op[cur].xsA[r], y0[r]);
      y1[r] = fmaf(op[cur].pB[1], op[cur].xsB[r], y1[r]);
    }
    const float sAc = op[cur].pA[0], sBc = op[cur].pB[0];
    if (t + 1 < TT) load_ops(t + 1, op[cur ^ 1]);
    __builtin_amdgcn_sched_barrier(0);
    if (t > 0) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        y0[r] = fmaf(sAp, acA[cur ^ 1][r], y0[r]);
        y1[r] = fmaf(sBp, acB[cur ^ 1][r], y1[r]);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    sAp = sAc;
    sBp = sBc;
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    y0[r] = fmaf(sAp, acA[(TT - 1) & 1][r], y0[r]);
    y1[r] = fmaf(sBp, acB[(TT - 1) & 1][r], y1[r]);
  }
#else
#pragma unroll
  for (int i = 0; i < S2; ++i) {
    const u32x4_t w0 = wb[2 * i], w1 = wb[2 * i + 1];
    uint32_t dA[4], dB[4];
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      dA[d] = lo8 ? w0[d] : w1[d];
      dB[d] = lo8 ? w1[d] : w0[d];
    }
    transpose4_lanerows(dA);      // dA[k]: dword ar of group k of row c
    transpose4_lanerows(dB);      // dB[k]: dword ar of group 4 + k of row c ^ 8
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int gA = GPL * i + k, gB = GPL * i + 4 + k;
      const f32x4_t xsA = *(const f32x4_t*)(xs + gA * 16 + 4 * ar);
      const f32x4_t xsB = *(const f32x4_t*)(xs + gB * 16 + 4 * ar);
      const bf16x8_t a0 = *(const bf16x8_t*)(xa + 64 * gA);
      const bf16x8_t a1 = *(const bf16x8_t*)(xa + 64 * gA + 8);
      const bf16x8_t b0 = *(const bf16x8_t*)(xa + 64 * gB);
      const bf16x8_t b1 = *(const bf16x8_t*)(xa + 64 * gB + 8);
      const f32x2_t pA = *(const f32x2_t*)(sz_c + 2 * gA);   // (s, -(128 + z) * s)
      const f32x2_t pB = *(const f32x2_t*)(sz_x + 2 * gB);
      const float sA = pA[0], czA = pA[1], sB = pB[0], czB = pB[1];
      f32x4_t accA = {0.f, 0.f, 0.f, 0.f}, accB = {0.f, 0.f, 0.f, 0.f};
      accA = mfma16x16x32(a0, unpack_crumb8_bf16(dA[k], 0, magic), accA);
      accB = mfma16x16x32(b0, unpack_crumb8_bf16(dB[k], 0, magic), accB);
      accA = mfma16x16x32(a1, unpack_crumb8_bf16(dA[k], 1, magic), accA);
      accB = mfma16x16x32(b1, unpack_crumb8_bf16(dB[k], 1, magic), accB);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        y0[r] = fmaf(czA, xsA[r], y0[r]);
        y1[r] = fmaf(czB, xsB[r], y1[r]);
        y0[r] = fmaf(sA, accA[r], y0[r]);
        y1[r] = fmaf(sB, accB[r], y1[r]);
      }
    }
  }
#endif
  float* pbase = a.part + (size_t)split * M * a.N + row0 + c;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const float vv = y0[r] + row_swap8(y1[r]);
    const int m = 4 * ar + r;
    if (tile_ok && m < M && c <= rlast) pbase[(size_t)m * a.N] = vv;
  }
}

// ---------------------------------------------------------------------------------------------
// int8 per-row decode kernel (M <= 16). A K-step is 64 codes: 64 bytes of each row, one 16-byte
// load per lane (lane row jl takes codes [16*jl, 16*jl+16)), feeding two MFMAs whose operands
// are (q + 128) as bf16 -- exact: q ^ 0x80 is q + 128 in 0..255, 8 significant bits -- against
// activations in natural order. The per-row scale factors out of K, so one accumulator runs
// over the whole row: y = s * (acc - 128 * sum(x)), the kernel form of the reference's `_ksk8`.
// ---------------------------------------------------------------------------------------------
constexpr int kStep8 = 64;

// 8 int8 codes (two dwords) -> bf16x8 of (q + 128), exact.
IMQ_DEV bf16x8_t biased_i8x8_bf16(uint32_t lo, uint32_t hi) {
  u32x4_t r;
  lo ^= 0x80808080u;
  hi ^= 0x80808080u;
  r[0] = cvt_pk_bf16((float)(lo & 0xffu), (float)((lo >> 8) & 0xffu));
  r[1] = cvt_pk_bf16((float)((lo >> 16) & 0xffu), (float)(lo >> 24));
  r[2] = cvt_pk_bf16((float)(hi & 0xffu), (float)((hi >> 8) & 0xffu));
  r[3] = cvt_pk_bf16((float)((hi >> 16) & 0xffu), (float)(hi >> 24));
  return __builtin_bit_cast(bf16x8_t, r);
}

// TL: weights in the line-tiled layout (a separate instantiation: the per-load address).
template <int S, int MC, int SDT, int MAXW, bool TL = false>
__global__ __launch_bounds__(64 * MAXW) void w8_skinny_kernel(SkinnyArgs a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int W = blockDim.x >> 6;
  const int nl = lane & 15;
  const int jl = lane >> 4;
  constexpr int RC = (MC < 4) ? MC : 4;

  const int KS = a.Kpad / kStep8;                   // a.Kpad carries K (a multiple of 64)
  const int CS = a.chunk_steps;
  const int nchunks = (KS + CS - 1) / CS;
  const int xls = CS * kStep8 + kXPad;
  uint16_t* xl = (uint16_t*)smem;                                    // [M][xls]
  float* xs = (float*)(smem + (size_t)a.M * xls * 2);                // [CS][16] step sums
  float* xtot = xs + (size_t)CS * 16;                                // [16] row sums
  float* red = xtot + 16;                                            // [2][W][256]
  const int NT = (a.N + 15) / 16;

  // stage steps [c0, c1) in natural order; per-step row sums reduced across the 8 lanes of a
  // step, then added to the row totals in step order (deterministic)
  auto stage = [&](int c0, int c1) {
    const int nblk = (c1 - c0) * 8;
    const int total = a.M * nblk;                    // a multiple of 8
    for (int base = 0; base < total; base += blockDim.x) {
      const int idx = base + threadIdx.x;
      const bool valid = idx < total;
      const int id = valid ? idx : total - 1;
      const int m = id / nblk;
      const int b = id - m * nblk;
      const u32x4_t v = *(const u32x4_t*)(a.x + (int64_t)m * a.sxm + (int64_t)c0 * kStep8 + 8 * b);
      float sum = bf16x8_sum(v);
      sum = half_row_sum8(sum);
      if (valid) {
        *(u32x4_t*)(xl + m * xls + 8 * b) = v;
        if ((b & 7) == 0) xs[(b >> 3) * 16 + m] = sum;
      }
    }
    lds_barrier();
    if ((int)threadIdx.x < a.M) {
      float t = xtot[threadIdx.x];
      for (int st = 0; st < c1 - c0; ++st) t += xs[st * 16 + threadIdx.x];
      xtot[threadIdx.x] = t;
    }
    lds_barrier();
  };

  const uint16_t* xlane = xl + (nl < a.M ? nl : a.M - 1) * xls + 16 * jl;
  int buf = 0;
  bool staged = false;

  for (int tile = blockIdx.x; tile < NT; tile += gridDim.x) {
    int row = tile * 16 + nl;
    row = row < a.N ? row : a.N - 1;
    const int8_t* qrow = a.q8 + (int64_t)row * a.sqn + 16 * jl;
    // line-tiled (N a multiple of 16): the 16 bytes at byte 64 st + 16 jl of tile row nl sit at
    // tile line-step st / 2, half h = nl / 8, slot (nl & 7) + 8 ((st & 1) ^ h) + 16 jl
    const int th = nl >> 3;
    const int8_t* qtile = a.q8 + (int64_t)tile * 16 * a.sqn + 1024 * th + 16 * (nl & 7) + 256 * jl;
    const int8_t* qte = qtile + 128 * th;
    const int8_t* qto = qtile + 128 * (1 - th);
    f32x4_t acc[4];                          // four independent MFMA chains
#pragma unroll
    for (int k = 0; k < 4; ++k) acc[k] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    for (int c = 0; c < nchunks; ++c) {
      const int c0 = c * CS;
      const int c1 = (c0 + CS < KS) ? c0 + CS : KS;
      if (nchunks > 1 || !staged) {
        if (c == 0) {                          // row totals restart with each pass over K
          lds_barrier();                       // (the previous tile's reduction has read them)
          if ((int)threadIdx.x < 16) xtot[threadIdx.x] = 0.f;
          lds_barrier();
        }
        stage(c0, c1);
        staged = true;
      }
      const int R = (c1 - c0 + W * S - 1) / (W * S);
      for (int rnd = 0; rnd < R; ++rnd) {
        const int sbase = c0 + (rnd * W + wave) * S;
        u32x4_t wv[S];
#pragma unroll
        for (int i = 0; i < S; ++i) {
          int st = sbase + i;
          st = st < c1 ? st : c1 - 1;
          if constexpr (TL)
            wv[i] = __builtin_nontemporal_load((const u32x4_t*)(((st & 1) ? qto : qte) + 2048 * (st >> 1)));
          else
            wv[i] = __builtin_nontemporal_load((const u32x4_t*)(qrow + (int64_t)st * kStep8));
        }
#pragma unroll
        for (int i = 0; i < S; ++i) {
          const int s0 = sbase + i;
          if (s0 < c1) {                               // uniform across the wave
            const int ls = s0 - c0;
            const bf16x8_t x0 = *(const bf16x8_t*)(xlane + ls * kStep8);
            const bf16x8_t x1 = *(const bf16x8_t*)(xlane + ls * kStep8 + 8);
            acc[2 * (i & 1)] = mfma16x16x32(x0, biased_i8x8_bf16(wv[i][0], wv[i][1]), acc[2 * (i & 1)]);
            acc[2 * (i & 1) + 1] = mfma16x16x32(x1, biased_i8x8_bf16(wv[i][2], wv[i][3]), acc[2 * (i & 1) + 1]);
          }
        }
      }
      if (nchunks > 1) lds_barrier();
    }

    float* rb = red + buf * (W * 256);
#pragma unroll
    for (int q = 0; q < 4; ++q) rb[wave * 256 + (4 * jl + q) * 16 + nl] = (acc[0][q] + acc[1][q]) + (acc[2][q] + acc[3][q]);
    lds_barrier();
    const int n0 = tile * 16;
    for (int e = threadIdx.x; e < 16 * a.M; e += blockDim.x) {
      const int m = e >> 4;
      const int n = e & 15;
      float sum = 0.f;
      for (int w = 0; w < W; ++w) sum += rb[w * 256 + e];
      if (n0 + n < a.N) {
        const float sc = load_as_f32<SDT>(a.sc, (int64_t)(n0 + n) * a.ssn);
        a.y[(int64_t)m * a.sym + n0 + n] = (uint16_t)f32_to_bf16_bits(sc * (sum - 128.f * xtot[m]));
      }
    }
    buf ^= 1;
  }
}

// ---------------------------------------------------------------------------------------------
// int8 decode line kernel (M <= 4): the int4 line kernel's structure for per-row int8. A
// line-step is 128 bytes of a row = 128 codes. One workgroup owns a 16-row tile and all of K; W
// waves split K in S2 line-steps each and issue all of their loads up front:
//   * two 16-byte loads per line-step cover 8 rows x a whole 128-byte line each: lane (c, ar)
//     keeps 16 codes of its own row c in the first half (K offset 16 ar) and 16 codes of row c ^ 8
//     in the second half (K offset 64 + 16 ar), so every lane of one MFMA reads the same K;
//   * operands are (q + 128) as bf16 (exact) against activations in natural order, staged in the
//     wave's LDS with per-64-code row sums; a line-step contributes acc - 128 * sum(x) per half;
//   * rows c ^ 8 are folded back with a row swap, partials reduce across waves in LDS, and the
//     per-row scale multiplies the sum: y = s * sum_k x * q, the kernel form of `_ksk8`.
// ---------------------------------------------------------------------------------------------
constexpr int kLine8 = 128;   // codes per int8 line-step (128 bytes of a row)

IMQ_HOST_DEV inline int line8_wave_lds(int M, int S2) { return M * (S2 * kLine8 + 8) * 2 + 2 * S2 * 16 * 4; }

template <int S2, int MC, int SDT, int MAXW>
__global__ __launch_bounds__(64 * MAXW) void w8_line_kernel(SkinnyArgs a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  constexpr int RC = MC < 4 ? MC : 4;                 // D registers that can hold a real row
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int W = blockDim.x >> 6;
  const int c = lane & 15, ar = lane >> 4;
  const bool lo8 = c < 8;
  const int M = MC <= 2 ? MC : a.M;                 // MC 1 and 2 launch exactly that M
  const int KL = a.Kpad / kLine8;                   // a.Kpad carries K (a multiple of 128)
  const int ls0 = wave * S2;
  const int row0 = blockIdx.x * 16;
  const int rlast = a.N - 1 - row0;                  // last valid row within the tile

  const int xrow = S2 * kLine8 + 8;
  const int wbytes = line8_wave_lds(M, S2);
  unsigned char* wl = smem + (size_t)wave * wbytes;
  uint16_t* xw = (uint16_t*)wl;                      // [M][xrow], natural order
  float* xs = (float*)(wl + M * xrow * 2);          // [2 * S2 half line-steps][16 rows]
  float* red = (float*)(smem + (size_t)W * wbytes);

  // 1) x: M rows x 16*S2 16-byte blocks of this wave's K range (clamped into the row)
  constexpr int XB = 16 * S2;
  constexpr int XU = (MC * XB + 63) / 64;
  const int xtot = M * XB;
  const uint16_t* xbase = a.x + (int64_t)ls0 * kLine8;
  const int xlim = a.Kpad - ls0 * kLine8 - 8;        // last valid block start in the range
  u32x4_t xv[XU];
#pragma unroll
  for (int u = 0; u < XU; ++u) {
    int idx = lane + 64 * u;
    idx = idx < xtot ? idx : xtot - 1;
    const int m = idx / XB, b = idx - m * XB;
    int kb = 8 * b;
    kb = kb < xlim ? kb : xlim;
    xv[u] = *(const u32x4_t*)(xbase + m * (int)a.sxm + kb);
  }
  // 2) weights: per line-step one full-line load for rows 0-7 and one for rows 8-15
  const int8_t* qt = a.q8 + (int64_t)row0 * a.sqn;
  const int8_t* q0;
  const int8_t* q1;
  int lst;
  line_bases(a, qt, lane, rlast, q0, q1, lst);
  u32x4_t wb[2 * S2];
#pragma unroll
  for (int i = 0; i < S2; ++i) {
    int l = ls0 + i;
    l = l < KL ? l : KL - 1;
    wb[2 * i] = __builtin_nontemporal_load((const u32x4_t*)(q0 + lst * l));
    wb[2 * i + 1] = __builtin_nontemporal_load((const u32x4_t*)(q1 + lst * l));
  }
  // 3) stage x with its per-64-code row sums
#pragma unroll
  for (int u = 0; u < XU; ++u) {
    const int idx = lane + 64 * u;
    const bool ok = idx < xtot;
    const int m = (ok ? idx : 0) / XB, b = (ok ? idx : 0) - m * XB;
    float sum = bf16x8_sum(xv[u]);
    // the 8 blocks of one half line-step are 8 consecutive idx (XB is a multiple of 8)
    sum = half_row_sum8(sum);
    if (ok) {
      *(u32x4_t*)(xw + m * xrow + 8 * b) = xv[u];
      if ((b & 7) == 0) xs[(b >> 3) * 16 + m] = sum;
    }
  }
  // LDS is written and read by this wave only; its LDS operations execute in order
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");

  // PAIRED (M == 2): A lane row m < M reads activation row m in the line-step's first half,
  // M <= m < 2M row m - M in its second half (64 codes on), other rows repeat row 0 (their D rows
  // are unused). Measured on the int8 lm_head 3584 -> 152064: M = 2 4811-4831 -> 5138-5508 GB/s;
  // at M = 1 it measured 2% slower, so M = 1 keeps the per-lane selects.
  constexpr bool PAIRED = MC == 2 && IMQ_LINE_PAIRED;
  const uint16_t* xa = PAIRED ? xw + (c < 2 * M ? c % M : 0) * xrow + 16 * ar + (c >= M && c < 2 * M ? 64 : 0)
                              : xw + (c < M ? c : M - 1) * xrow + 16 * ar;
  float y0[4] = {0.f, 0.f, 0.f, 0.f}, y1[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < S2; ++i) {
    // a line-step past K (its loads re-read the last one) contributes nothing
    const float v = ls0 + i < KL ? 1.f : 0.f;
    const f32x4_t xs0 = *(const f32x4_t*)(xs + (2 * i) * 16 + 4 * ar);
    const f32x4_t xs1 = *(const f32x4_t*)(xs + (2 * i + 1) * 16 + 4 * ar);
    const bf16x8_t a00 = *(const bf16x8_t*)(xa + i * kLine8);
    const bf16x8_t a01 = *(const bf16x8_t*)(xa + i * kLine8 + 8);
    const u32x4_t w0 = wb[2 * i], w1 = wb[2 * i + 1];
    if constexpr (PAIRED) {
      // each load feeds its MFMAs as loaded: lanes c < 8 of L0 (row c, first half) meet D rows
      // [0, M), lanes c >= 8 (row c ^ 8, second half) D rows [M, 2M); L1 the other way round
      f32x4_t p0 = {0.f, 0.f, 0.f, 0.f}, p1 = {0.f, 0.f, 0.f, 0.f};
      p0 = mfma16x16x32(a00, biased_i8x8_bf16(w0[0], w0[1]), p0);
      p1 = mfma16x16x32(a00, biased_i8x8_bf16(w1[0], w1[1]), p1);
      p0 = mfma16x16x32(a01, biased_i8x8_bf16(w0[2], w0[3]), p0);
      p1 = mfma16x16x32(a01, biased_i8x8_bf16(w1[2], w1[3]), p1);
#pragma unroll
      for (int r = 0; r < RC; ++r) {
        const float acc0 = lo8 ? p0[r] : p1[r];             // own row c, first half
        const float acc1 = lo8 ? p1[MC + r] : p0[MC + r];   // row c ^ 8, second half
        y0[r] = fmaf(v, fmaf(-128.f, xs0[r], acc0), y0[r]);
        y1[r] = fmaf(v, fmaf(-128.f, xs1[r], acc1), y1[r]);
      }
    } else {
      const bf16x8_t a10 = *(const bf16x8_t*)(xa + i * kLine8 + 64);
      const bf16x8_t a11 = *(const bf16x8_t*)(xa + i * kLine8 + 72);
      u32x4_t gA, gB;
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        gA[d] = lo8 ? w0[d] : w1[d];                   // own row c, first half
        gB[d] = lo8 ? w1[d] : w0[d];                   // row c ^ 8, second half
      }
      f32x4_t acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
      acc0 = mfma16x16x32(a00, biased_i8x8_bf16(gA[0], gA[1]), acc0);
      acc1 = mfma16x16x32(a10, biased_i8x8_bf16(gB[0], gB[1]), acc1);
      acc0 = mfma16x16x32(a01, biased_i8x8_bf16(gA[2], gA[3]), acc0);
      acc1 = mfma16x16x32(a11, biased_i8x8_bf16(gB[2], gB[3]), acc1);
#pragma unroll
      for (int r = 0; r < RC; ++r) {
        y0[r] = fmaf(v, fmaf(-128.f, xs0[r], acc0[r]), y0[r]);
        y1[r] = fmaf(v, fmaf(-128.f, xs1[r], acc1[r]), y1[r]);
      }
    }
  }
  // D row m = 4*ar + r; rows m < M <= 4 live in lanes ar == 0
  float* rb = red + wave * (RC * 16);
#pragma unroll
  for (int r = 0; r < RC; ++r) {
    const float vv = y0[r] + row_swap8(y1[r]);
    if (ar == 0) rb[r * 16 + c] = vv;
  }
  lds_barrier();
  for (int e = threadIdx.x; e < 16 * M; e += blockDim.x) {
    const int m = e >> 4, n = e & 15;
    float sum = 0.f;
    for (int w = 0; w < W; ++w) sum += red[w * (RC * 16) + m * 16 + n];
    if (n <= rlast) {
      const float sc = load_as_f32<SDT>(a.sc, (int64_t)(row0 + n) * a.ssn);
      a.y[(int64_t)m * a.sym + row0 + n] = (uint16_t)f32_to_bf16_bits(sc * sum);
    }
  }
}

// ---------------------------------------------------------------------------------------------
// Generic fallback: any bit width (2/4/8), any group size, any stride/alignment, M <= 16.
// One wave per output row; every weight is dequantized in fp32 as (q - bf16(z)) * bf16(s), the
// same un-rounded weight the fast kernels accumulate with, and accumulated in fp32. Slow but
// simple; used for shapes the fast kernels reject.
// ---------------------------------------------------------------------------------------------
struct GenericArgs {
  const uint16_t* x;
  int64_t sxm;
  int M;
  int64_t K;       // codes per row to reduce over (K_pad for int2/4, K for int8)
  const uint8_t* q;
  int64_t sqn;
  const void* sc;
  int64_t ssn, ssg;
  const void* zr;
  int64_t szn, szg;
  int64_t N;
  int64_t G;
  uint16_t* y;
  int64_t sym;
};

template <int BITS, int SDT, int ZDT>
__global__ __launch_bounds__(256) void generic_gemv_kernel(GenericArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= a.N) return;
  float acc[16];
#pragma unroll
  for (int m = 0; m < 16; ++m) acc[m] = 0.f;
  const uint8_t* qr = a.q + row * a.sqn;
  for (int64_t k = lane; k < a.K; k += 64) {
    float w;
    if constexpr (BITS == 8) {
      w = (float)((const int8_t*)qr)[k];
    } else {
      constexpr int CPB = 8 / BITS;
      const uint32_t byte = qr[k / CPB];
      const float code = (float)((byte >> (BITS * (k % CPB))) & ((1u << BITS) - 1u));
      const int64_t g = k / a.G;
      const float z = load_as_bf16_f32<ZDT>(a.zr, row * a.szn + g * a.szg);
      const float s = load_as_bf16_f32<SDT>(a.sc, row * a.ssn + g * a.ssg);
      w = (code - z) * s;
    }
#pragma unroll
    for (int m = 0; m < 16; ++m)
      if (m < a.M) acc[m] = fmaf(bf16_bits_to_f32(a.x[m * a.sxm + k]), w, acc[m]);
  }
#pragma unroll
  for (int m = 0; m < 16; ++m) {
    float v = acc[m];
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    acc[m] = v;
  }
  if (lane < a.M) {
    float v = 0.f;
#pragma unroll
    for (int m = 0; m < 16; ++m)
      if (m == lane) v = acc[m];
    if constexpr (BITS == 8) v *= load_as_f32<SDT>(a.sc, row * a.ssn);
    a.y[lane * a.sym + row] = (uint16_t)f32_to_bf16_bits(v);
  }
}

// ---------------------------------------------------------------------------------------------
// host dispatch
// ---------------------------------------------------------------------------------------------

template <typename K>
int launch_with_lds(K kern, dim3 grid, dim3 block, size_t lds, hipStream_t st, const SkinnyArgs& a) {
  if (lds > 65536) {
    hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return (int)e;
  }
  kern<<<grid, block, lds, st>>>(a);
  IMQ_LAUNCH_CHECK();
  return IMQ_OK;
}

// Register budget: a kernel compiled for up to MAXW waves per workgroup gets 512/(MAXW/4)
// VGPRs per lane at most; workgroups of <= 8 waves use the MAXW=8 build (no spills with the
// deep S=8 batches and fp16/fp32 scale conversion).
template <int S, int SDT, int ZDT, bool STRIP, int MAXW>
int skinny_resident_mw(const SkinnyArgs& a, size_t lds, int grid, int W, hipStream_t st) {
  const dim3 g(grid), b(64 * W);
  if (a.M == 1) return launch_with_lds(w4_skinny_kernel<S, 1, SDT, ZDT, STRIP, MAXW>, g, b, lds, st, a);
  if (a.M == 2) return launch_with_lds(w4_skinny_kernel<S, 2, SDT, ZDT, STRIP, MAXW>, g, b, lds, st, a);
  if (a.M <= 4) return launch_with_lds(w4_skinny_kernel<S, 4, SDT, ZDT, STRIP, MAXW>, g, b, lds, st, a);
  return launch_with_lds(w4_skinny_kernel<S, 16, SDT, ZDT, STRIP, MAXW>, g, b, lds, st, a);
}

template <int S, int SDT, int ZDT, bool STRIP>
int skinny_resident_m(const SkinnyArgs& a, size_t lds, int grid, int W, hipStream_t st) {
  if (W <= 8) return skinny_resident_mw<S, SDT, ZDT, STRIP, 8>(a, lds, grid, W, st);
  if constexpr (S == 8 && SDT != IMQ_DT_BF16) return IMQ_ERR_UNSUPPORTED;   // never dispatched
  else return skinny_resident_mw<S, SDT, ZDT, STRIP, 16>(a, lds, grid, W, st);
}

template <int S, int SDT, int ZDT>
int skinny_resident(const SkinnyArgs& a, size_t lds, int grid, int W, hipStream_t st) {
  constexpr int SZB = (SDT == IMQ_DT_FP32) ? 4 : 2;
  constexpr int ZZB = (ZDT == IMQ_DT_FP32) ? 4 : 2;
  const int KS = a.Kpad / kStep;
  const bool strip = a.G == kStep && (KS % S) == 0 && a.ssg == 1 && a.szg == 1 &&
                     ((uintptr_t)a.sc % 16) == 0 && ((uintptr_t)a.zr % 16) == 0 &&
                     ((a.ssn * SZB) % 16) == 0 && ((a.szn * ZZB) % 16) == 0;
  if (strip) return skinny_resident_m<S, SDT, ZDT, true>(a, lds, grid, W, st);
  return skinny_resident_m<S, SDT, ZDT, false>(a, lds, grid, W, st);
}

template <int W, int SDT, int ZDT>
int skinny_chunked(const SkinnyArgs& a, size_t lds, int grid, hipStream_t st) {
  const dim3 g(grid), b(64 * W);
  if (a.M == 1) return launch_with_lds(w4_skinny_chunked_kernel<W, 1, SDT, ZDT>, g, b, lds, st, a);
  if (a.M == 2) return launch_with_lds(w4_skinny_chunked_kernel<W, 2, SDT, ZDT>, g, b, lds, st, a);
  if (a.M <= 4) return launch_with_lds(w4_skinny_chunked_kernel<W, 4, SDT, ZDT>, g, b, lds, st, a);
  return launch_with_lds(w4_skinny_chunked_kernel<W, 16, SDT, ZDT>, g, b, lds, st, a);
}

// Workgroups of the resident kernel: enough to fill every CU several times over, each looping
// over ceil(NT / grid) tiles so the x staging is amortized over several tiles.
int skinny_grid(int NT, int W, size_t lds, const DevInfo& di) {
  int by_lds = lds > 0 ? (int)((size_t)di.max_lds / lds) : 8;
  int by_waves = 32 / W;                    // ~32 resident waves per CU
  int per_cu = by_lds < by_waves ? by_lds : by_waves;
  if (per_cu < 1) per_cu = 1;
  long g = (long)di.cus * per_cu;
  return (int)(g < NT ? g : NT);
}

// S steps (S KB of packed weights) per wave per round, W waves per tile (<= 16). Measured on
// MI355X at Llama-8B shapes: many tiles (N >= 16K) prefer deep batches (S=8) in persistent
// workgroups; fewer tiles prefer splitting K over more waves (S=4), one tile per workgroup while
// x is small. (S=8 with more than 8 waves and fp16/fp32 scales would exceed the 16-wave register
// budget.) Returns whether the deep form was chosen.
bool skinny_shape(int KS, int NT, bool bf16_scales, int* So, int* Wo) {
  const bool wide = NT >= 1024 && KS >= 16 && (bf16_scales || (KS + 7) / 8 <= 8);
  int S, W;
  if (wide) { S = 8; W = (KS + 7) / 8; }
  else { S = 4; W = (KS + 3) / 4; }
  if (W > 16) W = 16;
  if (W < 1) W = 1;
  *So = S;
  *Wo = W;
  return wide;
}

template <int SDT, int ZDT>
int skinny_dispatch(const SkinnyArgs& a0, const DevInfo& di, hipStream_t st) {
  SkinnyArgs a = a0;
  const int KS = a.Kpad / kStep;
  const int NT = (a.N + 15) / 16;
  int S, W;
  const bool wide = skinny_shape(KS, NT, SDT == IMQ_DT_BF16, &S, &W);
  const size_t resident = (size_t)a.M * (KS * kStep + kXPad) * 2 + (size_t)KS * 64 + (size_t)2 * W * 256 * 4;
  if (resident <= (size_t)di.max_lds) {
    a.chunk_steps = KS;
    // one tile per workgroup while staging x is cheap (M <= 4); otherwise persistent
    // workgroups that stage x once and loop over tiles
    const int grid = (a.M <= 4 && !wide) ? NT : skinny_grid(NT, W, resident, di);
    if (S == 8) return skinny_resident<8, SDT, ZDT>(a, resident, grid, W, st);
    return skinny_resident<4, SDT, ZDT>(a, resident, grid, W, st);
  }
  // chunked fallback
  const int Wc = 8;
  const size_t redc = (size_t)2 * Wc * 256 * 4;
  int cs = KS;
  auto need = [&](int c) { return (size_t)a.M * (c * kStep + kXPad) * 2 + (size_t)c * 64 + redc; };
  while (cs > 1 && need(cs) > (size_t)di.max_lds) cs = (cs + 1) / 2;
  if (need(cs) > (size_t)di.max_lds) return IMQ_ERR_UNSUPPORTED;
  a.chunk_steps = cs;
  int grid = di.cus;
  if (grid > NT) grid = NT;
  return skinny_chunked<8, SDT, ZDT>(a, need(cs), grid, st);
}

// Line kernel dispatch (M <= 4, G == 128, K_pad a multiple of 256 and at most 16384, unit group
// strides, same scale / zero dtype). Line-steps per wave S2: 2 (measured on MI355X at Llama-8B
// shapes), raised to 4 when W = ceil(KL / S2) would exceed 16 waves (line_plan). Deeper S2 (larger
// K) would exceed the 128-VGPR budget of 16-wave workgroups; such K take the K-split or skinny
// kernels.
template <int S2, int SDT>
int line_launch(const SkinnyArgs& a, int W, size_t lds, hipStream_t st) {
  const dim3 g((unsigned)((a.N + 15) / 16)), b(64 * W);
  if (a.M == 1) return launch_with_lds(w4_line_kernel<S2, 1, SDT, 16>, g, b, lds, st, a);
  if (a.M == 2) return launch_with_lds(w4_line_kernel<S2, 2, SDT, 16>, g, b, lds, st, a);
  return launch_with_lds(w4_line_kernel<S2, 4, SDT, 16>, g, b, lds, st, a);
}

template <int SDT>
int line_dispatch_s(const SkinnyArgs& a, int S2, int W, size_t lds, hipStream_t st) {
  if (S2 == 2) return line_launch<2, SDT>(a, W, lds, st);
  return line_launch<4, SDT>(a, W, lds, st);
}

// Eligibility and launch shape of the line kernel (restated by the CPU bounds model in the
// tests): returns false when the line kernel does not take the call.
bool line_plan(int64_t M, int64_t Kpad, int64_t G, int64_t N, int64_t sqn, int64_t sxm, int64_t ssn,
               int64_t ssg, int64_t szn, int64_t szg, int sdt, int zdt, int max_lds, int* S2o, int* Wo,
               size_t* ldso) {
  if (M < 1 || M > 4 || G != 128 || Kpad % kLine != 0 || sdt != zdt) return false;
  if (ssg != 1 || szg != 1 || N < 1) return false;
  const int vb = sdt == IMQ_DT_FP32 ? 4 : 2;
  if ((ssn * vb) % 4 != 0 || (szn * vb) % 4 != 0) return false;
  // 32-bit in-tile offsets
  if (16 * sqn >= (int64_t(1) << 31) || M * sxm * 2 >= (int64_t(1) << 31)) return false;
  if (16 * ssn * vb >= (int64_t(1) << 31) || 16 * szn * vb >= (int64_t(1) << 31)) return false;
  const int64_t KL = Kpad / kLine;
  // two line-steps per wave (four when K needs more than 16 waves): with the DPP / dot2 staging,
  // M = 1 gains from the shorter per-wave tail too (measured: C2 M=1 3806 -> 3863 GB/s, C1 1971 ->
  // 2080 against four; one line-step per wave 3250 at C2)
  int S2 = 2;
  if ((KL + S2 - 1) / S2 > 16) S2 = 4;
  const int64_t W = (KL + S2 - 1) / S2;
  if (W > 16) return false;
  const int rc = M <= 2 ? (int)M : 4;                // reduction rows of the launched M class
  const size_t lds = (size_t)W * line_wave_lds((int)M, S2, vb) + (size_t)W * rc * 16 * 4;
  if (lds > (size_t)max_lds) return false;
  *S2o = S2;
  *Wo = (int)W;
  *ldso = lds;
  return true;
}

int line_w4(const SkinnyArgs& a, int sdt, const DevInfo& di, hipStream_t st) {
  int S2, W;
  size_t lds;
  if (!line_plan(a.M, a.Kpad, a.G, a.N, a.sqn, a.sxm, a.ssn, a.ssg, a.szn, a.szg, sdt, sdt, di.max_lds,
                 &S2, &W, &lds))
    return IMQ_ERR_UNSUPPORTED;
  switch (sdt) {
    case IMQ_DT_BF16: return line_dispatch_s<IMQ_DT_BF16>(a, S2, W, lds, st);
    case IMQ_DT_FP16: return line_dispatch_s<IMQ_DT_FP16>(a, S2, W, lds, st);
    case IMQ_DT_FP32: return line_dispatch_s<IMQ_DT_FP32>(a, S2, W, lds, st);
  }
  return IMQ_ERR_UNSUPPORTED;
}

// K-split kernel plan (4 < M <= 16, G == 128, K_pad a multiple of 256, unit group strides, same
// scale / zero dtype, N % 4 == 0 for the vector reduction; restated by the CPU bounds model in the
// tests): S2 = 4 line-steps (1024 codes) per split, NW = 8 row tiles per workgroup while that still
// gives every CU a workgroup, else 4. Every workgroup restages its split's activations (M x 1024
// bf16), so 8 tiles halve that traffic per weight byte (measured at M = 16: down_proj 4096 x 14336
// 16.1 -> 14.8 us); below one workgroup per CU the 4-tile grid is faster. A 4-tile grid of at most
// two workgroups per CU splits K in 512-code pieces instead (twice the workgroups, half the
// activations each; measured at M = 16: qkv 4096 -> 6144 10.6 -> 9.9 us, o 4096 -> 4096 8.3 ->
// 8.0 us).
constexpr int kKsS2 = 4;

// Line-steps per split (4, or 2 for short grids) and tiles per workgroup of the K-split plan.
inline void ksplit_shape(int64_t Kpad, int64_t N, int cus, int* s2, int* nw) {
  const int64_t KL = Kpad / kLine;
  const int64_t splits4 = (KL + kKsS2 - 1) / kKsS2;
  *nw = splits4 * ((N + 127) / 128) >= (int64_t)cus ? 8 : 4;
  *s2 = *nw == 4 && splits4 * ((N + 63) / 64) <= 2 * (int64_t)cus ? 2 : kKsS2;
}

bool ksplit_plan(int64_t M, int64_t Kpad, int64_t G, int64_t N, int64_t sqn, int64_t sxm, int64_t ssn,
                 int64_t ssg, int64_t szn, int64_t szg, int sdt, int zdt, int max_lds, int cus, int* splitso,
                 int* nwo, int* s2o, size_t* ldso) {
  if (M <= 4 || M > 16 || G != 128 || Kpad % kLine != 0 || Kpad <= 0 || sdt != zdt) return false;
  if (N % 4 != 0 || sxm % 8 != 0) return false;
  if (ssg != 1 || szg != 1 || N < 1 || N > (1 << 30) || Kpad > (1 << 28)) return false;
  const int vb = sdt == IMQ_DT_FP32 ? 4 : 2;
  if ((ssn * vb) % 4 != 0 || (szn * vb) % 4 != 0) return false;
  if (16 * sqn >= (int64_t(1) << 31) || M * sxm * 2 >= (int64_t(1) << 31)) return false;
  if (16 * ssn * vb >= (int64_t(1) << 31) || 16 * szn * vb >= (int64_t(1) << 31)) return false;
  int s2, nw;
  ksplit_shape(Kpad, N, cus, &s2, &nw);
  const int64_t splits = (Kpad / kLine + s2 - 1) / s2;
  const int64_t rbs = (N + 16 * nw - 1) / (16 * nw);
  if (splits * rbs > 0x7fffffff) return false;
  const size_t lds = (size_t)ksplit_lds((int)M, s2, nw, vb);
  if (lds > (size_t)max_lds) return false;
  *splitso = (int)splits;
  *nwo = nw;
  *s2o = s2;
  *ldso = lds;
  return true;
}

// Workspace bytes of the K-split decode path for this shape on the current device (0: the shape
// does not use it).
int64_t ksplit_workspace_bytes(int64_t M, int64_t N, int64_t Kpad) {
  if (M < 1 || M > 16 || N <= 0 || Kpad <= 0 || Kpad % kLine != 0) return 0;
  // below 5 rows only line-tiled weights whose K exceeds the line kernel's 16 waves of 4 line-steps
  if (M <= 4 && Kpad / kLine <= 64) return 0;
  int s2, nw;
  ksplit_shape(Kpad, N, device_info().cus, &s2, &nw);
  return (Kpad / kLine + s2 - 1) / s2 * M * N * 4;
}

template <int SDT, int NW, int S2>
int ksplit_launch(const SkinnyArgs& a, int splits, size_t lds, hipStream_t st) {
  const int rbs = (a.N + 16 * NW - 1) / (16 * NW);
  const dim3 g((unsigned)(splits * rbs)), b(64 * NW);
  int rc;
  if (a.M <= 8) rc = launch_with_lds(w4_ksplit_kernel<S2, 8, SDT, NW>, g, b, lds, st, a);
  else rc = launch_with_lds(w4_ksplit_kernel<S2, 16, SDT, NW>, g, b, lds, st, a);
  if (rc != IMQ_OK) return rc;
  const int n4 = a.N / 4;
  splitk_rows_reduce_kernel<<<dim3((unsigned)((a.M * n4 + 255) / 256)), dim3(256), 0, st>>>(a.part, splits, a.M,
                                                                                           a.N, a.y, a.sym);
  IMQ_LAUNCH_CHECK();
  return IMQ_OK;
}

template <int SDT>
int ksplit_dispatch(const SkinnyArgs& a, int nw, int s2, int splits, size_t lds, hipStream_t st) {
  if (nw == 8) return ksplit_launch<SDT, 8, kKsS2>(a, splits, lds, st);
  if (s2 == 2) return ksplit_launch<SDT, 4, 2>(a, splits, lds, st);
  return ksplit_launch<SDT, 4, kKsS2>(a, splits, lds, st);
}

int ksplit_w4(const SkinnyArgs& a0, int sdt, void* ws, int64_t wsb, const DevInfo& di, hipStream_t st) {
  int splits, nw, s2;
  size_t lds;
  // line-tiled weights below 5 rows whose K the line kernel declines (the skinny kernel reads
  // rows): the plan of 5 rows, whose LDS covers the staging of fewer
  const int64_t pm = a0.tiled && a0.M < 5 ? 5 : a0.M;
  if (!ksplit_plan(pm, a0.Kpad, a0.G, a0.N, a0.sqn, a0.sxm, a0.ssn, a0.ssg, a0.szn, a0.szg, sdt, sdt,
                   di.max_lds, di.cus, &splits, &nw, &s2, &lds))
    return IMQ_ERR_UNSUPPORTED;
  const int64_t need = (int64_t)splits * a0.M * a0.N * 4;
  if (!ws || wsb < need || ((uintptr_t)ws & 15)) return IMQ_ERR_UNSUPPORTED;
  if (((uintptr_t)a0.y & 7) || (a0.sym & 3)) return IMQ_ERR_UNSUPPORTED;   // 8-byte y stores
  SkinnyArgs a = a0;
  a.part = (float*)ws;
  switch (sdt) {
    case IMQ_DT_BF16: return ksplit_dispatch<IMQ_DT_BF16>(a, nw, s2, splits, lds, st);
    case IMQ_DT_FP16: return ksplit_dispatch<IMQ_DT_FP16>(a, nw, s2, splits, lds, st);
    case IMQ_DT_FP32: return ksplit_dispatch<IMQ_DT_FP32>(a, nw, s2, splits, lds, st);
  }
  return IMQ_ERR_UNSUPPORTED;
}

// Wave-split plan (4 < M <= 16, G == 128, K_pad == 8 R 256 with R 1 or 2, unit group strides,
// same scale / zero dtype, 4-byte aligned scale / zero rows, the LDS of wsplit_lds within the
// device's, at least one row tile per CU; restated by the CPU bounds model in the tests): NW = 8
// waves, one workgroup per CU, the grid min(tiles, CUs). Returns R, or 0 when the kernel does not
// take the call. Every workgroup reads all of x (M x K_pad bf16) and the first tile waits for it,
// so the kernel gains most where a workgroup streams many tiles (measured at M = 16: gate_up
// 4096 -> 28672, 7 tiles per CU, 20.8 us against 24.0 us for K-split + reduction). With the
// activation group sums as v_dot2 and DPP row sums the staging is short enough that 1-2 tiles per
// CU also beat K-split + reduction (C2 M = 16 2458 -> 2487 GB/s, M = 8 2615 -> 2638 with qkv and
// o on this kernel); below one tile per CU the K-split grid has more workgroups. PD = 2 tiles of
// prefetch measured best (3, 4: no gain on gate_up, slower on short grids).
constexpr int kWsNW = 8;
#ifndef IMQ_WS_PD
#define IMQ_WS_PD 2
#endif
#ifndef IMQ_WS_MIN_TILES
#define IMQ_WS_MIN_TILES 1
#endif
int wsplit_plan(int64_t M, int64_t Kpad, int64_t G, int64_t N, int64_t sqn, int64_t sxm, int64_t ssn,
                int64_t ssg, int64_t szn, int64_t szg, int sdt, int zdt, int max_lds, int cus) {
  if (M <= 4 || M > 16 || G != 128 || sdt != zdt || ssg != 1 || szg != 1) return 0;
  if (Kpad != kWsNW * kLine && Kpad != 2 * kWsNW * kLine) return 0;
  if (N < 1 || N > (1 << 30) || sxm % 8 != 0) return 0;
  const int vb = sdt == IMQ_DT_FP32 ? 4 : 2;
  if ((ssn * vb) % 4 != 0 || (szn * vb) % 4 != 0) return 0;
  if (N * sqn >= (int64_t(1) << 46) || 16 * sqn >= (int64_t(1) << 31) || M * sxm * 2 >= (int64_t(1) << 31)) return 0;
  const int R = (int)(Kpad / (kWsNW * kLine));
  if (wsplit_lds(R, kWsNW) > max_lds || (N + 15) / 16 < IMQ_WS_MIN_TILES * (int64_t)cus) return 0;
  return R;
}

template <int SDT>
int wsplit_launch(const SkinnyArgs& a, int R, const DevInfo& di, hipStream_t st) {
  const int64_t T = (a.N + 15) / 16;
  const dim3 g((unsigned)(T < di.cus ? T : di.cus)), b(64 * kWsNW);
  const size_t lds = (size_t)wsplit_lds(R, kWsNW);
  auto kern = a.tiled ? (R == 1 ? w4_wsplit_kernel<1, SDT, kWsNW, IMQ_WS_PD, true>
                                 : w4_wsplit_kernel<2, SDT, kWsNW, IMQ_WS_PD, true>)
                      : (R == 1 ? w4_wsplit_kernel<1, SDT, kWsNW, IMQ_WS_PD, false>
                                : w4_wsplit_kernel<2, SDT, kWsNW, IMQ_WS_PD, false>);
  static int attr_set[4] = {0, 0, 0, 0};   // benign race: every caller sets the same value
  const int ai = 2 * a.tiled + R - 1;
  if (lds > 65536 && !__atomic_load_n(&attr_set[ai], __ATOMIC_ACQUIRE)) {
    hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return (int)e;
    __atomic_store_n(&attr_set[ai], 1, __ATOMIC_RELEASE);
  }
  kern<<<g, b, lds, st>>>(a);
  IMQ_LAUNCH_CHECK();
  return IMQ_OK;
}

// On line-tiled weights the wave-split kernel takes only grids of IMQ_WS_TILED_MIN_TILES row
// tiles per CU and more; below that the K-split kernel is faster on them (measured, M = 8 / 16,
// µs per linear: qkv 4096 -> 6144 8.1 / 9.1 against 9.3 / 9.9, o 4096 -> 4096 7.1 / 7.7 against
// 7.9 / 8.3), while gate_up's 7 tiles per CU keep the wave-split kernel (16.6 / 17.3 against
// 19.0 / 22.3).
#ifndef IMQ_WS_TILED_MIN_TILES
#define IMQ_WS_TILED_MIN_TILES 4
#endif

int wsplit_w4(const SkinnyArgs& a, int sdt, const DevInfo& di, hipStream_t st) {
  if (a.tiled && (a.N + 15) / 16 < (int64_t)IMQ_WS_TILED_MIN_TILES * di.cus) return IMQ_ERR_UNSUPPORTED;
  const int R = wsplit_plan(a.M, a.Kpad, a.G, a.N, a.sqn, a.sxm, a.ssn, a.ssg, a.szn, a.szg, sdt, sdt, di.max_lds, di.cus);
  if (!R) return IMQ_ERR_UNSUPPORTED;
  switch (sdt) {
    case IMQ_DT_BF16: return wsplit_launch<IMQ_DT_BF16>(a, R, di, st);
    case IMQ_DT_FP16: return wsplit_launch<IMQ_DT_FP16>(a, R, di, st);
    case IMQ_DT_FP32: return wsplit_launch<IMQ_DT_FP32>(a, R, di, st);
  }
  return IMQ_ERR_UNSUPPORTED;
}

// Workspace bytes the int4 decode dispatch (skinny_w4) uses for this call on the current device:
// the K-split partials when the K-split kernel is the first fast kernel that takes the call, else
// 0 (the line and wave-split kernels keep every partial in the workgroup). Pointer alignment is not
// known here and taken as satisfied; an unaligned call falls back to kernels without a workspace,
// so the figure stays an upper bound.
int64_t w4_decode_workspace_bytes(int64_t M, int64_t Kpad, int64_t G, int64_t N, int64_t sqn, int64_t sxm,
                                  int64_t ssn, int64_t ssg, int64_t szn, int64_t szg, int sdt, int zdt) {
  if (M < 1 || M > 16 || G % kStep != 0 || Kpad % G != 0 || Kpad <= 0 || sdt != zdt) return 0;
  if (((G / kStep) & (G / kStep - 1)) != 0 || (sqn & 15) || (sxm & 7) || N > (1 << 30) || Kpad > (1 << 28))
    return 0;
  const DevInfo di = device_info();
  int S2, W;
  size_t lds;
  if (line_plan(M, Kpad, G, N, sqn, sxm, ssn, ssg, szn, szg, sdt, zdt, di.max_lds, &S2, &W, &lds)) return 0;
  if (wsplit_plan(M, Kpad, G, N, sqn, sxm, ssn, ssg, szn, szg, sdt, zdt, di.max_lds, di.cus)) return 0;
  int splits, nw, s2;
  if (ksplit_plan(M, Kpad, G, N, sqn, sxm, ssn, ssg, szn, szg, sdt, zdt, di.max_lds, di.cus, &splits, &nw, &s2, &lds))
    return (int64_t)splits * M * N * 4;
  return 0;
}

// Fast path eligibility + launch. Returns IMQ_ERR_UNSUPPORTED when the caller must fall back.
// ws / wsb: the caller's optional workspace (the K-split path of 4 < M <= 16 needs one).
//
// tiled: qweight is in the line-tiled layout (see line_bases); only the line, wave-split and K-split
// kernels read it (the K-split kernel then also takes the M <= 4 calls the line kernel declines), so
// a call none of them takes returns IMQ_ERR_UNSUPPORTED and the caller must not fall back to a
// row-layout kernel.
int skinny_w4(const uint16_t* x, int64_t sxm, int64_t M, int64_t Kpad, const uint8_t* q, int64_t sqn,
              const void* sc, int64_t ssn, int64_t ssg, int sdt, const void* zr, int64_t szn, int64_t szg,
              int zdt, int64_t N, int64_t G, uint16_t* y, int64_t sym, void* ws, int64_t wsb, hipStream_t st,
              bool tiled) {
  if (M < 1 || M > 16 || G % kStep != 0 || Kpad % G != 0 || Kpad <= 0) return IMQ_ERR_UNSUPPORTED;
  if (((G / kStep) & (G / kStep - 1)) != 0) return IMQ_ERR_UNSUPPORTED;   // groups of 2^k steps
  if (((uintptr_t)q & 15) || (sqn & 15) || ((uintptr_t)x & 15) || (sxm & 7)) return IMQ_ERR_UNSUPPORTED;
  if (N > (1 << 30) || Kpad > (1 << 28)) return IMQ_ERR_UNSUPPORTED;
  if (sdt != zdt) return IMQ_ERR_UNSUPPORTED;
  const DevInfo di = device_info();
  SkinnyArgs a{x, sxm, (int)M, (int)Kpad, q, sqn, sc, ssn, ssg, zr, szn, szg, (int)N, (int)G, y, sym, 0};
  a.tiled = tiled ? 1 : 0;
  if (((uintptr_t)sc & 3) == 0 && ((uintptr_t)zr & 3) == 0) {
    int rc = line_w4(a, sdt, di, st);
    if (rc != IMQ_ERR_UNSUPPORTED) return rc;
    rc = wsplit_w4(a, sdt, di, st);
    if (rc != IMQ_ERR_UNSUPPORTED) return rc;
    rc = ksplit_w4(a, sdt, ws, wsb, di, st);
    if (rc != IMQ_ERR_UNSUPPORTED) return rc;
  }
  if (tiled) return IMQ_ERR_UNSUPPORTED;
  switch (sdt) {
    case IMQ_DT_BF16: return skinny_dispatch<IMQ_DT_BF16, IMQ_DT_BF16>(a, di, st);
    case IMQ_DT_FP16: return skinny_dispatch<IMQ_DT_FP16, IMQ_DT_FP16>(a, di, st);
    case IMQ_DT_FP32: return skinny_dispatch<IMQ_DT_FP32, IMQ_DT_FP32>(a, di, st);
  }
  return IMQ_ERR_INVALID;
}

template <int BITS, int SDT, int ZDT>
int launch_generic(const GenericArgs& a, hipStream_t st) {
  const int64_t blocks = imq_cdiv(a.N, 4);
  generic_gemv_kernel<BITS, SDT, ZDT><<<dim3((unsigned)blocks), dim3(256), 0, st>>>(a);
  IMQ_LAUNCH_CHECK();
  return IMQ_OK;
}

template <int BITS, int SDT>
int generic_z(const GenericArgs& a, int zdt, hipStream_t st) {
  switch (zdt) {
    case IMQ_DT_BF16: return launch_generic<BITS, SDT, IMQ_DT_BF16>(a, st);
    case IMQ_DT_FP16: return launch_generic<BITS, SDT, IMQ_DT_FP16>(a, st);
    case IMQ_DT_FP32: return launch_generic<BITS, SDT, IMQ_DT_FP32>(a, st);
  }
  return IMQ_ERR_INVALID;
}

template <int BITS>
int generic_gemv(const uint16_t* x, int64_t sxm, int64_t M, int64_t K, const uint8_t* q, int64_t sqn,
                 const void* sc, int64_t ssn, int64_t ssg, int sdt, const void* zr, int64_t szn,
                 int64_t szg, int zdt, int64_t N, int64_t G, uint16_t* y, int64_t sym, hipStream_t st) {
  // rows of x/y beyond 16 are handled by re-launching on 16-row slices
  for (int64_t m0 = 0; m0 < M; m0 += 16) {
    const int mm = (int)((M - m0) < 16 ? (M - m0) : 16);
    GenericArgs a{x + m0 * sxm, sxm, mm, K, q, sqn, sc, ssn, ssg, zr, szn, szg, N, G, y + m0 * sym, sym};
    int rc;
    switch (sdt) {
      case IMQ_DT_BF16: rc = generic_z<BITS, IMQ_DT_BF16>(a, BITS == 8 ? IMQ_DT_BF16 : zdt, st); break;
      case IMQ_DT_FP16: rc = generic_z<BITS, IMQ_DT_FP16>(a, BITS == 8 ? IMQ_DT_BF16 : zdt, st); break;
      case IMQ_DT_FP32: rc = generic_z<BITS, IMQ_DT_FP32>(a, BITS == 8 ? IMQ_DT_BF16 : zdt, st); break;
      default: return IMQ_ERR_INVALID;
    }
    if (rc != IMQ_OK) return rc;
  }
  return IMQ_OK;
}

template int generic_gemv<2>(const uint16_t*, int64_t, int64_t, int64_t, const uint8_t*, int64_t, const void*,
                             int64_t, int64_t, int, const void*, int64_t, int64_t, int, int64_t, int64_t,
                             uint16_t*, int64_t, hipStream_t);
template int generic_gemv<4>(const uint16_t*, int64_t, int64_t, int64_t, const uint8_t*, int64_t, const void*,
                             int64_t, int64_t, int, const void*, int64_t, int64_t, int, int64_t, int64_t,
                             uint16_t*, int64_t, hipStream_t);
template int generic_gemv<8>(const uint16_t*, int64_t, int64_t, int64_t, const uint8_t*, int64_t, const void*,
                             int64_t, int64_t, int, const void*, int64_t, int64_t, int, int64_t, int64_t,
                             uint16_t*, int64_t, hipStream_t);

}  // namespace imq

namespace imq {
// int2 / int8 decode fast paths: not specialised yet -> caller falls back to the generic kernel.
template <int S, int SDT, int ZDT, bool STRIP, int MAXW>
int w2_launch_mw(const SkinnyArgs& a, size_t lds, int grid, int W, hipStream_t st) {
  const dim3 g(grid), b(64 * W);
  if (a.M == 1) return launch_with_lds(w2_skinny_kernel<S, 1, SDT, ZDT, STRIP, MAXW>, g, b, lds, st, a);
  if (a.M <= 4) return launch_with_lds(w2_skinny_kernel<S, 4, SDT, ZDT, STRIP, MAXW>, g, b, lds, st, a);
  return launch_with_lds(w2_skinny_kernel<S, 16, SDT, ZDT, STRIP, MAXW>, g, b, lds, st, a);
}

template <int S, int SDT, int ZDT, bool STRIP>
int w2_launch_m(const SkinnyArgs& a, size_t lds, int grid, int W, hipStream_t st) {
  if (W <= 8) return w2_launch_mw<S, SDT, ZDT, STRIP, 8>(a, lds, grid, W, st);
  if constexpr (S == 16 && SDT != IMQ_DT_BF16) return IMQ_ERR_UNSUPPORTED;   // never dispatched
  else return w2_launch_mw<S, SDT, ZDT, STRIP, 16>(a, lds, grid, W, st);
}

template <int S, int SDT, int ZDT>
int w2_dispatch_s(const SkinnyArgs& a0, const DevInfo& di, hipStream_t st) {
  SkinnyArgs a = a0;
  constexpr int SZB = (SDT == IMQ_DT_FP32) ? 4 : 2;
  constexpr int ZZB = (ZDT == IMQ_DT_FP32) ? 4 : 2;
  const int KS = a.Kpad / kStep2;
  const int NT = (a.N + 15) / 16;
  int W = (KS + S - 1) / S;
  if (W > 16) W = 16;
  if (W < 1) W = 1;
  auto need = [&](int cs) { return (size_t)a.M * (cs * kStep2 + kXPad) * 2 + (size_t)cs * 64 + (size_t)2 * W * 256 * 4; };
  int cs = KS;
  if (need(cs) > (size_t)di.max_lds) {
    // chunks of whole rounds (W*S steps) while they fit, else of S steps
    cs = ((KS + W * S - 1) / (W * S)) * W * S;
    while (cs > W * S && need(cs) > (size_t)di.max_lds) cs -= W * S;
    while (cs > S && need(cs) > (size_t)di.max_lds) cs -= S;
    if (need(cs) > (size_t)di.max_lds) return IMQ_ERR_UNSUPPORTED;
  }
  a.chunk_steps = cs;
  const size_t lds = need(cs);
  // persistent workgroups: x is staged once per workgroup (resident) and amortized over tiles
  const int grid = skinny_grid(NT, W, lds, di);
  const bool strip = a.G == kStep2 && (KS % S) == 0 && (cs % S) == 0 && a.ssg == 1 && a.szg == 1 &&
                     ((uintptr_t)a.sc % 16) == 0 && ((uintptr_t)a.zr % 16) == 0 &&
                     ((a.ssn * SZB) % 16) == 0 && ((a.szn * ZZB) % 16) == 0;
  if (strip) return w2_launch_m<S, SDT, ZDT, true>(a, lds, grid, W, st);
  return w2_launch_m<S, SDT, ZDT, false>(a, lds, grid, W, st);
}

// S = 16 steps (4 KB of codes per wave per round); workgroups that need more than 8 waves with
// fp16/fp32 scale conversion take S = 8 so the 128-VGPR budget of 16-wave workgroups holds.
template <int SDT, int ZDT>
int w2_dispatch(const SkinnyArgs& a, const DevInfo& di, hipStream_t st) {
  const int KS = a.Kpad / kStep2;
  if (SDT != IMQ_DT_BF16 && (KS + 15) / 16 > 8) return w2_dispatch_s<8, SDT, ZDT>(a, di, st);
  return w2_dispatch_s<16, SDT, ZDT>(a, di, st);
}

// int2 line kernel plan (M <= 2, G == 64, K_pad a multiple of 512, unit group strides, same
// scale / zero dtype; restated by the CPU bounds model in the tests): S2 = 4 line-steps per wave
// at M == 1 (K_pad <= 32768), S2 = 2 at M == 2 (K_pad <= 16384). Larger M or K would hold more
// activation registers across the weight issue than the 16-wave budget of 128 VGPRs allows; they
// take the skinny kernel. Returns false when the line kernel does not take the call.
bool line2_plan(int64_t M, int64_t Kpad, int64_t G, int64_t N, int64_t sqn, int64_t sxm, int64_t ssn,
                int64_t ssg, int64_t szn, int64_t szg, int sdt, int zdt, int max_lds, int* S2o, int* Wo,
                size_t* ldso) {
  if (M < 1 || M > 2 || G != 64 || Kpad % kLine2 != 0 || sdt != zdt) return false;
  if (ssg != 1 || szg != 1 || N < 1) return false;
  const int vb = sdt == IMQ_DT_FP32 ? 4 : 2;
  if ((ssn * vb) % 4 != 0 || (szn * vb) % 4 != 0) return false;
  if (16 * sqn >= (int64_t(1) << 31) || M * sxm * 2 >= (int64_t(1) << 31)) return false;
  if (16 * ssn * vb >= (int64_t(1) << 31) || 16 * szn * vb >= (int64_t(1) << 31)) return false;
  const int64_t KL = Kpad / kLine2;
  const int S2 = M == 1 ? 4 : 2;
  const int64_t W = (KL + S2 - 1) / S2;
  if (W > 16) return false;
  const size_t lds = (size_t)W * line2_wave_lds((int)M, S2) + (size_t)W * M * 16 * 4;
  if (lds > (size_t)max_lds) return false;
  *S2o = S2;
  *Wo = (int)W;
  *ldso = lds;
  return true;
}

template <int SDT>
int line2_launch(const SkinnyArgs& a, int W, size_t lds, hipStream_t st) {
  const dim3 g((unsigned)((a.N + 15) / 16)), b(64 * W);
  if (a.M == 1) return launch_with_lds(w2_line_kernel<4, 1, SDT, 16>, g, b, lds, st, a);
  return launch_with_lds(w2_line_kernel<2, 2, SDT, 16>, g, b, lds, st, a);
}

int line_w2(const SkinnyArgs& a, int sdt, const DevInfo& di, hipStream_t st) {
  int S2, W;
  size_t lds;
  if (!line2_plan(a.M, a.Kpad, a.G, a.N, a.sqn, a.sxm, a.ssn, a.ssg, a.szn, a.szg, sdt, sdt, di.max_lds, &S2, &W,
                  &lds))
    return IMQ_ERR_UNSUPPORTED;
  switch (sdt) {
    case IMQ_DT_BF16: return line2_launch<IMQ_DT_BF16>(a, W, lds, st);
    case IMQ_DT_FP16: return line2_launch<IMQ_DT_FP16>(a, W, lds, st);
    case IMQ_DT_FP32: return line2_launch<IMQ_DT_FP32>(a, W, lds, st);
  }
  return IMQ_ERR_UNSUPPORTED;
}

// int2 K-split plan (4 < M <= 16, G == 64, K_pad a multiple of 512, N % 4 == 0, unit group strides,
// same scale / zero dtype; restated by the CPU bounds model in the tests): S2 = 2 line-steps (1024
// codes, the int4 K-split's split width) per split, NW = 4 row tiles per workgroup (three resident
// per CU at the kernel's register bound; measured at C3: 8 tiles per workgroup, one resident,
// M=8 1967 -> 2304 GB/s, M=16 1851 -> 2053).
#ifndef IMQ_KS2_S2
#define IMQ_KS2_S2 2
#endif
constexpr int kKs2S2 = IMQ_KS2_S2;
constexpr int kKs2NW = 4;
bool ksplit2_plan(int64_t M, int64_t Kpad, int64_t G, int64_t N, int64_t sqn, int64_t sxm, int64_t ssn,
                  int64_t ssg, int64_t szn, int64_t szg, int sdt, int zdt, int max_lds, int cus, int* splitso,
                  int* nwo, size_t* ldso) {
  if (M <= 4 || M > 16 || G != 64 || Kpad % kLine2 != 0 || Kpad <= 0 || sdt != zdt) return false;
  if (N % 4 != 0 || sxm % 8 != 0 || ssg != 1 || szg != 1 || N < 1 || N > (1 << 30) || Kpad > (1 << 28))
    return false;
  const int vb = sdt == IMQ_DT_FP32 ? 4 : 2;
  if ((ssn * vb) % 4 != 0 || (szn * vb) % 4 != 0) return false;
  if (16 * sqn >= (int64_t(1) << 31) || M * sxm * 2 >= (int64_t(1) << 31)) return false;
  if (16 * ssn * vb >= (int64_t(1) << 31) || 16 * szn * vb >= (int64_t(1) << 31)) return false;
  const int64_t splits = (Kpad / kLine2 + kKs2S2 - 1) / kKs2S2;
  const int nw = kKs2NW;
  const int64_t rbs = (N + 16 * nw - 1) / (16 * nw);
  if (splits * rbs > 0x7fffffff) return false;
  const size_t lds = (size_t)ksplit2_lds((int)M, kKs2S2, nw);
  if (lds > (size_t)max_lds) return false;
  *splitso = (int)splits;
  *nwo = nw;
  *ldso = lds;
  return true;
}

template <int SDT, int NW>
int ksplit2_launch(const SkinnyArgs& a, int splits, size_t lds, hipStream_t st) {
  const int rbs = (a.N + 16 * NW - 1) / (16 * NW);
  const dim3 g((unsigned)(splits * rbs)), b(64 * NW);
  int rc;
  if (a.M <= 8) rc = launch_with_lds(w2_ksplit_kernel<kKs2S2, 8, SDT, NW>, g, b, lds, st, a);
  else rc = launch_with_lds(w2_ksplit_kernel<kKs2S2, 16, SDT, NW>, g, b, lds, st, a);
  if (rc != IMQ_OK) return rc;
  const int n4 = a.N / 4;
  splitk_rows_reduce_kernel<<<dim3((unsigned)((a.M * n4 + 255) / 256)), dim3(256), 0, st>>>(a.part, splits, a.M,
                                                                                           a.N, a.y, a.sym);
  IMQ_LAUNCH_CHECK();
  return IMQ_OK;
}

int ksplit_w2(const SkinnyArgs& a0, int sdt, void* ws, int64_t wsb, const DevInfo& di, hipStream_t st) {
  int splits, nw;
  size_t lds;
  // line-tiled weights below 5 rows (the line kernel declined: M 3..4, or K too long for its 16
  // waves; the skinny kernel reads rows): the plan of 5 rows, whose LDS covers the staging of fewer
  const int64_t pm = a0.tiled && a0.M < 5 ? 5 : a0.M;
  if (!ksplit2_plan(pm, a0.Kpad, a0.G, a0.N, a0.sqn, a0.sxm, a0.ssn, a0.ssg, a0.szn, a0.szg, sdt, sdt,
                    di.max_lds, di.cus, &splits, &nw, &lds))
    return IMQ_ERR_UNSUPPORTED;
  const int64_t need = (int64_t)splits * a0.M * a0.N * 4;
  if (!ws || wsb < need || ((uintptr_t)ws & 15)) return IMQ_ERR_UNSUPPORTED;
  if (((uintptr_t)a0.y & 7) || (a0.sym & 3)) return IMQ_ERR_UNSUPPORTED;   // 8-byte y stores
  SkinnyArgs a = a0;
  a.part = (float*)ws;
  switch (sdt) {
    case IMQ_DT_BF16: return ksplit2_launch<IMQ_DT_BF16, kKs2NW>(a, splits, lds, st);
    case IMQ_DT_FP16: return ksplit2_launch<IMQ_DT_FP16, kKs2NW>(a, splits, lds, st);
    case IMQ_DT_FP32: return ksplit2_launch<IMQ_DT_FP32, kKs2NW>(a, splits, lds, st);
  }
  return IMQ_ERR_UNSUPPORTED;
}

// The int2 K-split kernel's partials [splits][M][N] where it may run: 4 < M <= 16, and on
// line-tiled weights also M 3..4 and the M <= 2 shapes whose K is too long for the line kernel
// (more than 16 waves of its line-steps).
int64_t ksplit2_workspace_bytes(int64_t M, int64_t N, int64_t Kpad) {
  if (M < 1 || M > 16 || N <= 0 || Kpad <= 0 || Kpad % kLine2 != 0) return 0;
  const int64_t KL = Kpad / kLine2;
  if (M <= 2 && (KL + (M == 1 ? 4 : 2) - 1) / (M == 1 ? 4 : 2) <= 16) return 0;
  return (KL + kKs2S2 - 1) / kKs2S2 * M * N * 4;
}

// ws / wsb: the caller's optional workspace (the K-split path of 4 < M <= 16 needs one).
// tiled: qweight in the line-tiled layout; only the line and K-split kernels read it (the K-split
// kernel then also takes every M the line kernel declines), so a call neither takes returns
// IMQ_ERR_UNSUPPORTED.
int skinny_w2(const uint16_t* x, int64_t sxm, int64_t M, int64_t Kpad, const uint8_t* q, int64_t sqn,
              const void* sc, int64_t ssn, int64_t ssg, int sdt, const void* zr, int64_t szn, int64_t szg,
              int zdt, int64_t N, int64_t G, uint16_t* y, int64_t sym, void* ws, int64_t wsb, hipStream_t st,
              bool tiled) {
  if (M < 1 || M > 16 || G % kStep2 != 0 || Kpad % G != 0 || Kpad <= 0) return IMQ_ERR_UNSUPPORTED;
  if (((G / kStep2) & (G / kStep2 - 1)) != 0) return IMQ_ERR_UNSUPPORTED;   // groups of 2^k steps
  if (((uintptr_t)q & 15) || (sqn & 15) || ((uintptr_t)x & 15) || (sxm & 7)) return IMQ_ERR_UNSUPPORTED;
  if ((Kpad / kStep2) % 4 != 0) return IMQ_ERR_UNSUPPORTED;   // whole 4-step (64-byte) load units
  if (N > (1 << 30) || Kpad > (1 << 28)) return IMQ_ERR_UNSUPPORTED;
  if (sdt != zdt) return IMQ_ERR_UNSUPPORTED;
  const DevInfo di = device_info();
  SkinnyArgs a{x, sxm, (int)M, (int)Kpad, q, sqn, sc, ssn, ssg, zr, szn, szg, (int)N, (int)G, y, sym, 0};
  a.tiled = tiled ? 1 : 0;
  if (((uintptr_t)sc & 3) == 0 && ((uintptr_t)zr & 3) == 0) {
    int rc = line_w2(a, sdt, di, st);
    if (rc != IMQ_ERR_UNSUPPORTED) return rc;
    rc = ksplit_w2(a, sdt, ws, wsb, di, st);
    if (rc != IMQ_ERR_UNSUPPORTED) return rc;
  }
  if (tiled) return IMQ_ERR_UNSUPPORTED;
  switch (sdt) {
    case IMQ_DT_BF16: return w2_dispatch<IMQ_DT_BF16, IMQ_DT_BF16>(a, di, st);
    case IMQ_DT_FP16: return w2_dispatch<IMQ_DT_FP16, IMQ_DT_FP16>(a, di, st);
    case IMQ_DT_FP32: return w2_dispatch<IMQ_DT_FP32, IMQ_DT_FP32>(a, di, st);
  }
  return IMQ_ERR_INVALID;
}
template <int SDT, int MAXW, bool TL>
int w8_launch_tl(const SkinnyArgs& a, size_t lds, int grid, int W, hipStream_t st) {
  constexpr int S = 8;
  const dim3 g(grid), b(64 * W);
  if (a.M == 1) return launch_with_lds(w8_skinny_kernel<S, 1, SDT, MAXW, TL>, g, b, lds, st, a);
  if (a.M <= 4) return launch_with_lds(w8_skinny_kernel<S, 4, SDT, MAXW, TL>, g, b, lds, st, a);
  return launch_with_lds(w8_skinny_kernel<S, 16, SDT, MAXW, TL>, g, b, lds, st, a);
}

template <int SDT, int MAXW>
int w8_launch_mw(const SkinnyArgs& a, size_t lds, int grid, int W, hipStream_t st) {
  if (a.tiled) return w8_launch_tl<SDT, MAXW, true>(a, lds, grid, W, st);
  return w8_launch_tl<SDT, MAXW, false>(a, lds, grid, W, st);
}

template <int SDT>
int w8_dispatch(const SkinnyArgs& a0, const DevInfo& di, hipStream_t st) {
  SkinnyArgs a = a0;
  constexpr int S = 8;                     // 8 x 16 bytes per lane = 8 KB per wave per round
  const int KS = a.Kpad / kStep8;
  const int NT = (a.N + 15) / 16;
  int W = (KS + S - 1) / S;
  if (W > 16) W = 16;
  if (W < 1) W = 1;
  auto need = [&](int cs) {
    return (size_t)a.M * (cs * kStep8 + kXPad) * 2 + (size_t)cs * 64 + 64 + (size_t)2 * W * 256 * 4;
  };
  int cs = KS;
  if (need(cs) > (size_t)di.max_lds) {
    cs = ((KS + W * S - 1) / (W * S)) * W * S;
    while (cs > W * S && need(cs) > (size_t)di.max_lds) cs -= W * S;
    while (cs > S && need(cs) > (size_t)di.max_lds) cs -= S;
    if (need(cs) > (size_t)di.max_lds) return IMQ_ERR_UNSUPPORTED;
  }
  a.chunk_steps = cs;
  const size_t lds = need(cs);
  const int grid = skinny_grid(NT, W, lds, di);
  if (W <= 8) return w8_launch_mw<SDT, 8>(a, lds, grid, W, st);
  return w8_launch_mw<SDT, 16>(a, lds, grid, W, st);
}

// int8 line kernel plan (M <= 4, K a multiple of 128; restated by the CPU bounds model in the
// tests): S2 = 4 line-steps per wave (8 when K needs more than 16 waves of 4), W <= 16 waves.
bool line8_plan(int64_t M, int64_t K, int64_t N, int64_t sqn, int64_t sxm, int max_lds, int* S2o, int* Wo,
                size_t* ldso) {
  if (M < 1 || M > 4 || K <= 0 || K % kLine8 != 0 || N < 1) return false;
  if (16 * sqn >= (int64_t(1) << 31) || M * sxm * 2 >= (int64_t(1) << 31)) return false;
  const int64_t KL = K / kLine8;
  int S2 = 4;
  if ((KL + S2 - 1) / S2 > 16) S2 = 8;
  const int64_t W = (KL + S2 - 1) / S2;
  if (W > 16) return false;
  const int rc = M <= 2 ? (int)M : 4;
  const size_t lds = (size_t)W * line8_wave_lds((int)M, S2) + (size_t)W * rc * 16 * 4;
  if (lds > (size_t)max_lds) return false;
  *S2o = S2;
  *Wo = (int)W;
  *ldso = lds;
  return true;
}

template <int S2, int SDT>
int line8_launch(const SkinnyArgs& a, int W, size_t lds, hipStream_t st) {
  const dim3 g((unsigned)((a.N + 15) / 16)), b(64 * W);
  if (a.M == 1) return launch_with_lds(w8_line_kernel<S2, 1, SDT, 16>, g, b, lds, st, a);
  if (a.M == 2) return launch_with_lds(w8_line_kernel<S2, 2, SDT, 16>, g, b, lds, st, a);
  return launch_with_lds(w8_line_kernel<S2, 4, SDT, 16>, g, b, lds, st, a);
}

template <int SDT>
int line8_dispatch(const SkinnyArgs& a, int S2, int W, size_t lds, hipStream_t st) {
  if (S2 == 8) return line8_launch<8, SDT>(a, W, lds, st);
  return line8_launch<4, SDT>(a, W, lds, st);
}

// tiled: q in the line-tiled layout (N a multiple of 16, dense rows of K a multiple of 128 bytes):
// the line kernel and the skinny kernel's tiled form read it.
int skinny_w8(const uint16_t* x, int64_t sxm, int64_t M, int64_t K, const int8_t* q, int64_t sqn,
              const void* sc, int64_t ssn, int sdt, int64_t N, uint16_t* y, int64_t sym, hipStream_t st,
              bool tiled) {
  if (M < 1 || M > 16 || K <= 0 || K % kStep8 != 0) return IMQ_ERR_UNSUPPORTED;
  if (((uintptr_t)q & 15) || (sqn & 15) || ((uintptr_t)x & 15) || (sxm & 7)) return IMQ_ERR_UNSUPPORTED;
  if (N > (1 << 30) || K > (1 << 28)) return IMQ_ERR_UNSUPPORTED;
  if (tiled && (N % 16 != 0 || K % kLine8 != 0 || sqn != K)) return IMQ_ERR_UNSUPPORTED;
  const DevInfo di = device_info();
  SkinnyArgs a{x, sxm, (int)M, (int)K, nullptr, sqn, sc, ssn, 0, nullptr, 0, 0, (int)N, 0, y, sym, 0};
  a.q8 = q;
  a.tiled = tiled ? 1 : 0;
  {
    int S2, W;
    size_t lds;
    if (line8_plan(M, K, N, sqn, sxm, di.max_lds, &S2, &W, &lds)) {
      switch (sdt) {
        case IMQ_DT_BF16: return line8_dispatch<IMQ_DT_BF16>(a, S2, W, lds, st);
        case IMQ_DT_FP16: return line8_dispatch<IMQ_DT_FP16>(a, S2, W, lds, st);
        case IMQ_DT_FP32: return line8_dispatch<IMQ_DT_FP32>(a, S2, W, lds, st);
      }
      return IMQ_ERR_INVALID;
    }
  }
  switch (sdt) {
    case IMQ_DT_BF16: return w8_dispatch<IMQ_DT_BF16>(a, di, st);
    case IMQ_DT_FP16: return w8_dispatch<IMQ_DT_FP16>(a, di, st);
    case IMQ_DT_FP32: return w8_dispatch<IMQ_DT_FP32>(a, di, st);
  }
  return IMQ_ERR_INVALID;
}

// The decode launchers' plans for a shape, without a device: the same plan functions the
// launchers call, with the device's LDS bytes and CU count as arguments. in = {M, K_pad, G, N,
// q_row_stride, x_row_stride, s_stride_n, s_dtype, max_lds, cus} (unit group strides, zero
// strides and dtype equal to the scale's); out = {taken, p1, p2, p3, lds}.
int decode_plan_query(int kind, const int64_t* in, int64_t* out) {
  const int64_t M = in[0], Kpad = in[1], G = in[2], N = in[3], sqn = in[4], sxm = in[5], ssn = in[6];
  const int sdt = (int)in[7], max_lds = (int)in[8], cus = (int)in[9];
  int p1 = 0, p2 = 0, p3 = 0;
  size_t lds = 0;
  bool ok = false;
  switch (kind) {
    case IMQ_PLAN_W4_LINE:
      ok = line_plan(M, Kpad, G, N, sqn, sxm, ssn, 1, ssn, 1, sdt, sdt, max_lds, &p1, &p2, &lds);
      break;
    case IMQ_PLAN_W4_KSPLIT:
      ok = ksplit_plan(M, Kpad, G, N, sqn, sxm, ssn, 1, ssn, 1, sdt, sdt, max_lds, cus, &p1, &p2, &p3, &lds);
      break;
    case IMQ_PLAN_W4_WSPLIT:
      p1 = wsplit_plan(M, Kpad, G, N, sqn, sxm, ssn, 1, ssn, 1, sdt, sdt, max_lds, cus);
      ok = p1 != 0;
      if (ok) {
        p2 = kWsNW;
        lds = (size_t)wsplit_lds(p1, kWsNW);
      }
      break;
    case IMQ_PLAN_W4_SKINNY:
      if (Kpad <= 0 || Kpad % kStep != 0 || N < 1) break;
      skinny_shape((int)(Kpad / kStep), (int)((N + 15) / 16), sdt == IMQ_DT_BF16, &p1, &p2);
      ok = true;
      break;
    case IMQ_PLAN_W2_LINE:
      ok = line2_plan(M, Kpad, G, N, sqn, sxm, ssn, 1, ssn, 1, sdt, sdt, max_lds, &p1, &p2, &lds);
      break;
    case IMQ_PLAN_W2_KSPLIT:
      ok = ksplit2_plan(M, Kpad, G, N, sqn, sxm, ssn, 1, ssn, 1, sdt, sdt, max_lds, cus, &p1, &p2, &lds);
      break;
    case IMQ_PLAN_W8_LINE:
      ok = line8_plan(M, Kpad, N, sqn, sxm, max_lds, &p1, &p2, &lds);
      break;
    default:
      return IMQ_ERR_INVALID;
  }
  out[0] = ok ? 1 : 0;
  out[1] = ok ? p1 : 0;
  out[2] = ok ? p2 : 0;
  out[3] = ok ? p3 : 0;
  out[4] = ok ? (int64_t)lds : 0;
  return IMQ_OK;
}
}  // namespace imq
