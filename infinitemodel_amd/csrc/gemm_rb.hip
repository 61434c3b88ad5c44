// Prefill-regime fused dequant GEMM with the weights dequantized straight into MFMA B operands
// ("register-B" form), for int4 group-wise and int8 per-row weights on gfx950.
//
// y[M, N] = x[M, K] . dequant(W[N, K])^T, bf16 activations, fp32 accumulation, bf16 output: the
// contract of the reference's `_k` / `_k8` GEMM kernels (worker_quant.py:1098-1126, 953-980).
//
// Structure. A workgroup of NW waves computes a BM x (64 NW) output tile; wave w owns all BM rows
// of columns [64 w, 64 w + 64), as IB x 2 blocks of v_mfma_f32_32x32x16_bf16 (BM = 32 IB).
//   * Activations: the workgroup stages the BM x 64 tile of each K step in LDS (three buffers,
//     XOR-swizzled 16-byte chunks, one barrier per step), loaded from global two steps ahead;
//     every wave reads all BM rows from LDS, one MFMA slice ahead of use.
//   * Weights never touch LDS: each wave loads its own 64 columns' packed bytes from global memory
//     (one 16-byte load per lane per 32-column block per step for int4, two for int8, two steps
//     ahead) and converts them in registers into the MFMA B fragments -- every weight is
//     dequantized exactly once per workgroup and the LDS carries only the activations, so LDS
//     bytes per flop are 1 / 64 (against 1 / 32 for a 64 x 64 wave tile with both operands in LDS).
//   * K order inside a step is permuted consistently for A and B: MFMA slice s of half h
//     (lanes 32 h .. 32 h + 31) covers K [32 h + 8 s, +8), so a lane's B codes for the whole step
//     are 32 consecutive columns of its row (one contiguous load) and its A chunks are LDS chunks
//     4 h + s. The sum over K is unchanged.
//   * int4: w = bf16((q - z) s) with z, s taken to bf16 first -- the exact product rounded once,
//     the reference GEMM's weight tile (worker_quant.py:1121-1122). int8: the exact integer, the
//     per-row scale applied to the fp32 accumulator in the epilogue.
//   * Tiles are dealt XCD-aware and in groups of 8 tile-rows (as the LDS-dequant GEMM); when the
//     tiles do not fill the CUs K is split across workgroups into fp32 partials [split][M][N]
//     that a second launch sums in split order.
#include "imq_common.h"

#include <type_traits>

namespace imq {

int64_t rb_workspace_bytes(int bits, int64_t M, int64_t N, int64_t K, int cus);

namespace {

constexpr int RB_GROUP_M = 8;
constexpr int RB_BK = 64;
// VALU instructions the scheduler places after each MFMA (int4 dequant / int8 conversion work):
// chosen per format as the pattern that keeps the 256-row variants within the register file.
#ifndef RB_VALU_PER_MFMA_4
#define RB_VALU_PER_MFMA_4 5
#endif
#ifndef RB_VALU_PER_MFMA_8
#define RB_VALU_PER_MFMA_8 3
#endif

struct RbArgs {
  const uint16_t* x;
  int64_t sxm;
  int M, K;
  const uint8_t* q;
  int64_t sqn;
  const void* sc;
  int64_t ssn, ssg;
  const void* zr;
  int64_t szn, szg;
  int N, gsh;
  uint16_t* y;
  int64_t sym;
  int tiles_m, tiles_n;
  int splits, kps;
  float* part;
};

IMQ_DEV int rb_swz(int row, int c) { return (row * 8 + (c ^ ((row >> 1) & 7))) * 8; }

// w & m computed in a register the compiler cannot see through, so the byte extractions below
// stay single v_cvt_f32_ubyteN instructions instead of being re-folded into per-nibble bit-field
// extracts (the result only feeds VALU conversions, never an MFMA operand directly).
IMQ_DEV uint32_t rb_and(uint32_t w, uint32_t m) {
  uint32_t r;
  asm("v_and_b32 %0, %1, %2" : "=v"(r) : "v"(w), "v"(m));
  return r;
}

// 8 int4 codes of one dword (code i at bits 4i) -> 4 dwords of bf16 (c - z) s in K order: the
// even codes sit in the bytes of lo, the odd ones in the bytes of hi, each one v_cvt_f32_ubyteN
// from fp32; fma(c, s, -z s) is the exact (c - z) s, rounded once by the pack.
IMQ_DEV u32x4_t rb_dequant4(uint32_t w, float s, float nzs) {
  const uint32_t lo = rb_and(w, 0x0F0F0F0Fu), hi = rb_and(w >> 4, 0x0F0F0F0Fu);
  u32x4_t r;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float c0 = (float)((lo >> (8 * i)) & 0xffu);
    const float c1 = (float)((hi >> (8 * i)) & 0xffu);
    r[i] = cvt_pk_bf16(fmaf(c0, s, nzs), fmaf(c1, s, nzs));
  }
  return r;
}

// 8 int8 codes (two dwords) -> 4 dwords of bf16, exact.
IMQ_DEV u32x4_t rb_convert8(uint32_t lo, uint32_t hi) {
  u32x4_t r;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const uint32_t w = i ? hi : lo;
    r[2 * i] = cvt_pk_bf16((float)(int8_t)(w & 0xff), (float)(int8_t)((w >> 8) & 0xff));
    r[2 * i + 1] = cvt_pk_bf16((float)(int8_t)((w >> 16) & 0xff), (float)(int8_t)(w >> 24));
  }
  return r;
}

template <int BITS, int SDT, int ZDT, int IB, int NW>
__global__ __launch_bounds__(64 * NW, 1) void gemm_rb_kernel(RbArgs a) {
  constexpr int BM = 32 * IB, BN = 64 * NW, BK = RB_BK, NTHR = 64 * NW;
  constexpr int A_EL = BM * BK;                    // bf16 elements of one LDS buffer
  constexpr int XC = BM * 8 / NTHR;                // 16-byte activation chunks per thread per step
  constexpr int QV = BITS == 8 ? 2 : 1;            // 16-byte weight loads per lane per column block
  static_assert((BM * 8) % NTHR == 0, "activation chunks must divide evenly");
  extern __shared__ __align__(16) uint16_t lds[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int h = lane >> 5, c = lane & 31;

  // ---- tile mapping: XCD-aware, grouped by RB_GROUP_M tile-rows; split-K index outermost ------
  const int T = a.tiles_m * a.tiles_n;
  const int split = blockIdx.x / T;
  int L = blockIdx.x - split * T;
  if ((T & 7) == 0) L = (L & 7) * (T >> 3) + (L >> 3);
  const int per_group = RB_GROUP_M * a.tiles_n;
  const int grp = L / per_group;
  const int first_m = grp * RB_GROUP_M;
  const int gm = (a.tiles_m - first_m) < RB_GROUP_M ? (a.tiles_m - first_m) : RB_GROUP_M;
  const int in_grp = L - grp * per_group;
  const int m0 = (first_m + in_grp % gm) * BM;
  const int n0 = (in_grp / gm) * BN;

  // ---- activation load plan (32-bit offsets from the tile's first row) -------------------------
  const uint16_t* xtile = a.x + (int64_t)m0 * a.sxm;
  int xo[XC], xl[XC];
#pragma unroll
  for (int j = 0; j < XC; ++j) {
    const int id = tid + NTHR * j;
    const int row = id >> 3, ch = id & 7;
    const int r = m0 + row < a.M ? row : a.M - 1 - m0;
    xo[j] = (int)(r * a.sxm) + ch * 8;
    xl[j] = rb_swz(row, ch);
  }

  // ---- weight load plan: columns n0 + 64 wave + 32 j + c, K bytes [32 h, +32) codes per step ---
  const uint8_t* qb[2];
  int64_t sb[2], zb[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    int n = n0 + 64 * wave + 32 * j + c;
    n = n < a.N ? n : a.N - 1;
    qb[j] = a.q + (int64_t)n * a.sqn + (BITS == 8 ? 32 : 16) * h;
    sb[j] = (int64_t)n * a.ssn;
    zb[j] = (int64_t)n * a.szn;
  }

  u32x4_t xr[2][XC];
  u32x4_t qr[2][2][QV];
  uint32_t sr[2][2], zr[2][2];
  const int kt0 = split * a.kps;
  const int KT = (a.K / BK - kt0) < a.kps ? (a.K / BK - kt0) : a.kps;

  auto load_a = [&](auto setc, int ktl) {
    constexpr int set = decltype(setc)::value;
    const int kt = kt0 + (ktl < KT ? ktl : KT - 1);
#pragma unroll
    for (int j = 0; j < XC; ++j) xr[set][j] = *(const u32x4_t*)(xtile + kt * BK + xo[j]);
  };
  auto load_b = [&](auto setc, int ktl) {
    constexpr int set = decltype(setc)::value;
    const int kt = kt0 + (ktl < KT ? ktl : KT - 1);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
#pragma unroll
      for (int v = 0; v < QV; ++v) qr[set][j][v] = *(const u32x4_t*)(qb[j] + kt * (BK * BITS / 8) + 16 * v);
      if constexpr (BITS != 8) {
        const int g = (kt * BK + 32 * h) >> a.gsh;
        sr[set][j] = load_raw_bits<SDT>(a.sc, sb[j] + (int64_t)g * a.ssg);
        zr[set][j] = load_raw_bits<ZDT>(a.zr, zb[j] + (int64_t)g * a.szg);
      }
    }
  };
  auto store_a = [&](auto setc, uint16_t* A) {
    constexpr int set = decltype(setc)::value;
#pragma unroll
    for (int j = 0; j < XC; ++j) *(u32x4_t*)(A + xl[j]) = xr[set][j];
  };

  f32x16_t acc[IB][2];
#pragma unroll
  for (int i = 0; i < IB; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
  int aoff[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) aoff[s] = rb_swz(c, 4 * h + s);   // + 32 rows (2048 elements) per i

  bf16x8_t af[2][IB];        // A fragments of slice s live in af[s & 1], B fragments in bq[s & 1]
  bf16x8_t bq[2][2];         // (4 slices: the parity pattern repeats every step)
  auto read_frags = [&](auto pc, const uint16_t* A, int s) {
    constexpr int p = decltype(pc)::value;
#pragma unroll
    for (int i = 0; i < IB; ++i) af[p][i] = *(const bf16x8_t*)(A + aoff[s] + i * 32 * BK);
  };

  // The scale / zero of a B register set as (s, -z s), both taken to bf16 first.
  auto scale_pair = [&](auto bsc, float* sv, float* nz) {
    constexpr int bs = decltype(bsc)::value;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      if constexpr (BITS != 8) {
        float s_ = raw_bits_to_f32<SDT>(sr[bs][j]);
        float z_ = raw_bits_to_f32<ZDT>(zr[bs][j]);
        if constexpr (SDT != IMQ_DT_BF16) s_ = round_to<IMQ_DT_BF16>(s_);
        if constexpr (ZDT != IMQ_DT_BF16) z_ = round_to<IMQ_DT_BF16>(z_);
        sv[j] = s_;
        nz[j] = -z_ * s_;
      } else {
        sv[j] = nz[j] = 0.f;
      }
    }
  };
  auto b_frag = [&](auto bsc, int s, int j, float sv, float nz) -> bf16x8_t {
    constexpr int bs = decltype(bsc)::value;
    u32x4_t d;
    if constexpr (BITS == 8) d = rb_convert8(qr[bs][j][s >> 1][2 * (s & 1)], qr[bs][j][s >> 1][2 * (s & 1) + 1]);
    else d = rb_dequant4(qr[bs][j][0][s], sv, nz);
    return __builtin_bit_cast(bf16x8_t, d);
  };

  // LDS: three buffers of BM x 64 activations; step kt reads buffer kt % 3 and writes A(kt+1) into
  // buffer (kt+1) % 3, whose last reads (steps kt-2 and the slice-0 prefetch at the end of kt-3)
  // all precede the barrier of step kt-1 -- so one barrier per step suffices, placed after
  // slice 1 once its MFMAs are queued.
  //
  // Step kt (B register set kt & 1, A register set (kt+1) & 1 holding A(kt+1)):
  //   slice s: dequantize B(kt) slice s; read the A fragments of slice s+1 (slice 0 of step
  //            kt+1 from the new buffer at s = 3); MFMAs of slice s on the fragments read one
  //            slice earlier;
  //   slice 0: also write A(kt+1) into the next buffer;
  //   slice 1: then wait for the LDS writes, barrier, and load A(kt+3) into the freed A set;
  //   after slice 3: load B(kt+2) into the freed B set.
  auto step = [&](int kt, int rb, int wb, auto bsc) {
    constexpr int bs = decltype(bsc)::value;     // kt & 1
    constexpr int as = 1 - bs;                   // A(kt+1) lives in set (kt+1) & 1
    const uint16_t* Ar = lds + rb * A_EL;
    uint16_t* Aw = lds + wb * A_EL;
    float sv[2], nz[2];
    scale_pair(bsc, sv, nz);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      // operands of the next slice (slice 0 of step kt+1 at s = 3) into the other register pair,
      // while this slice's MFMAs read the pair filled one slice earlier
      if (s < 3) {
        if ((s & 1) == 0) {
#pragma unroll
          for (int j = 0; j < 2; ++j) bq[1][j] = b_frag(bsc, s + 1, j, sv[j], nz[j]);
          read_frags(std::integral_constant<int, 1>{}, Ar, s + 1);
        } else {
#pragma unroll
          for (int j = 0; j < 2; ++j) bq[0][j] = b_frag(bsc, s + 1, j, sv[j], nz[j]);
          read_frags(std::integral_constant<int, 0>{}, Ar, s + 1);
        }
      } else {
        float sv2[2], nz2[2];
        scale_pair(std::integral_constant<int, 1 - bs>{}, sv2, nz2);
#pragma unroll
        for (int j = 0; j < 2; ++j) bq[0][j] = b_frag(std::integral_constant<int, 1 - bs>{}, 0, j, sv2[j], nz2[j]);
        read_frags(std::integral_constant<int, 0>{}, Aw, 0);
      }
      if ((s & 1) == 0) {
#pragma unroll
        for (int i = 0; i < IB; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j) acc[i][j] = mfma32x32x16(af[0][i], bq[0][j], acc[i][j]);
      } else {
#pragma unroll
        for (int i = 0; i < IB; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j) acc[i][j] = mfma32x32x16(af[1][i], bq[1][j], acc[i][j]);
      }
      if (s == 0) store_a(std::integral_constant<int, as>{}, Aw);
      if (s == 1) {
        lds_barrier();
        load_a(std::integral_constant<int, as>{}, kt + 3);
        __builtin_amdgcn_sched_barrier(0);
      }
      // one MFMA, then a few VALU and one LDS read, repeated: keeps the dequant and the fragment
      // reads between MFMAs instead of bunched before them
#pragma unroll
      for (int k = 0; k < 2 * IB; ++k) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, BITS == 8 ? RB_VALU_PER_MFMA_8 : RB_VALU_PER_MFMA_4, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    load_b(bsc, kt + 2);
    __builtin_amdgcn_sched_barrier(0);
  };

  // Prologue, in the loop's steady-state load order (A(kt+1), B(kt), A(kt+2), B(kt+1) outstanding
  // at the top of step kt) so the waits the compiler places at the loop head match the loop's:
  // A(0) is loaded and written to buffer 0 first, then A(1), B(0), A(2), B(1).
  load_a(std::integral_constant<int, 0>{}, 0);
  __builtin_amdgcn_sched_barrier(0);
  load_a(std::integral_constant<int, 1>{}, 1);
  __builtin_amdgcn_sched_barrier(0);
  load_b(std::integral_constant<int, 0>{}, 0);
  __builtin_amdgcn_sched_barrier(0);
  store_a(std::integral_constant<int, 0>{}, lds);
  __builtin_amdgcn_sched_barrier(0);
  load_a(std::integral_constant<int, 0>{}, 2);
  __builtin_amdgcn_sched_barrier(0);
  load_b(std::integral_constant<int, 1>{}, 1);
  __builtin_amdgcn_sched_barrier(0);
  lds_barrier();
  read_frags(std::integral_constant<int, 0>{}, lds, 0);
  {
    float sv0[2], nz0[2];
    scale_pair(std::integral_constant<int, 0>{}, sv0, nz0);
#pragma unroll
    for (int j = 0; j < 2; ++j) bq[0][j] = b_frag(std::integral_constant<int, 0>{}, 0, j, sv0[j], nz0[j]);
  }

  int rb = 0;
  int kt = 0;
  for (; kt + 1 < KT; kt += 2) {
    const int wb = rb == 2 ? 0 : rb + 1;
    step(kt, rb, wb, std::integral_constant<int, 0>{});
    const int wb2 = wb == 2 ? 0 : wb + 1;
    step(kt + 1, wb, wb2, std::integral_constant<int, 1>{});
    rb = wb2;
  }
  if (kt < KT) step(kt, rb, rb == 2 ? 0 : rb + 1, std::integral_constant<int, 0>{});

  // ---- epilogue: D lane l holds column l % 32, element r at row 8 (r / 4) + 4 (l / 32) + r % 4 ---
  if (a.splits > 1) {
    float* pbase = a.part + (size_t)split * a.M * a.N;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int n = n0 + 64 * wave + 32 * j + c;
      if (n >= a.N) continue;
#pragma unroll
      for (int i = 0; i < IB; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int m = m0 + 32 * i + 8 * (r >> 2) + 4 * h + (r & 3);
          if (m < a.M) pbase[(size_t)m * a.N + n] = acc[i][j][r];
        }
    }
    return;
  }
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int n = n0 + 64 * wave + 32 * j + c;
    if (n >= a.N) continue;
    float sc8 = 1.f;
    if constexpr (BITS == 8) sc8 = load_as_f32<SDT>(a.sc, (int64_t)n * a.ssn);
#pragma unroll
    for (int i = 0; i < IB; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = m0 + 32 * i + 8 * (r >> 2) + 4 * h + (r & 3);
        if (m < a.M) a.y[(int64_t)m * a.sym + n] = (uint16_t)cvt_pk_bf16(acc[i][j][r] * sc8, 0.f);
      }
  }
}

// y[m, n] = bf16(sum_s part[s][m][n] * scale[n]) over the splits in order; 4 columns per thread.
template <int BITS, int SDT>
__global__ __launch_bounds__(256) void rb_reduce_kernel(const float* __restrict__ part, int splits, int M, int N,
                                                        const void* __restrict__ sc, int64_t ssn,
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

// Tile plan (measured on the C4 shapes): 256 rows per wave (IB 8) whenever those tiles cover at
// least half of the CUs, else 128 rows (IB 4); then K is split in two or four while the grid still
// fits the CUs (each split costs a pass over fp32 partials), with at least 16 K steps per split.
#ifndef IMQ_RB_FORCE_IB
#define IMQ_RB_FORCE_IB 0
#endif
inline void rb_plan(int64_t M, int64_t N, int64_t K, int cus, int* ib, int* splits) {
  const int64_t T8 = imq_cdiv(M, 256) * imq_cdiv(N, 256), T4 = imq_cdiv(M, 128) * imq_cdiv(N, 256);
  *ib = IMQ_RB_FORCE_IB ? IMQ_RB_FORCE_IB : (M > 128 && 2 * T8 >= cus ? 8 : 4);
  const int64_t T = *ib == 8 ? T8 : T4;
  const int KT = (int)(K / RB_BK);
  int s = 1;
  while (s < 4 && 2 * T * s <= cus && KT / (2 * s) >= 16) s *= 2;
  *splits = s;
}

template <int BITS, int SDT, int ZDT, int IB>
int rb_launch(const RbArgs& a0, void* ws, int64_t wsb, hipStream_t st) {
  constexpr int NW = 4, BM = 32 * IB, BN = 64 * NW;
  RbArgs a = a0;
  a.tiles_m = (a.M + BM - 1) / BM;
  a.tiles_n = (a.N + BN - 1) / BN;
  const int64_t T = (int64_t)a.tiles_m * a.tiles_n;
  const int KT = a.K / RB_BK;
  int ib_plan, s;
  rb_plan(a.M, a.N, a.K, device_info().cus, &ib_plan, &s);
  const int64_t need = (int64_t)s * a.M * a.N * 4;
  if (s > 1 && (!ws || wsb < need || ((uintptr_t)ws & 15))) s = 1;
  a.splits = s;
  a.kps = (KT + s - 1) / s;
  a.part = s > 1 ? (float*)ws : nullptr;
  if (T * s > 0x7fffffff) return IMQ_ERR_UNSUPPORTED;
  const size_t lds = (size_t)3 * BM * RB_BK * 2;
  auto kern = gemm_rb_kernel<BITS, SDT, ZDT, IB, NW>;
  if (lds > 65536) {
    static int attr_set = 0;   // benign race: every caller sets the same value
    if (!__atomic_load_n(&attr_set, __ATOMIC_ACQUIRE)) {
      hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
      if (e != hipSuccess) return (int)e;
      __atomic_store_n(&attr_set, 1, __ATOMIC_RELEASE);
    }
  }
  kern<<<dim3((unsigned)(T * s)), dim3(64 * NW), lds, st>>>(a);
  IMQ_LAUNCH_CHECK();
  if (s > 1) {
    const int64_t total = (int64_t)a.M * ((a.N + 3) / 4);
    const int64_t blocks = imq_cdiv(total, 256) < 8192 ? imq_cdiv(total, 256) : 8192;
    rb_reduce_kernel<BITS, SDT><<<dim3((unsigned)blocks), dim3(256), 0, st>>>(a.part, s, a.M, a.N, a.sc, a.ssn, a.y,
                                                                             a.sym);
    IMQ_LAUNCH_CHECK();
  }
  return IMQ_OK;
}

template <int BITS, int SDT, int ZDT>
int rb_ib_dispatch(const RbArgs& a, void* ws, int64_t wsb, hipStream_t st) {
  int ib, s;
  rb_plan(a.M, a.N, a.K, device_info().cus, &ib, &s);
  if (ib == 8) return rb_launch<BITS, SDT, ZDT, 8>(a, ws, wsb, st);
  return rb_launch<BITS, SDT, ZDT, 4>(a, ws, wsb, st);
}

template <int BITS, int SDT>
int rb_z(const RbArgs& a, int zdt, void* ws, int64_t wsb, hipStream_t st) {
  if constexpr (BITS == 8) {
    return rb_ib_dispatch<8, SDT, SDT>(a, ws, wsb, st);
  } else {
    switch (zdt) {
      case IMQ_DT_BF16: return rb_ib_dispatch<BITS, SDT, IMQ_DT_BF16>(a, ws, wsb, st);
      case IMQ_DT_FP16: return rb_ib_dispatch<BITS, SDT, IMQ_DT_FP16>(a, ws, wsb, st);
      case IMQ_DT_FP32: return rb_ib_dispatch<BITS, SDT, IMQ_DT_FP32>(a, ws, wsb, st);
    }
    return IMQ_ERR_INVALID;
  }
}

}  // namespace

// Whether the register-B GEMM takes this call: int4 with power-of-two groups >= 32, or int8; K a
// multiple of 64; more than 512 rows (measured: at 512 rows and below the LDS-dequant GEMM's
// 128 / 256-row tiles with two waves per SIMD are as fast or faster).
bool rb_takes(int bits, int64_t M, int64_t N, int64_t K, int64_t G) {
  if (bits != 4 && bits != 8) return false;
  if (M <= 512 || N <= 0 || K <= 0 || K % RB_BK != 0) return false;
  if (bits == 4 && (G < 32 || (G & (G - 1)) != 0)) return false;
  return M <= 0x7fffffff && N <= 0x7fffffff && K <= 0x7fffffff;
}

int64_t rb_workspace_bytes(int bits, int64_t M, int64_t N, int64_t K, int cus) {
  if (!rb_takes(bits, M, N, K, 128)) return 0;
  int ib, s;
  rb_plan(M, N, K, cus, &ib, &s);
  return s > 1 ? (int64_t)s * M * N * 4 : 0;
}

// Launch for a call rb_takes accepted. Returns IMQ_ERR_UNSUPPORTED for layouts it does not cover
// (misaligned operands, offsets beyond 32 bits); the caller then uses the LDS-dequant GEMM.
int gemm_rb(int bits, const uint16_t* x, int64_t sxm, int64_t M, int64_t K, const uint8_t* q, int64_t sqn,
            const void* sc, int64_t ssn, int64_t ssg, int sdt, const void* zr, int64_t szn, int64_t szg, int zdt,
            int64_t N, int64_t G, uint16_t* y, int64_t sym, void* ws, int64_t wsb, hipStream_t st) {
  if (((uintptr_t)x & 15) || (sxm & 7) || ((uintptr_t)q & 15) || (sqn & 15)) return IMQ_ERR_UNSUPPORTED;
  if (sxm < 0 || sqn < 0 || 256 * sxm > 0x7fffffff) return IMQ_ERR_UNSUPPORTED;
  int gsh = 0;
  if (bits == 4) {
    while ((1 << gsh) < G) ++gsh;
    if (ssg < 0 || szg < 0) return IMQ_ERR_UNSUPPORTED;
  }
  RbArgs a{x, sxm, (int)M, (int)K, q, sqn, sc, ssn, ssg, zr, szn, szg, (int)N, gsh, y, sym, 0, 0, 1, 0, nullptr};
  switch (sdt) {
    case IMQ_DT_BF16: return bits == 8 ? rb_z<8, IMQ_DT_BF16>(a, zdt, ws, wsb, st) : rb_z<4, IMQ_DT_BF16>(a, zdt, ws, wsb, st);
    case IMQ_DT_FP16: return bits == 8 ? rb_z<8, IMQ_DT_FP16>(a, zdt, ws, wsb, st) : rb_z<4, IMQ_DT_FP16>(a, zdt, ws, wsb, st);
    case IMQ_DT_FP32: return bits == 8 ? rb_z<8, IMQ_DT_FP32>(a, zdt, ws, wsb, st) : rb_z<4, IMQ_DT_FP32>(a, zdt, ws, wsb, st);
  }
  return IMQ_ERR_INVALID;
}

}  // namespace imq
