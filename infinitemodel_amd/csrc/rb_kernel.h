// The register-B GEMM kernel (weights dequantized straight into MFMA B operands) for int4
// group-wise and int8 per-row weights on gfx950, shared by the dense launchers (gemm_rb.hip)
// and the grouped MoE launchers (moe_rb.hip).
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
#pragma once
#include "imq_common.h"

#include <type_traits>

namespace imq {
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
#ifndef RB_VALU_PER_MFMA_FOLD
#define RB_VALU_PER_MFMA_FOLD 4
#endif
// FOLD: 1 unpacks a step's four B slices at its top (step_fold), 0 one slice ahead (step)
#ifndef RB_FOLD_EARLY_UNPACK
#define RB_FOLD_EARLY_UNPACK 1
#endif
// Dense form: 1 loads activations, weights and scale / zero through buffer resources (see the kernel)
#ifndef IMQ_RB_BUF
#define IMQ_RB_BUF 1
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
  // grouped MoE forms (MOE != 0): a tile is (row block, column tile); mtl[2 b] = expert and
  // mtl[2 b + 1] = first sorted row of block b, *nmt blocks in all; off = [E + 1] sorted offsets,
  // perm = sorted position -> routed row
  const int32_t* mtl = nullptr;
  const int32_t* nmt = nullptr;
  const int32_t* off = nullptr;
  const int32_t* perm = nullptr;
  int64_t sqe = 0, sse = 0;           // expert strides: packed bytes, scale / zero elements
  int k = 1, I = 0;                   // top_k; intermediate size (gate_up)
  const void* bias = nullptr;         // per-expert row bias [E][rows] or null
  int64_t sbe = 0;
  int bdt = 0;
  float alpha = 0.f, limit = 0.f;     // gpt-oss activation
  float* yr = nullptr;                // MOE 3: fp32 rows [B][N] in routed order
  uint16_t* yrb = nullptr;            // MOE 3, instead: bf16 rows [B][N] in routed order
  // scale-folded form (FOLD): per-row sums of the activations over each group of 128 K,
  // rs[row][g] (row = token for gate_up, sorted position for down), groups >= rs_groups read 0;
  // gate_up also writes the group sums of its bf16 h rows into hrs[p][tn] (down's rs)
  const float* rs = nullptr;
  int rs_stride = 0, rs_groups = 0;
  float* hrs = nullptr;
  int hrs_stride = 0;
  // MoE forms: valid x columns (a multiple of the K step, <= K; 0 means K): the K steps past them
  // are skipped -- their activations are zero -- so rows need not be zero-padded to K
  int xk = 0;
};

// Bias element i as the raw aligned dword holding it (which lies in the element's page), read
// without a branch so it can go out with the first loads (a null bias reads `fb`'s first word);
// rb_bias_of converts it where it is used.
IMQ_DEV uint32_t rb_bias_word(const void* p, int dt, int64_t i, const void* fb, bool& hi) {
  const char* b = p != nullptr ? (const char*)p : (const char*)fb;
  const int64_t off = p != nullptr ? i * (dt == IMQ_DT_FP32 ? 4 : 2) : 0;
  const int mis = (int)(((uintptr_t)b + (uintptr_t)off) & 3);
  hi = mis != 0;
  return *(const uint32_t*)(b + off - mis);
}
IMQ_DEV float rb_bias_of(uint32_t w, bool hi, int dt) {
  const uint32_t h = hi ? (w >> 16) : (w & 0xffffu);
  return dt == IMQ_DT_FP32 ? __uint_as_float(w) : dt == IMQ_DT_FP16 ? f16_bits_to_f32(h) : bf16_bits_to_f32(h);
}

IMQ_DEV int rb_swz(int row, int c) { return (row * 8 + (c ^ ((row >> 1) & 7))) * 8; }

// A raw buffer resource over `base` (offsets are kept below 2^31 by the launcher, so the range
// check never clips) and its loads: the per-lane offset in a VGPR, the per-step one in an SGPR.
IMQ_DEV __amdgpu_buffer_rsrc_t rb_rsrc(const void* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, 0x7fffffff, 0x00020000);
}
IMQ_DEV u32x4_t rb_bload128(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, 0));
}
template <int DT>
IMQ_DEV uint32_t rb_bload_raw(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  if constexpr (DT == IMQ_DT_FP32) return __builtin_amdgcn_raw_buffer_load_b32(r, (int)voff, (int)soff, 0);
  else return __builtin_amdgcn_raw_buffer_load_b16(r, (int)voff, (int)soff, 0);
}

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

// MOE 0: the dense GEMM. Grouped MoE forms (int4; one hit expert's sorted rows per row block,
// gathered): MOE 1 gate_up with SiLU-GLU -- wave w's first column block holds gate rows, its
// second the matching up rows, so h = silu(gate) * up is formed in registers and written as bf16
// in sorted order; MOE 2 gpt-oss gate_up (interleaved gate / up rows in adjacent lanes, its
// clamped GLU); MOE 3 down (fp32 rows plus the row bias, scattered to routed order).
//
// PD: register sets of the global -> register pipeline; B(kt) is loaded PD steps ahead and A(kt)
// PD + 1 steps ahead (the dense GEMM's long steps need 2, the MoE forms' short ones more).
//
// FOLD (MoE forms, int4, groups of 128 = two K steps): the B operand is the exact bf16 128 + q
// (the code dropped into the mantissa of 0x4300: 7 integer ops per 8 codes instead of 23 for
// the dequantized bf16 (q - z) s), the MFMAs of one group accumulate into fresh registers which
// are folded into the total with the group's scale s -- sum_g s_g sum_{k in g} x_k (128 + q_k) --
// and the remaining -s_g (128 + z_g) sum_{k in g} x_k terms are one fp32 32x32x2 MFMA chain per
// block over the groups, from the rows' group sums rs. The activations' K order inside each
// 8-element chunk is permuted to the order the magic unpack produces. Every product is exact
// and no weight is rounded to bf16, so the sums are within fp32 accumulation error of the exact
// (q - z) s products (the dequantizing form rounds each weight to bf16 first).
// TL: the dense int4 form on weights in the line-tiled layout (16-byte pieces permuted within
// 16-row tiles), a separate instantiation so the row-layout loop is unchanged.
template <int BITS, int SDT, int ZDT, int IB, int NW, int MOE = 0, int PD = 2, bool FOLD = false, bool TL = false>
__global__ __launch_bounds__(64 * NW, 1) void gemm_rb_kernel(RbArgs a) {
  static_assert(!FOLD || (MOE != 0 && BITS == 4 && PD % 2 == 0), "the folded form: int4 MoE, even pipeline depth");
  static_assert(!TL || MOE == 0, "line-tiled weights: the dense forms");
  constexpr int BM = 32 * IB, BN = 64 * NW, BK = RB_BK, NTHR = 64 * NW;
  constexpr int A_EL = BM * BK;                    // bf16 elements of one LDS buffer
  constexpr int XC = BM * 8 / NTHR;                // 16-byte activation chunks per thread per step
  constexpr int QV = BITS == 8 ? 2 : 1;            // 16-byte weight loads per lane per column block
  static_assert((BM * 8) % NTHR == 0, "activation chunks must divide evenly");
  extern __shared__ __align__(16) uint16_t lds[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int h = lane >> 5, c = lane & 31;

  // ---- tile mapping ------------------------------------------------------------------------------
  int split = 0, m0 = 0, n0, tn = 0;
  int e = 0, prow0 = 0, cnt = 0;                    // MOE: expert, first sorted row, rows of the block
  if constexpr (MOE == 0) {
    // XCD-aware, grouped by RB_GROUP_M tile-rows; split-K index outermost
    const int T = a.tiles_m * a.tiles_n;
    split = blockIdx.x / T;
    int L = blockIdx.x - split * T;
    if ((T & 7) == 0) L = (L & 7) * (T >> 3) + (L >> 3);
    const int per_group = RB_GROUP_M * a.tiles_n;
    const int grp = L / per_group;
    const int first_m = grp * RB_GROUP_M;
    const int gm = (a.tiles_m - first_m) < RB_GROUP_M ? (a.tiles_m - first_m) : RB_GROUP_M;
    const int in_grp = L - grp * per_group;
    m0 = (first_m + in_grp % gm) * BM;
    n0 = (in_grp / gm) * BN;
  } else {
    // The grid covers the most blocks the routing can produce; the Tr tiles that exist are dealt
    // so that dispatch index b (which runs on XCD b % 8) gets a contiguous run of tiles per XCD,
    // column tiles fastest: the tiles reading one block's gathered rows share an L2.
    const int Tr = *a.nmt * a.tiles_n;
    const int b = blockIdx.x;
    if (b >= Tr) return;                            // uniform over the workgroup
    const int x8 = b & 7, q8 = Tr >> 3, r8 = Tr & 7;
    const int lid = x8 * q8 + (x8 < r8 ? x8 : r8) + (b >> 3);
    const int mt = lid / a.tiles_n;
    tn = lid - mt * a.tiles_n;
    const int ec = a.mtl[2 * mt];                   // expert | rows of the block (<= BM) << 16
    e = ec & 0xffff;
    cnt = ec >> 16;
    prow0 = a.mtl[2 * mt + 1];
    n0 = tn * BN;
  }
  // MoE forms: the epilogue's row biases of this lane (MOE 1: gate and up column; MOE 2: the gate
  // / up pair of both column blocks; MOE 3: both column blocks), read before the K loop
  constexpr int NBW = MOE == 2 ? 4 : 2;
  uint32_t bw_w[NBW];
  bool bw_h[NBW];
  if constexpr (MOE != 0) {
#pragma unroll
    for (int q = 0; q < NBW; ++q) {
      int row;
      if constexpr (MOE == 1) {
        row = (q ? a.I : 0) + tn * (32 * NW) + 32 * (tid >> 6) + (tid & 31);
      } else {
        const int n = n0 + 64 * (tid >> 6) + 32 * (MOE == 2 ? q >> 1 : q) + (tid & 31) + (MOE == 2 ? (q & 1) : 0);
        row = n < a.N ? n : a.N - 1;
      }
      bw_w[q] = rb_bias_word(a.bias, a.bdt, (int64_t)e * a.sbe + row, a.q, bw_h[q]);
    }
  }

  // ---- activation load plan (32-bit offsets from the tile's first row); the MoE forms gather
  // rows through perm, so the folded form runs it after its first weight loads are out ------
  // Dense form (BUF): every load goes through a buffer resource whose base is uniform over the
  // workgroup (the tile's first activation row, weight row, scale and zero row); a lane's offset
  // into it is fixed for the whole K loop and the step's offset is a scalar operand, so a step's
  // loads cost no vector address arithmetic (64-bit per-lane addresses were a fifth of the loop's
  // VALU instructions). gemm_rb keeps every offset below 2^31.
  constexpr bool BUF = MOE == 0 && IMQ_RB_BUF;
  const uint16_t* xtile = a.x + (int64_t)m0 * a.sxm;
  int xo[XC], xl[XC];
  // MoE forms: the block's routed rows RID[row] = perm[prow0 + row] (0 past cnt), staged in LDS by
  // plan_a for the row-sum staging and down's scatter. A wave's lanes of chunk j cover 8
  // consecutive rows, whose perm entries are one scalar load (the workspace keeps BM spare
  // entries past perm's B): scalar loads count on lgkmcnt, so the gather's addresses do not wait
  // behind the weight loads issued before them on the in-order vmcnt.
  int* const RID = (int*)((char*)lds + (size_t)3 * A_EL * 2 + (size_t)(a.K >> a.gsh) * BN * 4 +
                          (FOLD ? (size_t)(a.K >> a.gsh) * BM * 4 : 0));
  auto plan_a = [&]() {
#pragma unroll
    for (int j = 0; j < XC; ++j) {
      const int id = tid + NTHR * j;
      const int row = id >> 3, ch = id & 7;
      int r;
      if constexpr (MOE == 0) {
        r = m0 + row < a.M ? row : a.M - 1 - m0;
      } else {
        typedef int32_t v8i __attribute__((ext_vector_type(8), aligned(4)));
        // the wave's first row of chunk j (row = rb8 + lane / 8), uniform
        const int rb8 = (64 * __builtin_amdgcn_readfirstlane(wave) + NTHR * j) >> 3;
        const v8i pv = *(const __attribute__((address_space(4))) v8i*)(a.perm + prow0 + rb8);
        int pr = pv[0];
#pragma unroll
        for (int i = 1; i < 8; ++i) pr = (lane >> 3) == i ? pv[i] : pr;
        const bool ok = row < cnt;
        if (ch == 0) RID[row] = ok ? pr : 0;
        // down reads h in sorted order (rows past cnt repeat the last), gate_up gathers hidden rows
        // (rows past cnt read token 0; their results are never stored)
        r = MOE == 3 ? prow0 + (ok ? row : cnt - 1) : (ok ? pr / a.k : 0);
      }
      xo[j] = ((int)(r * a.sxm) + ch * 8) * (BUF ? 2 : 1);   // BUF: bytes
      xl[j] = 2 * rb_swz(row, ch);                    // bytes
    }
  };
  // ---- weight load plan: columns n0 + 64 wave + 32 j + c (MOE 1: gate column tn 32 NW + 32 wave
  // + c for j = 0, the matching up column I + that for j = 1), K bytes [32 h, +32) codes per step --
  const uint8_t* qb[2];
  int64_t sb[2], zb[2];
  uint32_t qvo[2], svo[2], zvo[2];                  // BUF: byte offsets from the tile's rows
  uint32_t qto[2][2] = {{0u, 0u}, {0u, 0u}};        // line-tiled weights: lane offsets by (kt / 2) & 1
  constexpr int SES = SDT == IMQ_DT_FP32 ? 4 : 2, ZES = ZDT == IMQ_DT_FP32 ? 4 : 2;
  const int gh = (32 * h) >> a.gsh;                 // the lane half's group within a step (groups < 64)
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    int n = MOE == 1 ? (j ? a.I : 0) + tn * (32 * NW) + 32 * wave + c : n0 + 64 * wave + 32 * j + c;
    n = n < a.N ? n : a.N - 1;
    qb[j] = a.q + (int64_t)e * a.sqe + (int64_t)n * a.sqn + (BITS == 8 ? 32 : 16) * h;
    sb[j] = (int64_t)e * a.sse + (int64_t)n * a.ssn;
    zb[j] = (int64_t)e * a.sse + (int64_t)n * a.szn;
    qvo[j] = (uint32_t)((n - n0) * (int)a.sqn + (BITS == 8 ? 32 : 16) * h);
    svo[j] = (uint32_t)(((n - n0) * (int)a.ssn + gh * (int)a.ssg) * SES);
    zvo[j] = (uint32_t)(((n - n0) * (int)a.szn + gh * (int)a.szg) * ZES);
    if constexpr (TL) {
      // line-tiled weights: the lane's bytes of a K step of row n (tile-relative rr) sit at tile
      // rr / 16, half hr = (rr / 8) & 1, slot (rr & 7) + 8 (sel ^ hr) + 16 (piece & 3) of the
      // step's line-step. int4 (16 bytes at 32 kt + 16 h): line-step kt / 4, piece 2 (kt & 1) + h,
      // sel = (kt / 2) & 1; int8 (two pieces at 64 kt + 32 h + 16 v): line-step kt / 2, piece 2 h
      // + v, sel = kt & 1. A lane offset per value of sel plus the step's uniform part (rb_tl_step).
      const int rr = n - n0, hr = (rr >> 3) & 1;
      const uint32_t tb = (uint32_t)((rr >> 4) * 16 * (int)a.sqn + 1024 * hr + 16 * (rr & 7) + (BITS == 8 ? 512 : 256) * h);
      qto[j][0] = tb + 128 * hr;
      qto[j][1] = tb + 128 * (1 - hr);
    }
  }
  // (built unconditionally; the forms that do not use them drop them)
  const __amdgpu_buffer_rsrc_t xrs = rb_rsrc(xtile);
  const __amdgpu_buffer_rsrc_t qrs = rb_rsrc(a.q + (int64_t)n0 * a.sqn);
  const __amdgpu_buffer_rsrc_t srs = rb_rsrc((const char*)a.sc + (int64_t)n0 * a.ssn * SES);
  const __amdgpu_buffer_rsrc_t zrs = rb_rsrc((const char*)a.zr + (int64_t)n0 * a.szn * ZES);

  // MoE forms: the tile's scale / zero pairs for all K groups are staged in LDS once, as
  // [group][tile column] dwords (bf16 scale | bf16 zero << 16, both rounded to bf16 as the
  // dequantization uses them); each step then reads one dword per column block from LDS instead
  // of two strided global loads per column block -- those loads touch a separate cache line per
  // lane and, issued every step, kept the texture unit busier than the weight stream itself.
  uint32_t* SZ = (uint32_t*)(lds + 3 * A_EL);
  // FOLD's step unpacks all of a step's weights at its top (step_fold); else one slice ahead
  constexpr bool EARLY = FOLD && RB_FOLD_EARLY_UNPACK;
  // The MoE forms' staging into LDS (the caller places the barrier after it): the block rows'
  // group sums (FOLD, needs the row plan), and the scale / zero pairs -- with 16-byte aligned
  // scale rows (unit group stride) one 16-byte load covers 16 / sizeof(scale) groups of a column
  // (the row's allocated stride covers the last chunk), issued apart from their LDS stores when
  // a thread has at most four such loads; else element by element.
  auto stage_rs = [&]() {
    if constexpr (MOE != 0) {
      // FOLD: the block rows' group sums too, as [group][BM rows] floats after the pairs -- read by
      // the final correction's MFMA operands (lane: row c of block i, group g0 + h)
      if constexpr (FOLD) {
        float* RS = (float*)(SZ + (a.K >> a.gsh) * BN);
        const int ng = a.K >> a.gsh, total = ng * BM;
        for (int base = 0; base < total; base += 8 * NTHR) {
          float v[8];
          int at[8];
#pragma unroll
          for (int u = 0; u < 8; ++u) {
            const int idx = base + u * NTHR + tid;
            const int id = idx < total ? idx : total - 1;
            const int row = id / ng, g = id - row * ng;   // consecutive threads: consecutive groups of a row
            const int rid = MOE == 3 ? prow0 + (row < cnt ? row : cnt - 1) : RID[row] / a.k;
            v[u] = g < a.rs_groups ? a.rs[(int64_t)rid * a.rs_stride + g] : 0.f;
            at[u] = idx < total ? g * BM + row : -1;
          }
#pragma unroll
          for (int u = 0; u < 8; ++u)
            if (at[u] >= 0) RS[at[u]] = v[u];
        }
      }
    }
  };
  constexpr int ES = SDT == IMQ_DT_FP32 ? 4 : 2;
  constexpr int VG = 16 / ES;
  const int ngs = a.K >> a.gsh;
  const int nch = (ngs + VG - 1) / VG;
  const bool sz_vec = MOE != 0 && a.ssg == 1 && a.szg == 1 && ((a.ssn * ES) & 15) == 0 &&
                      ((a.szn * ES) & 15) == 0 && ((a.sse * ES) & 15) == 0 &&
                      ((((uintptr_t)a.sc) | ((uintptr_t)a.zr)) & 15) == 0 && BN * nch <= 4 * NTHR;
  u32x4_t szs[4], szz[4];
  auto sz_issue = [&]() {   // sz_vec: the loads
    if constexpr (MOE != 0) {
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int it = u * NTHR + tid;
        const int id = it < BN * nch ? it : BN * nch - 1;
        const int tc = id / nch, ch = id - tc * nch;
        const int w_ = tc >> 6, j_ = (tc >> 5) & 1, c_ = tc & 31;
        int n = MOE == 1 ? (j_ ? a.I : 0) + tn * (32 * NW) + 32 * w_ + c_ : n0 + tc;
        n = n < a.N ? n : a.N - 1;
        const int64_t eb = (int64_t)e * a.sse + (int64_t)ch * VG;
        szs[u] = *(const u32x4_t*)((const char*)a.sc + (eb + (int64_t)n * a.ssn) * ES);
        szz[u] = *(const u32x4_t*)((const char*)a.zr + (eb + (int64_t)n * a.szn) * ES);
      }
    }
  };
  auto sz_store = [&]() {   // sz_vec: the LDS stores
    if constexpr (MOE != 0) {
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int it = u * NTHR + tid;
        const int tc = it / nch, ch = it - tc * nch;
#pragma unroll
        for (int v = 0; v < VG; ++v) {
          const uint32_t sraw = ES == 4 ? szs[u][v] : ((szs[u][v >> 1] >> (16 * (v & 1))) & 0xffffu);
          const uint32_t zraw = ES == 4 ? szz[u][v] : ((szz[u][v >> 1] >> (16 * (v & 1))) & 0xffffu);
          const float s_ = round_to<IMQ_DT_BF16>(raw_bits_to_f32<SDT>(sraw));
          const float z_ = round_to<IMQ_DT_BF16>(raw_bits_to_f32<ZDT>(zraw));
          const int g = ch * VG + v;
          if (it < BN * nch && g < ngs) SZ[g * BN + tc] = (__float_as_uint(s_) >> 16) | (__float_as_uint(z_) & 0xffff0000u);
        }
      }
    }
  };
  auto sz_scalar = [&]() {   // !sz_vec
    if constexpr (MOE != 0) {
      // batches of 16 elements per thread, all loads of a batch issued before any is consumed;
      // consecutive threads take consecutive groups of one column (one scale row segment)
      constexpr int SB = 16;
      const int ng = a.K >> a.gsh, total = ng * BN;
      for (int base = 0; base < total; base += SB * NTHR) {
        uint32_t sv[SB], zv[SB];
        int at[SB];
#pragma unroll
        for (int u = 0; u < SB; ++u) {
          const int idx = base + u * NTHR + tid;
          const int id = idx < total ? idx : total - 1;
          const int tc = id / ng, g = id - tc * ng;
          const int w_ = tc >> 6, j_ = (tc >> 5) & 1, c_ = tc & 31;
          int n = MOE == 1 ? (j_ ? a.I : 0) + tn * (32 * NW) + 32 * w_ + c_ : n0 + tc;
          n = n < a.N ? n : a.N - 1;
          const int64_t gb = (int64_t)e * a.sse + (int64_t)g * a.ssg;
          sv[u] = load_raw_bits<SDT>(a.sc, gb + (int64_t)n * a.ssn);
          zv[u] = load_raw_bits<ZDT>(a.zr, gb + (int64_t)n * a.szn);
          at[u] = idx < total ? g * BN + tc : -1;
        }
#pragma unroll
        for (int u = 0; u < SB; ++u) {
          const float s_ = round_to<IMQ_DT_BF16>(raw_bits_to_f32<SDT>(sv[u]));
          const float z_ = round_to<IMQ_DT_BF16>(raw_bits_to_f32<ZDT>(zv[u]));
          if (at[u] >= 0) SZ[at[u]] = (__float_as_uint(s_) >> 16) | (__float_as_uint(z_) & 0xffff0000u);
        }
      }
    }
  };
  auto stage_moe = [&]() {
    stage_rs();
    if (sz_vec) {
      sz_issue();
      sz_store();
    } else {
      sz_scalar();
    }
  };
  if constexpr (!EARLY) plan_a();
  if constexpr (MOE != 0 && !EARLY) {
    lds_barrier();     // RID, read by the row-sum staging
    stage_moe();
    __syncthreads();   // the prologue's weight-set loads read pairs other threads staged
  }

  static_assert(PD >= 2 && PD <= 4, "pipeline depth 2..4");
  u32x4_t xr[PD][XC];
  u32x4_t qr[PD][2][QV];
  uint32_t sr[PD][2], zr[PD][2];
  const int kt0 = split * a.kps;
  const int KS = ((MOE != 0 && a.xk > 0) ? a.xk : a.K) / BK;   // K steps with nonzero activations
  const int KT = (KS - kt0) < a.kps ? (KS - kt0) : a.kps;

  auto load_a = [&](auto setc, int ktl) {
    constexpr int set = decltype(setc)::value;
    const int kt = kt0 + (ktl < KT ? ktl : KT - 1);
#pragma unroll
    for (int j = 0; j < XC; ++j) {
      if constexpr (BUF) xr[set][j] = rb_bload128(xrs, xo[j], kt * (BK * 2));
      else xr[set][j] = *(const u32x4_t*)(xtile + kt * BK + xo[j]);
    }
  };
  auto load_b = [&](auto setc, int ktl) {
    constexpr int set = decltype(setc)::value;
    const int kt = kt0 + (ktl < KT ? ktl : KT - 1);
    if constexpr (BUF) {
      const uint32_t gs = (uint32_t)((kt * BK) >> a.gsh);
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        if constexpr (TL) {
          const int sel = BITS == 8 ? (kt & 1) : ((kt >> 1) & 1);
          const uint32_t so = BITS == 8 ? 2048 * (kt >> 1) : 2048 * (kt >> 2) + 512 * (kt & 1);
#pragma unroll
          for (int v = 0; v < QV; ++v) qr[set][j][v] = rb_bload128(qrs, (sel ? qto[j][1] : qto[j][0]) + 256 * v, so);
        } else {
#pragma unroll
          for (int v = 0; v < QV; ++v) qr[set][j][v] = rb_bload128(qrs, qvo[j] + 16 * v, kt * (BK * BITS / 8));
        }
        if constexpr (BITS != 8) {
          sr[set][j] = rb_bload_raw<SDT>(srs, svo[j], gs * (uint32_t)a.ssg * SES);
          zr[set][j] = rb_bload_raw<ZDT>(zrs, zvo[j], gs * (uint32_t)a.szg * ZES);
        }
      }
      return;
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      if constexpr (TL) {
        const int sel = BITS == 8 ? (kt & 1) : ((kt >> 1) & 1);
        const uint32_t so = BITS == 8 ? 2048 * (kt >> 1) : 2048 * (kt >> 2) + 512 * (kt & 1);
#pragma unroll
        for (int v = 0; v < QV; ++v)
          qr[set][j][v] = *(const u32x4_t*)(a.q + (int64_t)n0 * a.sqn + (sel ? qto[j][1] : qto[j][0]) + 256 * v + so);
      } else {
#pragma unroll
        for (int v = 0; v < QV; ++v) qr[set][j][v] = *(const u32x4_t*)(qb[j] + kt * (BK * BITS / 8) + 16 * v);
      }
      if constexpr (MOE == 0 && BITS != 8) {
        const int g = (kt * BK + 32 * h) >> a.gsh;
        sr[set][j] = load_raw_bits<SDT>(a.sc, sb[j] + (int64_t)g * a.ssg);
        zr[set][j] = load_raw_bits<ZDT>(a.zr, zb[j] + (int64_t)g * a.szg);
      }
    }
  };
  // MoE forms: the scale / zero pair of a weight set, from the staged LDS copy
  auto load_s = [&](auto setc, int ktl) {
    if constexpr (MOE != 0) {
      constexpr int set = decltype(setc)::value;
      const int kt = kt0 + (ktl < KT ? ktl : KT - 1);
      const int g = (kt * BK + 32 * h) >> a.gsh;
#pragma unroll
      for (int j = 0; j < 2; ++j) sr[set][j] = SZ[g * BN + 64 * wave + 32 * j + c];
    }
  };
  auto store_a = [&](auto setc, uint16_t* A) {
    constexpr int set = decltype(setc)::value;
#pragma unroll
    for (int j = 0; j < XC; ++j) *(u32x4_t*)((char*)A + xl[j]) = FOLD ? permute_x8(xr[set][j]) : xr[set][j];
  };

  // acc: the running sums (FOLD: the current group's sums of x (128 + q)); tot: FOLD's total
  f32x16_t acc[IB][2];
  f32x16_t tot[FOLD ? IB : 1][2];
#pragma unroll
  for (int i = 0; i < IB; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        acc[i][j][r] = 0.f;
        if constexpr (FOLD) tot[i][j][r] = 0.f;
      }
  const uint32_t magic = FOLD ? magic_bf16_128x2() : 0u;
  float sfold[2] = {0.f, 0.f};   // FOLD: scale of the group whose sums acc holds
  int aoff[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) aoff[s] = 2 * rb_swz(c, 4 * h + s);   // bytes; + 32 rows (4096 bytes) per i

  bf16x8_t af[2][IB];        // A fragments of slice s live in af[s & 1], B fragments in bq[s & 1]
  bf16x8_t bq[2][2];         // (4 slices: the parity pattern repeats every step)
  auto read_frags = [&](auto pc, const uint16_t* A, int s) {
    constexpr int p = decltype(pc)::value;
#pragma unroll
    for (int i = 0; i < IB; ++i) af[p][i] = *(const bf16x8_t*)((const char*)A + aoff[s] + i * 64 * BK);
  };

  // The scale / zero of a B register set as (s, -z s), both taken to bf16 first.
  auto scale_pair = [&](auto bsc, float* sv, float* nz) {
    constexpr int bs = decltype(bsc)::value;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      if constexpr (MOE != 0) {
        const float s_ = __uint_as_float(sr[bs][j] << 16), z_ = __uint_as_float(sr[bs][j] & 0xffff0000u);
        sv[j] = s_;
        nz[j] = -z_ * s_;
      } else if constexpr (BITS != 8) {
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
    if constexpr (FOLD) return unpack_nib8_bf16(qr[bs][j][0][s], magic);
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
  // Step kt (B register set kt % PD, A register set (kt+1) % PD holding A(kt+1)):
  //   slice s: dequantize B(kt) slice s; read the A fragments of slice s+1 (slice 0 of step
  //            kt+1 from the new buffer at s = 3, dequantized from B(kt+1)); MFMAs of slice s on
  //            the fragments read one slice earlier;
  //   slice 0: also write A(kt+1) into the next buffer;
  //   slice 1: then wait for the LDS writes, barrier, and load A(kt+1+PD) into the freed A set;
  //   after slice 3: load B(kt+PD) into the freed B set.
  auto step = [&](int kt, int rb, int wb, auto bsc) {
    constexpr int bs = decltype(bsc)::value;     // kt % PD
    constexpr int as = (bs + 1) % PD;            // A(kt+1) and B(kt+1) live in set (kt+1) % PD
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
        scale_pair(std::integral_constant<int, as>{}, sv2, nz2);
#pragma unroll
        for (int j = 0; j < 2; ++j) bq[0][j] = b_frag(std::integral_constant<int, as>{}, 0, j, sv2[j], nz2[j]);
        read_frags(std::integral_constant<int, 0>{}, Aw, 0);
      }
      if ((s & 1) == 0) {
        // FOLD, first slice of a group (even step): fold the previous group's sums into the
        // total with its scale, then start the group's sums from zero
        constexpr bool group_start = FOLD && bs % 2 == 0;
#pragma unroll
        for (int i = 0; i < IB; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            if (group_start && s == 0) {
              if constexpr (FOLD) {
#pragma unroll
                for (int r = 0; r < 16; ++r) tot[i][j][r] = fmaf(sfold[j], acc[i][j][r], tot[i][j][r]);
              }
              acc[i][j] = mfma32x32x16(af[0][i], bq[0][j], f32x16_t{});
            } else {
              acc[i][j] = mfma32x32x16(af[0][i], bq[0][j], acc[i][j]);
            }
          }
        if (group_start && s == 0) {
          sfold[0] = sv[0];
          sfold[1] = sv[1];
        }
      } else {
#pragma unroll
        for (int i = 0; i < IB; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j) acc[i][j] = mfma32x32x16(af[1][i], bq[1][j], acc[i][j]);
      }
      if (s == 0) store_a(std::integral_constant<int, as>{}, Aw);
      if (s == 1) {
        lds_barrier();
        load_a(std::integral_constant<int, as>{}, kt + 1 + PD);
        __builtin_amdgcn_sched_barrier(0);
      }
      // one MFMA, then a few VALU and one LDS read, repeated: keeps the dequant and the fragment
      // reads between MFMAs instead of bunched before them
#pragma unroll
      for (int k = 0; k < 2 * IB; ++k) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, FOLD ? RB_VALU_PER_MFMA_FOLD : BITS == 8 ? RB_VALU_PER_MFMA_8 : RB_VALU_PER_MFMA_4, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    load_b(bsc, kt + PD);
    load_s(bsc, kt + PD);
    __builtin_amdgcn_sched_barrier(0);
  };

  // FOLD's step (PD 2). The magic unpack is cheap, so all four slices of B(kt) are unpacked at
  // the top of the step and B(kt+2) is issued at once into the freed register set: a weight load
  // has two full steps to arrive (the dequantizing step above unpacks the next step's first
  // slice in its last one, so B(kt+1) must land within the step it was issued after). At the
  // first slice of a group (even step) the previous group's sums are folded into the total with
  // its scale and the group's sums restart from zero.
  bf16x8_t bq4[FOLD ? 4 : 1][2];
  auto step_fold = [&](int kt, int rb, int wb, auto bsc) {
    constexpr int bs = decltype(bsc)::value;     // kt % 2
    constexpr int as = (bs + 1) % PD;
    constexpr bool group_start = bs % 2 == 0;
    const uint16_t* Ar = lds + rb * A_EL;
    uint16_t* Aw = lds + wb * A_EL;
    float sv[2], nz[2];
    scale_pair(bsc, sv, nz);
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int j = 0; j < 2; ++j) bq4[FOLD ? s : 0][j] = b_frag(bsc, s, j, sv[j], nz[j]);
    __builtin_amdgcn_sched_barrier(0);
    load_b(bsc, kt + PD);
    load_s(bsc, kt + PD);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      if (s < 3) {
        if ((s & 1) == 0) read_frags(std::integral_constant<int, 1>{}, Ar, s + 1);
        else read_frags(std::integral_constant<int, 0>{}, Ar, s + 1);
      } else {
        read_frags(std::integral_constant<int, 0>{}, Aw, 0);
      }
#pragma unroll
      for (int i = 0; i < IB; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const bf16x8_t av = (s & 1) ? af[1][i] : af[0][i];
          if (group_start && s == 0) {
            if constexpr (FOLD) {
#pragma unroll
              for (int r = 0; r < 16; ++r) tot[i][j][r] = fmaf(sfold[j], acc[i][j][r], tot[i][j][r]);
            }
            acc[i][j] = mfma32x32x16(av, bq4[FOLD ? s : 0][j], f32x16_t{});
          } else {
            acc[i][j] = mfma32x32x16(av, bq4[FOLD ? s : 0][j], acc[i][j]);
          }
        }
      if (group_start && s == 0) {
        sfold[0] = sv[0];
        sfold[1] = sv[1];
      }
      if (s == 0) store_a(std::integral_constant<int, as>{}, Aw);
      if (s == 1) {
        lds_barrier();
        load_a(std::integral_constant<int, as>{}, kt + 1 + PD);
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int k = 0; k < 2 * IB; ++k) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  };

  // Prologue, in the loop's steady-state load order (A(kt+1), B(kt), ..., A(kt+PD), B(kt+PD-1)
  // outstanding at the top of step kt) so the waits the compiler places at the loop head match
  // the loop's: A(0) is loaded first, then A(1), B(0), ..., with A(0) written to buffer 0 just
  // before A(PD) takes its register set.
  if constexpr (EARLY) {
    // the fold step's steady state has B(kt), A(kt+1), B(kt+1), A(kt+2) outstanding at the top
    // of step kt
    static_assert(PD == 2, "the fold step keeps two register sets");
    // weights and scales need only the tile: their loads go out before the gathered rows' plan
    // (a dependent load of perm), so the two latencies overlap
    load_b(std::integral_constant<int, 0>{}, 0);
    __builtin_amdgcn_sched_barrier(0);
    load_b(std::integral_constant<int, 1>{}, 1);
    __builtin_amdgcn_sched_barrier(0);
    if (sz_vec) sz_issue();
    __builtin_amdgcn_sched_barrier(0);
    plan_a();
    load_a(std::integral_constant<int, 0>{}, 0);
    __builtin_amdgcn_sched_barrier(0);
    load_a(std::integral_constant<int, 1>{}, 1);
    __builtin_amdgcn_sched_barrier(0);
    if (sz_vec) sz_store();
    else sz_scalar();
    lds_barrier();     // RID, read by the row-sum staging
    stage_rs();
    __syncthreads();
    load_s(std::integral_constant<int, 0>{}, 0);
    load_s(std::integral_constant<int, 1>{}, 1);
    store_a(std::integral_constant<int, 0>{}, lds);
    __builtin_amdgcn_sched_barrier(0);
    load_a(std::integral_constant<int, 0>{}, 2);
    __builtin_amdgcn_sched_barrier(0);
    lds_barrier();
    read_frags(std::integral_constant<int, 0>{}, lds, 0);
  } else {
    load_a(std::integral_constant<int, 0>{}, 0);
    __builtin_amdgcn_sched_barrier(0);
    auto prologue_pair = [&](auto jc) {
      constexpr int j = decltype(jc)::value;
      if constexpr (j + 1 == PD) {
        store_a(std::integral_constant<int, 0>{}, lds);
        __builtin_amdgcn_sched_barrier(0);
      }
      load_a(std::integral_constant<int, (j + 1) % PD>{}, j + 1);
      __builtin_amdgcn_sched_barrier(0);
      load_b(jc, j);
      load_s(jc, j);
      __builtin_amdgcn_sched_barrier(0);
    };
    prologue_pair(std::integral_constant<int, 0>{});
    prologue_pair(std::integral_constant<int, 1>{});
    if constexpr (PD > 2) prologue_pair(std::integral_constant<int, 2>{});
    if constexpr (PD > 3) prologue_pair(std::integral_constant<int, 3>{});
    lds_barrier();
    read_frags(std::integral_constant<int, 0>{}, lds, 0);
    {
      float sv0[2], nz0[2];
      scale_pair(std::integral_constant<int, 0>{}, sv0, nz0);
#pragma unroll
      for (int j = 0; j < 2; ++j) bq[0][j] = b_frag(std::integral_constant<int, 0>{}, 0, j, sv0[j], nz0[j]);
    }
  }

  // main loop unrolled by PD so every register set index is a compile-time constant
  int rb = 0;
  int kt = 0;
  auto run_step = [&](auto uc) {
    const int wb = rb == 2 ? 0 : rb + 1;
    if constexpr (EARLY) step_fold(kt + decltype(uc)::value, rb, wb, uc);
    else step(kt + decltype(uc)::value, rb, wb, uc);
    rb = wb;
  };
  for (; kt + PD - 1 < KT; kt += PD) {
    run_step(std::integral_constant<int, 0>{});
    run_step(std::integral_constant<int, 1>{});
    if constexpr (PD > 2) run_step(std::integral_constant<int, 2>{});
    if constexpr (PD > 3) run_step(std::integral_constant<int, 3>{});
  }
  if (kt < KT) run_step(std::integral_constant<int, 0>{});
  if constexpr (PD > 2)
    if (kt + 1 < KT) run_step(std::integral_constant<int, 1>{});
  if constexpr (PD > 3)
    if (kt + 2 < KT) run_step(std::integral_constant<int, 2>{});

  if constexpr (FOLD) {
    // the last group's fold, then the -s_g (128 + z_g) sum_{k in g} x_k terms: one fp32
    // 32x32x2 MFMA per pair of groups, A = the rows' group sums (lane: row c, group g0 + h),
    // B = -s (128 + z) of the lane's column and group g0 + h
#pragma unroll
    for (int i = 0; i < IB; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) tot[i][j][r] = fmaf(sfold[j], acc[i][j][r], tot[i][j][r]);
    const int ng = a.K >> a.gsh;
    const float* RS = (const float*)(SZ + ng * BN);   // staged [group][BM rows] (zero past rs_groups)
    for (int g0 = 0; g0 < ng; g0 += 2) {
      const int g = g0 + h;
      float av[IB], bv[2];
#pragma unroll
      for (int i = 0; i < IB; ++i) av[i] = g < ng ? RS[g * BM + 32 * i + c] : 0.f;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const uint32_t pr = g < ng ? SZ[g * BN + 64 * wave + 32 * j + c] : 0u;
        bv[j] = -(128.f + __uint_as_float(pr & 0xffff0000u)) * __uint_as_float(pr << 16);
      }
#pragma unroll
      for (int i = 0; i < IB; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) tot[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i], bv[j], tot[i][j], 0, 0, 0);
    }
  }
  // the finished sums of block (i, j)
  auto res = [&](int i, int j) -> const f32x16_t& {
    if constexpr (FOLD) return tot[i][j];
    else return acc[i][j];
  };

  // ---- epilogue: D lane l holds column l % 32, element r at row 8 (r / 4) + 4 (l / 32) + r % 4 ---
  if constexpr (MOE != 0) {
    const bool has_bias = a.bias != nullptr;
    auto bias_q = [&](int q) -> float { return has_bias ? rb_bias_of(bw_w[q], bw_h[q], a.bdt) : 0.f; };
    if constexpr (MOE == 1 || MOE == 2) {
      // h through LDS as [BM][HS] bf16 (rows padded against bank conflicts): the tile's 128 h
      // columns then leave as 16-byte row segments, and their sum per row (the bf16 values down
      // reads) is the group sum hrs[p][tn] of down's folded form
      constexpr int HS = 136;
      uint16_t* Ht = lds;              // the activation buffers: every wave is past its last step
      __syncthreads();
      if constexpr (MOE == 1) {
        const int hc = 32 * wave + c;                   // tile-local h column; I % 128 == 0
        const int g = tn * (32 * NW) + hc;
        const float bg = bias_q(0), bu = bias_q(1);   // rows g, I + g
#pragma unroll
        for (int i = 0; i < IB; ++i)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int m = 32 * i + 8 * (r >> 2) + 4 * h + (r & 3);
            const float gv = res(i, 0)[r] + bg, uv = res(i, 1)[r] + bu;
            Ht[m * HS + hc] = (uint16_t)cvt_pk_bf16(gv / (1.f + __expf(-gv)) * uv, 0.f);
          }
      } else {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int n = n0 + 64 * wave + 32 * j + c;    // even lanes: gate rows, odd: the up rows
          const int hc = (64 * wave + 32 * j + c) >> 1;
          const float bg = n < a.N ? bias_q(2 * j) : 0.f, bu = n + 1 < a.N ? bias_q(2 * j + 1) : 0.f;
#pragma unroll
          for (int i = 0; i < IB; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const float v = res(i, j)[r];
              const float up = __shfl_xor(v, 1, 64);
              const int m = 32 * i + 8 * (r >> 2) + 4 * h + (r & 3);
              if ((c & 1) == 0) {
                float gv = v + bg, uv = up + bu;
                gv = gv > a.limit ? a.limit : gv;
                uv = uv > a.limit ? a.limit : (uv < -a.limit ? -a.limit : uv);
                const float hv = (uv + 1.f) * (gv / (1.f + __expf(-a.alpha * gv)));
                Ht[m * HS + hc] = n < a.N ? (uint16_t)cvt_pk_bf16(hv, 0.f) : (uint16_t)0;   // past I: zero
              }
            }
        }
      }
      __syncthreads();
      // four threads per row, 32 columns (64 bytes) each
      const int q = tid & 3;
#pragma unroll
      for (int row = tid >> 2; row < BM; row += NTHR / 4) {
        u32x4_t v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) v[u] = *(const u32x4_t*)(Ht + row * HS + 32 * q + 8 * u);
        float sum = 0.f;
#pragma unroll
        for (int u = 0; u < 4; ++u) sum += bf16x8_sum(v[u]);
        sum = quad_sum4(sum);
        if (row < cnt) {
          uint16_t* dst = a.y + (int64_t)(prow0 + row) * a.sym + tn * 128 + 32 * q;
#pragma unroll
          for (int u = 0; u < 4; ++u) *(u32x4_t*)(dst + 8 * u) = v[u];
          if (a.hrs != nullptr && q == 0) a.hrs[(int64_t)(prow0 + row) * a.hrs_stride + tn] = sum;
        }
      }
    } else if (a.yrb != nullptr) {
      // bf16 rows through LDS as [BM][YS] (rows padded against bank conflicts): 16-byte row
      // segments to the routed rows (N % 64 == 0, so a segment lies wholly inside or past N)
      constexpr int YS = BN + 8;
      uint16_t* Yt = lds;              // every wave is past its last step and the correction
      // this thread's routed rows, read before the row tile may overwrite RID
      constexpr int NIT = BM * (BN / 8) / NTHR;
      static_assert(BM * (BN / 8) % NTHR == 0, "whole row-tile passes");
      int rr[NIT];
#pragma unroll
      for (int i = 0; i < NIT; ++i) rr[i] = RID[(tid + NTHR * i) / (BN / 8)];
      __syncthreads();
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int col = 64 * wave + 32 * j + c;
        const float bn = n0 + col < a.N ? bias_q(j) : 0.f;
#pragma unroll
        for (int i = 0; i < IB; ++i)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int m = 32 * i + 8 * (r >> 2) + 4 * h + (r & 3);
            Yt[m * YS + col] = (uint16_t)cvt_pk_bf16(res(i, j)[r] + bn, 0.f);
          }
      }
      __syncthreads();
#pragma unroll
      for (int i = 0; i < NIT; ++i) {
        const int it = tid + NTHR * i;
        const int row = it / (BN / 8), ch = it - row * (BN / 8);
        const int n = n0 + 8 * ch;
        if (row < cnt && n < a.N)
          *(u32x4_t*)(a.yrb + (int64_t)rr[i] * a.N + n) = *(const u32x4_t*)(Yt + row * YS + 8 * ch);
      }
    } else {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int n = n0 + 64 * wave + 32 * j + c;
        if (n >= a.N) continue;
        const float bn = bias_q(j);
#pragma unroll
        for (int i = 0; i < IB; ++i)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int m = 32 * i + 8 * (r >> 2) + 4 * h + (r & 3);
            if (m < cnt) a.yr[(int64_t)RID[m] * a.N + n] = res(i, j)[r] + bn;
          }
      }
    }
    return;
  }
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

}  // namespace
}  // namespace imq
