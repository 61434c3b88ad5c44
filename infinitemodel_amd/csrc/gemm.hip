// Prefill-regime (M > 16) fused dequant GEMM for gfx950.
//
// y[M, N] = x[M, K] . dequant(W[N, K])^T with bf16 activations, packed int4 / int2 (group-wise
// asymmetric) or int8 (per-row symmetric) weights, fp32 accumulation and bf16 output: the
// contract of the reference's `_k` / `_k2` / `_k8` GEMM kernels (worker_quant.py:1098-1126,
// 1795-1828, 953-980).
//
// Structure (a workgroup computes a BM x 128 output tile; each wave a WM x WN sub-tile with
// v_mfma_f32_32x32x16_bf16, which issues at twice the rate of the 16x16x32 form on gfx950):
//   * K advances in steps of 64 through two LDS buffers. Global loads run two steps ahead (one
//     in registers); at the end of step kt every thread writes step kt+1 into the other buffer --
//     activations as loaded, weights dequantized to bf16 (q - z) * s rounded once (the exact
//     product of two bf16 values fits fp32) for int4/int2, the exact integer for int8 (its
//     per-row scale multiplies the fp32 accumulator in the epilogue) -- then issues the loads of
//     step kt+2 into the freed registers, all interleaved with the step's MFMAs. One barrier per
//     step.
//   * Each weight is dequantized once per workgroup and feeds BM activation rows from LDS.
//   * LDS rows are 64 bf16 (8 chunks of 16 B) with the chunk index XOR-swizzled by the row, so
//     the 16-lane row-strided fragment reads spread over the banks.
//   * Workgroups are mapped XCD-aware: consecutive logical tiles land on one XCD (blockIdx is
//     dealt round-robin over the 8 XCDs), and logical tiles run in groups of 8 tile-rows so the
//     activation rows and weight columns a group shares stay in that XCD's L2.
#include "imq_common.h"
#include "splitk_sum.h"

#include <type_traits>

namespace imq {

bool rb_takes(int bits, int64_t M, int64_t N, int64_t K, int64_t G);
int64_t rb_workspace_bytes(int bits, int64_t M, int64_t N, int64_t K, int cus);
int gemm_rb(int bits, const uint16_t* x, int64_t sxm, int64_t M, int64_t K, const uint8_t* q, int64_t sqn,
            const void* sc, int64_t ssn, int64_t ssg, int sdt, const void* zr, int64_t szn, int64_t szg, int zdt,
            int64_t N, int64_t G, uint16_t* y, int64_t sym, void* ws, int64_t wsb, hipStream_t st, bool tiled);

namespace {

constexpr int GROUP_M = 8;

// BM x BN workgroup tile, K steps of BK, WAVES_M x WAVES_N waves, at least MINB workgroups per CU
// (bounds the registers so that many fit).
template <int BM_, int BN_, int BK_, int WAVES_M_, int WAVES_N_, int MINB_>
struct Cfg {
  static constexpr int BM = BM_, BN = BN_, BK = BK_, MINB = MINB_;
  static constexpr int CH = BK / 8;              // 16-byte chunks per LDS row
  static constexpr int KS = BK / 16;             // MFMA K slices per step
  static constexpr int SH = BK == 128 ? 0 : (BK == 64 ? 1 : 2);   // swizzle row shift: 256 B / row bytes
  static constexpr int WAVES_M = WAVES_M_, WAVES_N = WAVES_N_;
  static constexpr int NTHR = 64 * WAVES_M * WAVES_N;
  static constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;
  static constexpr int XC = BM * CH / NTHR;      // 16-byte activation chunks per thread per step
  static constexpr int WC = BN * BK / NTHR;      // weight codes per thread per step
  static constexpr int A_EL = BM * BK, B_EL = BN * BK;
  static constexpr int LDS = 2 * (A_EL + B_EL) * 2;
  static_assert(XC >= 1 && (BM * CH) % NTHR == 0, "activation chunks must divide evenly");
  static_assert(WC == 16 || WC == 32 || WC == 64, "16, 32 or 64 weight codes per thread");
  static_assert(WM % 32 == 0 && WN % 32 == 0, "wave tile of 32x32 blocks");
};

struct GemmArgs {
  const uint16_t* x;
  int64_t sxm;
  int M, K;
  const uint8_t* q;
  int64_t sqn;
  const void* sc;
  int64_t ssn, ssg;
  const void* zr;
  int64_t szn, szg;
  int N, gsh;          // group = 1 << gsh codes
  uint16_t* y;
  int64_t sym;
  int tiles_m, tiles_n;
  int splits, kps;     // split-K: K steps [split * kps, +kps) per workgroup; 1 = no split
  float* part;         // split-K partials [splits][M][N] fp32
  // grouped MoE form (the kernel's MOE != 0): a tile is (row block mt, column tile tn);
  // mtl[2 mt] = expert, mtl[2 mt + 1] = first sorted row of the block, *nmt blocks in all
  const int32_t* mtl = nullptr;
  const int32_t* nmt = nullptr;
  const int32_t* off = nullptr;       // [E + 1] sorted offsets
  const int32_t* perm = nullptr;      // sorted position -> routed row
  int64_t sqe = 0, sse = 0;           // expert strides: packed bytes, scale / zero elements
  int k = 1, I = 0;                   // top_k; intermediate size (gate_up)
  const void* bias = nullptr;         // per-expert row bias [E][rows] or null
  int64_t sbe = 0;
  int bdt = 0;
  float alpha = 0.f, limit = 0.f;     // gpt-oss activation
  float* yr = nullptr;                // MOE 3: fp32 rows [B][N] in routed order
};

// Element i of a per-expert bias row in the bias dtype.
IMQ_DEV float gemm_bias(const void* p, int dt, int64_t i) {
  if (dt == IMQ_DT_FP32) return ((const float*)p)[i];
  if (dt == IMQ_DT_FP16) return f16_bits_to_f32(((const uint16_t*)p)[i]);
  return bf16_bits_to_f32(((const uint16_t*)p)[i]);
}

// LDS element offset of 16-byte chunk c of row `row`: the chunk index is XOR-ed with the row's
// position inside a 256-byte bank period, so 8 consecutive rows read at one chunk hit 8 bank groups.
template <class C>
IMQ_DEV int swz(int row, int c) {
  return (row * C::CH + (c ^ ((row >> C::SH) & (C::CH - 1)))) * 8;
}

// 8 codes (BITS 4: nibbles of a dword; BITS 2: crumbs in the low 16 bits) -> 4 dwords of bf16
// (c - z) * s in K order.
template <int BITS>
IMQ_DEV u32x4_t dequant8(uint32_t w, float s, float nzs) {
  u32x4_t r;
  if constexpr (BITS == 4) {
    // even codes in the bytes of lo, odd codes in the bytes of hi: each code is then one
    // v_cvt_f32_ubyteN away from fp32
    const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float c0 = (float)((lo >> (8 * i)) & 0xffu);
      const float c1 = (float)((hi >> (8 * i)) & 0xffu);
      r[i] = cvt_pk_bf16(fmaf(c0, s, nzs), fmaf(c1, s, nzs));
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float c0 = (float)((w >> (4 * i)) & 3u);
      const float c1 = (float)((w >> (4 * i + 2)) & 3u);
      r[i] = cvt_pk_bf16(fmaf(c0, s, nzs), fmaf(c1, s, nzs));
    }
  }
  return r;
}

// 8 int8 codes (two dwords) -> 4 dwords of bf16, exact.
IMQ_DEV u32x4_t convert8_i8(uint32_t lo, uint32_t hi) {
  u32x4_t r;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const uint32_t w = i ? hi : lo;
    r[2 * i] = cvt_pk_bf16((float)(int8_t)(w & 0xff), (float)(int8_t)((w >> 8) & 0xff));
    r[2 * i + 1] = cvt_pk_bf16((float)(int8_t)((w >> 16) & 0xff), (float)(int8_t)(w >> 24));
  }
  return r;
}

// Packed weight bytes one thread loads per step: WC codes of BITS bits.
template <int BITS, int WC>
struct WRegs {
  static constexpr int BYTES = WC * BITS / 8;     // 4, 8, 16 or 32
  static constexpr int DW = BYTES / 4;
  uint32_t d[DW];
};

template <int BITS, int WC>
IMQ_DEV void load_w(WRegs<BITS, WC>& r, const uint8_t* p) {
  constexpr int B = WRegs<BITS, WC>::BYTES;
  if constexpr (B == 4) {
    r.d[0] = *(const uint32_t*)p;
  } else if constexpr (B == 8) {
    const u32x2_t v = *(const u32x2_t*)p;
    r.d[0] = v[0];
    r.d[1] = v[1];
  } else if constexpr (B == 16) {
    const u32x4_t v = *(const u32x4_t*)p;
#pragma unroll
    for (int i = 0; i < 4; ++i) r.d[i] = v[i];
  } else {
#pragma unroll
    for (int v = 0; v < B / 16; ++v) {
      const u32x4_t t = *(const u32x4_t*)(p + 16 * v);
#pragma unroll
      for (int i = 0; i < 4; ++i) r.d[4 * v + i] = t[i];
    }
  }
}

// Chunk c (8 codes, c < WC/8) of a thread's weight registers -> 4 dwords of bf16.
template <int BITS, int WC>
IMQ_DEV u32x4_t weight_chunk(const WRegs<BITS, WC>& r, int c, float s, float nzs) {
  if constexpr (BITS == 4) {
    return dequant8<4>(r.d[c], s, nzs);
  } else if constexpr (BITS == 2) {
    return dequant8<2>(r.d[c >> 1] >> (16 * (c & 1)), s, nzs);
  } else {
    return convert8_i8(r.d[2 * c], r.d[2 * c + 1]);
  }
}

// MOE 0: the dense GEMM. Grouped MoE forms (int4, rows of one hit expert per block, gathered):
// MOE 1 gate_up with SiLU-GLU (the tile's first BN/2 weight rows are gate rows, the rest the
// matching up rows; h = silu(gate) * up written as bf16 in sorted order), MOE 2 gpt-oss gate_up
// (consecutive interleaved rows, its clamped GLU), MOE 3 down (fp32 rows plus the row bias, in
// routed order, for the combine).
// TL: the dense int4 form on weights in the line-tiled layout (a separate instantiation, so the
// row-layout loop is unchanged).
template <class C, int BITS, int SDT, int ZDT, int MOE = 0, bool TL = false>
__global__ __launch_bounds__(C::NTHR, C::MINB) void gemm_wq_kernel(GemmArgs a) {
  static_assert(!TL || MOE == 0, "line-tiled weights: the dense forms");
  constexpr int BM = C::BM, BN = C::BN, WM = C::WM, WN = C::WN, XC = C::XC, WC = C::WC;
  constexpr int BK = C::BK, CH = C::CH, KS = C::KS;
  constexpr int PD = 2;   // register sets of loaded-but-not-yet-stored steps
  constexpr int NTHR = C::NTHR;
  extern __shared__ __align__(16) uint16_t lds[];
  uint16_t* As = lds;
  uint16_t* Bs = lds + 2 * C::A_EL;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;

  // ---- tile mapping: XCD-aware, grouped by GROUP_M tile-rows; split-K index outermost ---------
  int split = 0, tn, m0, n0;
  int e = 0, prow0 = 0, cnt = 0;                    // MOE: expert, first sorted row, rows of the block
  if constexpr (MOE == 0) {
    const int T = a.tiles_m * a.tiles_n;
    split = blockIdx.x / T;                         // the splits of one tile run the same XCD
    const int tile_id = blockIdx.x - split * T;
    int L = tile_id;
    if ((T & 7) == 0) L = (L & 7) * (T >> 3) + (L >> 3);
    const int per_group = GROUP_M * a.tiles_n;
    const int grp = L / per_group;
    const int first_m = grp * GROUP_M;
    const int gm = (a.tiles_m - first_m) < GROUP_M ? (a.tiles_m - first_m) : GROUP_M;
    const int in_grp = L - grp * per_group;
    const int tm = first_m + in_grp % gm;
    tn = in_grp / gm;
    m0 = tm * BM;
    n0 = tn * BN;
  } else {
    const int mt = blockIdx.x / a.tiles_n;
    tn = blockIdx.x - mt * a.tiles_n;
    if (mt >= *a.nmt) return;                       // uniform over the workgroup
    const int ec = a.mtl[2 * mt];                   // expert | rows of the block (<= BM) << 16
    e = ec & 0xffff;
    cnt = ec >> 16;
    prow0 = a.mtl[2 * mt + 1];
    m0 = 0;
    n0 = tn * BN;
  }

  // ---- global -> register load plan ----------------------------------------------------------
  // per-thread element offsets from the tile's first row (32-bit) + a uniform per-step base, so
  // the loads can take the scalar-base + vector-offset form
  const uint16_t* xtile = a.x + (int64_t)m0 * a.sxm;
  int xo[XC];
  int xl[XC];
#pragma unroll
  for (int j = 0; j < XC; ++j) {
    const int id = tid + NTHR * j;
    const int row = id / CH, c = id % CH;
    int r = row;
    if constexpr (MOE == 0) {
      if (m0 + r >= a.M) r = a.M - 1 - m0;
    } else {
      const int p = prow0 + (r < cnt ? r : cnt - 1);                  // sorted position
      r = MOE == 3 ? p : a.perm[p] / a.k;           // down reads h in sorted order, gate_up gathers
    }
    xo[j] = (int)(r * a.sxm) + c * 8;
    xl[j] = swz<C>(row, c);
  }
  constexpr int PARTS = BK / WC;                    // threads per weight row per step
  const int wrow = tid / PARTS, part = tid % PARTS;
  int gn = n0 + wrow;
  if constexpr (MOE == 1)   // gate rows then the matching up rows
    gn = wrow < BN / 2 ? tn * (BN / 2) + wrow : a.I + tn * (BN / 2) + (wrow - BN / 2);
  gn = gn < a.N ? gn : a.N - 1;
  constexpr int BYTES_STEP = BK * BITS / 8;
  const uint8_t* wtile = MOE == 0 ? a.q + (int64_t)n0 * a.sqn : a.q + (int64_t)e * a.sqe;
  const int wo = (int)((gn - (MOE == 0 ? n0 : 0)) * a.sqn) + part * (WC * BITS / 8);
  // line-tiled weights (K steps of 64 codes: 64 bytes of an int8 row, 32 of an int4 row, 16 of an
  // int2 row): the thread's bytes at SB kt + o of tile-relative row rr sit at tile rr / 16,
  // line-step SB kt / 128, half hr, slot (rr & 7) + 8 ((p / 4) ^ hr) + 16 (p & 3) for piece
  // p = (SB kt + o) / 16 of the line, byte o & 15 of the piece. int8: p = 4 (kt & 1) + o / 16,
  // line-step kt / 2; int4: p = 2 (kt & 3) + o / 16, line-step kt / 4; int2: p = kt & 7,
  // line-step kt / 8. p / 4 is uniform per step, so a thread offset for each of its values plus
  // the step's uniform part (tl_step) address every step; a 32-byte int8 load is two pieces 256
  // bytes apart.
  int wta = 0, wtb = 0;
  if constexpr (TL) {
    static_assert(BK == 64 && (WC * BITS / 8 <= 16 || (BITS == 8 && WC == 32)),
                  "a thread's bytes of a step: one 16-byte piece, or two of an int8 row");
    const int rr = gn - n0, hr = (rr >> 3) & 1, o = part * (WC * BITS / 8);
    const int tb = (rr >> 4) * 16 * (int)a.sqn + 1024 * hr + 16 * (rr & 7) + 256 * (o >> 4) + (o & 15);
    wta = tb + 128 * hr;
    wtb = tb + 128 * (1 - hr);
  }
  // uniform part of a step's tiled offset, and the step's (p / 4) bit
  auto tl_step = [&](int kt) {
    return BITS == 8 ? 2048 * (kt >> 1) : BITS == 4 ? 2048 * (kt >> 2) + 512 * (kt & 1) : 2048 * (kt >> 3) + 256 * (kt & 3);
  };
  auto tl_sel = [&](int kt) { return BITS == 8 ? (kt & 1) : BITS == 4 ? ((kt >> 1) & 1) : ((kt >> 2) & 1); };
  int bl[WC / 8];
#pragma unroll
  for (int c = 0; c < WC / 8; ++c) bl[c] = swz<C>(wrow, (WC / 8) * part + c);
  const int64_t sbase = (int64_t)gn * a.ssn + (int64_t)e * a.sse, zbase = (int64_t)gn * a.szn + (int64_t)e * a.sse;
  const int ssg = (int)a.ssg, szg = (int)a.szg;

  u32x4_t xr[PD][XC];
  WRegs<BITS, WC> wr[PD];
  uint32_t sraw[PD], zraw[PD];   // raw bits: converted only when consumed (loads stay in flight)

  const int kt0 = split * a.kps;                    // first K step of this workgroup
  auto gload = [&](int set, int ktl) {
    const int kt = kt0 + ktl;
#pragma unroll
    for (int j = 0; j < XC; ++j) xr[set][j] = *(const u32x4_t*)(xtile + kt * BK + xo[j]);
    if constexpr (TL && WRegs<BITS, WC>::BYTES == 32) {   // int8, two pieces
      const uint8_t* p = wtile + (tl_sel(kt) ? wtb : wta) + tl_step(kt);
      const u32x4_t v0 = *(const u32x4_t*)p, v1 = *(const u32x4_t*)(p + 256);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        wr[set].d[i] = v0[i];
        wr[set].d[4 + i] = v1[i];
      }
    } else if constexpr (TL)
      load_w(wr[set], wtile + (tl_sel(kt) ? wtb : wta) + tl_step(kt));
    else
      load_w(wr[set], wtile + kt * BYTES_STEP + wo);
    if constexpr (BITS != 8) {
      const int g = (kt * BK + WC * part) >> a.gsh;
      sraw[set] = load_raw_bits<SDT>(a.sc, sbase + g * ssg);
      zraw[set] = load_raw_bits<ZDT>(a.zr, zbase + g * szg);
    }
  };

  auto lstore = [&](int set, int buf) {
    uint16_t* A = As + buf * C::A_EL;
    uint16_t* B = Bs + buf * C::B_EL;
#pragma unroll
    for (int j = 0; j < XC; ++j) *(u32x4_t*)(A + xl[j]) = xr[set][j];
    float s = 0.f, nzs = 0.f;
    if constexpr (BITS != 8) {
      // scale / zero taken to bf16 first, as the reference dequant `_dequant(torch.bfloat16)` does
      s = raw_bits_to_f32<SDT>(sraw[set]);
      float z = raw_bits_to_f32<ZDT>(zraw[set]);
      if constexpr (SDT != IMQ_DT_BF16) s = round_to<IMQ_DT_BF16>(s);
      if constexpr (ZDT != IMQ_DT_BF16) z = round_to<IMQ_DT_BF16>(z);
      nzs = -z * s;
    }
#pragma unroll
    for (int c = 0; c < WC / 8; ++c) *(u32x4_t*)(B + bl[c]) = weight_chunk(wr[set], c, s, nzs);
  };

  // ---- compute plan ----------------------------------------------------------------------------
  // v_mfma_f32_32x32x16_bf16 blocks; a K step is BK/16 slices of 16 (two 16-byte chunks each:
  // lane l reads chunk 2*slice + l/32 of row l%32 of its block)
  const int wm = wave / C::WAVES_N, wn = wave % C::WAVES_N;
  constexpr int IB = WM / 32, JB = WN / 32;
  f32x16_t acc[IB][JB];
#pragma unroll
  for (int i = 0; i < IB; ++i)
#pragma unroll
    for (int j = 0; j < JB; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
  int aoff[IB][KS], boff[JB][KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
    for (int i = 0; i < IB; ++i) aoff[i][ks] = swz<C>(wm * WM + i * 32 + (lane & 31), 2 * ks + (lane >> 5));
#pragma unroll
    for (int j = 0; j < JB; ++j) boff[j][ks] = swz<C>(wn * WN + j * 32 + (lane & 31), 2 * ks + (lane >> 5));
  }

  auto compute = [&](int buf) {
    const uint16_t* A = As + buf * C::A_EL;
    const uint16_t* B = Bs + buf * C::B_EL;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      bf16x8_t af[IB], bfr[JB];
#pragma unroll
      for (int i = 0; i < IB; ++i) af[i] = *(const bf16x8_t*)(A + aoff[i][ks]);
#pragma unroll
      for (int j = 0; j < JB; ++j) bfr[j] = *(const bf16x8_t*)(B + boff[j][ks]);
#pragma unroll
      for (int i = 0; i < IB; ++i)
#pragma unroll
        for (int j = 0; j < JB; ++j) acc[i][j] = mfma32x32x16(af[i], bfr[j], acc[i][j]);
    }
  };

  // One step with the next step's LDS writes spread over the K slices: slice ks writes the
  // activation chunks j == ks (mod KS) and dequantizes / writes the weight chunks c == ks (mod KS),
  // so the VALU dequant sits between MFMAs instead of after them.
  auto step = [&](int cur, auto rsc) {
    constexpr int rs = decltype(rsc)::value;          // register set holding the next step
    const uint16_t* A = As + cur * C::A_EL;
    const uint16_t* B = Bs + cur * C::B_EL;
    uint16_t* An = As + (cur ^ 1) * C::A_EL;
    uint16_t* Bn = Bs + (cur ^ 1) * C::B_EL;
    float s = 0.f, nzs = 0.f;
    if constexpr (BITS != 8) {
      s = raw_bits_to_f32<SDT>(sraw[rs]);
      float z = raw_bits_to_f32<ZDT>(zraw[rs]);
      if constexpr (SDT != IMQ_DT_BF16) s = round_to<IMQ_DT_BF16>(s);
      if constexpr (ZDT != IMQ_DT_BF16) z = round_to<IMQ_DT_BF16>(z);
      nzs = -z * s;
    }
    // all fragment reads of the step go out first (in order of use), so the LDS latency of slice
    // ks+1.. hides behind the MFMAs of slice ks
    bf16x8_t af[KS][IB], bfr[KS][JB];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
      for (int i = 0; i < IB; ++i) af[ks][i] = *(const bf16x8_t*)(A + aoff[i][ks]);
#pragma unroll
      for (int j = 0; j < JB; ++j) bfr[ks][j] = *(const bf16x8_t*)(B + boff[j][ks]);
    }
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
      for (int i = 0; i < IB; ++i)
#pragma unroll
        for (int j = 0; j < JB; ++j) acc[i][j] = mfma32x32x16(af[ks][i], bfr[ks][j], acc[i][j]);
#pragma unroll
      for (int j = ks; j < XC; j += KS) *(u32x4_t*)(An + xl[j]) = xr[rs][j];
#pragma unroll
      for (int c = ks; c < WC / 8; c += KS) *(u32x4_t*)(Bn + bl[c]) = weight_chunk(wr[rs], c, s, nzs);
    }
  };

  // Prologue: step 0 into LDS buffer 0; step 1 in register set 1.
  const int KT = (a.K / BK - kt0) < a.kps ? (a.K / BK - kt0) : a.kps;   // this workgroup's K steps
  gload(0, 0);
  lstore(0, 0);
  gload(1, KT > 1 ? 1 : 0);
  __syncthreads();

  // Step kt: load step kt+2 into the register set freed by step kt (written to LDS during step
  // kt-1), then MFMAs on LDS buffer kt&1 while register set (kt+1)&1 -- loaded a whole step
  // earlier -- is dequantized into the other buffer. The body is branch-free so the dequant, LDS
  // writes and loads interleave with the MFMAs: past the end the loads re-read the last step (in
  // bounds) and the final writes land in the buffer no later step reads. Unrolled by two so the
  // register sets are compile-time indexed.
  auto iter = [&](int kt, auto setc) {
    constexpr int set = decltype(setc)::value;       // == kt & 1
    gload(set, kt + 2 < KT ? kt + 2 : KT - 1);
    step(set, std::integral_constant<int, 1 - set>{});
    __syncthreads();
  };
  int kt = 0;
  for (; kt + 1 < KT; kt += 2) {
    iter(kt, std::integral_constant<int, 0>{});
    iter(kt + 1, std::integral_constant<int, 1>{});
  }
  if (kt < KT) iter(kt, std::integral_constant<int, 0>{});

  // ---- grouped MoE epilogues --------------------------------------------------------------------
  if constexpr (MOE != 0) {
    auto bias_at = [&](int row) -> float {
      return a.bias != nullptr ? gemm_bias(a.bias, a.bdt, (int64_t)e * a.sbe + row) : 0.f;
    };
    if constexpr (MOE == 3) {
#pragma unroll
      for (int j = 0; j < JB; ++j) {
        const int n = n0 + wn * WN + j * 32 + (lane & 31);
        if (n >= a.N) continue;
        const float b = bias_at(n);
#pragma unroll
        for (int i = 0; i < IB; ++i)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int m = wm * WM + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
            if (m < cnt) a.yr[(int64_t)a.perm[prow0 + m] * a.N + n] = acc[i][j][r] + b;
          }
      }
    } else if constexpr (MOE == 2) {
      // interleaved (gate, up) columns sit in adjacent lanes
#pragma unroll
      for (int j = 0; j < JB; ++j) {
        const int n = n0 + wn * WN + j * 32 + (lane & 31);   // even lanes: gate rows
        const float bg = n < a.N ? bias_at(n) : 0.f, bu = n + 1 < a.N ? bias_at(n + 1) : 0.f;
#pragma unroll
        for (int i = 0; i < IB; ++i)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const float v = acc[i][j][r];
            const float up = __shfl_xor(v, 1, 64);
            const int m = wm * WM + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
            if ((lane & 1) == 0 && m < cnt && n < a.N) {
              float g = v + bg, u = up + bu;
              g = g > a.limit ? a.limit : g;
              u = u > a.limit ? a.limit : (u < -a.limit ? -a.limit : u);
              const float hv = (u + 1.f) * (g / (1.f + __expf(-a.alpha * g)));
              a.y[(int64_t)(prow0 + m) * a.sym + (n >> 1)] = (uint16_t)cvt_pk_bf16(hv, 0.f);
            }
          }
      }
    } else {
      // gate columns live in the waves of the left column half, up columns in the right half:
      // the up sums go through LDS
      constexpr int HW = C::WAVES_N / 2;
      static_assert(C::WAVES_N % 2 == 0 && BM * (BN / 2) * 4 <= C::LDS, "MOE 1 pairs the tile's column halves");
      float* U = (float*)lds;                        // [BM][BN/2], the K-loop buffers are done
      const int wcol = (wn % HW) * WN;
#pragma unroll
      for (int j = 0; j < JB; ++j)
#pragma unroll
        for (int i = 0; i < IB; ++i)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int m = wm * WM + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
            const int col = wcol + j * 32 + (lane & 31);
            if (wn >= HW) U[m * (BN / 2) + col] = acc[i][j][r];
          }
      __syncthreads();
      if (wn < HW) {
#pragma unroll
        for (int j = 0; j < JB; ++j) {
          const int col = wcol + j * 32 + (lane & 31);
          const int hc = tn * (BN / 2) + col;        // h column = gate row
          const float bg = bias_at(hc), bu = bias_at(a.I + hc);
#pragma unroll
          for (int i = 0; i < IB; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const int m = wm * WM + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
              if (m < cnt) {
                const float g = acc[i][j][r] + bg, u = U[m * (BN / 2) + col] + bu;
                a.y[(int64_t)(prow0 + m) * a.sym + hc] = (uint16_t)cvt_pk_bf16(g / (1.f + __expf(-g)) * u, 0.f);
              }
            }
        }
      }
    }
    return;
  }

  // ---- split-K: each split stores its fp32 partial tile into [split][M][N]; splitk_sum_kernel
  // sums the splits in order (deterministic) and writes y. A second launch instead of arrival
  // counters: the device-scope fences a last-arriving reduction needs would write back and
  // invalidate the XCD's whole L2 once per workgroup, evicting the shared activation tiles.
  if (a.splits > 1) {
    float* pbase = a.part + (size_t)split * a.M * a.N;
#pragma unroll
    for (int j = 0; j < JB; ++j) {
      const int n = n0 + wn * WN + j * 32 + (lane & 31);
      if (n >= a.N) continue;
#pragma unroll
      for (int i = 0; i < IB; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int m = m0 + wm * WM + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
          if (m < a.M) pbase[(size_t)m * a.N + n] = acc[i][j][r];
        }
    }
    return;
  }

  // ---- epilogue: D lane l holds column l%32, element r at row 8*(r/4) + 4*(l/32) + r%4 -------
#pragma unroll
  for (int j = 0; j < JB; ++j) {
    const int n = n0 + wn * WN + j * 32 + (lane & 31);
    if (n >= a.N) continue;
    float sc8 = 1.f;
    if constexpr (BITS == 8) sc8 = load_as_f32<SDT>(a.sc, (int64_t)n * a.ssn);
#pragma unroll
    for (int i = 0; i < IB; ++i) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = m0 + wm * WM + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (m < a.M) a.y[(int64_t)m * a.sym + n] = (uint16_t)cvt_pk_bf16(acc[i][j][r] * sc8, 0.f);
      }
    }
  }
}

// Split-K factor for a launch of T tiles over KT steps of K: 1 while the tiles fill at least
// three quarters of the CUs, else the smallest power of two reaching one tile per CU, capped at 8
// and at 8 K steps per split.
inline int split_plan(int64_t T, int KT, int cus) {
  if (4 * T >= 3 * (int64_t)cus) return 1;
  int s = 1;
  while (s < 8 && T * s < cus && KT / (2 * s) >= 8) s *= 2;
  return s;
}

template <class C>
int64_t split_bytes(int64_t M, int64_t N, int64_t K, int cus, int* splits_out = nullptr) {
  const int64_t T = imq_cdiv(M, C::BM) * imq_cdiv(N, C::BN);
  const int s = split_plan(T, (int)(K / C::BK), cus);
  if (splits_out) *splits_out = s;
  if (s == 1) return 0;
  return (int64_t)s * M * N * 4;
}

template <class C, int BITS, int SDT, int ZDT, bool TL = false>
int launch_cfg(const GemmArgs& a0, void* ws, int64_t ws_bytes, hipStream_t st) {
  GemmArgs a = a0;
  a.tiles_m = (a.M + C::BM - 1) / C::BM;
  a.tiles_n = (a.N + C::BN - 1) / C::BN;
  const int64_t T = (int64_t)a.tiles_m * a.tiles_n;
  if (T > 0x7fffffff) return IMQ_ERR_UNSUPPORTED;
  const int KT = a.K / C::BK;
  int s = 1;
  const int64_t need = split_bytes<C>(a.M, a.N, a.K, device_info().cus, &s);
  if (s > 1 && (!ws || ws_bytes < need || ((uintptr_t)ws & 15))) s = 1;
  a.splits = s;
  a.kps = (KT + s - 1) / s;
  a.part = s > 1 ? (float*)ws : nullptr;
  if (T * s > 0x7fffffff) return IMQ_ERR_UNSUPPORTED;
  auto kern = gemm_wq_kernel<C, BITS, SDT, ZDT, 0, TL>;
  if (C::LDS > 65536) {
    static int attr_set = 0;   // benign race: every caller sets the same attribute value
    if (!__atomic_load_n(&attr_set, __ATOMIC_ACQUIRE)) {
      hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, C::LDS);
      if (e != hipSuccess) return (int)e;
      __atomic_store_n(&attr_set, 1, __ATOMIC_RELEASE);
    }
  }
  kern<<<dim3((unsigned)(T * s)), dim3(C::NTHR), C::LDS, st>>>(a);
  IMQ_LAUNCH_CHECK();
  if (s > 1) return splitk_sum<BITS, SDT>(a.part, s, a.M, a.N, a.sc, a.ssn, a.y, a.sym, st);
  return IMQ_OK;
}

// Tile configurations (selected on the host by how many workgroup tiles the shape yields).
#ifndef IMQ_GEMM_CFG_BIG
#define IMQ_GEMM_CFG_BIG 256, 128, 64, 4, 2, 1
#endif
#ifndef IMQ_GEMM_CFG_SMALL
#define IMQ_GEMM_CFG_SMALL 128, 128, 64, 2, 2, 2
#endif
using CfgBig = Cfg<IMQ_GEMM_CFG_BIG>;
using CfgSmall = Cfg<IMQ_GEMM_CFG_SMALL>;

// 256 x 128 tiles once M spans two 128-row tiles, else 128 x 128; either splits K when its tiles
// do not fill the CUs.
inline bool use_big(int64_t M) { return M > 128; }

template <int BITS, int SDT, int ZDT, bool TL = false>
int launch_gemm(const GemmArgs& a, void* ws, int64_t wsb, hipStream_t st) {
  if (use_big(a.M)) return launch_cfg<CfgBig, BITS, SDT, ZDT, TL>(a, ws, wsb, st);
  return launch_cfg<CfgSmall, BITS, SDT, ZDT, TL>(a, ws, wsb, st);
}

template <int BITS, int SDT>
int gemm_z(const GemmArgs& a, int zdt, void* ws, int64_t wsb, hipStream_t st) {
  if constexpr (BITS == 8) {
    return launch_gemm<8, SDT, SDT>(a, ws, wsb, st);
  } else {
    switch (zdt) {
      case IMQ_DT_BF16: return launch_gemm<BITS, SDT, IMQ_DT_BF16>(a, ws, wsb, st);
      case IMQ_DT_FP16: return launch_gemm<BITS, SDT, IMQ_DT_FP16>(a, ws, wsb, st);
      case IMQ_DT_FP32: return launch_gemm<BITS, SDT, IMQ_DT_FP32>(a, ws, wsb, st);
    }
    return IMQ_ERR_INVALID;
  }
}

template <int BITS>
int gemm_bits(const GemmArgs& a, int sdt, int zdt, void* ws, int64_t wsb, hipStream_t st) {
  switch (sdt) {
    case IMQ_DT_BF16: return gemm_z<BITS, IMQ_DT_BF16>(a, zdt, ws, wsb, st);
    case IMQ_DT_FP16: return gemm_z<BITS, IMQ_DT_FP16>(a, zdt, ws, wsb, st);
    case IMQ_DT_FP32: return gemm_z<BITS, IMQ_DT_FP32>(a, zdt, ws, wsb, st);
  }
  return IMQ_ERR_INVALID;
}

}  // namespace

// Workspace bytes a split-K launch of this shape may use (0: no launch splits K): the larger of
// the register-B GEMM's plan (int4 / int8) and the LDS-dequant GEMM's (int2, other layouts).
// The LDS-dequant GEMM's tile and split plan for an M x N x K call on a device of `cus` CUs,
// without a device: out = {1, tile rows, tile columns, K splits}.
void gemm_plan_query(int64_t M, int64_t N, int64_t K, int cus, int64_t* out) {
  int s = 1;
  if (use_big(M)) split_bytes<CfgBig>(M, N, K, cus, &s);
  else split_bytes<CfgSmall>(M, N, K, cus, &s);
  out[0] = 1;
  out[1] = use_big(M) ? CfgBig::BM : CfgSmall::BM;
  out[2] = use_big(M) ? CfgBig::BN : CfgSmall::BN;
  out[3] = s;
}

int64_t gemm_workspace_bytes(int64_t M, int64_t N, int64_t K) {
  if (M <= 16 || N <= 0 || K % 64 != 0) return 0;
  const int cus = device_info().cus;
  const int64_t lds = use_big(M) ? split_bytes<CfgBig>(M, N, K, cus) : split_bytes<CfgSmall>(M, N, K, cus);
  const int64_t rb = rb_workspace_bytes(4, M, N, K, cus);
  return lds > rb ? lds : rb;
}

namespace {
// Grouped MoE GEMM (int4, G = 128): BM x BN tiles of one hit expert's sorted rows; see the
// kernel's MOE forms. Tiles past the device-side block count exit at once.
#ifndef IMQ_MOE_GEMM_CFG
#define IMQ_MOE_GEMM_CFG 64, 128, 64, 2, 2, 2
#endif
using CfgMoe = Cfg<IMQ_MOE_GEMM_CFG>;
template <int SDT, int MOE>
int moe_gemm_launch(const GemmArgs& a, int64_t max_mt, hipStream_t st) {
  const int64_t grid = max_mt * a.tiles_n;
  if (grid > 0x7fffffff || grid <= 0) return grid <= 0 ? IMQ_OK : IMQ_ERR_UNSUPPORTED;
  auto kern = gemm_wq_kernel<CfgMoe, 4, SDT, SDT, MOE>;
  if (CfgMoe::LDS > 65536) {
    static int attr_set = 0;   // benign race: every caller sets the same attribute value
    if (!__atomic_load_n(&attr_set, __ATOMIC_ACQUIRE)) {
      hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, CfgMoe::LDS);
      if (e != hipSuccess) return (int)e;
      __atomic_store_n(&attr_set, 1, __ATOMIC_RELEASE);
    }
  }
  kern<<<dim3((unsigned)grid), dim3(CfgMoe::NTHR), CfgMoe::LDS, st>>>(a);
  IMQ_LAUNCH_CHECK();
  return IMQ_OK;
}
}  // namespace

int moe_gemm_bm() { return CfgMoe::BM; }
int moe_gemm_bn() { return CfgMoe::BN; }

// mode 1: gate_up SiLU-GLU (N = 2I, I a multiple of BN / 2), 2: gate_up gpt-oss (N = 2I), 3: down (N = H).
// x rows: hidden (modes 1, 2: row perm[p] / k) or h (mode 3: row p), stride sxm, K columns.
// check_only: validate the shape and layout, launch nothing.
int moe_gemm_w4(int mode, const uint16_t* x, int64_t sxm, int64_t xrows, int64_t K, const uint8_t* q, int64_t sqe,
                int64_t sqn,
                const void* sc, const void* zr, int64_t sse, int64_t ssn, int sdt, int64_t N, int64_t I,
                const int32_t* mtl, const int32_t* nmt, int64_t max_mt, const int32_t* off, const int32_t* perm, int k,
                const void* bias, int64_t sbe, int bdt, float alpha, float limit, uint16_t* h, int64_t hs,
                float* yr, hipStream_t st, bool check_only) {
  if (K % CfgMoe::BK != 0 || K <= 0 || N <= 0 || (mode == 1 && I % (CfgMoe::BN / 2) != 0)) return IMQ_ERR_UNSUPPORTED;
  if (((uintptr_t)x & 15) || (sxm & 7) || ((uintptr_t)q & 15) || (sqn & 15) || (sqe & 15)) return IMQ_ERR_UNSUPPORTED;
  if (128 * sqn > 0x7fffffff || N * sqn > 0x7fffffff || xrows * sxm > 0x7fffffff) return IMQ_ERR_UNSUPPORTED;
  if (check_only) return IMQ_OK;
  GemmArgs a{x, sxm, 0, (int)K, q, sqn, sc, ssn, 1, zr, ssn, 1, (int)N, 7, h, hs, 0, 0, 1, 0, nullptr};
  a.tiles_n = mode == 1 ? (int)(I / (CfgMoe::BN / 2)) : (int)((N + CfgMoe::BN - 1) / CfgMoe::BN);
  a.kps = (int)(K / CfgMoe::BK);
  a.mtl = mtl;
  a.nmt = nmt;
  a.off = off;
  a.perm = perm;
  a.sqe = sqe;
  a.sse = sse;
  a.k = k;
  a.I = (int)I;
  a.bias = bias;
  a.sbe = sbe;
  a.bdt = bdt;
  a.alpha = alpha;
  a.limit = limit;
  a.yr = yr;
#define IMQ_MG(S) (mode == 1 ? moe_gemm_launch<S, 1>(a, max_mt, st) : mode == 2 ? moe_gemm_launch<S, 2>(a, max_mt, st) \
                                                                              : moe_gemm_launch<S, 3>(a, max_mt, st))
  switch (sdt) {
    case IMQ_DT_BF16: return IMQ_MG(IMQ_DT_BF16);
    case IMQ_DT_FP16: return IMQ_MG(IMQ_DT_FP16);
    case IMQ_DT_FP32: return IMQ_MG(IMQ_DT_FP32);
  }
#undef IMQ_MG
  return IMQ_ERR_INVALID;
}

// Prefill GEMM entry used by imq_linear_w4 / _w2 / _w8 for M > 16. Returns IMQ_ERR_UNSUPPORTED
// for shapes the tiled kernel does not cover (K not a multiple of 64, groups below 32 codes or
// not a power of two, misaligned operands, offsets beyond 32 bits); the caller then uses the
// generic kernel. Without a large enough workspace the launch does not split K.
namespace {
int gemm_wq_any(int bits, const uint16_t* x, int64_t sxm, int64_t M, int64_t K, const uint8_t* q, int64_t sqn,
                const void* sc, int64_t ssn, int64_t ssg, int sdt, const void* zr, int64_t szn, int64_t szg,
                int zdt, int64_t N, int64_t G, uint16_t* y, int64_t sym, void* ws, int64_t wsb, hipStream_t st,
                bool tiled) {
  if (M <= 0 || N <= 0) return IMQ_OK;
  if (K % 64 != 0 || M > 0x7fffffff || N > 0x7fffffff || K > 0x7fffffff) return IMQ_ERR_UNSUPPORTED;
  int gsh = 0;
  if (bits != 8) {
    if (G < 32 || (G & (G - 1)) != 0) return IMQ_ERR_UNSUPPORTED;   // power-of-two groups >= 32
    while ((1 << gsh) < G) ++gsh;
    const int64_t gmax = ssg > szg ? ssg : szg;
    if (ssg < 0 || szg < 0 || (K >> gsh) * gmax > 0x7fffffff) return IMQ_ERR_UNSUPPORTED;   // 32-bit offsets
  }
  if (((uintptr_t)x & 15) || (sxm & 7)) return IMQ_ERR_UNSUPPORTED;
  if (sxm < 0 || sqn < 0 || 256 * sxm > 0x7fffffff || 128 * sqn > 0x7fffffff) return IMQ_ERR_UNSUPPORTED;
  // widest weight load of either tile configuration: 16 B (int4, int8 as 2 x 16 B), 8 B (int2)
  const int wbytes = bits == 2 ? 8 : 16;
  if (((uintptr_t)q % wbytes) || (sqn % wbytes)) return IMQ_ERR_UNSUPPORTED;
  if (rb_takes(bits, M, N, K, G)) {
    const int rc = gemm_rb(bits, x, sxm, M, K, q, sqn, sc, ssn, ssg, sdt, zr, szn, szg, zdt, N, G, y, sym, ws, wsb, st,
                           tiled);
    if (rc != IMQ_ERR_UNSUPPORTED) return rc;
  }
  GemmArgs a{x, sxm, (int)M, (int)K, q, sqn, sc, ssn, ssg, zr, szn, szg, (int)N, gsh, y, sym, 0, 0, 1, 0,
             nullptr};
  if (tiled) {   // line-tiled weights: scale and zero of one dtype (int8: the scale's)
    if (sdt != zdt && bits != 8) return IMQ_ERR_UNSUPPORTED;
    if (bits == 8) {
      switch (sdt) {
        case IMQ_DT_BF16: return launch_gemm<8, IMQ_DT_BF16, IMQ_DT_BF16, true>(a, ws, wsb, st);
        case IMQ_DT_FP16: return launch_gemm<8, IMQ_DT_FP16, IMQ_DT_FP16, true>(a, ws, wsb, st);
        case IMQ_DT_FP32: return launch_gemm<8, IMQ_DT_FP32, IMQ_DT_FP32, true>(a, ws, wsb, st);
      }
    } else if (bits == 4) {
      switch (sdt) {
        case IMQ_DT_BF16: return launch_gemm<4, IMQ_DT_BF16, IMQ_DT_BF16, true>(a, ws, wsb, st);
        case IMQ_DT_FP16: return launch_gemm<4, IMQ_DT_FP16, IMQ_DT_FP16, true>(a, ws, wsb, st);
        case IMQ_DT_FP32: return launch_gemm<4, IMQ_DT_FP32, IMQ_DT_FP32, true>(a, ws, wsb, st);
      }
    } else if (bits == 2) {
      switch (sdt) {
        case IMQ_DT_BF16: return launch_gemm<2, IMQ_DT_BF16, IMQ_DT_BF16, true>(a, ws, wsb, st);
        case IMQ_DT_FP16: return launch_gemm<2, IMQ_DT_FP16, IMQ_DT_FP16, true>(a, ws, wsb, st);
        case IMQ_DT_FP32: return launch_gemm<2, IMQ_DT_FP32, IMQ_DT_FP32, true>(a, ws, wsb, st);
      }
    }
    return IMQ_ERR_UNSUPPORTED;
  }
  switch (bits) {
    case 4: return gemm_bits<4>(a, sdt, zdt, ws, wsb, st);
    case 2: return gemm_bits<2>(a, sdt, zdt, ws, wsb, st);
    case 8: return gemm_bits<8>(a, sdt, zdt, ws, wsb, st);
  }
  return IMQ_ERR_INVALID;
}
}  // namespace

int gemm_wq(int bits, const uint16_t* x, int64_t sxm, int64_t M, int64_t K, const uint8_t* q, int64_t sqn,
            const void* sc, int64_t ssn, int64_t ssg, int sdt, const void* zr, int64_t szn, int64_t szg,
            int zdt, int64_t N, int64_t G, uint16_t* y, int64_t sym, void* ws, int64_t wsb, hipStream_t st) {
  return gemm_wq_any(bits, x, sxm, M, K, q, sqn, sc, ssn, ssg, sdt, zr, szn, szg, zdt, N, G, y, sym, ws, wsb, st,
                     false);
}

// int4 groups of 128 in the line-tiled layout (rows of K / 2 bytes, N a multiple of 16, K a
// multiple of 256): the same kernels and results as gemm_wq on the row layout; shapes they
// decline return IMQ_ERR_UNSUPPORTED (no row-layout fallback may read these bytes).
int gemm_wq_tiled(int bits, const uint16_t* x, int64_t sxm, int64_t M, int64_t K, const uint8_t* q, const void* sc,
                  int64_t ssn, int64_t ssg, int sdt, const void* zr, int64_t szn, int64_t szg, int zdt, int64_t N,
                  uint16_t* y, int64_t sym, void* ws, int64_t wsb, hipStream_t st) {
  if ((bits != 8 && bits != 4 && bits != 2) || N % 16 != 0 || (K * bits / 8) % 128 != 0) return IMQ_ERR_UNSUPPORTED;
  return gemm_wq_any(bits, x, sxm, M, K, q, K * bits / 8, sc, ssn, ssg, sdt, zr, szn, szg, zdt, N,
                     bits == 8 ? 0 : bits == 4 ? 128 : 64, y, sym, ws, wsb, st, true);
}

}  // namespace imq
