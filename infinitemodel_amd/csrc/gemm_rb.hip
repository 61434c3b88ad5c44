// Prefill-regime fused dequant GEMM with the weights dequantized straight into MFMA B operands
// ("register-B" form): the dense launchers (tile plan, split-K partials and their reduction).
// The kernel and its structure are described in rb_kernel.h.
#include "rb_kernel.h"
#include "splitk_sum.h"

namespace imq {

int64_t rb_workspace_bytes(int bits, int64_t M, int64_t N, int64_t K, int cus);

namespace {

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

template <int BITS, int SDT, int ZDT, int IB, bool TL>
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
  auto kern = gemm_rb_kernel<BITS, SDT, ZDT, IB, NW, 0, 2, false, TL>;
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
  if (s > 1) return splitk_sum<BITS, SDT>(a.part, s, a.M, a.N, a.sc, a.ssn, a.y, a.sym, st);
  return IMQ_OK;
}

template <int BITS, int SDT, int ZDT, bool TL = false>
int rb_ib_dispatch(const RbArgs& a, void* ws, int64_t wsb, hipStream_t st) {
  int ib, s;
  rb_plan(a.M, a.N, a.K, device_info().cus, &ib, &s);
  if (ib == 8) return rb_launch<BITS, SDT, ZDT, 8, TL>(a, ws, wsb, st);
  return rb_launch<BITS, SDT, ZDT, 4, TL>(a, ws, wsb, st);
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

// The register-B GEMM's plan for an M x N x K call (int4 groups of G, or int8) on a device of
// `cus` CUs, without a device: out = {takes the call, 32-row blocks per wave, K splits}.
void rb_plan_query(int bits, int64_t M, int64_t N, int64_t K, int64_t G, int cus, int64_t* out) {
  int ib = 0, s = 0;
  const bool takes = rb_takes(bits, M, N, K, G);
  if (takes) rb_plan(M, N, K, cus, &ib, &s);
  out[0] = takes ? 1 : 0;
  out[1] = ib;
  out[2] = s;
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
            int64_t N, int64_t G, uint16_t* y, int64_t sym, void* ws, int64_t wsb, hipStream_t st, bool tiled) {
  if (((uintptr_t)x & 15) || (sxm & 7) || ((uintptr_t)q & 15) || (sqn & 15)) return IMQ_ERR_UNSUPPORTED;
  if (tiled && (N % 16 != 0 || (K * bits / 8) % 128 != 0 || sqn != K * bits / 8)) return IMQ_ERR_UNSUPPORTED;
  if (sxm < 0 || sqn < 0 || 256 * sxm > 0x7fffffff) return IMQ_ERR_UNSUPPORTED;
  // the kernel's buffer offsets from a tile's first row (activations, weights, scale / zero)
  if ((256 * sxm + K) * 2 > 0x7fffffff || 256 * sqn + K > 0x7fffffff) return IMQ_ERR_UNSUPPORTED;
  int gsh = 0;
  if (bits == 4) {
    while ((1 << gsh) < G) ++gsh;
    if (ssg < 0 || szg < 0 || ssn < 0 || szn < 0) return IMQ_ERR_UNSUPPORTED;
    const int64_t ng = K / G + 1;
    if ((256 * ssn + ng * ssg) * 4 > 0x7fffffff || (256 * szn + ng * szg) * 4 > 0x7fffffff) return IMQ_ERR_UNSUPPORTED;
  }
  RbArgs a{x, sxm, (int)M, (int)K, q, sqn, sc, ssn, ssg, zr, szn, szg, (int)N, gsh, y, sym, 0, 0, 1, 0, nullptr};
  if (tiled) {   // line-tiled weights: int4 with scale and zero of one dtype, or int8
    if (bits == 4 && sdt != zdt) return IMQ_ERR_UNSUPPORTED;
    switch (sdt) {
      case IMQ_DT_BF16:
        return bits == 8 ? rb_ib_dispatch<8, IMQ_DT_BF16, IMQ_DT_BF16, true>(a, ws, wsb, st)
                         : rb_ib_dispatch<4, IMQ_DT_BF16, IMQ_DT_BF16, true>(a, ws, wsb, st);
      case IMQ_DT_FP16:
        return bits == 8 ? rb_ib_dispatch<8, IMQ_DT_FP16, IMQ_DT_FP16, true>(a, ws, wsb, st)
                         : rb_ib_dispatch<4, IMQ_DT_FP16, IMQ_DT_FP16, true>(a, ws, wsb, st);
      case IMQ_DT_FP32:
        return bits == 8 ? rb_ib_dispatch<8, IMQ_DT_FP32, IMQ_DT_FP32, true>(a, ws, wsb, st)
                         : rb_ib_dispatch<4, IMQ_DT_FP32, IMQ_DT_FP32, true>(a, ws, wsb, st);
    }
    return IMQ_ERR_INVALID;
  }
  switch (sdt) {
    case IMQ_DT_BF16: return bits == 8 ? rb_z<8, IMQ_DT_BF16>(a, zdt, ws, wsb, st) : rb_z<4, IMQ_DT_BF16>(a, zdt, ws, wsb, st);
    case IMQ_DT_FP16: return bits == 8 ? rb_z<8, IMQ_DT_FP16>(a, zdt, ws, wsb, st) : rb_z<4, IMQ_DT_FP16>(a, zdt, ws, wsb, st);
    case IMQ_DT_FP32: return bits == 8 ? rb_z<8, IMQ_DT_FP32>(a, zdt, ws, wsb, st) : rb_z<4, IMQ_DT_FP32>(a, zdt, ws, wsb, st);
  }
  return IMQ_ERR_INVALID;
}

}  // namespace imq
