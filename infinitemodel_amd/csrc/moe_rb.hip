// Grouped MoE forms of the register-B GEMM (rb_kernel.h): one hit expert's sorted, gathered
// rows per row block, SiLU-GLU / gpt-oss GLU in gate_up's epilogue, down's rows scattered to
// routed order. Built with the MFMA results in VGPRs (build flag), which the folded form's
// per-group fold reads with plain VALU ops.
#include "rb_kernel.h"

namespace imq {
namespace {

#ifndef IMQ_MOE_RB_PD
#define IMQ_MOE_RB_PD 2
#endif
// 1: the MoE forms run scale-folded (magic-128 operands, per-group fold, row-sum correction)
#ifndef IMQ_MOE_RB_FOLD
#define IMQ_MOE_RB_FOLD 1
#endif
// The MoE forms stage K / 128 groups of scale / zero pairs (and, folded, of the block rows' group
// sums) in LDS beside the three 64-row activation buffers (24 KiB): up to 40 groups (K <= 5120),
// 74 KiB per workgroup at most, two workgroups per CU.
constexpr int kMoeRbMaxGroups = 40;
template <int SDT, int IB, int MOE>
constexpr size_t moe_rb_lds(int ng) {
  return (size_t)3 * 32 * IB * RB_BK * 2 + (size_t)ng * 256 * 4 + (IMQ_MOE_RB_FOLD ? (size_t)ng * 32 * IB * 4 : 0) +
         (size_t)32 * IB * 4;   // RID: the block's routed rows
}
template <int SDT, int IB, int MOE>
int moe_rb_launch(const RbArgs& a, int64_t max_mt, hipStream_t st) {
  constexpr int NW = 4;
  const int64_t grid = max_mt * a.tiles_n;
  if (grid <= 0) return IMQ_OK;
  if (grid > 0x7fffffff) return IMQ_ERR_UNSUPPORTED;
  size_t lds = moe_rb_lds<SDT, IB, MOE>(a.K >> a.gsh);
  if (MOE == 3 && a.yrb != nullptr && lds < (size_t)32 * IB * (64 * NW + 8) * 2)
    lds = (size_t)32 * IB * (64 * NW + 8) * 2;   // the bf16 row tile of the epilogue
  auto kern = gemm_rb_kernel<4, SDT, SDT, IB, NW, MOE, IMQ_MOE_RB_PD, IMQ_MOE_RB_FOLD != 0>;
  if (lds > 65536) {
    static int attr_set = 0;   // benign race: every caller sets the same value
    if (!__atomic_load_n(&attr_set, __ATOMIC_ACQUIRE)) {
      hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                                         (int)moe_rb_lds<SDT, IB, MOE>(kMoeRbMaxGroups));
      if (e != hipSuccess) return (int)e;
      __atomic_store_n(&attr_set, 1, __ATOMIC_RELEASE);
    }
  }
  kern<<<dim3((unsigned)grid), dim3(64 * NW), lds, st>>>(a);
  IMQ_LAUNCH_CHECK();
  return IMQ_OK;
}

template <int SDT, int IB>
int moe_rb_mode(int mode, const RbArgs& a, int64_t max_mt, hipStream_t st) {
  switch (mode) {
    case 1: return moe_rb_launch<SDT, IB, 1>(a, max_mt, st);
    case 2: return moe_rb_launch<SDT, IB, 2>(a, max_mt, st);
    case 3: return moe_rb_launch<SDT, IB, 3>(a, max_mt, st);
  }
  return IMQ_ERR_INVALID;
}

template <int SDT>
int moe_rb_ib(int mode, const RbArgs& a, int64_t max_mt, hipStream_t st) {
  return moe_rb_mode<SDT, 2>(mode, a, max_mt, st);
}

}  // namespace

// Whether the MoE forms run scale-folded (then the caller supplies the rows' group sums).
bool moe_rb_folded() { return IMQ_MOE_RB_FOLD != 0; }

// Grouped MoE launch of the register-B kernel (int4, groups of 128 codes, scale / zero
// [E][N][groups] with a unit group stride, 64 sorted rows per block: ib 2, the sort's block size;
// measured on MI355X, 128-row blocks never paid: the folded form's registers then allow one wave
// per SIMD and the dequantizing one dequantizes twice the MFMA work per weight load). mode 1: gate_up SiLU-GLU (N = 2I, I a multiple of 128); 2: gpt-oss gate_up
// (N = 2I, interleaved rows); 3: down (N = H). x rows: hidden (modes 1, 2: row perm[p] / k) or h
// (mode 3: row p), stride sxm, K columns of which the first xk (a multiple of the 64-column K
// step; 0: all) are read -- the K steps past them hold zero activations and are skipped; down
// writes yr as fp32 rows, or bf16 ones with yr_bf16
// (N % 64 == 0). check_only: validate the shape and layout, launch
// nothing. IMQ_ERR_UNSUPPORTED for what the kernel does not cover.
int moe_rb(int mode, int ib, const uint16_t* x, int64_t sxm, int64_t xrows, int64_t K, int64_t xk, const uint8_t* q,
           int64_t sqe, int64_t sqn, const void* sc, const void* zr, int64_t sse, int64_t ssn, int sdt, int64_t N,
           int64_t I, const int32_t* mtl, const int32_t* nmt, int64_t max_mt, const int32_t* off,
           const int32_t* perm, int k, const void* bias, int64_t sbe, int bdt, float alpha, float limit,
           uint16_t* h, int64_t hs, float* yr, bool yr_bf16, const float* rs, int rs_stride, int rs_groups,
           float* hrs, int hrs_stride, hipStream_t st, bool check_only) {
  if (ib != 2 || mode < 1 || mode > 3) return IMQ_ERR_UNSUPPORTED;
  if (K <= 0 || K % 128 || K / 128 > kMoeRbMaxGroups || N <= 0 || N > 0x7fffffff) return IMQ_ERR_UNSUPPORTED;
  if (mode == 1 && (I % 128 || N != 2 * I)) return IMQ_ERR_UNSUPPORTED;
  if (mode == 2 && (N % 2 || N != 2 * I)) return IMQ_ERR_UNSUPPORTED;
  if (((uintptr_t)x & 15) || (sxm & 7) || ((uintptr_t)q & 15) || (sqn & 15) || (sqe & 15)) return IMQ_ERR_UNSUPPORTED;
  if (xk <= 0) xk = K;
  if (xk % RB_BK || xk > K) return IMQ_ERR_UNSUPPORTED;
  if (sxm < xk || sqn < K / 2 || xrows <= 0 || (xrows + 1) * sxm > 0x7fffffff) return IMQ_ERR_UNSUPPORTED;
  if (mode != 3 && (hs % 8 || ((uintptr_t)h & 15))) return IMQ_ERR_UNSUPPORTED;   // 16-byte h row segments
  if (mode == 3 && yr_bf16 && (N % 64 || ((uintptr_t)yr & 15))) return IMQ_ERR_UNSUPPORTED;   // 16-byte y segments
  if (check_only) return IMQ_OK;
  if (moe_rb_folded() && (!rs || rs_stride < rs_groups || rs_groups < 0)) return IMQ_ERR_INVALID;
  RbArgs a{x, sxm, 0, (int)K, q, sqn, sc, ssn, 1, zr, ssn, 1, (int)N, 7, h, hs, 1, 0, 1, (int)(K / RB_BK), nullptr};
  a.xk = (int)xk;
  a.rs = rs;
  a.rs_stride = rs_stride;
  a.rs_groups = rs_groups;
  a.hrs = hrs;
  a.hrs_stride = hrs_stride;
  a.tiles_n = mode == 1 ? (int)(I / 128) : (int)((N + 255) / 256);
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
  a.yr = yr_bf16 ? nullptr : yr;
  a.yrb = yr_bf16 ? (uint16_t*)yr : nullptr;
  switch (sdt) {
    case IMQ_DT_BF16: return moe_rb_ib<IMQ_DT_BF16>(mode, a, max_mt, st);
    case IMQ_DT_FP16: return moe_rb_ib<IMQ_DT_FP16>(mode, a, max_mt, st);
    case IMQ_DT_FP32: return moe_rb_ib<IMQ_DT_FP32>(mode, a, max_mt, st);
  }
  return IMQ_ERR_INVALID;
}

}  // namespace imq
