// C-ABI entry points of the fused dequant linear family (imq_linear_w4 / _w2 / _w8) and the
// ABI metadata calls. Dispatch: decode rows (M <= 16) go to the MFMA skinny GEMV, prefill rows
// to the LDS-dequant MFMA GEMM; shapes or alignments a fast kernel rejects fall back to the
// generic dequantize-then-matmul kernel (never wrong, just slower).
//
// imq_linear_w4_noalloc is imq_linear_w4 with its workspace taken from a static per-device
// scratch array instead of a caller buffer (for callers that cannot allocate device memory).
#include <atomic>
#include <mutex>

#include "imq_common.h"

namespace imq {
int skinny_w4(const uint16_t* x, int64_t sxm, int64_t M, int64_t Kpad, const uint8_t* q, int64_t sqn,
              const void* sc, int64_t ssn, int64_t ssg, int sdt, const void* zr, int64_t szn, int64_t szg,
              int zdt, int64_t N, int64_t G, uint16_t* y, int64_t sym, void* ws, int64_t wsb, hipStream_t st,
              bool tiled);
int64_t ksplit_workspace_bytes(int64_t M, int64_t N, int64_t Kpad);
int64_t w4_decode_workspace_bytes(int64_t M, int64_t Kpad, int64_t G, int64_t N, int64_t sqn, int64_t sxm,
                                  int64_t ssn, int64_t ssg, int64_t szn, int64_t szg, int sdt, int zdt);
int skinny_w2(const uint16_t* x, int64_t sxm, int64_t M, int64_t Kpad, const uint8_t* q, int64_t sqn,
              const void* sc, int64_t ssn, int64_t ssg, int sdt, const void* zr, int64_t szn, int64_t szg,
              int zdt, int64_t N, int64_t G, uint16_t* y, int64_t sym, void* ws, int64_t wsb, hipStream_t st,
              bool tiled);
int64_t ksplit2_workspace_bytes(int64_t M, int64_t N, int64_t Kpad);
int skinny_w8(const uint16_t* x, int64_t sxm, int64_t M, int64_t K, const int8_t* q, int64_t sqn,
              const void* sc, int64_t ssn, int sdt, int64_t N, uint16_t* y, int64_t sym, hipStream_t st,
              bool tiled);
int gemm_wq(int bits, const uint16_t* x, int64_t sxm, int64_t M, int64_t K, const uint8_t* q, int64_t sqn,
            const void* sc, int64_t ssn, int64_t ssg, int sdt, const void* zr, int64_t szn, int64_t szg,
            int zdt, int64_t N, int64_t G, uint16_t* y, int64_t sym, void* ws, int64_t wsb, hipStream_t st);
int gemm_wq_tiled(int bits, const uint16_t* x, int64_t sxm, int64_t M, int64_t K, const uint8_t* q, const void* sc,
                  int64_t ssn, int64_t ssg, int sdt, const void* zr, int64_t szn, int64_t szg, int zdt, int64_t N,
                  uint16_t* y, int64_t sym, void* ws, int64_t wsb, hipStream_t st);
int64_t gemm_workspace_bytes(int64_t M, int64_t N, int64_t K);
int decode_plan_query(int kind, const int64_t* in, int64_t* out);
void gemm_plan_query(int64_t M, int64_t N, int64_t K, int cus, int64_t* out);
void rb_plan_query(int bits, int64_t M, int64_t N, int64_t K, int64_t G, int cus, int64_t* out);
template <int BITS>
int generic_gemv(const uint16_t* x, int64_t sxm, int64_t M, int64_t K, const uint8_t* q, int64_t sqn,
                 const void* sc, int64_t ssn, int64_t ssg, int sdt, const void* zr, int64_t szn,
                 int64_t szg, int zdt, int64_t N, int64_t G, uint16_t* y, int64_t sym, hipStream_t st);
}  // namespace imq

namespace {

bool dt_ok(int d) { return d == IMQ_DT_BF16 || d == IMQ_DT_FP16 || d == IMQ_DT_FP32; }

// Shared argument validation of the group-wise formats (int4 / int2).
int check_g(int bits, const void* x, int64_t sxm, int64_t M, int64_t Kpad, const void* q, int64_t sqn,
            const void* sc, int sdt, const void* zr, int zdt, int64_t N, int64_t G, const void* y,
            int64_t sym) {
  if (!x || !q || !sc || !zr || !y) return IMQ_ERR_INVALID;
  if (M < 0 || N < 0 || Kpad <= 0 || G <= 0 || Kpad % G != 0) return IMQ_ERR_INVALID;
  if ((Kpad * bits) % 8 != 0 || sqn < Kpad * bits / 8) return IMQ_ERR_INVALID;
  if (sxm < Kpad || sym < N) return IMQ_ERR_INVALID;
  if (!dt_ok(sdt) || !dt_ok(zdt)) return IMQ_ERR_INVALID;
  return IMQ_OK;
}

}  // namespace

extern "C" int imq_abi_version(void) { return IMQ_ABI_VERSION; }

extern "C" int64_t imq_linear_workspace_bytes(int64_t M, int64_t N, int64_t K_pad) {
  if (M < 0 || N < 0 || K_pad <= 0) return -1;
  const int64_t g = imq::gemm_workspace_bytes(M, N, K_pad);
  const int64_t d = imq::ksplit_workspace_bytes(M, N, K_pad);
  const int64_t d2 = imq::ksplit2_workspace_bytes(M, N, K_pad);
  const int64_t gd = g > d ? g : d;
  return gd > d2 ? gd : d2;
}

extern "C" int64_t imq_linear_w4_workspace_bytes(int64_t M, int64_t K_pad, int64_t N, int64_t group_size,
                                                 int64_t q_row_stride, int64_t x_row_stride, int64_t s_stride_n,
                                                 int64_t s_stride_g, int s_dtype, int64_t z_stride_n,
                                                 int64_t z_stride_g, int z_dtype) {
  if (M < 0 || N < 0 || K_pad <= 0 || group_size <= 0 || K_pad % group_size) return -1;
  if (M == 0 || N == 0) return 0;
  if (M > 16) return imq::gemm_workspace_bytes(M, N, K_pad);
  return imq::w4_decode_workspace_bytes(M, K_pad, group_size, N, q_row_stride, x_row_stride, s_stride_n, s_stride_g,
                                        z_stride_n, z_stride_g, s_dtype, z_dtype);
}

extern "C" int imq_launch_plan(int kind, const int64_t* in, int64_t* out) {
  if (!in || !out) return IMQ_ERR_INVALID;
  for (int i = 0; i < 5; ++i) out[i] = 0;
  const int64_t M = in[0], K = in[1], G = in[2], N = in[3];
  const int cus = (int)in[9];
  if (kind == IMQ_PLAN_GEMM) {
    if (M <= 16 || N <= 0 || K <= 0 || K % 64 != 0 || cus <= 0) return IMQ_OK;
    imq::gemm_plan_query(M, N, K, cus, out);
    return IMQ_OK;
  }
  if (kind == IMQ_PLAN_GEMM_RB) {
    if (cus <= 0) return IMQ_OK;
    imq::rb_plan_query(G == 0 ? 8 : 4, M, N, K, G == 0 ? 128 : G, cus, out);
    return IMQ_OK;
  }
  if (in[7] != IMQ_DT_BF16 && in[7] != IMQ_DT_FP16 && in[7] != IMQ_DT_FP32) return IMQ_ERR_INVALID;
  return imq::decode_plan_query(kind, in, out);
}

extern "C" const char* imq_strerror(int status) {
  switch (status) {
    case IMQ_OK: return "ok";
    case IMQ_ERR_INVALID: return "invalid argument (shape, stride, dtype or null pointer)";
    case IMQ_ERR_UNSUPPORTED: return "configuration not supported by this kernel family";
    case IMQ_ERR_ALIGN: return "pointer or stride misaligned for this kernel";
    case IMQ_ERR_SCRATCH:
      return "workspace need exceeds the static scratch of the allocation-free entry point "
             "(IMQ_NOALLOC_SCRATCH_BYTES)";
  }
  if (status > 0) return hipGetErrorString((hipError_t)status);
  return "unknown status";
}

extern "C" int imq_linear_w4(const void* x, int64_t x_row_stride, int64_t M, int64_t K_pad,
                             const void* qweight, int64_t q_row_stride, const void* scale,
                             int64_t s_stride_n, int64_t s_stride_g, int s_dtype, const void* zero,
                             int64_t z_stride_n, int64_t z_stride_g, int z_dtype, int64_t N,
                             int64_t group_size, void* y, int64_t y_row_stride, void* workspace,
                             int64_t workspace_bytes, void* stream) {
  int rc = check_g(4, x, x_row_stride, M, K_pad, qweight, q_row_stride, scale, s_dtype, zero, z_dtype, N,
                   group_size, y, y_row_stride);
  if (rc != IMQ_OK) return rc;
  if (M == 0 || N == 0) return IMQ_OK;
  hipStream_t st = (hipStream_t)stream;
  const uint16_t* xb = (const uint16_t*)x;
  uint16_t* yb = (uint16_t*)y;
  const uint8_t* q = (const uint8_t*)qweight;
  if (M <= 16) {
    rc = imq::skinny_w4(xb, x_row_stride, M, K_pad, q, q_row_stride, scale, s_stride_n, s_stride_g, s_dtype,
                        zero, z_stride_n, z_stride_g, z_dtype, N, group_size, yb, y_row_stride, workspace,
                        workspace_bytes, st, false);
  } else {
    rc = imq::gemm_wq(4, xb, x_row_stride, M, K_pad, q, q_row_stride, scale, s_stride_n, s_stride_g,
                      s_dtype, zero, z_stride_n, z_stride_g, z_dtype, N, group_size, yb, y_row_stride,
                      workspace, workspace_bytes, st);
  }
  if (rc != IMQ_ERR_UNSUPPORTED) return rc;
  return imq::generic_gemv<4>(xb, x_row_stride, M, K_pad, q, q_row_stride, scale, s_stride_n, s_stride_g,
                              s_dtype, zero, z_stride_n, z_stride_g, z_dtype, N, group_size, yb,
                              y_row_stride, st);
}

// int4 weights in the line-tiled layout: the arguments and results of imq_linear_w4. The layout
// permutes 16-byte pieces within each 16-row tile (N a multiple of 16, dense rows of K_pad / 2
// bytes, K_pad a multiple of 256, groups of 128); the kernels that read it are the decode line,
// wave-split and K-split kernels and the two prefill GEMMs. A call none of them takes returns
// IMQ_ERR_UNSUPPORTED: no row-layout kernel may read these bytes.
extern "C" int imq_linear_w4_tiled(const void* x, int64_t x_row_stride, int64_t M, int64_t K_pad,
                                   const void* qweight, int64_t q_row_stride, const void* scale,
                                   int64_t s_stride_n, int64_t s_stride_g, int s_dtype, const void* zero,
                                   int64_t z_stride_n, int64_t z_stride_g, int z_dtype, int64_t N,
                                   int64_t group_size, void* y, int64_t y_row_stride, void* workspace,
                                   int64_t workspace_bytes, void* stream) {
  int rc = check_g(4, x, x_row_stride, M, K_pad, qweight, q_row_stride, scale, s_dtype, zero, z_dtype, N,
                   group_size, y, y_row_stride);
  if (rc != IMQ_OK) return rc;
  if (N % 16 != 0 || K_pad % 256 != 0 || group_size != 128 || q_row_stride != K_pad / 2) return IMQ_ERR_INVALID;
  if (M == 0 || N == 0) return IMQ_OK;
  hipStream_t st = (hipStream_t)stream;
  const uint16_t* xb = (const uint16_t*)x;
  uint16_t* yb = (uint16_t*)y;
  const uint8_t* q = (const uint8_t*)qweight;
  if (M <= 16)
    return imq::skinny_w4(xb, x_row_stride, M, K_pad, q, q_row_stride, scale, s_stride_n, s_stride_g, s_dtype,
                          zero, z_stride_n, z_stride_g, z_dtype, N, group_size, yb, y_row_stride, workspace,
                          workspace_bytes, st, true);
  return imq::gemm_wq_tiled(4, xb, x_row_stride, M, K_pad, q, scale, s_stride_n, s_stride_g, s_dtype, zero,
                            z_stride_n, z_stride_g, z_dtype, N, yb, y_row_stride, workspace, workspace_bytes, st);
}

// int2 weights in the line-tiled layout: the arguments and results of imq_linear_w2 (N a multiple of
// 16, dense rows of K_pad / 4 bytes, K_pad a multiple of 512, groups of 64); the decode line and
// K-split kernels and the LDS-dequant GEMM read it, other calls return IMQ_ERR_UNSUPPORTED.
extern "C" int imq_linear_w2_tiled(const void* x, int64_t x_row_stride, int64_t M, int64_t K_pad,
                                   const void* qweight, int64_t q_row_stride, const void* scale,
                                   int64_t s_stride_n, int64_t s_stride_g, int s_dtype, const void* zero,
                                   int64_t z_stride_n, int64_t z_stride_g, int z_dtype, int64_t N,
                                   int64_t group_size, void* y, int64_t y_row_stride, void* workspace,
                                   int64_t workspace_bytes, void* stream) {
  int rc = check_g(2, x, x_row_stride, M, K_pad, qweight, q_row_stride, scale, s_dtype, zero, z_dtype, N,
                   group_size, y, y_row_stride);
  if (rc != IMQ_OK) return rc;
  if (N % 16 != 0 || K_pad % 512 != 0 || group_size != 64 || q_row_stride != K_pad / 4) return IMQ_ERR_INVALID;
  if (M == 0 || N == 0) return IMQ_OK;
  hipStream_t st = (hipStream_t)stream;
  const uint16_t* xb = (const uint16_t*)x;
  uint16_t* yb = (uint16_t*)y;
  const uint8_t* q = (const uint8_t*)qweight;
  if (M <= 16)
    return imq::skinny_w2(xb, x_row_stride, M, K_pad, q, q_row_stride, scale, s_stride_n, s_stride_g, s_dtype,
                          zero, z_stride_n, z_stride_g, z_dtype, N, group_size, yb, y_row_stride, workspace,
                          workspace_bytes, st, true);
  return imq::gemm_wq_tiled(2, xb, x_row_stride, M, K_pad, q, scale, s_stride_n, s_stride_g, s_dtype, zero,
                            z_stride_n, z_stride_g, z_dtype, N, yb, y_row_stride, workspace, workspace_bytes, st);
}

// int8 weights in the line-tiled layout: the arguments and results of imq_linear_w8 (N a multiple of
// 16, dense rows of K bytes, K a multiple of 128); the decode line and skinny kernels and both
// prefill GEMMs read it, other calls return IMQ_ERR_UNSUPPORTED.
extern "C" int imq_linear_w8_tiled(const void* x, int64_t x_row_stride, int64_t M, int64_t K,
                                   const void* qweight, int64_t q_row_stride, const void* scale,
                                   int64_t s_stride_n, int s_dtype, int64_t N, void* y, int64_t y_row_stride,
                                   void* workspace, int64_t workspace_bytes, void* stream) {
  if (!x || !qweight || !scale || !y || M < 0 || N < 0 || K <= 0) return IMQ_ERR_INVALID;
  if (q_row_stride < K || x_row_stride < K || y_row_stride < N || !dt_ok(s_dtype)) return IMQ_ERR_INVALID;
  if (N % 16 != 0 || K % 128 != 0 || q_row_stride != K) return IMQ_ERR_INVALID;
  if (M == 0 || N == 0) return IMQ_OK;
  hipStream_t st = (hipStream_t)stream;
  const uint16_t* xb = (const uint16_t*)x;
  uint16_t* yb = (uint16_t*)y;
  if (M <= 16)
    return imq::skinny_w8(xb, x_row_stride, M, K, (const int8_t*)qweight, q_row_stride, scale, s_stride_n, s_dtype,
                          N, yb, y_row_stride, st, true);
  return imq::gemm_wq_tiled(8, xb, x_row_stride, M, K, (const uint8_t*)qweight, scale, s_stride_n, 0, s_dtype,
                            nullptr, 0, 0, s_dtype, N, yb, y_row_stride, workspace, workspace_bytes, st);
}

// ---- allocation-free variant of imq_linear_w4 ----------------------------------------------------
// The scratch array: each device the library runs on holds its own copy until the process ends.
// Host code never uses the name `scratch` as an address (on the host it is only a stand-in for
// the symbol): the device address comes from hipGetSymbolAddress, once per device, and only that
// pointer is passed to kernels.
static __device__ __align__(256) unsigned char scratch[IMQ_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
std::atomic<void*> g_scratch_ptr[kMaxDevices];

// Device address of the current device's scratch array, resolved on the first call per device
// (with that device current) and cached.
int scratch_ptr(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= kMaxDevices) return IMQ_ERR_UNSUPPORTED;
  void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (!p) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
    if (!p) {
      e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (e != hipSuccess) return (int)e;
      if (!p) return IMQ_ERR_UNSUPPORTED;
      g_scratch_ptr[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return IMQ_OK;
}

}  // namespace

extern "C" int imq_linear_w4_noalloc(const void* x, int64_t x_row_stride, int64_t M, int64_t K_pad,
                                     const void* qweight, int64_t q_row_stride, const void* scale,
                                     int64_t s_stride_n, int64_t s_stride_g, int s_dtype, const void* zero,
                                     int64_t z_stride_n, int64_t z_stride_g, int z_dtype, int64_t N,
                                     int64_t group_size, void* y, int64_t y_row_stride, void* stream) {
  int rc = check_g(4, x, x_row_stride, M, K_pad, qweight, q_row_stride, scale, s_dtype, zero, z_dtype, N,
                   group_size, y, y_row_stride);
  if (rc != IMQ_OK) return rc;
  if (M == 0 || N == 0) return IMQ_OK;
  // The partials of the K-split / split-K launches need no initialisation (every element a
  // reduction reads is written first by the same call), so the array is never cleared. The need
  // is this call's own (the dispatcher's plans for these strides on this device): shapes whose
  // kernels keep their partials in the workgroup need none, whatever their size.
  const int64_t need = imq_linear_w4_workspace_bytes(M, K_pad, N, group_size, q_row_stride, x_row_stride, s_stride_n,
                                                     s_stride_g, s_dtype, z_stride_n, z_stride_g, z_dtype);
  if (need > IMQ_NOALLOC_SCRATCH_BYTES) return IMQ_ERR_SCRATCH;
  void* ws = nullptr;
  rc = scratch_ptr(&ws);
  if (rc != IMQ_OK) return rc;
  return imq_linear_w4(x, x_row_stride, M, K_pad, qweight, q_row_stride, scale, s_stride_n, s_stride_g, s_dtype,
                       zero, z_stride_n, z_stride_g, z_dtype, N, group_size, y, y_row_stride, ws,
                       IMQ_NOALLOC_SCRATCH_BYTES, stream);
}

extern "C" int imq_linear_w2(const void* x, int64_t x_row_stride, int64_t M, int64_t K_pad,
                             const void* qweight, int64_t q_row_stride, const void* scale,
                             int64_t s_stride_n, int64_t s_stride_g, int s_dtype, const void* zero,
                             int64_t z_stride_n, int64_t z_stride_g, int z_dtype, int64_t N,
                             int64_t group_size, void* y, int64_t y_row_stride, void* workspace,
                             int64_t workspace_bytes, void* stream) {
  int rc = check_g(2, x, x_row_stride, M, K_pad, qweight, q_row_stride, scale, s_dtype, zero, z_dtype, N,
                   group_size, y, y_row_stride);
  if (rc != IMQ_OK) return rc;
  if (M == 0 || N == 0) return IMQ_OK;
  hipStream_t st = (hipStream_t)stream;
  const uint16_t* xb = (const uint16_t*)x;
  uint16_t* yb = (uint16_t*)y;
  const uint8_t* q = (const uint8_t*)qweight;
  if (M <= 16) {
    rc = imq::skinny_w2(xb, x_row_stride, M, K_pad, q, q_row_stride, scale, s_stride_n, s_stride_g, s_dtype,
                        zero, z_stride_n, z_stride_g, z_dtype, N, group_size, yb, y_row_stride, workspace,
                        workspace_bytes, st, false);
  } else {
    rc = imq::gemm_wq(2, xb, x_row_stride, M, K_pad, q, q_row_stride, scale, s_stride_n, s_stride_g,
                      s_dtype, zero, z_stride_n, z_stride_g, z_dtype, N, group_size, yb, y_row_stride,
                      workspace, workspace_bytes, st);
  }
  if (rc != IMQ_ERR_UNSUPPORTED) return rc;
  return imq::generic_gemv<2>(xb, x_row_stride, M, K_pad, q, q_row_stride, scale, s_stride_n, s_stride_g,
                              s_dtype, zero, z_stride_n, z_stride_g, z_dtype, N, group_size, yb,
                              y_row_stride, st);
}

extern "C" int imq_linear_w8(const void* x, int64_t x_row_stride, int64_t M, int64_t K,
                             const void* qweight, int64_t q_row_stride, const void* scale,
                             int64_t s_stride_n, int s_dtype, int64_t N, void* y, int64_t y_row_stride,
                             void* workspace, int64_t workspace_bytes, void* stream) {
  if (!x || !qweight || !scale || !y || M < 0 || N < 0 || K <= 0) return IMQ_ERR_INVALID;
  if (q_row_stride < K || x_row_stride < K || y_row_stride < N || !dt_ok(s_dtype)) return IMQ_ERR_INVALID;
  if (M == 0 || N == 0) return IMQ_OK;
  hipStream_t st = (hipStream_t)stream;
  const uint16_t* xb = (const uint16_t*)x;
  uint16_t* yb = (uint16_t*)y;
  int rc;
  if (M <= 16) {
    rc = imq::skinny_w8(xb, x_row_stride, M, K, (const int8_t*)qweight, q_row_stride, scale, s_stride_n,
                        s_dtype, N, yb, y_row_stride, st, false);
  } else {
    rc = imq::gemm_wq(8, xb, x_row_stride, M, K, (const uint8_t*)qweight, q_row_stride, scale, s_stride_n,
                      0, s_dtype, nullptr, 0, 0, s_dtype, N, 0, yb, y_row_stride, workspace, workspace_bytes, st);
  }
  if (rc != IMQ_ERR_UNSUPPORTED) return rc;
  return imq::generic_gemv<8>(xb, x_row_stride, M, K, (const uint8_t*)qweight, q_row_stride, scale,
                              s_stride_n, 0, s_dtype, nullptr, 0, 0, s_dtype, N, 1, yb, y_row_stride, st);
}
