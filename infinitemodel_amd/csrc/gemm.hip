// Prefill-regime (M > 16) fused dequant GEMM for gfx950.
#include "imq_common.h"

namespace imq {
int skinny_w4(const uint16_t* x, int64_t sxm, int64_t M, int64_t Kpad, const uint8_t* q, int64_t sqn,
              const void* sc, int64_t ssn, int64_t ssg, int sdt, const void* zr, int64_t szn, int64_t szg,
              int zdt, int64_t N, int64_t G, uint16_t* y, int64_t sym, hipStream_t st);

int gemm_wq(int bits, const uint16_t* x, int64_t sxm, int64_t M, int64_t K, const uint8_t* q, int64_t sqn,
            const void* sc, int64_t ssn, int64_t ssg, int sdt, const void* zr, int64_t szn, int64_t szg,
            int zdt, int64_t N, int64_t G, uint16_t* y, int64_t sym, hipStream_t st) {
  if (bits != 4) return IMQ_ERR_UNSUPPORTED;
  // Interim: 16-row slices through the decode kernel.
  for (int64_t m0 = 0; m0 < M; m0 += 16) {
    const int64_t mm = (M - m0) < 16 ? (M - m0) : 16;
    int rc = skinny_w4(x + m0 * sxm, sxm, mm, K, q, sqn, sc, ssn, ssg, sdt, zr, szn, szg, zdt, N, G,
                       y + m0 * sym, sym, st);
    if (rc != IMQ_OK) return rc;
  }
  return IMQ_OK;
}
}  // namespace imq
