// Ragged grouped f16 / bf16 GEMMs with [G][K][N] weights read in place
// (grouped_kn.h).
#include "grouped_kn.h"

using namespace gkn;

namespace intent {
// zeros in the rows the groups cover (dense_gemm.hip)
int grouped_empty_k(const int32_t* offsets, int64_t G, const int32_t* routes, int64_t rows, void* out, int64_t out_ld,
                    int64_t N, void* stream);
}  // namespace intent

extern "C" int intent_grouped_gemm_kn(const void* x, int64_t rows, int64_t K, int64_t x_ld, const int32_t* offsets,
                                      int64_t G, const void* w, int64_t N, int64_t w_ld, int64_t w_group_stride,
                                      int bf16, void* out, int64_t out_ld, void* stream) {
  intent::clear_error();
  INTENT_REQUIRE(rows >= 0 && K >= 0 && N >= 0 && G >= 0 && rows <= INT32_MAX && K <= INT32_MAX && N <= INT32_MAX &&
                     G <= (1 << 20),
                 INTENT_ERR_INVALID_ARGUMENT, "bad extents");
  if (rows == 0 || N == 0 || G == 0) return INTENT_OK;
  if (K == 0) return intent::grouped_empty_k(offsets, G, nullptr, rows, out, out_ld, N, stream);
  int st = kn_shape_check(K, N, w_ld, w, "grouped_gemm_kn");
  if (st != INTENT_OK) return st;
  INTENT_REQUIRE(x && offsets && out, INTENT_ERR_INVALID_ARGUMENT, "null pointer argument");
  INTENT_REQUIRE(x_ld >= K && out_ld >= N && w_group_stride >= K * w_ld, INTENT_ERR_INVALID_ARGUMENT,
                 "leading stride smaller than the row");
  INTENT_REQUIRE(intent::aligned16(x) && x_ld % 8 == 0 && w_group_stride % 8 == 0, INTENT_ERR_ALIGNMENT,
                 "x must be 16-byte aligned with 16-byte row strides");
  INTENT_REQUIRE(intent::fits_offset(rows, x_ld * 2), INTENT_ERR_UNSUPPORTED,
                 "grouped_gemm_kn: x exceeds 31-bit buffer offsets");
  const int64_t ntiles = (rows + GTile::BM - 1) / GTile::BM + G;
  INTENT_REQUIRE(ntiles * ((N + GTile::BN - 1) / GTile::BN) < (1ll << 31), INTENT_ERR_UNSUPPORTED, "grid too large");
  hipStream_t s = (hipStream_t)stream;
  if (bf16)
    launch_grouped<mp::BF16Math, false, GEpi::kStore16>(x, x_ld, offsets, G, rows, nullptr, nullptr, 1, 1, nullptr, w,
                                                        w_ld, w_group_stride, N, K, (int)ntiles, out, out_ld, s);
  else
    launch_grouped<mp::F16Math, false, GEpi::kStore16>(x, x_ld, offsets, G, rows, nullptr, nullptr, 1, 1, nullptr, w,
                                                       w_ld, w_group_stride, N, K, (int)ntiles, out, out_ld, s);
  return intent::launch_status(bf16 ? "grouped_kn_kernel<bf16>" : "grouped_kn_kernel<f16>");
}

