// Dense weight-only contractions on the shared f16 MFMA tile GEMM:
//   W4A16 (asymmetric group-quant nibbles) and W8A16 (per-channel int8).
#include "common.h"
#include "gemm_f16.h"
#include "internal.h"

namespace {

using namespace gemm;

struct ClampRows {
  int n0;
  int N;
  INTENT_DEVICE int operator()(int c) const {
    const int n = n0 + c;
    return n < N ? n : N - 1;  // tail rows read a valid row; their outputs are dropped
  }
};

template <class T, class WSrc, bool kColScale>
__global__ __launch_bounds__(T::NT, 2) void dense_gemm_kernel(DenseRows rows, WSrc w, int N, int K, f16* __restrict__ y,
                                                           int64_t ldy, const f16* __restrict__ colscale,
                                                           int mblocks) {
  __shared__ typename T::Shared tile;
  const int bid = xcd_swizzle(blockIdx.x, gridDim.x);
  const int m0 = (bid % mblocks) * T::BM;
  const int n0 = (bid / mblocks) * T::BN;
  f32x16 acc[T::TI][T::TJ];
  mainloop<T>(rows, m0, w, ClampRows{n0, N}, K, tile, acc);
#pragma unroll
  for (int j = 0; j < T::TJ; ++j) {
    const int col = n0 + T::acc_col(j);
    if (col >= N) continue;
    const float cs = kColScale ? (float)colscale[col] : 1.0f;
#pragma unroll
    for (int i = 0; i < T::TI; ++i)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int row = m0 + T::acc_row(i, v);
        if (row < rows.M) {
          const float val = kColScale ? acc[i][j][v] * cs : acc[i][j][v];
          y[(int64_t)row * ldy + col] = (f16)val;
        }
      }
  }
}

template <class T, class WSrc, bool kColScale>
int launch_tile(const f16* x, int64_t ldx, int M, int N, int K, const WSrc& w, f16* y, int64_t ldy,
                const f16* colscale, hipStream_t st, const char* name) {
  const int mblocks = (M + T::BM - 1) / T::BM;
  const int nblocks = (N + T::BN - 1) / T::BN;
  const int64_t grid = (int64_t)mblocks * nblocks;
  INTENT_REQUIRE(grid < (1ll << 31), INTENT_ERR_UNSUPPORTED, "%s: grid too large", name);
  hipLaunchKernelGGL((dense_gemm_kernel<T, WSrc, kColScale>), dim3((unsigned)grid), dim3(T::NT), 0, st,
                     DenseRows{x, ldx, M}, w, N, K, y, ldy, colscale, mblocks);
  return intent::launch_status(name);
}

// Tile choice: 256 x 128 (128 x 64 per wave) once M fills it, else 128 x 128.
template <class WSrc, bool kColScale>
int launch_dense(const f16* x, int64_t ldx, int M, int N, int K, const WSrc& w, f16* y, int64_t ldy,
                 const f16* colscale, hipStream_t st, const char* name) {
  if (M > 128) return launch_tile<Tile<256, 128, 2, 2>, WSrc, kColScale>(x, ldx, M, N, K, w, y, ldy, colscale, st, name);
  return launch_tile<Tile<128, 128, 2, 2>, WSrc, kColScale>(x, ldx, M, N, K, w, y, ldy, colscale, st, name);
}

}  // namespace

namespace intent {

int w4a16_check(const void* x, int64_t M, int64_t K, int64_t x_ld, const uint8_t* packed, int64_t N,
                int64_t packed_ld, const void* scales, const uint8_t* zeros, int64_t qparam_ld, int64_t gs,
                const void* y, int64_t y_ld);
int w4a16_gemv_launch(const void* x, int64_t M, int64_t K, int64_t x_ld, const uint8_t* packed, int64_t N,
                      int64_t packed_ld, const void* scales, const uint8_t* zeros, int64_t qparam_ld, int64_t gs,
                      void* y, int64_t y_ld, void* stream);

int w8a16_gemv_launch(const void* x, int64_t M, int64_t K, int64_t x_ld, const int8_t* w, int64_t N, int64_t w_ld,
                      const void* scales, void* y, int64_t y_ld, void* stream);

int w4a16_gemm_launch(const void* x, int64_t M, int64_t K, int64_t x_ld, const uint8_t* packed, int64_t N,
                      int64_t packed_ld, const void* scales, const uint8_t* zeros, int64_t qparam_ld, int64_t gs,
                      void* y, int64_t y_ld, void* stream) {
  if (M == 0 || N == 0) return INTENT_OK;
  INTENT_REQUIRE(gs == 32 || gs % 64 == 0, INTENT_ERR_UNSUPPORTED,
                 "the tiled GEMM needs group_size 32 or a multiple of 64, got %lld", (long long)gs);
  INTENT_REQUIRE(intent::fits_offset(N, packed_ld) && intent::fits_offset(N, qparam_ld * 2) &&
                     intent::fits_offset(256 + 1, x_ld * 2),
                 INTENT_ERR_UNSUPPORTED, "w4a16_gemm: operand too large for 31-bit buffer offsets");
  W4Source w{packed, packed_ld, (const f16*)scales, zeros, qparam_ld, (int)gs};
  return launch_dense<W4Source, false>((const f16*)x, x_ld, (int)M, (int)N, (int)K, w, (f16*)y, y_ld, nullptr,
                                       (hipStream_t)stream, "w4a16_gemm");
}

}  // namespace intent

extern "C" int intent_w4a16_matmul(const void* x, int64_t M, int64_t K, int64_t x_ld, const uint8_t* packed, int64_t N,
                                   int64_t packed_ld, const void* scales, const uint8_t* zeros, int64_t qparam_ld,
                                   int64_t group_size, void* y, int64_t y_ld, void* stream) {
  intent::clear_error();
  int st = intent::w4a16_check(x, M, K, x_ld, packed, N, packed_ld, scales, zeros, qparam_ld, group_size, y, y_ld);
  if (st != INTENT_OK) return st;
  if (M <= 16)
    return intent::w4a16_gemv_launch(x, M, K, x_ld, packed, N, packed_ld, scales, zeros, qparam_ld, group_size, y,
                                     y_ld, stream);
  return intent::w4a16_gemm_launch(x, M, K, x_ld, packed, N, packed_ld, scales, zeros, qparam_ld, group_size, y, y_ld,
                                   stream);
}

extern "C" int intent_w4a16_gemv(const void* x, int64_t M, int64_t K, int64_t x_ld, const uint8_t* packed, int64_t N,
                                 int64_t packed_ld, const void* scales, const uint8_t* zeros, int64_t qparam_ld,
                                 int64_t group_size, void* y, int64_t y_ld, void* stream) {
  intent::clear_error();
  int st = intent::w4a16_check(x, M, K, x_ld, packed, N, packed_ld, scales, zeros, qparam_ld, group_size, y, y_ld);
  if (st != INTENT_OK) return st;
  return intent::w4a16_gemv_launch(x, M, K, x_ld, packed, N, packed_ld, scales, zeros, qparam_ld, group_size, y, y_ld,
                                   stream);
}

extern "C" int intent_w4a16_gemm(const void* x, int64_t M, int64_t K, int64_t x_ld, const uint8_t* packed, int64_t N,
                                 int64_t packed_ld, const void* scales, const uint8_t* zeros, int64_t qparam_ld,
                                 int64_t group_size, void* y, int64_t y_ld, void* stream) {
  intent::clear_error();
  int st = intent::w4a16_check(x, M, K, x_ld, packed, N, packed_ld, scales, zeros, qparam_ld, group_size, y, y_ld);
  if (st != INTENT_OK) return st;
  return intent::w4a16_gemm_launch(x, M, K, x_ld, packed, N, packed_ld, scales, zeros, qparam_ld, group_size, y, y_ld,
                                   stream);
}

extern "C" int intent_w8a16_matmul(const void* x, int64_t M, int64_t K, int64_t x_ld, const int8_t* w, int64_t N,
                                   int64_t w_ld, const void* scales, void* y, int64_t y_ld, void* stream) {
  intent::clear_error();
  INTENT_REQUIRE(M >= 0 && N >= 0 && K >= 0, INTENT_ERR_INVALID_ARGUMENT, "negative extent");
  INTENT_REQUIRE(M <= INT32_MAX && N <= INT32_MAX && K <= INT32_MAX, INTENT_ERR_UNSUPPORTED, "extent exceeds int32");
  INTENT_REQUIRE(K % 64 == 0, INTENT_ERR_UNSUPPORTED, "K must be a multiple of 64, got %lld", (long long)K);
  if (M == 0 || N == 0) return INTENT_OK;
  INTENT_REQUIRE(x && w && scales && y, INTENT_ERR_INVALID_ARGUMENT, "null pointer argument");
  INTENT_REQUIRE(x_ld >= K && w_ld >= K && y_ld >= N, INTENT_ERR_INVALID_ARGUMENT, "leading stride smaller than the row");
  INTENT_REQUIRE(intent::aligned16(x) && intent::aligned16(w) && x_ld % 8 == 0 && w_ld % 16 == 0, INTENT_ERR_ALIGNMENT,
                 "x and w must be 16-byte aligned with 16-byte row strides");
  if (M <= 16) return intent::w8a16_gemv_launch(x, M, K, x_ld, w, N, w_ld, scales, y, y_ld, stream);
  INTENT_REQUIRE(intent::fits_offset(N, w_ld) && intent::fits_offset(256 + 1, x_ld * 2), INTENT_ERR_UNSUPPORTED,
                 "w8a16_matmul: operand too large for 31-bit buffer offsets");
  W8Source ws{w, w_ld};
  return launch_dense<W8Source, true>((const f16*)x, x_ld, (int)M, (int)N, (int)K, ws, (f16*)y, y_ld,
                                      (const f16*)scales, (hipStream_t)stream, "w8a16_matmul");
}
