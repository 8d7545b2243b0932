// W8A8 int8 GEMM on v_mfma_i32_32x32x32_i8 (gfx950), exact int32 accumulation.
//
// Tile: 128 x 128 outputs, BK = 128 bytes (64 when K is not a multiple of 128), 256 threads = 4 waves (2 x 2), each
// wave 64 x 64 = 2 x 2 MFMA tiles. Both operands are K-contiguous int8 rows
// staged through LDS with a register prefetch of the next k-tile.
// Epilogues: bf16(f32(acc) * a_scale[m] * w_scale[n]) or int32 acc + bias[n].
#include "common.h"
#include "internal.h"

namespace {

constexpr int BM = 128;
constexpr int BN = 128;
constexpr int NTHREADS = 256;

// BK bytes of K per step; rows padded by 16 bytes against bank aliasing.
template <int BK>
struct I8Tile {
  int8_t a[BM][BK + 16];
  int8_t b[BN][BK + 16];
};

enum class Epi { kBf16Scaled, kI32Bias };

template <Epi E, int BK>
__global__ __launch_bounds__(NTHREADS) void i8_gemm_kernel(const int8_t* __restrict__ a, int64_t lda, int M,
                                                           const int8_t* __restrict__ w, int64_t ldw, int N, int K,
                                                           const float* __restrict__ a_scales,
                                                           const float* __restrict__ w_scales,
                                                           const int32_t* __restrict__ bias, void* __restrict__ out,
                                                           int64_t ldo, int mblocks) {
  __shared__ I8Tile<BK> t;
  constexpr int CPR = BK / 16;                 // 16-byte chunks per row
  constexpr int NCH = BM * CPR / NTHREADS;     // chunks per thread per operand
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave & 1;
  const int wn = wave >> 1;
  const int bid = xcd_swizzle(blockIdx.x, gridDim.x);
  const int m0 = (bid % mblocks) * BM;
  const int n0 = (bid / mblocks) * BN;

  // Staging: chunk c = tid + 256*i covers row c/CPR, bytes (c%CPR)*16. Rows
  // past the end read a clamped valid row; their outputs are never stored.
  const int8_t* ap[NCH];
  const int8_t* wp[NCH];
  int srow[NCH], scol[NCH];
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    const int c = tid + NTHREADS * i;
    srow[i] = c / CPR;
    scol[i] = (c % CPR) * 16;
    const int m = m0 + srow[i];
    const int n = n0 + srow[i];
    ap[i] = a + (int64_t)(m < M ? m : M - 1) * lda + scol[i];
    wp[i] = w + (int64_t)(n < N ? n : N - 1) * ldw + scol[i];
  }

  i32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0;

  const int nk = K / BK;
  u32x4 ar[NCH], wr[NCH];
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    ar[i] = load16(ap[i]);
    wr[i] = load16(wp[i]);
  }
  for (int kt = 0; kt < nk; ++kt) {
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      *reinterpret_cast<u32x4*>(&t.a[srow[i]][scol[i]]) = ar[i];
      *reinterpret_cast<u32x4*>(&t.b[srow[i]][scol[i]]) = wr[i];
    }
    __syncthreads();
    if (kt + 1 < nk) {
#pragma unroll
      for (int i = 0; i < NCH; ++i) {
        ar[i] = load16(ap[i] + (int64_t)(kt + 1) * BK);
        wr[i] = load16(wp[i] + (int64_t)(kt + 1) * BK);
      }
    }
#pragma unroll
    for (int kk = 0; kk < BK / 32; ++kk) {
      i32x4 af[2], bf[2];
      const int kof = kk * 32 + (lane >> 5) * 16;
#pragma unroll
      for (int i = 0; i < 2; ++i) af[i] = *reinterpret_cast<const i32x4*>(&t.a[wm * 64 + i * 32 + (lane & 31)][kof]);
#pragma unroll
      for (int j = 0; j < 2; ++j) bf[j] = *reinterpret_cast<const i32x4*>(&t.b[wn * 64 + j * 32 + (lane & 31)][kof]);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[i], bf[j], acc[i][j], 0, 0, 0);
    }
    __syncthreads();
  }

  // 32x32 layout: lane l holds column l%32, rows (v/4)*8 + (l/32)*4 + v%4.
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int col = n0 + wn * 64 + j * 32 + (lane & 31);
    if (col >= N) continue;
    float ws = 0.f;
    int32_t bs = 0;
    if (E == Epi::kBf16Scaled) ws = w_scales[col];
    if (E == Epi::kI32Bias && bias) bs = bias[col];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int row = m0 + wm * 64 + i * 32 + (v >> 2) * 8 + (lane >> 5) * 4 + (v & 3);
        if (row >= M) continue;
        if (E == Epi::kBf16Scaled) {
          float f = (float)acc[i][j][v];
          f = f * a_scales[row];
          f = f * ws;
          reinterpret_cast<uint16_t*>(out)[(int64_t)row * ldo + col] = f32_to_bf16_rne(f);
        } else {
          reinterpret_cast<int32_t*>(out)[(int64_t)row * ldo + col] =
              (int32_t)((uint32_t)acc[i][j][v] + (uint32_t)bs);
        }
      }
  }
}

int check_i8(const int8_t* a, int64_t M, int64_t K, int64_t a_ld, const int8_t* w, int64_t N, int64_t w_ld,
             const void* out, int64_t out_ld) {
  INTENT_REQUIRE(M >= 0 && N >= 0 && K >= 0, INTENT_ERR_INVALID_ARGUMENT, "negative extent");
  INTENT_REQUIRE(M <= INT32_MAX && N <= INT32_MAX && K <= INT32_MAX, INTENT_ERR_UNSUPPORTED, "extent exceeds int32");
  INTENT_REQUIRE(K % 64 == 0, INTENT_ERR_UNSUPPORTED, "K must be a multiple of 64, got %lld", (long long)K);
  if (M == 0 || N == 0) return INTENT_OK;
  INTENT_REQUIRE(a && w && out, INTENT_ERR_INVALID_ARGUMENT, "null pointer argument");
  INTENT_REQUIRE(a_ld >= K && w_ld >= K && out_ld >= N, INTENT_ERR_INVALID_ARGUMENT,
                 "leading stride smaller than the row");
  INTENT_REQUIRE(intent::aligned16(a) && intent::aligned16(w) && a_ld % 16 == 0 && w_ld % 16 == 0,
                 INTENT_ERR_ALIGNMENT, "a and w must be 16-byte aligned with 16-byte row strides");
  return INTENT_OK;
}

template <Epi E>
int launch_i8(const int8_t* a, int64_t M, int64_t K, int64_t a_ld, const float* sa, const int8_t* w, int64_t N,
              int64_t w_ld, const float* sw, const int32_t* bias, void* out, int64_t out_ld, void* stream,
              const char* name) {
  const int mblocks = (int)((M + BM - 1) / BM);
  const int nblocks = (int)((N + BN - 1) / BN);
  const int64_t grid = (int64_t)mblocks * nblocks;
  INTENT_REQUIRE(grid < (1ll << 31), INTENT_ERR_UNSUPPORTED, "%s: grid too large", name);
  if (K % 128 == 0)
    hipLaunchKernelGGL((i8_gemm_kernel<E, 128>), dim3((unsigned)grid), dim3(NTHREADS), 0, (hipStream_t)stream, a,
                       a_ld, (int)M, w, w_ld, (int)N, (int)K, sa, sw, bias, out, out_ld, mblocks);
  else
    hipLaunchKernelGGL((i8_gemm_kernel<E, 64>), dim3((unsigned)grid), dim3(NTHREADS), 0, (hipStream_t)stream, a,
                       a_ld, (int)M, w, w_ld, (int)N, (int)K, sa, sw, bias, out, out_ld, mblocks);
  return intent::launch_status(name);
}

}  // namespace

extern "C" int intent_w8a8_gemm(const int8_t* a, int64_t M, int64_t K, int64_t a_ld, const float* a_scales,
                                const int8_t* w, int64_t N, int64_t w_ld, const float* w_scales, void* out,
                                int64_t out_ld, void* stream) {
  intent::clear_error();
  int st = check_i8(a, M, K, a_ld, w, N, w_ld, out, out_ld);
  if (st != INTENT_OK || M == 0 || N == 0) return st;
  INTENT_REQUIRE(a_scales && w_scales, INTENT_ERR_INVALID_ARGUMENT, "null scale pointer");
  return launch_i8<Epi::kBf16Scaled>(a, M, K, a_ld, a_scales, w, N, w_ld, w_scales, nullptr, out, out_ld, stream,
                                     "w8a8_gemm");
}

extern "C" int intent_i8_gemm_i32(const int8_t* a, int64_t M, int64_t K, int64_t a_ld, const int8_t* w, int64_t N,
                                  int64_t w_ld, const int32_t* bias, int32_t* c, int64_t c_ld, void* stream) {
  intent::clear_error();
  int st = check_i8(a, M, K, a_ld, w, N, w_ld, c, c_ld);
  if (st != INTENT_OK || M == 0 || N == 0) return st;
  return launch_i8<Epi::kI32Bias>(a, M, K, a_ld, nullptr, w, N, w_ld, nullptr, bias, c, c_ld, stream, "i8_gemm_i32");
}
