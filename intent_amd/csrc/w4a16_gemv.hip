// W4A16 decode GEMV (M <= 16) for gfx950.
//
// Work split: one workgroup owns 16*NT output columns (weight rows n) and all
// M <= 16 activation rows. Its KW waves split K in 128-wide steps, interleaved
// (wave w takes steps w, w+KW, ...), so at any moment the waves of a group
// stream KW*64 contiguous bytes of every weight row.
//
// Per step a lane (r = lane%16, quad = lane/16) loads 16 bytes = 32 nibbles of
// weight row n0+r (k = step*128 + quad*32 .. +32) with one 128-bit load, and
// the matching 32 activations of row m = r. Nibbles are dequantized in
// registers ((q - z) * s in packed f16) and fed to v_mfma_f32_16x16x32_f16:
// MFMA t (t = 0..3) consumes k = step*128 + quad*32 + t*8 + [0..7] from both
// operands, so four MFMAs cover the 128 k of the step. Activation rows m >= M
// are zero and never loaded. Partial sums of the KW waves are reduced through
// LDS in a fixed order and rounded to f16 once.
#include "common.h"
#include "internal.h"

namespace {

template <int NT, int KW>
__global__ __launch_bounds__(64 * KW) void w4a16_gemv_kernel(
    const f16* __restrict__ x, int64_t ldx, int M, int K,
    const uint8_t* __restrict__ wq, int64_t ldw,
    const f16* __restrict__ sc, const uint8_t* __restrict__ zp, int64_t ldq, int gs,
    f16* __restrict__ y, int64_t ldy, int N) {
  __shared__ f32x4 red[KW][NT][64];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int r = lane & 15;
  const int quad = lane >> 4;
  const int n_base = blockIdx.x * 16 * NT;
  const int nsteps = K >> 7;

  const uint8_t* wrow[NT];
  const f16* srow[NT];
  const uint8_t* zrow[NT];
#pragma unroll
  for (int j = 0; j < NT; ++j) {
    int n = n_base + j * 16 + r;
    n = n < N ? n : N - 1;  // tail rows compute on a valid row; their outputs are dropped
    wrow[j] = wq + (int64_t)n * ldw + quad * 16;
    srow[j] = sc + (int64_t)n * ldq;
    zrow[j] = zp + (int64_t)n * ldq;
  }
  const bool mvalid = r < M;
  const f16* xrow = x + (int64_t)(mvalid ? r : 0) * ldx + quad * 32;

  f32x4 acc[NT];
#pragma unroll
  for (int j = 0; j < NT; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};

  int s = wave;
  u32x4 wv[NT];
  u32x4 xv[4];
  if (s < nsteps) {
#pragma unroll
    for (int j = 0; j < NT; ++j) wv[j] = load16(wrow[j] + (int64_t)s * 64);
#pragma unroll
    for (int t = 0; t < 4; ++t) xv[t] = mvalid ? load16(xrow + (int64_t)s * 128 + t * 8) : u32x4{0, 0, 0, 0};
  }
  while (s < nsteps) {
    const int g = (s * 128 + quad * 32) / gs;
    f16x2 zoff[NT], scale[NT];
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      zoff[j] = splat2((f16)(float)(1024 + zrow[j][g]));
      scale[j] = splat2(srow[j][g]);
    }
    u32x4 wc[NT], xc[4];
#pragma unroll
    for (int j = 0; j < NT; ++j) wc[j] = wv[j];
#pragma unroll
    for (int t = 0; t < 4; ++t) xc[t] = xv[t];
    const int sn = s + KW;
    if (sn < nsteps) {  // prefetch the next step before the math of this one
#pragma unroll
      for (int j = 0; j < NT; ++j) wv[j] = load16(wrow[j] + (int64_t)sn * 64);
#pragma unroll
      for (int t = 0; t < 4; ++t) xv[t] = mvalid ? load16(xrow + (int64_t)sn * 128 + t * 8) : u32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int j = 0; j < NT; ++j) {
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        f16x8 b = dequant8(wc[j][t], zoff[j], scale[j]);
        f16x8 a = bit_cast<f16x8>(xc[t]);
        acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, acc[j], 0, 0, 0);
      }
    }
    s = sn;
  }

#pragma unroll
  for (int j = 0; j < NT; ++j) red[wave][j][lane] = acc[j];
  __syncthreads();
  // 16x16 MFMA result layout: lane l holds column l%16, rows (l/16)*4 + i.
  for (int o = threadIdx.x; o < 256 * NT; o += 64 * KW) {
    const int j = o >> 8;
    const int m = (o >> 4) & 15;
    const int nc = o & 15;
    const int src = (m >> 2) * 16 + nc;
    float sum = 0.f;
#pragma unroll
    for (int w = 0; w < KW; ++w) sum += red[w][j][src][m & 3];
    const int n = n_base + j * 16 + nc;
    if (m < M && n < N) y[(int64_t)m * ldy + n] = (f16)sum;
  }
}

template <int NT, int KW>
void launch_gemv(const f16* x, int64_t ldx, int M, int K, const uint8_t* wq, int64_t ldw, const f16* sc,
                 const uint8_t* zp, int64_t ldq, int gs, f16* y, int64_t ldy, int N, hipStream_t st) {
  const int tiles = (N + 16 * NT - 1) / (16 * NT);
  hipLaunchKernelGGL((w4a16_gemv_kernel<NT, KW>), dim3(tiles), dim3(64 * KW), 0, st, x, ldx, M, K, wq, ldw, sc, zp,
                     ldq, gs, y, ldy, N);
}

}  // namespace

namespace intent {

int w4a16_check(const void* x, int64_t M, int64_t K, int64_t x_ld, const uint8_t* packed, int64_t N,
                int64_t packed_ld, const void* scales, const uint8_t* zeros, int64_t qparam_ld, int64_t gs,
                const void* y, int64_t y_ld) {
  INTENT_REQUIRE(M >= 0 && N >= 0 && K >= 0, INTENT_ERR_INVALID_ARGUMENT, "negative extent (M=%lld N=%lld K=%lld)",
                 (long long)M, (long long)N, (long long)K);
  INTENT_REQUIRE(M <= INT32_MAX && N <= INT32_MAX && K <= INT32_MAX, INTENT_ERR_UNSUPPORTED, "extent exceeds int32");
  INTENT_REQUIRE(gs > 0 && gs % 32 == 0, INTENT_ERR_UNSUPPORTED, "group_size must be a positive multiple of 32, got %lld",
                 (long long)gs);
  INTENT_REQUIRE(K % 128 == 0 && K % gs == 0, INTENT_ERR_UNSUPPORTED,
                 "K must be a multiple of 128 and of group_size (K=%lld group=%lld)", (long long)K, (long long)gs);
  if (M == 0 || N == 0) return INTENT_OK;
  INTENT_REQUIRE(x && packed && scales && zeros && y, INTENT_ERR_INVALID_ARGUMENT, "null pointer argument");
  INTENT_REQUIRE(x_ld >= K && packed_ld >= K / 2 && qparam_ld >= K / gs && y_ld >= N, INTENT_ERR_INVALID_ARGUMENT,
                 "leading stride smaller than the row (x_ld=%lld packed_ld=%lld qparam_ld=%lld y_ld=%lld)",
                 (long long)x_ld, (long long)packed_ld, (long long)qparam_ld, (long long)y_ld);
  INTENT_REQUIRE(aligned16(x) && aligned16(packed) && x_ld % 8 == 0 && packed_ld % 16 == 0, INTENT_ERR_ALIGNMENT,
                 "x and packed must be 16-byte aligned with 16-byte row strides");
  return INTENT_OK;
}

int w4a16_gemv_launch(const void* x, int64_t M, int64_t K, int64_t x_ld, const uint8_t* packed, int64_t N,
                      int64_t packed_ld, const void* scales, const uint8_t* zeros, int64_t qparam_ld, int64_t gs,
                      void* y, int64_t y_ld, void* stream) {
  INTENT_REQUIRE(M <= 16, INTENT_ERR_UNSUPPORTED, "the GEMV kernel covers M <= 16, got M=%lld", (long long)M);
  if (M == 0 || N == 0) return INTENT_OK;
  hipStream_t st = (hipStream_t)stream;
  const f16* xx = (const f16*)x;
  const f16* ss = (const f16*)scales;
  f16* yy = (f16*)y;
  const int steps = (int)(K / 128);
  if (steps >= 16)
    launch_gemv<1, 16>(xx, x_ld, (int)M, (int)K, packed, packed_ld, ss, zeros, qparam_ld, (int)gs, yy, y_ld, (int)N, st);
  else if (steps >= 8)
    launch_gemv<1, 8>(xx, x_ld, (int)M, (int)K, packed, packed_ld, ss, zeros, qparam_ld, (int)gs, yy, y_ld, (int)N, st);
  else
    launch_gemv<1, 4>(xx, x_ld, (int)M, (int)K, packed, packed_ld, ss, zeros, qparam_ld, (int)gs, yy, y_ld, (int)N, st);
  return launch_status("w4a16_gemv");
}

}  // namespace intent
