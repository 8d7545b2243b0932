// Per-token symmetric int8 activation quantizer for gfx950 (the producer of
// the W8A8 GEMM's int8 activations and f32 per-token scales), bit-exact:
//   absmax[m] = max_k |f32(x[m,k])|
//   scale[m]  = absmax / 127                 (IEEE f32 division)
//   inv[m]    = 127 / absmax                 (IEEE f32 division)
//   q[m,k]    = rne(clamp(f32(x[m,k]) * inv, -128, 127))
// An all-zero row gets scale 0 and q 0. Clamping before rounding to nearest
// even is the reference's integer quantization rule
// (lib/Conversion/KIRToGPU/Quantization.cpp:191-203); the f16 and bf16 inputs
// widen to f32 exactly. Inputs are finite.
//
// One 256-lane workgroup per row. A lane owns 8-column chunks c = lane + 256*i
// (16-byte loads, so a wave reads 1 KB contiguous per load). For K <= 8192 a
// lane keeps its (at most four) chunks in registers between the absmax and the
// encode; longer rows are read a second time (from L2) for the encode. K = 0
// gives scale 0 for every row.
#include "common.h"
#include "internal.h"

namespace {

template <bool kBf16>
INTENT_DEVICE void widen8(u32x4 raw, float (&v)[8]) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    if constexpr (kBf16) {
      v[2 * j] = bit_cast<float>(raw[j] << 16);
      v[2 * j + 1] = bit_cast<float>(raw[j] & 0xffff0000u);
    } else {
      const f16x2 h = bit_cast<f16x2>(raw[j]);
      v[2 * j] = (float)h[0];
      v[2 * j + 1] = (float)h[1];
    }
  }
}

INTENT_DEVICE float chunk_absmax(u32x4 raw, bool bf16) {
  float v[8];
  if (bf16) widen8<true>(raw, v);
  else widen8<false>(raw, v);
  float m = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) m = fmaxf(m, fabsf(v[j]));
  return m;
}

template <bool kBf16>
INTENT_DEVICE u32x2 encode8(u32x4 raw, float inv) {
  float v[8];
  widen8<kBf16>(raw, v);
  uint32_t w[2] = {0u, 0u};
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float t = fminf(fmaxf(v[j] * inv, -128.0f), 127.0f);
    const int qi = (int)__builtin_rintf(t);
    w[j >> 2] |= ((uint32_t)qi & 0xffu) << (8 * (j & 3));
  }
  return u32x2{w[0], w[1]};
}

template <bool kBf16, int R>  // R = chunks per lane kept in registers (0: stream twice)
__global__ __launch_bounds__(256) void i8_per_token_kernel(const uint16_t* __restrict__ x, int64_t ldx, int K,
                                                           int8_t* __restrict__ q, int64_t ldq,
                                                           float* __restrict__ scales) {
  __shared__ float wave_max[4];
  const int row = blockIdx.x;
  const int lane = threadIdx.x;
  const int nchunks = K >> 3;
  const uint16_t* xr = x + (int64_t)row * ldx;
  int8_t* qr = q + (int64_t)row * ldq;

  float amax = 0.f;
  u32x4 keep[R > 0 ? R : 1];
  if constexpr (R > 0) {
#pragma unroll
    for (int i = 0; i < R; ++i) {
      const int c = lane + 256 * i;
      // read once: non-temporal (19.7 -> 17.2 us at 4096 x 8192; the same hint on the
      // int8 stores measured slower)
      keep[i] = c < nchunks ? __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(xr + (int64_t)c * 8))
                            : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int i = 0; i < R; ++i) amax = fmaxf(amax, chunk_absmax(keep[i], kBf16));
  } else {
    for (int c = lane; c < nchunks; c += 256) amax = fmaxf(amax, chunk_absmax(load16(xr + (int64_t)c * 8), kBf16));
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
  if ((lane & 63) == 0) wave_max[lane >> 6] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(wave_max[0], wave_max[1]), fmaxf(wave_max[2], wave_max[3]));

  const bool zero = amax == 0.f;
  const float scale = zero ? 0.f : __fdiv_rn(amax, 127.0f);
  const float inv = zero ? 0.f : __fdiv_rn(127.0f, amax);
  if (lane == 0) scales[row] = scale;
  if constexpr (R > 0) {
#pragma unroll
    for (int i = 0; i < R; ++i) {
      const int c = lane + 256 * i;
      if (c < nchunks) *reinterpret_cast<u32x2*>(qr + (int64_t)c * 8) = encode8<kBf16>(keep[i], inv);
    }
  } else {
    for (int c = lane; c < nchunks; c += 256)
      *reinterpret_cast<u32x2*>(qr + (int64_t)c * 8) = encode8<kBf16>(load16(xr + (int64_t)c * 8), inv);
  }
}

template <bool kBf16>
void launch_i8q(const void* x, int64_t ldx, int M, int K, int8_t* q, int64_t ldq, float* scales, hipStream_t st) {
  const int chunks = (K / 8 + 255) / 256;
  const uint16_t* xx = (const uint16_t*)x;
  if (chunks <= 1)
    hipLaunchKernelGGL((i8_per_token_kernel<kBf16, 1>), dim3(M), dim3(256), 0, st, xx, ldx, K, q, ldq, scales);
  else if (chunks <= 2)
    hipLaunchKernelGGL((i8_per_token_kernel<kBf16, 2>), dim3(M), dim3(256), 0, st, xx, ldx, K, q, ldq, scales);
  else if (chunks <= 4)
    hipLaunchKernelGGL((i8_per_token_kernel<kBf16, 4>), dim3(M), dim3(256), 0, st, xx, ldx, K, q, ldq, scales);
  else
    hipLaunchKernelGGL((i8_per_token_kernel<kBf16, 0>), dim3(M), dim3(256), 0, st, xx, ldx, K, q, ldq, scales);
}

}  // namespace

extern "C" int intent_i8_per_token_quantize(const void* x, int x_is_bf16, int64_t M, int64_t K, int64_t x_ld,
                                            int8_t* q, int64_t q_ld, float* scales, void* stream) {
  intent::clear_error();
  INTENT_REQUIRE(M >= 0 && K >= 0 && M <= INT32_MAX && K <= INT32_MAX, INTENT_ERR_INVALID_ARGUMENT,
                 "bad extents (M=%lld K=%lld)", (long long)M, (long long)K);
  INTENT_REQUIRE(K % 8 == 0, INTENT_ERR_UNSUPPORTED, "K must be a multiple of 8, got %lld", (long long)K);
  // one 256-lane workgroup per row: the grid's work items stay below 2^32
  INTENT_REQUIRE(M < ((int64_t)1 << 24), INTENT_ERR_UNSUPPORTED,
                 "M=%lld rows exceed the %lld a launch covers (one 256-lane workgroup per row)", (long long)M,
                 (long long)((int64_t)1 << 24));
  if (M == 0) return INTENT_OK;
  INTENT_REQUIRE(scales != nullptr, INTENT_ERR_INVALID_ARGUMENT, "null scales");
  if (K > 0) {  // empty rows read and write nothing but their zero scales
    INTENT_REQUIRE(x && q, INTENT_ERR_INVALID_ARGUMENT, "null pointer argument");
    INTENT_REQUIRE(x_ld >= K && q_ld >= K, INTENT_ERR_INVALID_ARGUMENT, "leading stride smaller than the row");
    INTENT_REQUIRE(intent::aligned16(x) && x_ld % 8 == 0 && (reinterpret_cast<uintptr_t>(q) & 7) == 0 &&
                       q_ld % 8 == 0,
                   INTENT_ERR_ALIGNMENT,
                   "x must be 16-byte aligned with x_ld %% 8 == 0; q 8-byte aligned, q_ld %% 8 == 0");
  }
  hipStream_t st = (hipStream_t)stream;
  if (x_is_bf16) launch_i8q<true>(x, x_ld, (int)M, (int)K, q, q_ld, scales, st);
  else launch_i8q<false>(x, x_ld, (int)M, (int)K, q, q_ld, scales, st);
  return intent::launch_status_fmt("i8_per_token_kernel<%s>", x_is_bf16 ? "bf16" : "f16");
}
