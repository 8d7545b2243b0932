// Groupwise FP8 (OCP E4M3FN) activation quantizers for gfx950, bit-exact:
//   scale = max(absmax over a group of 128 columns, eps) / 448
//   q     = e4m3fn(min(max(x / scale, -448), 448)), round to nearest even
// (examples/kernels/quantization/fp8.py:11-69; eps 1e-12 for bf16 input,
// 1e-4 for f32 input). Every division is IEEE f32; the E4M3FN rounding is done
// in integer arithmetic, so the bytes equal a CPU evaluation of the formula.
#include "common.h"
#include "internal.h"

namespace {

// Thread t of a 32-lane half-wave holds columns 4t..4t+3 of its group.
template <bool kBf16>
__global__ __launch_bounds__(256) void fp8_groupwise_kernel(const void* __restrict__ xv, int64_t ldx, int M, int N,
                                                            int G, float eps, uint8_t* __restrict__ q, int64_t ldq,
                                                            float* __restrict__ scales, int64_t lds) {
  const int pair = blockIdx.x * 8 + (threadIdx.x >> 5);
  const bool active = pair < M * G;
  const int row = active ? pair / G : 0;
  const int g = active ? pair % G : 0;
  const int c = g * 128 + (threadIdx.x & 31) * 4;
  const bool has = active && c < N;  // N % 4 == 0: all four columns or none
  float v[4] = {0.f, 0.f, 0.f, 0.f};
  if (has) {
    if constexpr (kBf16) {
      const u32x2 w = *reinterpret_cast<const u32x2*>(reinterpret_cast<const uint16_t*>(xv) + (int64_t)row * ldx + c);
      v[0] = bit_cast<float>(w[0] << 16);
      v[1] = bit_cast<float>(w[0] & 0xffff0000u);
      v[2] = bit_cast<float>(w[1] << 16);
      v[3] = bit_cast<float>(w[1] & 0xffff0000u);
    } else {
      const f32x4 w = *reinterpret_cast<const f32x4*>(reinterpret_cast<const float*>(xv) + (int64_t)row * ldx + c);
      v[0] = w[0], v[1] = w[1], v[2] = w[2], v[3] = w[3];
    }
  }
  float amax = has ? fmaxf(fmaxf(fmaxf(v[0], -v[0]), fmaxf(v[1], -v[1])), fmaxf(fmaxf(v[2], -v[2]), fmaxf(v[3], -v[3])))
                   : -INFINITY;
#pragma unroll
  for (int off = 16; off >= 1; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
  const float scale = __fdiv_rn(fmaxf(amax, eps), 448.0f);
  if (has) {
    uint32_t packed = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float t = fminf(fmaxf(__fdiv_rn(v[i], scale), -448.0f), 448.0f);
      packed |= f32_to_e4m3fn(t) << (8 * i);
    }
    *reinterpret_cast<uint32_t*>(q + (int64_t)row * ldq + c) = packed;
  }
  if (active && (threadIdx.x & 31) == 0) scales[(int64_t)row * lds + g] = scale;
}

}  // namespace

extern "C" int intent_fp8_groupwise_quantize(const void* x, int x_is_bf16, int64_t M, int64_t N, int64_t x_ld,
                                             uint8_t* q, int64_t q_ld, float* scales, int64_t G, int64_t scales_ld,
                                             void* stream) {
  intent::clear_error();
  INTENT_REQUIRE(M >= 0 && N >= 0 && G >= 0 && M <= INT32_MAX && N <= INT32_MAX && M * G <= INT32_MAX,
                 INTENT_ERR_INVALID_ARGUMENT, "bad extents (M=%lld N=%lld G=%lld)", (long long)M, (long long)N,
                 (long long)G);
  INTENT_REQUIRE(G * 128 >= N, INTENT_ERR_INVALID_ARGUMENT, "%lld groups of 128 do not cover N=%lld", (long long)G,
                 (long long)N);
  INTENT_REQUIRE(N % 4 == 0, INTENT_ERR_UNSUPPORTED, "N must be a multiple of 4, got %lld", (long long)N);
  if (M == 0 || G == 0) return INTENT_OK;
  INTENT_REQUIRE(x && q && scales, INTENT_ERR_INVALID_ARGUMENT, "null pointer argument");
  INTENT_REQUIRE(x_ld >= N && q_ld >= N && scales_ld >= G, INTENT_ERR_INVALID_ARGUMENT,
                 "leading stride smaller than the row");
  const uintptr_t xa = reinterpret_cast<uintptr_t>(x);
  INTENT_REQUIRE((x_is_bf16 ? (xa & 7) == 0 : (xa & 15) == 0) && x_ld % 4 == 0 && intent::aligned4(q) &&
                     q_ld % 4 == 0,
                 INTENT_ERR_ALIGNMENT, "x must be 8 (bf16) / 16 (f32) byte aligned with x_ld %% 4 == 0; q 4-byte aligned");
  const unsigned blocks = (unsigned)((M * G + 7) / 8);
  if (x_is_bf16)
    hipLaunchKernelGGL((fp8_groupwise_kernel<true>), dim3(blocks), dim3(256), 0, (hipStream_t)stream, x, x_ld, (int)M,
                       (int)N, (int)G, 1.0e-12f, q, q_ld, scales, scales_ld);
  else
    hipLaunchKernelGGL((fp8_groupwise_kernel<false>), dim3(blocks), dim3(256), 0, (hipStream_t)stream, x, x_ld,
                       (int)M, (int)N, (int)G, 1.0e-4f, q, q_ld, scales, scales_ld);
  return intent::launch_status("fp8_groupwise_quantize");
}

// ---- NVFP4 quantization (examples/kernels/quantization/nvfp4.py) --------------------
// One thread per (row, group of 16 values). CPU baseline cpu_runtime.py:1325-1340:
//   scale = e4m3fn(max((amax / 6) * gs, 1.5258789e-5)), multiplier = gs / f32(scale),
//   v = x * multiplier, code = E2M1 thresholds on |v| (> 0.25, >= 0.75, > 1.25,
//   >= 1.75, > 2.5, >= 3.5, > 5.0), sign bit of v; two codes per byte, low = even
//   column. The group's scale byte goes to scales[row/128][group/4][row%32]
//   [(row%128)/32][group%4] (the reference's 128 x 4 swizzled block).
namespace {

INTENT_DEVICE float e4m3fn_to_f32(uint32_t v) {
  const uint32_t e = (v >> 3) & 15u, m = v & 7u;
  float mag;
  if (e == 15u && m == 7u) mag = __builtin_nanf("");
  else if (e == 0u) mag = (float)m * 0.001953125f;  // m * 2^-9
  else mag = bit_cast<float>(((e + 120u) << 23) | (m << 20));
  return (v & 0x80u) ? -mag : mag;
}

INTENT_DEVICE uint32_t e2m1_code(float v) {
  const float a = fabsf(v);
  uint32_t c = a > 0.25f ? 1u : 0u;
  c = a >= 0.75f ? 2u : c;
  c = a > 1.25f ? 3u : c;
  c = a >= 1.75f ? 4u : c;
  c = a > 2.5f ? 5u : c;
  c = a >= 3.5f ? 6u : c;
  c = a > 5.0f ? 7u : c;
  return c | ((bit_cast<uint32_t>(v) >> 31) << 3);
}

__global__ __launch_bounds__(256) void nvfp4_quantize_kernel(const uint16_t* __restrict__ x, int64_t ldx, int M,
                                                             int G, const float* __restrict__ global_scale,
                                                             uint8_t* __restrict__ packed, int64_t ldp,
                                                             uint8_t* __restrict__ scales, int NT) {
  const int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= (int64_t)M * G) return;
  const int row = (int)(id / G), g = (int)(id % G);
  const float gs = global_scale[0];
  const uint16_t* src = x + (int64_t)row * ldx + g * 16;
  float v[16];
  if ((((uintptr_t)src) & 15) == 0) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const u32x4 w = *reinterpret_cast<const u32x4*>(src + 8 * h);
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        v[8 * h + 2 * d] = bit_cast<float>(w[d] << 16);
        v[8 * h + 2 * d + 1] = bit_cast<float>(w[d] & 0xffff0000u);
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < 16; ++i) v[i] = bit_cast<float>((uint32_t)src[i] << 16);
  }
  float amax = fabsf(v[0]);
#pragma unroll
  for (int i = 1; i < 16; ++i) amax = fmaxf(amax, fabsf(v[i]));
  const float s = fmaxf(__fmul_rn(__fdiv_rn(amax, 6.0f), gs), 1.5258789e-05f);
  // The E4M3FN cast of the CPU formula (torch's) rounds (448, 464] to 448 and
  // turns anything above into NaN (0x7f); a NaN scale leaves every value of the
  // group NaN, which encodes as code 0.
  const bool nan_scale = !(s <= 464.0f);
  const uint32_t sbyte = nan_scale ? 0x7fu : f32_to_e4m3fn(s);
  const float mult = __fdiv_rn(gs, e4m3fn_to_f32(sbyte));
  uint32_t lo = 0, hi = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t b = e2m1_code(__fmul_rn(v[2 * i], mult)) | (e2m1_code(__fmul_rn(v[2 * i + 1], mult)) << 4);
    if (i < 4) lo |= b << (8 * i);
    else hi |= b << (8 * (i - 4));
  }
  if (nan_scale) lo = hi = 0u;
  uint8_t* dst = packed + (int64_t)row * ldp + g * 8;
  if ((((uintptr_t)dst) & 7) == 0) {
    *reinterpret_cast<u32x2*>(dst) = u32x2{lo, hi};
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      dst[i] = (uint8_t)(lo >> (8 * i));
      dst[4 + i] = (uint8_t)(hi >> (8 * i));
    }
  }
  const int64_t sidx = ((((int64_t)(row / 128) * NT + g / 4) * 32 + row % 32) * 4 + (row % 128) / 32) * 4 + g % 4;
  scales[sidx] = (uint8_t)sbyte;
}

}  // namespace

extern "C" int intent_nvfp4_quantize(const void* x, int64_t M, int64_t N, int64_t x_ld, const float* global_scale,
                                     uint8_t* packed, int64_t packed_ld, uint8_t* scales, void* stream) {
  intent::clear_error();
  INTENT_REQUIRE(M >= 0 && N >= 0 && M <= INT32_MAX && N <= INT32_MAX, INTENT_ERR_INVALID_ARGUMENT, "bad extents");
  INTENT_REQUIRE(N % 16 == 0, INTENT_ERR_UNSUPPORTED, "N must be a multiple of 16, got %lld", (long long)N);
  if (M == 0 || N == 0) return INTENT_OK;
  INTENT_REQUIRE(x && global_scale && packed && scales, INTENT_ERR_INVALID_ARGUMENT, "null pointer argument");
  INTENT_REQUIRE(x_ld >= N && packed_ld >= N / 2, INTENT_ERR_INVALID_ARGUMENT, "leading stride smaller than the row");
  const int64_t G = N / 16;
  const int64_t total = M * G;
  INTENT_REQUIRE(total / 256 < (1ll << 31), INTENT_ERR_UNSUPPORTED, "nvfp4_quantize: grid too large");
  hipLaunchKernelGGL(nvfp4_quantize_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                     (const uint16_t*)x, x_ld, (int)M, (int)G, global_scale, packed, packed_ld, scales,
                     (int)((G + 3) / 4));
  return intent::launch_status("nvfp4_quantize");
}
