// Generic-shape paths of the weight-only and int8 contractions.
//
// The tiled kernels need K in whole stages (64 or 128 k) and 16-byte aligned
// rows. Shapes outside that (any K, any row stride, any alignment) run here:
// one output element per thread, scalar loads, the same per-element
// arithmetic and the same epilogue as the fast kernels, so the results meet
// the same bar (bit-exact int32 sums and bf16 epilogue; f32 sums of the same
// f16 products for the weight-only forms). Throughput is not the point of
// these kernels; they keep the operator surface as wide as the reference's
// (examples/kernels/contraction/weight_only_int4.py:18-51, gemm.py:29-39,
// the W8 kernels of runtime/cpu_runtime.py), whose DSL kernels take any shape.
// fill_launch writes a constant: the epilogue of an empty K, where a
// contraction sums nothing (doc/dsl/core.en.md:213).
#include "common.h"
#include "internal.h"

#include <atomic>
#include <type_traits>

namespace {

constexpr int kThreads = 256;

// y[m, n] = f16(sum_k f32(x[m, k]) * f32(f16((q - z) * s))), nibble k of row n
// = low nibble of byte k/2 for even k, high for odd k; group k / gs.
__global__ __launch_bounds__(kThreads) void w4a16_generic_kernel(const f16* __restrict__ x, int64_t ldx,
                                                                 const uint8_t* __restrict__ q, int64_t ldq,
                                                                 const f16* __restrict__ sc,
                                                                 const uint8_t* __restrict__ zp, int64_t ldp, int gs,
                                                                 int K, int N, f16* __restrict__ y, int64_t ldy) {
  const int n = blockIdx.x * kThreads + threadIdx.x;
  const int m = blockIdx.y;
  if (n >= N) return;
  const f16* xr = x + (int64_t)m * ldx;
  const uint8_t* qr = q + (int64_t)n * ldq;
  float acc = 0.f;
  for (int g0 = 0; g0 < K; g0 += gs) {
    const int g = g0 / gs;
    const f16 s = sc[(int64_t)n * ldp + g];
    const f16 z = (f16)(float)zp[(int64_t)n * ldp + g];
    const int g1 = g0 + gs < K ? g0 + gs : K;
    for (int k = g0; k < g1; ++k) {
      const uint32_t byte = qr[k >> 1];
      const f16 nib = (f16)(float)((k & 1) ? (byte >> 4) : (byte & 15u));
      const f16 w = (f16)((float)(f16)((float)nib - (float)z) * (float)s);  // (q - z) exact, one f16 rounding
      acc = __builtin_fmaf((float)xr[k], (float)w, acc);
    }
  }
  y[(int64_t)m * ldy + n] = (f16)acc;
}

// y[m, n] = f16(sum_k f32(x[m, k]) * w[n, k] * scale[n]).
__global__ __launch_bounds__(kThreads) void w8a16_generic_kernel(const f16* __restrict__ x, int64_t ldx,
                                                                 const int8_t* __restrict__ w, int64_t ldw,
                                                                 const f16* __restrict__ sc, int K, int N,
                                                                 f16* __restrict__ y, int64_t ldy) {
  const int n = blockIdx.x * kThreads + threadIdx.x;
  const int m = blockIdx.y;
  if (n >= N) return;
  const f16* xr = x + (int64_t)m * ldx;
  const int8_t* wr = w + (int64_t)n * ldw;
  float acc = 0.f;
  for (int k = 0; k < K; ++k) acc = __builtin_fmaf((float)xr[k], (float)wr[k], acc);
  y[(int64_t)m * ldy + n] = (f16)(acc * (float)sc[n]);
}

// acc = sum_k a[m, k] * w[n, k] in int32 arithmetic modulo 2^32, then
// bf16(f32(acc) * a_scale[m] * w_scale[n]) (scaled) or acc + bias[n] (int32).
template <bool kScaled>
__global__ __launch_bounds__(kThreads) void i8_generic_kernel(const int8_t* __restrict__ a, int64_t lda,
                                                              const int8_t* __restrict__ w, int64_t ldw, int K, int N,
                                                              const float* __restrict__ sa,
                                                              const float* __restrict__ sw,
                                                              const int32_t* __restrict__ bias,
                                                              void* __restrict__ out, int64_t ldo) {
  const int n = blockIdx.x * kThreads + threadIdx.x;
  const int m = blockIdx.y;
  if (n >= N) return;
  const int8_t* ar = a + (int64_t)m * lda;
  const int8_t* wr = w + (int64_t)n * ldw;
  uint32_t acc = 0;
  for (int k = 0; k < K; ++k) acc += (uint32_t)((int32_t)ar[k] * (int32_t)wr[k]);
  if constexpr (kScaled) {
    reinterpret_cast<uint16_t*>(out)[(int64_t)m * ldo + n] = f32_to_bf16_rne(((float)(int32_t)acc * sa[m]) * sw[n]);
  } else {
    reinterpret_cast<int32_t*>(out)[(int64_t)m * ldo + n] = (int32_t)(acc + (uint32_t)(bias ? bias[n] : 0));
  }
}

dim3 grid_for(int64_t M, int64_t N) { return dim3((unsigned)((N + kThreads - 1) / kThreads), (unsigned)M); }

// out[r * ld + c] = bits for r < rows, c < cols; elements of EB bytes.
template <int EB>
__global__ __launch_bounds__(kThreads) void fill_kernel(void* __restrict__ out, int64_t rows, int64_t cols,
                                                        int64_t ld, uint32_t bits) {
  using E = std::conditional_t<EB == 1, uint8_t, std::conditional_t<EB == 2, uint16_t, uint32_t>>;
  const int64_t c = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (c >= cols) return;
  for (int64_t r = blockIdx.y; r < rows; r += gridDim.y) reinterpret_cast<E*>(out)[r * ld + c] = (E)bits;
}

}  // namespace

namespace intent {

bool generic_grid_ok(int64_t M, int64_t N) { return M <= 65535 && (N + kThreads - 1) / kThreads < (1ll << 31); }

int w4a16_generic_launch(const void* x, int64_t M, int64_t K, int64_t x_ld, const uint8_t* packed, int64_t N,
                         int64_t packed_ld, const void* scales, const uint8_t* zeros, int64_t qparam_ld, int64_t gs,
                         void* y, int64_t y_ld, void* stream) {
  INTENT_REQUIRE(generic_grid_ok(M, N), INTENT_ERR_UNSUPPORTED, "w4a16 generic path: M above 65535");
  hipLaunchKernelGGL(w4a16_generic_kernel, grid_for(M, N), dim3(kThreads), 0, (hipStream_t)stream, (const f16*)x,
                     x_ld, packed, packed_ld, (const f16*)scales, zeros, qparam_ld, (int)gs, (int)K, (int)N, (f16*)y,
                     y_ld);
  return launch_status("w4a16_generic_kernel");
}

int w8a16_generic_launch(const void* x, int64_t M, int64_t K, int64_t x_ld, const int8_t* w, int64_t N, int64_t w_ld,
                         const void* scales, void* y, int64_t y_ld, void* stream) {
  INTENT_REQUIRE(generic_grid_ok(M, N), INTENT_ERR_UNSUPPORTED, "w8a16 generic path: M above 65535");
  hipLaunchKernelGGL(w8a16_generic_kernel, grid_for(M, N), dim3(kThreads), 0, (hipStream_t)stream, (const f16*)x,
                     x_ld, w, w_ld, (const f16*)scales, (int)K, (int)N, (f16*)y, y_ld);
  return launch_status("w8a16_generic_kernel");
}

int cu_count() {
  constexpr int kMaxDevices = 64;
  static std::atomic<int> known[kMaxDevices] = {};
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 0;
  int n = known[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n < 0) n = 0;
    known[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

int fill_launch(void* out, int64_t rows, int64_t cols, int64_t ld, int elem_bytes, uint32_t bits, void* stream) {
  if (rows == 0 || cols == 0) return INTENT_OK;
  INTENT_REQUIRE(out, INTENT_ERR_INVALID_ARGUMENT, "null output");
  INTENT_REQUIRE(ld >= cols, INTENT_ERR_INVALID_ARGUMENT, "leading stride smaller than the row");
  INTENT_REQUIRE((cols + kThreads - 1) / kThreads < (1ll << 31), INTENT_ERR_UNSUPPORTED, "fill: row too long");
  const dim3 grid((unsigned)((cols + kThreads - 1) / kThreads), (unsigned)(rows < 65535 ? rows : 65535));
  if (elem_bytes == 1)
    hipLaunchKernelGGL(fill_kernel<1>, grid, dim3(kThreads), 0, (hipStream_t)stream, out, rows, cols, ld, bits);
  else if (elem_bytes == 2)
    hipLaunchKernelGGL(fill_kernel<2>, grid, dim3(kThreads), 0, (hipStream_t)stream, out, rows, cols, ld, bits);
  else
    hipLaunchKernelGGL(fill_kernel<4>, grid, dim3(kThreads), 0, (hipStream_t)stream, out, rows, cols, ld, bits);
  return launch_status("fill_kernel");
}

int i8_generic_launch(const int8_t* a, int64_t M, int64_t K, int64_t a_ld, const int8_t* w, int64_t N, int64_t w_ld,
                      const float* sa, const float* sw, const int32_t* bias, void* out, int64_t out_ld, bool scaled,
                      void* stream) {
  INTENT_REQUIRE(generic_grid_ok(M, N), INTENT_ERR_UNSUPPORTED, "int8 generic path: M above 65535");
  if (scaled)
    hipLaunchKernelGGL(i8_generic_kernel<true>, grid_for(M, N), dim3(kThreads), 0, (hipStream_t)stream, a, a_ld, w,
                       w_ld, (int)K, (int)N, sa, sw, bias, out, out_ld);
  else
    hipLaunchKernelGGL(i8_generic_kernel<false>, grid_for(M, N), dim3(kThreads), 0, (hipStream_t)stream, a, a_ld, w,
                       w_ld, (int)K, (int)N, sa, sw, bias, out, out_ld);
  return launch_status(scaled ? "i8_generic_kernel<scaled>" : "i8_generic_kernel<i32>");
}

}  // namespace intent
