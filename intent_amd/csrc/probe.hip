// HBM read-floor probe: the fastest plain read of a buffer, used to measure
// what any kernel that streams the same bytes once can reach (the decode
// GEMV's own floor at its size). Not part of any operator.
//
// A workgroup of 256 lanes reads 256 * U * 16 contiguous bytes: lane t loads
// 16 bytes at t, t + 256, ... (U loads, all issued before any is used). The
// values are folded with XOR and stored only if they hit a magic word, which
// keeps the loads live without writing anything in practice.
#include "../../include/intent_amd_probes.h"
#include "common.h"
#include "internal.h"

namespace {

template <int U, int kMode>  // kMode bit 0: one store per wave; bit 1: non-temporal loads
__global__ __launch_bounds__(256) void hbm_read_probe_kernel(const u32x4* __restrict__ src, int64_t n16,
                                                             uint32_t* __restrict__ sink) {
  constexpr bool kStore = (kMode & 1) != 0, kNT = (kMode & 2) != 0;
  const int64_t base = (int64_t)blockIdx.x * 256 * U + threadIdx.x;
  u32x4 v[U];
#pragma unroll
  for (int i = 0; i < U; ++i) {
    const int64_t idx = base + (int64_t)i * 256;
    v[i] = idx < n16 ? (kNT ? __builtin_nontemporal_load(src + idx) : src[idx]) : u32x4{0u, 0u, 0u, 0u};
  }
  uint32_t s = 0;
#pragma unroll
  for (int i = 0; i < U; ++i) s ^= v[i][0] ^ v[i][1] ^ v[i][2] ^ v[i][3];
  if (kStore) {
    // every lane's value decides whether it stores, so no lane's loads can
    // be dropped; lane 0 always stores (a lane on a hash hit rewrites the
    // second word of its wave's pair)
    const int lane = threadIdx.x & 63;
    const int64_t w = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (lane == 0) *reinterpret_cast<u32x2*>(sink + 2 * w) = u32x2{s, s ^ 1u};
    else if (s == 0x9e3779b9u) sink[2 * w + 1] = s;
  } else if (s == 0x9e3779b9u) {
    sink[blockIdx.x & 255] = s;
  }
}

template <int U>
void launch_probe(const void* buf, int64_t n16, int mode, uint32_t* sink, hipStream_t st) {
  const int64_t per = 256 * U;
  const unsigned blocks = (unsigned)((n16 + per - 1) / per);
  const u32x4* src = (const u32x4*)buf;
  switch (mode) {
    case 0: hipLaunchKernelGGL((hbm_read_probe_kernel<U, 0>), dim3(blocks), dim3(256), 0, st, src, n16, sink); break;
    case 1: hipLaunchKernelGGL((hbm_read_probe_kernel<U, 1>), dim3(blocks), dim3(256), 0, st, src, n16, sink); break;
    case 2: hipLaunchKernelGGL((hbm_read_probe_kernel<U, 2>), dim3(blocks), dim3(256), 0, st, src, n16, sink); break;
    default: hipLaunchKernelGGL((hbm_read_probe_kernel<U, 3>), dim3(blocks), dim3(256), 0, st, src, n16, sink); break;
  }
}

// MFMA issue-rate probe: every wave runs `iters` rounds of four independent
// 32x32 MFMAs on register operands (no memory traffic), so the measured rate
// is the matrix cores' sustained throughput at the clock the chip holds under
// that load. kind 0: v_mfma_f32_32x32x16_f16 (32768 flops each); kind 1:
// v_mfma_i32_32x32x32_i8 (65536 ops each).
template <int kKind>
__global__ __launch_bounds__(256) void mfma_peak_probe_kernel(int64_t iters, uint32_t* __restrict__ sink) {
  const uint32_t seed = threadIdx.x * 2654435761u + blockIdx.x;
  if constexpr (kKind == 0) {
    const f16x8 a = bit_cast<f16x8>(u32x4{seed, seed ^ 1u, seed ^ 2u, seed ^ 3u} & 0x3bff3bffu);
    const f16x8 b = bit_cast<f16x8>(u32x4{seed ^ 5u, seed ^ 6u, seed ^ 7u, seed ^ 8u} & 0x3bff3bffu);
    f32x16 c0 = {}, c1 = {}, c2 = {}, c3 = {};
    for (int64_t i = 0; i < iters; ++i) {
      c0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c0, 0, 0, 0);
      c1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(b, a, c1, 0, 0, 0);
      c2 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, a, c2, 0, 0, 0);
      c3 = __builtin_amdgcn_mfma_f32_32x32x16_f16(b, b, c3, 0, 0, 0);
    }
    const float t = c0[0] + c1[1] + c2[2] + c3[3];
    if (t == 1234.5f) sink[blockIdx.x & 255] = 1u;
  } else {
    const i32x4 a4 = {(int)seed, (int)(seed ^ 1u), (int)(seed ^ 2u), (int)(seed ^ 3u)};
    const i32x4 b4 = {(int)(seed ^ 5u), (int)(seed ^ 6u), (int)(seed ^ 7u), (int)(seed ^ 8u)};
    i32x16 c0 = {}, c1 = {}, c2 = {}, c3 = {};
    for (int64_t i = 0; i < iters; ++i) {
      c0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a4, b4, c0, 0, 0, 0);
      c1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(b4, a4, c1, 0, 0, 0);
      c2 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a4, a4, c2, 0, 0, 0);
      c3 = __builtin_amdgcn_mfma_i32_32x32x32_i8(b4, b4, c3, 0, 0, 0);
    }
    const int t = c0[0] + c1[1] + c2[2] + c3[3];
    if (t == 1234567) sink[blockIdx.x & 255] = 1u;
  }
}

}  // namespace

extern "C" int intent_mfma_peak_probe(int kind, int64_t iters, int64_t workgroups, uint32_t* sink, void* stream) {
  INTENT_REQUIRE(sink, INTENT_ERR_INVALID_ARGUMENT, "null sink");
  INTENT_REQUIRE(iters > 0 && workgroups > 0 && workgroups <= (1 << 20), INTENT_ERR_INVALID_ARGUMENT,
                 "bad iters / workgroups");
  hipStream_t st = (hipStream_t)stream;
  if (kind == 0)
    hipLaunchKernelGGL(mfma_peak_probe_kernel<0>, dim3((unsigned)workgroups), dim3(256), 0, st, iters, sink);
  else if (kind == 1)
    hipLaunchKernelGGL(mfma_peak_probe_kernel<1>, dim3((unsigned)workgroups), dim3(256), 0, st, iters, sink);
  else
    return intent::fail(INTENT_ERR_UNSUPPORTED, "kind must be 0 (f16) or 1 (i8), got %d", kind);
  return intent::launch_status_fmt("mfma_peak_probe_kernel<%d>", kind);
}

extern "C" int intent_hbm_read_probe(const void* buf, int64_t bytes, int unroll, int store, uint32_t* sink,
                                     int64_t sink_words, void* stream) {
  INTENT_REQUIRE(buf && sink, INTENT_ERR_INVALID_ARGUMENT, "null pointer argument");
  INTENT_REQUIRE(bytes > 0 && bytes % 16 == 0, INTENT_ERR_INVALID_ARGUMENT, "bytes must be a positive multiple of 16");
  INTENT_REQUIRE(intent::aligned16(buf) && intent::aligned4(sink), INTENT_ERR_ALIGNMENT,
                 "buffer must be 16-byte aligned, sink 4-byte aligned");
  INTENT_REQUIRE(unroll == 1 || unroll == 2 || unroll == 4 || unroll == 8 || unroll == 16, INTENT_ERR_UNSUPPORTED,
                 "unroll must be 1, 2, 4, 8 or 16, got %d", unroll);
  INTENT_REQUIRE(store >= 0 && store <= 3, INTENT_ERR_INVALID_ARGUMENT, "store must be 0..3, got %d", store);
  const int64_t waves = 4 * ((bytes + 4096LL * unroll - 1) / (4096LL * unroll));
  const int64_t need = (store & 1) ? 2 * waves : 256;
  INTENT_REQUIRE(sink_words >= need, INTENT_ERR_INVALID_ARGUMENT, "sink needs %lld words, got %lld", (long long)need,
                 (long long)sink_words);
  const int64_t n16 = bytes / 16;
  hipStream_t st = (hipStream_t)stream;
  switch (unroll) {
    case 1: launch_probe<1>(buf, n16, store, sink, st); break;
    case 2: launch_probe<2>(buf, n16, store, sink, st); break;
    case 4: launch_probe<4>(buf, n16, store, sink, st); break;
    case 8: launch_probe<8>(buf, n16, store, sink, st); break;
    default: launch_probe<16>(buf, n16, store, sink, st); break;
  }
  return intent::launch_status_fmt("hbm_read_probe_kernel<%d, %d>", unroll, store);
}
