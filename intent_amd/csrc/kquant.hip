// GGUF K-quant records on gfx950: Q8_K quantization of f32 activations and the
// Q4_K x Q8_K dot product, composed into the quantized projection
//   y[n] = quantized_dot(W[n], quantize(x)).
//
// Record formats and numerics follow doc/dsl/quantized-operations.en.md:11-70:
//   Q4_K (144 B): f16 d, f16 dmin, 12 bytes of 6-bit sub-block scales sc[8]
//                 and mins m[8], 128 bytes of nibbles;
//   Q8_K (292 B): f32 ds, 256 x i8, 16 x i16 bsum (sums of 16 values).
// Per record pair: S = sum_s sc[s] * dot32_s (int32, exact), T = sum_s m[s] *
// (bsum[2s] + bsum[2s+1]) (int32, exact), v = ds * (d*S - dmin*T) with every
// f32 operation rounded once (no contraction: built with -ffp-contract=off),
// and the row result is the f32 sum of v in increasing record order starting
// from +0. The kernels reproduce that order exactly, so results are bit-equal
// to a sequential CPU evaluation.
#include "common.h"
#include <atomic>
#include <mutex>

#include "internal.h"

namespace {

constexpr int kQ4Bytes = 144;
constexpr int kQ8Bytes = 292;

// ---- Q8_K quantization: one wave per 256-value record --------------------------
// Lane l holds values 4l..4l+3 (v). Extremes reduce exactly across the wave; the
// record's inverse and ds use IEEE division; q = saturate(rne(v * inverse)).
struct Q8Lane {
  float ds;         // the record's scale (every lane)
  uint32_t packed;  // the lane's four i8 values
  int bsum;         // sum of the lane's quad (bsum[lane / 4]; every lane of the quad)
};

INTENT_DEVICE Q8Lane quantize_lane(const f32x4 v) {
  float mx = fmaxf(fmaxf(v[0], v[1]), fmaxf(v[2], v[3]));
  float mn = fminf(fminf(v[0], v[1]), fminf(v[2], v[3]));
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    mx = fmaxf(mx, __shfl_xor(mx, off));
    mn = fminf(mn, __shfl_xor(mn, off));
  }
  const float extreme = fabsf(mx) > fabsf(mn) ? mx : mn;  // ties pick the minimum
  float inverse = 0.f, ds = 0.f;
  int q[4] = {0, 0, 0, 0};
  if (extreme != 0.f) {
    inverse = __fdiv_rn(-127.0f, extreme);
    ds = __fdiv_rn(1.0f, inverse);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float t = rintf(__fmul_rn(v[i], inverse));
      q[i] = t > 127.f ? 127 : t < -128.f ? -128 : (int)t;
    }
  }
  Q8Lane r;
  r.ds = ds;
  r.packed = (uint32_t)(q[0] & 255) | ((uint32_t)(q[1] & 255) << 8) | ((uint32_t)(q[2] & 255) << 16) |
             ((uint32_t)(q[3] & 255) << 24);
  int sum = q[0] + q[1] + q[2] + q[3];
  sum += __shfl_xor(sum, 1);
  sum += __shfl_xor(sum, 2);
  r.bsum = sum;
  return r;
}

// Writes the lane's share of a 292-byte Q8_K record.
INTENT_DEVICE void store_q8_record(uint8_t* rec, const Q8Lane& q, int lane) {
  *reinterpret_cast<uint32_t*>(rec + 4 + 4 * lane) = q.packed;
  if ((lane & 3) == 0) *reinterpret_cast<int16_t*>(rec + 260 + 2 * (lane >> 2)) = (int16_t)q.bsum;
  if (lane == 0) *reinterpret_cast<float*>(rec) = q.ds;
}

__global__ __launch_bounds__(256) void q8k_quantize_kernel(const float* __restrict__ x, int64_t ldx, int G,
                                                           uint8_t* __restrict__ out, int64_t ld_out) {
  const int lane = threadIdx.x & 63;
  const int g = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (g >= G) return;  // wave-uniform
  const f32x4 v = *reinterpret_cast<const f32x4*>(x + (int64_t)g * ldx + 4 * lane);
  store_q8_record(out + (int64_t)g * ld_out, quantize_lane(v), lane);
}

// ---- Q4_K x Q8_K GEMV ------------------------------------------------------------
// A wave owns RW weight rows. Records go 16 at a time: lane l takes record
// c0 + l/4 and quarter u = l%4 of it, i.e. sub-blocks 2u (low nibbles of
// packed group u) and 2u+1 (high nibbles), 64 elements. The integer dots use
// v_dot4_i32_i8 (nibbles are non-negative, so signed bytes are exact); S and T
// are summed over the record's four lanes (integer, exact); lane 4b computes
// v_b and the wave adds v_b one record at a time into the row total.

// v_b of the record pair a lane's quad works on (the same value in the four
// lanes): hdr = bytes 0..15 of the Q4_K record, q0/q1 = packed group u
// (bytes 16+32u .. 47+32u), xqv = the 64 i8 activations 64u..64u+63,
// bsum_lo/hi = bsum[4u]+bsum[4u+1] and bsum[4u+2]+bsum[4u+3], ds its scale.
INTENT_DEVICE float record_value(const u32x4 hdr, const u32x4 q0, const u32x4 q1, const uint32_t (&xqv)[16],
                                 int bsum_lo, int bsum_hi, float ds, int u) {
  const uint32_t qw[8] = {q0[0], q0[1], q0[2], q0[3], q1[0], q1[1], q1[2], q1[3]};
  int dlo = 0, dhi = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    dlo = __builtin_amdgcn_sdot4((int)(qw[i] & 0x0F0F0F0Fu), (int)xqv[i], dlo, false);
    dhi = __builtin_amdgcn_sdot4((int)((qw[i] >> 4) & 0x0F0F0F0Fu), (int)xqv[8 + i], dhi, false);
  }
  // The 6-bit scale sc[i] and min m[i] of sub-blocks i = 2u and 2u + 1
  // (doc/dsl/quantized-operations.en.md:21-36), without branching on u: with
  // t = i % 4, A = header byte 4 + t, B = byte 8 + t, C = byte 12 + t;
  // i < 4: sc = A & 63, m = B & 63; i >= 4: sc = (C & 15) | (A >> 6) << 4,
  // m = (C >> 4) | (B >> 6) << 4.
  const bool high = u >= 2;
  int sc[2], mn[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const uint32_t sh = 8u * (uint32_t)((2 * u + h) & 3);
    const uint32_t A = __builtin_amdgcn_ubfe(hdr[1], sh, 8);
    const uint32_t B = __builtin_amdgcn_ubfe(hdr[2], sh, 8);
    const uint32_t C = __builtin_amdgcn_ubfe(hdr[3], sh, 8);
    sc[h] = (int)(high ? ((C & 15u) | ((A >> 6) << 4)) : (A & 63u));
    mn[h] = (int)(high ? ((C >> 4) | ((B >> 6) << 4)) : (B & 63u));
  }
  // |products| < 2^22: 24-bit multiplies are exact
  int S = __mul24(sc[0], dlo) + __mul24(sc[1], dhi);
  int T = __mul24(mn[0], bsum_lo) + __mul24(mn[1], bsum_hi);
  // sums over the quad (integer, so the order does not matter): quad_perm [1,0,3,2], [2,3,0,1]
  S += __builtin_amdgcn_mov_dpp(S, 0xB1, 0xF, 0xF, false);
  T += __builtin_amdgcn_mov_dpp(T, 0xB1, 0xF, 0xF, false);
  S += __builtin_amdgcn_mov_dpp(S, 0x4E, 0xF, 0xF, false);
  T += __builtin_amdgcn_mov_dpp(T, 0x4E, 0xF, 0xF, false);
  const float d = (float)bit_cast<f16>((uint16_t)(hdr[0] & 0xFFFFu));
  const float dmin = (float)bit_cast<f16>((uint16_t)(hdr[0] >> 16));
  const float p = __fmul_rn(d, (float)S);
  const float nn = __fmul_rn(dmin, (float)T);
  return __fmul_rn(ds, __fsub_rn(p, nn));
}

// Adds v of records c0 .. c0+cnt-1 (lane 4k holds record c0 + k) to t in order.
INTENT_DEVICE float add_in_order(float t, float v, int cnt) {
  for (int k = 0; k < cnt; ++k) t = __fadd_rn(t, bit_cast<float>(__builtin_amdgcn_readlane(bit_cast<int>(v), 4 * k)));
  return t;
}

// The weight bytes a lane needs of record b of a row: header and group u.
struct Q4Frag {
  u32x4 hdr, q0, q1;
};
INTENT_DEVICE Q4Frag load_q4(__amdgpu_buffer_rsrc_t row, int b, int u) {
  const uint32_t o = (uint32_t)(b * kQ4Bytes);
  return Q4Frag{__builtin_amdgcn_raw_buffer_load_b128(row, o, 0, 0),
                __builtin_amdgcn_raw_buffer_load_b128(row, o + 16 + 32 * u, 0, 0),
                __builtin_amdgcn_raw_buffer_load_b128(row, o + 32 + 32 * u, 0, 0)};
}

template <int RW>
__global__ __launch_bounds__(256) void q4k_gemv_kernel(const uint8_t* __restrict__ w, int64_t ldw, int N, int G,
                                                       const uint8_t* __restrict__ xq, float* __restrict__ y) {
  const int lane = threadIdx.x & 63;
  const int row0 = (blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6)) * RW;
  if (row0 >= N) return;  // wave-uniform
  const int u = lane & 3;
  const auto xr = make_rsrc(xq);
  float total[RW];
#pragma unroll
  for (int r = 0; r < RW; ++r) total[r] = 0.f;

  for (int c0 = 0; c0 < G; c0 += 16) {
    const int b = c0 + (lane >> 2) < G ? c0 + (lane >> 2) : G - 1;
    // Activation fragment: 64 i8 (elements 64u..64u+63), bsum[4u..4u+3], ds.
    const uint32_t xo = (uint32_t)b * kQ8Bytes;
    uint32_t xqv[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) xqv[i] = __builtin_amdgcn_raw_buffer_load_b32(xr, xo + 4 + 64 * u + 4 * i, 0, 0);
    const uint32_t bs01 = __builtin_amdgcn_raw_buffer_load_b32(xr, xo + 260 + 8 * u, 0, 0);
    const uint32_t bs23 = __builtin_amdgcn_raw_buffer_load_b32(xr, xo + 264 + 8 * u, 0, 0);
    const float ds = bit_cast<float>(__builtin_amdgcn_raw_buffer_load_b32(xr, xo, 0, 0));
    const int bsum_lo = (int)(int16_t)(bs01 & 0xFFFFu) + (int)(int16_t)(bs01 >> 16);
    const int bsum_hi = (int)(int16_t)(bs23 & 0xFFFFu) + (int)(int16_t)(bs23 >> 16);
    const int cnt = G - c0 < 16 ? G - c0 : 16;
#pragma unroll
    for (int r = 0; r < RW; ++r) {
      const int n = row0 + r < N ? row0 + r : N - 1;
      const Q4Frag f = load_q4(make_rsrc(w + (int64_t)n * ldw), b, u);
      total[r] = add_in_order(total[r], record_value(f.hdr, f.q0, f.q1, xqv, bsum_lo, bsum_hi, ds, u), cnt);
    }
  }
  if (lane < RW) {
    float out = 0.f;
#pragma unroll
    for (int r = 0; r < RW; ++r)
      if (r == lane) out = total[r];
    if (row0 + lane < N) y[row0 + lane] = out;
  }
}

// ---- fused projection: quantize into LDS, then the GEMV ------------------------
// Every workgroup quantizes the whole activation vector (G <= kFusedMaxG
// records, a few KB of VALU work) into LDS records padded to 304 bytes (ds at
// 0, q at 16, bsum at 272, so fragments are 16-byte aligned); workgroup 0 also
// writes the Q8_K records out. The activation loads are issued first, then
// the weight loads of the first 16 records, so the weights stream in while
// the records are being quantized. One launch instead of two.
constexpr int kFusedMaxG = 64;
constexpr int kLdsRec = 304;

// NWV waves per workgroup, RW rows per wave: the workgroup's NWV waves share
// both the quantization (record g goes to wave g % NWV) and the rows.
template <int RW, int NWV>
__global__ __launch_bounds__(64 * NWV) void q4k_projection_kernel(const uint8_t* __restrict__ w, int64_t ldw, int N,
                                                                  int G, const float* __restrict__ x, int64_t ldx,
                                                                  uint8_t* __restrict__ xq_out, float* __restrict__ y) {
  __shared__ __attribute__((aligned(16))) uint8_t xs[kFusedMaxG * kLdsRec];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int row0 = (blockIdx.x * NWV + wave) * RW;
  const int u = lane & 3;
  // Records g = wave + NWV i of this wave (up to kFusedMaxG / NWV).
  constexpr int kPerWave = kFusedMaxG / NWV;
  f32x4 xv[kPerWave];
#pragma unroll
  for (int i = 0; i < kPerWave; ++i) {
    const int g = wave + NWV * i;
    if (g < G) xv[i] = *reinterpret_cast<const f32x4*>(x + (int64_t)g * ldx + 4 * lane);
  }
  const int b0 = (lane >> 2) < G ? (lane >> 2) : G - 1;
  Q4Frag f0[RW];
#pragma unroll
  for (int r = 0; r < RW; ++r) {
    const int n = row0 + r < N ? row0 + r : N - 1;
    f0[r] = load_q4(make_rsrc(w + (int64_t)n * ldw), b0, u);
  }
#pragma unroll
  for (int i = 0; i < kPerWave; ++i) {
    const int g = wave + NWV * i;
    if (g < G) {
      const Q8Lane q = quantize_lane(xv[i]);
      uint8_t* r = xs + g * kLdsRec;
      *reinterpret_cast<uint32_t*>(r + 16 + 4 * lane) = q.packed;
      if ((lane & 3) == 0) *reinterpret_cast<int16_t*>(r + 272 + 2 * (lane >> 2)) = (int16_t)q.bsum;
      if (lane == 0) *reinterpret_cast<float*>(r) = q.ds;
      if (blockIdx.x == 0) store_q8_record(xq_out + (int64_t)g * kQ8Bytes, q, lane);
    }
  }
  __syncthreads();
  if (row0 >= N) return;  // wave-uniform, after the barrier

  float total[RW];
#pragma unroll
  for (int r = 0; r < RW; ++r) total[r] = 0.f;
  for (int c0 = 0; c0 < G; c0 += 16) {
    const int b = c0 + (lane >> 2) < G ? c0 + (lane >> 2) : G - 1;
    const uint8_t* rec = xs + b * kLdsRec;
    uint32_t xqv[16];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const u32x4 v = *reinterpret_cast<const u32x4*>(rec + 16 + 64 * u + 16 * i);
      xqv[4 * i] = v[0], xqv[4 * i + 1] = v[1], xqv[4 * i + 2] = v[2], xqv[4 * i + 3] = v[3];
    }
    const u32x2 bs = *reinterpret_cast<const u32x2*>(rec + 272 + 8 * u);
    const float ds = *reinterpret_cast<const float*>(rec);
    const int bsum_lo = (int)(int16_t)(bs[0] & 0xFFFFu) + (int)(int16_t)(bs[0] >> 16);
    const int bsum_hi = (int)(int16_t)(bs[1] & 0xFFFFu) + (int)(int16_t)(bs[1] >> 16);
    const int cnt = G - c0 < 16 ? G - c0 : 16;
#pragma unroll
    for (int r = 0; r < RW; ++r) {
      Q4Frag f = f0[r];
      if (c0 > 0) {
        const int n = row0 + r < N ? row0 + r : N - 1;
        f = load_q4(make_rsrc(w + (int64_t)n * ldw), b, u);
      }
      total[r] = add_in_order(total[r], record_value(f.hdr, f.q0, f.q1, xqv, bsum_lo, bsum_hi, ds, u), cnt);
    }
  }
  if (lane < RW) {
    float out = 0.f;
#pragma unroll
    for (int r = 0; r < RW; ++r)
      if (r == lane) out = total[r];
    if (row0 + lane < N) y[row0 + lane] = out;
  }
}

constexpr int kRows = 4;
// Projection workgroups: 16 waves of one row each. Each wave quantizes one
// record and computes one row, so the 16 waves of a CU split both phases
// (N = K = 4096: 5.07 us, against 7.97 us for 4 waves of 4 rows, 6.06 us for
// 8 waves of one row and 6.90 us for 16 waves of 2 rows).
constexpr int kProjWaves = 16;  // waves per projection workgroup
constexpr int kProjRows = 1;    // rows per projection wave

__global__ void zero_fill_kernel(float* __restrict__ y, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) y[i] = 0.f;
}

int quantize_check(const float* x, int64_t G, int64_t x_ld, const uint8_t* out, int64_t out_ld) {
  INTENT_REQUIRE(G >= 0 && G <= INT32_MAX / 4, INTENT_ERR_INVALID_ARGUMENT, "bad record count %lld", (long long)G);
  if (G == 0) return INTENT_OK;
  INTENT_REQUIRE(x && out, INTENT_ERR_INVALID_ARGUMENT, "null pointer argument");
  INTENT_REQUIRE(x_ld >= 256 && out_ld >= kQ8Bytes, INTENT_ERR_INVALID_ARGUMENT, "leading stride smaller than the row");
  INTENT_REQUIRE(intent::aligned16(x) && x_ld % 4 == 0 && intent::aligned4(out) && out_ld % 4 == 0,
                 INTENT_ERR_ALIGNMENT, "x must be 16-byte aligned (row stride a multiple of 4), records 4-byte aligned");
  return INTENT_OK;
}

}  // namespace

extern "C" int intent_q8k_quantize(const float* x, int64_t G, int64_t x_ld, uint8_t* records, int64_t records_ld,
                                   void* stream) {
  intent::clear_error();
  int st = quantize_check(x, G, x_ld, records, records_ld);
  if (st != INTENT_OK || G == 0) return st;
  hipLaunchKernelGGL(q8k_quantize_kernel, dim3((unsigned)((G + 3) / 4)), dim3(256), 0, (hipStream_t)stream, x, x_ld,
                     (int)G, records, records_ld);
  return intent::launch_status("q8k_quantize");
}

extern "C" int intent_q4k_q8k_gemv(const uint8_t* w, int64_t N, int64_t G, int64_t w_ld, const uint8_t* xq,
                                   float* y, void* stream) {
  intent::clear_error();
  INTENT_REQUIRE(N >= 0 && G >= 0 && N <= INT32_MAX && G <= INT32_MAX / kQ8Bytes, INTENT_ERR_INVALID_ARGUMENT,
                 "bad extents (N=%lld G=%lld)", (long long)N, (long long)G);
  if (N == 0) return INTENT_OK;
  INTENT_REQUIRE(y, INTENT_ERR_INVALID_ARGUMENT, "null output");
  if (G == 0) {  // empty dot: +0 for every row, no reads (a fill kernel, not a memset node)
    hipLaunchKernelGGL(zero_fill_kernel, dim3((unsigned)((N + 255) / 256)), dim3(256), 0, (hipStream_t)stream, y,
                       (int)N);
    return intent::launch_status("q4k_q8k_gemv");
  }
  INTENT_REQUIRE(w && xq, INTENT_ERR_INVALID_ARGUMENT, "null pointer argument");
  INTENT_REQUIRE(w_ld >= G * kQ4Bytes, INTENT_ERR_INVALID_ARGUMENT, "weight row stride smaller than G records");
  INTENT_REQUIRE(intent::aligned16(w) && w_ld % 16 == 0 && intent::aligned4(xq), INTENT_ERR_ALIGNMENT,
                 "weights must be 16-byte aligned with 16-byte row strides; Q8_K records 4-byte aligned");
  const int64_t waves = (N + kRows - 1) / kRows;
  hipLaunchKernelGGL((q4k_gemv_kernel<kRows>), dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, (hipStream_t)stream,
                     w, w_ld, (int)N, (int)G, xq, y);
  return intent::launch_status("q4k_q8k_gemv");
}

extern "C" int intent_q4k_projection(const uint8_t* w, int64_t N, int64_t G, int64_t w_ld, const float* x,
                                     int64_t x_ld, uint8_t* xq_records, float* y, void* stream) {
  intent::clear_error();
  int st = quantize_check(x, G, x_ld, xq_records, kQ8Bytes);
  if (st != INTENT_OK) return st;
  if (G > 0 && G <= kFusedMaxG && N > 0) {
    INTENT_REQUIRE(w && y, INTENT_ERR_INVALID_ARGUMENT, "null pointer argument");
    INTENT_REQUIRE(N <= INT32_MAX, INTENT_ERR_INVALID_ARGUMENT, "bad extent N=%lld", (long long)N);
    INTENT_REQUIRE(w_ld >= G * kQ4Bytes, INTENT_ERR_INVALID_ARGUMENT, "weight row stride smaller than G records");
    INTENT_REQUIRE(intent::aligned16(w) && w_ld % 16 == 0, INTENT_ERR_ALIGNMENT,
                   "weights must be 16-byte aligned with 16-byte row strides");
    const int64_t waves = (N + kProjRows - 1) / kProjRows;
    hipLaunchKernelGGL((q4k_projection_kernel<kProjRows, kProjWaves>),
                       dim3((unsigned)((waves + kProjWaves - 1) / kProjWaves)), dim3(64 * kProjWaves), 0,
                       (hipStream_t)stream, w, w_ld, (int)N, (int)G, x, x_ld, xq_records, y);
    return intent::launch_status("q4k_projection");
  }
  if (G > 0) {
    hipLaunchKernelGGL(q8k_quantize_kernel, dim3((unsigned)((G + 3) / 4)), dim3(256), 0, (hipStream_t)stream, x,
                       x_ld, (int)G, xq_records, (int64_t)kQ8Bytes);
    st = intent::launch_status("q8k_quantize");
    if (st != INTENT_OK) return st;
  }
  return intent_q4k_q8k_gemv(w, N, G, w_ld, xq_records, y, stream);
}

// ---- allocation-free Q4_K projection ----------------------------------------------
// intent_q4k_projection_noalloc keeps the Q8_K records of the activation in
// `scratch`, a fixed device array (one copy per GPU, held until the process
// ends), instead of a caller workspace: for callers that cannot allocate
// (code under HIP graph capture, tight serving loops). The records are fully
// written by each call before they are read, so nothing needs clearing; calls
// that overlap on one GPU share the array and race.
constexpr int64_t kScratchMaxG = 1024;  // K <= 262144; 299,008 bytes
static __device__ __align__(256) uint8_t scratch[kScratchMaxG * kQ8Bytes];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
std::atomic<uint8_t*> g_scratch_ptr[kMaxDevices] = {};

// Device address of the current device's `scratch` (looked up once per device,
// with that device current; the array's name is not a device address in host code).
int current_scratch(uint8_t** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return intent::fail(INTENT_ERR_LAUNCH, "hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return intent::fail(INTENT_ERR_UNSUPPORTED, "device %d out of range", dev);
  // after the first call on a device the address is read without the lock
  uint8_t* known = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (known == nullptr) {
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    known = g_scratch_ptr[dev].load(std::memory_order_relaxed);
    if (known == nullptr) {
      void* p = nullptr;
      e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (e != hipSuccess || p == nullptr)
        return intent::fail(INTENT_ERR_LAUNCH, "hipGetSymbolAddress(scratch) on device %d: %s", dev,
                            hipGetErrorString(e));
      known = (uint8_t*)p;
      g_scratch_ptr[dev].store(known, std::memory_order_release);
    }
  }
  *out = known;
  return INTENT_OK;
}

}  // namespace

extern "C" int intent_q4k_projection_noalloc(const uint8_t* w, int64_t N, int64_t G, int64_t w_ld, const float* x,
                                             int64_t x_ld, float* y, void* stream) {
  intent::clear_error();
  INTENT_REQUIRE(G >= 0 && G <= kScratchMaxG, INTENT_ERR_UNSUPPORTED,
                 "G=%lld records exceed the allocation-free limit of %lld (K <= %lld)", (long long)G,
                 (long long)kScratchMaxG, (long long)(kScratchMaxG * 256));
  uint8_t* records = nullptr;
  const int st = current_scratch(&records);
  if (st != INTENT_OK) return st;
  return intent_q4k_projection(w, N, G, w_ld, x, x_ld, records, y, stream);
}
