// W8A8 int8 GEMM on v_mfma_i32_32x32x32_i8 (gfx950), exact int32 accumulation.
//
// Tiles of 256 x 256 with 8 waves in 4 x 2 (or 128 x 128 with 4 waves for
// small problems) on the pipelined core in mfma_pipe.h: both K-contiguous int8 operands are
// staged global -> VGPR -> LDS, 128 k per stage, two stages in flight.
// Epilogues: bf16(f32(acc) * a_scale[m] * w_scale[n]) or int32 acc + bias[n].
#include "common.h"
#include "internal.h"
#include "mfma_pipe.h"

namespace intent {
int i8_generic_launch(const int8_t* a, int64_t M, int64_t K, int64_t a_ld, const int8_t* w, int64_t N, int64_t w_ld,
                      const float* sa, const float* sw, const int32_t* bias, void* out, int64_t out_ld, bool scaled,
                      void* stream);
}  // namespace intent

namespace {

using T256 = mp::Tile<256, 256, 4, 2>;  // 8 waves of 64 x 128 (two per SIMD)
using T128 = mp::Tile<128, 128, 2, 2>;  // small problems: more workgroups

enum class Epi { kBf16Scaled, kI32Bias };

// Lane holds m = row(i) and n = col(j, g) + 0..3 in acc[i][j][4g..4g+3].
template <class T, Epi E>
INTENT_DEVICE void store_tile(const i32x16 (&acc)[T::TI][T::TJ], int m0, int n0, int M, int N,
                              const float* __restrict__ a_scales, const float* __restrict__ w_scales,
                              const int32_t* __restrict__ bias, void* __restrict__ out, int64_t ldo) {
  if constexpr ((INTENT_ABLATE & 4) != 0)
    if (ldo > 0) return;  // measurement build: no stores (ldo is unknown here, so the sums stay live)
  const bool vec = (ldo & 3) == 0 && (((uintptr_t)out) & 7) == 0;
#pragma unroll
  for (int i = 0; i < T::TI; ++i) {
    const int m = m0 + T::row(i);
    if (m >= M) continue;
    const float sa = E == Epi::kBf16Scaled ? a_scales[m] : 0.f;
#pragma unroll
    for (int j = 0; j < T::TJ; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int n = n0 + T::col(j, g);
        if (E == Epi::kBf16Scaled) {
          uint16_t* o = reinterpret_cast<uint16_t*>(out) + (int64_t)m * ldo + n;
          if (vec && n + 3 < N) {
            const f32x4 ws = *reinterpret_cast<const f32x4*>(w_scales + n);
            const uint32_t lo = bf16x2_rne(((float)acc[i][j][4 * g] * sa) * ws[0],
                                           ((float)acc[i][j][4 * g + 1] * sa) * ws[1]);
            const uint32_t hi = bf16x2_rne(((float)acc[i][j][4 * g + 2] * sa) * ws[2],
                                           ((float)acc[i][j][4 * g + 3] * sa) * ws[3]);
            *reinterpret_cast<u32x2*>(o) = u32x2{lo, hi};
          } else {
#pragma unroll
            for (int c = 0; c < 4; ++c)
              if (n + c < N) o[c] = (uint16_t)bf16x2_rne(((float)acc[i][j][4 * g + c] * sa) * w_scales[n + c], 0.f);
          }
        } else {
          int32_t* o = reinterpret_cast<int32_t*>(out) + (int64_t)m * ldo + n;
#pragma unroll
          for (int c = 0; c < 4; ++c)
            if (n + c < N) o[c] = (int32_t)((uint32_t)acc[i][j][4 * g + c] + (uint32_t)(bias ? bias[n + c] : 0));
        }
      }
  }

}

// The scaled bf16 epilogue through LDS (a stage buffer is free after the main
// loop): each wave converts its 32-row blocks one at a time into a private
// [32][128] bf16 block (256-byte rows, 16-byte piece p of row r in slot
// p ^ (r % 16), so the 8-byte writes of 16 rows and the 16-byte reads of one
// row fall in distinct banks), reads it back as 16-byte row pieces and stores
// whole 256-byte row segments, where the register layout would store 16-byte
// pieces of 32 rows per instruction. lds: NW * 8 KB no longer read by any wave.
// scales: the tile's BM row scales, then its BN column scales (LDS; zero past
// M and N).
template <class T>
INTENT_DEVICE void store_bf16_lds(const i32x16 (&acc)[T::TI][T::TJ], char* lds, const float* scales, int m0, int n0,
                                  int M, int N, uint16_t* __restrict__ out, int64_t ldo) {
  static_assert(T::WTN == 128, "128-column wave tiles");
  constexpr int RS = 256;  // LDS row bytes
  const int lane = threadIdx.x & 63;
  char* blk = lds + T::wave() * 32 * RS;
  const int wm = m0 + T::wave_m() * T::WTM, wn = n0 + T::wave_n() * T::WTN;
  const bool vec_out = (ldo & 7) == 0 && (((uintptr_t)out) & 15) == 0;
  f32x4 ws[T::TJ][4];
#pragma unroll
  for (int j = 0; j < T::TJ; ++j)
#pragma unroll
    for (int g = 0; g < 4; ++g) ws[j][g] = *reinterpret_cast<const f32x4*>(scales + T::BM + T::col(j, g));
#pragma unroll
  for (int i = 0; i < T::TI; ++i) {
    const float sa = scales[T::row(i)];
#pragma unroll
    for (int j = 0; j < T::TJ; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const uint32_t lo = bf16x2_rne(((float)acc[i][j][4 * g] * sa) * ws[j][g][0],
                                       ((float)acc[i][j][4 * g + 1] * sa) * ws[j][g][1]);
        const uint32_t hi = bf16x2_rne(((float)acc[i][j][4 * g + 2] * sa) * ws[j][g][2],
                                       ((float)acc[i][j][4 * g + 3] * sa) * ws[j][g][3]);
        const int cb = (T::col(j, g) - T::wave_n() * T::WTN) * 2;  // byte in the row
        const int r = lane & 31;
        *reinterpret_cast<u32x2*>(blk + r * RS + ((((cb >> 4) ^ (r & 15))) << 4) + (cb & 15)) = u32x2{lo, hi};
      }
    // rows r = 4q + lane / 16 of the block, 16-byte piece lane % 16
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int r = 4 * q + (lane >> 4), c8 = (lane & 15) * 8;
      const u32x4 v = *reinterpret_cast<const u32x4*>(blk + r * RS + (((lane & 15) ^ (r & 15)) << 4));
      const int gm = wm + i * 32 + r, gn = wn + c8;
      if (gm >= M) continue;
      uint16_t* dst = out + (int64_t)gm * ldo + gn;
      if (vec_out && gn + 7 < N) {
        *reinterpret_cast<u32x4*>(dst) = v;
      } else {
#pragma unroll
        for (int c = 0; c < 8; ++c)
          if (gn + c < N) dst[c] = (uint16_t)(v[c >> 1] >> (16 * (c & 1)));
      }
    }
  }
}

// One workgroup per output tile; 128 k per LDS stage, the last one possibly 64.
template <class T, Epi E, bool kHalf>
__global__ __launch_bounds__(T::NT, 1) void i8_gemm_kernel(const int8_t* __restrict__ a, int64_t lda, int M,
                                                                const int8_t* __restrict__ w, int64_t ldw, int N,
                                                                int K, const float* __restrict__ a_scales,
                                                                const float* __restrict__ w_scales,
                                                                const int32_t* __restrict__ bias,
                                                                void* __restrict__ out, int64_t ldo, int mblocks) {
  __shared__ __attribute__((aligned(16))) char buf0[T::STAGE_BYTES];
  __shared__ __attribute__((aligned(16))) char buf1[T::STAGE_BYTES];
  // XCD-grouped tile order (4 row blocks x 8 column blocks per XCD round): 1% faster here
  // than plain m-fastest dispatch, which beat xcd_swizzle alone.
  int tmb, tnb;
  grid_tile(mblocks, 4, tmb, tnb);
  const int m0 = tmb * T::BM;
  const int n0 = tnb * T::BN;
  const int wave = T::wave();
  const int nk = (K + mp::ROWB - 1) / mp::ROWB;
  const bool half = kHalf;
  mp::RegRowsOperand<T::BN, mp::DenseRows, kHalf, T::NW> bop;
  bop.init(mp::DenseRows{w, ldw, N}, n0, wave, half ? nk - 1 : -1);
  i32x16 acc[T::TI][T::TJ];
  mp::RegRowsOperand<T::BM, mp::DenseRows, kHalf, T::NW> aop;
  aop.init(mp::DenseRows{a, lda, M}, m0, wave, half ? nk - 1 : -1);
  constexpr bool kLdsEpi = E == Epi::kBf16Scaled && T::WTN == 128 && T::NW * 32 * 256 <= T::STAGE_BYTES &&
                           T::NT == T::BM + T::BN && (INTENT_ABLATE & 4) == 0;
  // kLdsEpi: thread t's scale (row t, or column t - BM), loaded before the main
  // loop, whose first wait retires it
  __shared__ float scales[kLdsEpi ? T::BM + T::BN : 1];
  float my_scale = 0.f;
  if constexpr (kLdsEpi) {
    const int t = threadIdx.x;
    const int idx = t < T::BM ? m0 + t : n0 + (t - T::BM);
    const int lim = t < T::BM ? M : N;
    my_scale = idx < lim ? (t < T::BM ? a_scales : w_scales)[idx] : 0.f;
  }
  mp::mainloop<T, mp::I8Math>(aop, bop, nk, buf0, buf1, acc, half);

  if constexpr (kLdsEpi) {
    scales[threadIdx.x] = my_scale;
    __syncthreads();  // every wave's last fragment reads are done; the scales are in
    store_bf16_lds<T>(acc, buf0, scales, m0, n0, M, N, reinterpret_cast<uint16_t*>(out), ldo);
    return;
  }
  store_tile<T, E>(acc, m0, n0, M, N, a_scales, w_scales, bias, out, ldo);
}

// Low-bit weight x int8 activation contractions with exact int32 outputs.
// W4A8 (weight_only_int4.py:54-91): out[n, m] = sum_k sext4(W[n, k]) * a[m, k],
//   so the weight rows are the tile's M side and the output is [N, M].
// BitNet int2 (weight_only_int4.py:94-124): out[m, n] = sum_k a[m, k] * W2[n, k]
//   with weights 0..3 in the interleaved 2-bit packing.
// The packed weights are decoded to int8 while staged into LDS; the rest is
// the int8 pipeline above (128 k per stage, K % 128 == 0). For K <= kX16MaxK
// the W4A8 nibbles are staged as 16 * value (LowBit::kSignedNibbleX16: two
// logic ops per packed dword instead of a sign extension) and the int32
// accumulators shifted right by 4 before the store.
template <class T, bool kBitNet, bool kX16 = false>
__global__ __launch_bounds__(T::NT, 1) void lowbit_gemm_kernel(const int8_t* __restrict__ act, int64_t ld_act,
                                                               int M, const uint8_t* __restrict__ wq,
                                                               int64_t ld_w, int N, int K,
                                                               int32_t* __restrict__ out, int64_t ldo,
                                                               int mblocks) {
  __shared__ __attribute__((aligned(16))) char buf0[T::STAGE_BYTES];
  __shared__ __attribute__((aligned(16))) char buf1[T::STAGE_BYTES];
  // Tile rows come from the side that is the output's row dimension.
  const int rows = kBitNet ? M : N;
  const int cols = kBitNet ? N : M;
  const int r0 = (blockIdx.x % mblocks) * T::BM;
  const int c0 = (blockIdx.x / mblocks) * T::BN;
  const int wave = T::wave();
  const int nk = K / mp::ROWB;
  i32x16 acc[T::TI][T::TJ];
  if constexpr (kBitNet) {
    mp::RegRowsOperand<T::BM, mp::DenseRows, false, T::NW> aop;
    aop.init(mp::DenseRows{act, ld_act, M}, r0, wave);
    mp::LowBitRowsOperand<T::BN, mp::LowBit::kInt2, T::NW> bop;
    bop.init(wq, ld_w, N, c0, wave);
    mp::mainloop<T, mp::I8Math>(aop, bop, nk, buf0, buf1, acc);
  } else {
    mp::LowBitRowsOperand<T::BM, kX16 ? mp::LowBit::kSignedNibbleX16 : mp::LowBit::kSignedNibble, T::NW> aop;
    aop.init(wq, ld_w, N, r0, wave);
    mp::RegRowsOperand<T::BN, mp::DenseRows, false, T::NW> bop;
    bop.init(mp::DenseRows{act, ld_act, M}, c0, wave);
    mp::mainloop<T, mp::I8Math>(aop, bop, nk, buf0, buf1, acc);
    if constexpr (kX16) {
#pragma unroll
      for (int i = 0; i < T::TI; ++i)
#pragma unroll
        for (int j = 0; j < T::TJ; ++j)
#pragma unroll
          for (int e = 0; e < 16; ++e) acc[i][j][e] >>= 4;  // exact: every product is a multiple of 16
    }
  }
  store_tile<T, Epi::kI32Bias>(acc, r0, c0, rows, cols, nullptr, nullptr, nullptr, out, ldo);
}

// Large W4A8 / BitNet problems on producer/consumer workgroups
// (mainloop_ws): four consumer waves only read fragments and issue MFMAs;
// four producer waves copy the int8 activation rows by LDS DMA and load,
// decode and store the packed weight rows as int8. The activations are the
// tile's A side (rows m), the weights its B side (rows n). For W4A8 (output
// [N, M]) the MFMA operands are swapped so that a lane holds one weight row n
// and four consecutive activation rows m per register group, four adjacent
// int32 of the output; BitNet's output is [M, N], the usual lane layout.
using TWs = mp::Tile<256, 192, 2, 2>;  // consumers of 128 x 96

template <class T, bool kBitNet, bool kX16 = false>
__global__ __launch_bounds__(T::NT_WS, 1) void lowbit_ws_kernel(const int8_t* __restrict__ act, int64_t ld_act, int M,
                                                                const uint8_t* __restrict__ wq, int64_t ld_w, int N,
                                                                int K, int32_t* __restrict__ out, int64_t ldo,
                                                                int mblocks) {
  __shared__ __attribute__((aligned(16))) char buf0[T::STAGE_BYTES];
  __shared__ __attribute__((aligned(16))) char buf1[T::STAGE_BYTES];
  char* const bufs[2] = {buf0, buf1};
  // Plain m-fastest order: the XCD-grouped order (grid_tile) measured 0.7% slower here.
  const int m0 = (blockIdx.x % mblocks) * T::BM;
  const int n0 = (blockIdx.x / mblocks) * T::BN;
  const int pw = T::wave() % T::NW;
  mp::DmaRowsOperand<T::BM, mp::DenseRows, T::NW> aop;
  aop.init(mp::DenseRows{act, ld_act, M}, m0, pw);
  constexpr mp::LowBit kFmt =
      kBitNet ? mp::LowBit::kInt2 : (kX16 ? mp::LowBit::kSignedNibbleX16 : mp::LowBit::kSignedNibble);
  mp::LowBitRowsOperand<T::BN, kFmt, T::NW> bop;
  bop.init(wq, ld_w, N, n0, pw);
  i32x16 acc[T::TI][T::TJ];
  if (!mp::mainloop_ws<T, mp::I8Math, 2, mp::DenseRows, decltype(bop), !kBitNet>(aop, bop, K / mp::ROWB, bufs, acc))
    return;
  if constexpr (kX16) {
#pragma unroll
    for (int i = 0; i < T::TI; ++i)
#pragma unroll
      for (int j = 0; j < T::TJ; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[i][j][e] >>= 4;  // exact: every product is a multiple of 16
  }
  if constexpr (kBitNet) {
    store_tile<T, Epi::kI32Bias>(acc, m0, n0, M, N, nullptr, nullptr, nullptr, out, ldo);
    return;
  }
  // acc[i][j][4g + c]: n = col j, lane % 32; m = row block i, 8g + 4h + c.
  const int lane = threadIdx.x & 63;
  const bool vec = (ldo & 3) == 0 && (((uintptr_t)out) & 15) == 0;
  // Through LDS: after the main loop's last barrier the stage buffer of
  // stage nk - 2 (none, for nk = 1) is neither read nor written again (the
  // producers drained their DMA before it and issue nothing after it). Each
  // consumer wave passes 32 n x 64 m blocks through a private part of it
  // (rows padded by 16 bytes: the 16-byte writes of 16 rows fall in distinct
  // bank groups) and stores 256-byte row segments, where the register layout
  // stores 32 bytes of each of 32 rows per instruction.
  constexpr int RS = 64 * 4 + 16;
  if constexpr (T::TI % 2 == 0 && T::NW * 32 * RS <= T::STAGE_BYTES) {
    char* blk = (((K / mp::ROWB) & 1) ? buf1 : buf0) + T::wave() * 32 * RS;
#pragma unroll
    for (int j = 0; j < T::TJ; ++j)
#pragma unroll
      for (int ih = 0; ih < T::TI / 2; ++ih) {
#pragma unroll
        for (int i2 = 0; i2 < 2; ++i2)
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const int i = 2 * ih + i2;
            *reinterpret_cast<i32x4*>(blk + (lane & 31) * RS + (i2 * 32 + g * 8 + (lane >> 5) * 4) * 4) =
                i32x4{acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]};
          }
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          const int p = q * 64 + lane, r = p / 16, c = (p % 16) * 4;
          const i32x4 v = *reinterpret_cast<const i32x4*>(blk + r * RS + c * 4);
          const int n = n0 + T::wave_n() * T::WTN + j * 32 + r;
          const int m = m0 + T::wave_m() * T::WTM + ih * 64 + c;
          if (n >= N) continue;
          int32_t* dst = out + (int64_t)n * ldo + m;
          if (vec && m + 3 < M) {
            *reinterpret_cast<i32x4*>(dst) = v;
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (m + e < M) dst[e] = v[e];
          }
        }
      }
    return;
  }
#pragma unroll
  for (int j = 0; j < T::TJ; ++j) {
    const int n = n0 + T::wave_n() * T::WTN + j * 32 + (lane & 31);
    if (n >= N) continue;
    int32_t* row = out + (int64_t)n * ldo;
#pragma unroll
    for (int i = 0; i < T::TI; ++i)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int m = m0 + T::wave_m() * T::WTM + i * 32 + g * 8 + (lane >> 5) * 4;
        if (vec && m + 3 < M) {
          *reinterpret_cast<i32x4*>(row + m) =
              i32x4{acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]};
        } else {
#pragma unroll
          for (int c = 0; c < 4; ++c)
            if (m + c < M) row[m + c] = acc[i][j][4 * g + c];
        }
      }
  }
}

int check_i8(const int8_t* a, int64_t M, int64_t K, int64_t a_ld, const int8_t* w, int64_t N, int64_t w_ld,
             const void* out, int64_t out_ld) {
  INTENT_REQUIRE(M >= 0 && N >= 0 && K >= 0, INTENT_ERR_INVALID_ARGUMENT, "negative extent");
  INTENT_REQUIRE(M <= INT32_MAX && N <= INT32_MAX && K <= INT32_MAX, INTENT_ERR_UNSUPPORTED, "extent exceeds int32");
  if (M == 0 || N == 0) return INTENT_OK;
  // an empty K reads no operand (the generic kernel applies the epilogue to zero)
  INTENT_REQUIRE(out && (K == 0 || (a && w)), INTENT_ERR_INVALID_ARGUMENT, "null pointer argument");
  INTENT_REQUIRE(a_ld >= K && w_ld >= K && out_ld >= N, INTENT_ERR_INVALID_ARGUMENT,
                 "leading stride smaller than the row");
  return INTENT_OK;
}

// The tiled kernels take whole 64-k stages of 16-byte aligned rows.
bool i8_fast(const int8_t* a, int64_t K, int64_t a_ld, const int8_t* w, int64_t w_ld) {
  return K > 0 && K % 64 == 0 && intent::aligned16(a) && intent::aligned16(w) && a_ld % 16 == 0 && w_ld % 16 == 0;
}

template <class T, Epi E>
int launch_tile(const int8_t* a, int64_t M, int64_t K, int64_t a_ld, const float* sa, const int8_t* w, int64_t N,
                int64_t w_ld, const float* sw, const int32_t* bias, void* out, int64_t out_ld, void* stream,
                const char* name) {
  const int mblocks = (int)((M + T::BM - 1) / T::BM);
  const int nblocks = (int)((N + T::BN - 1) / T::BN);
  const int64_t grid = (int64_t)mblocks * nblocks;
  INTENT_REQUIRE(grid < (1ll << 31), INTENT_ERR_UNSUPPORTED, "%s: grid too large", name);
  INTENT_REQUIRE(intent::fits_offset(M, a_ld) && intent::fits_offset(N, w_ld), INTENT_ERR_UNSUPPORTED,
                 "%s: operand too large for 31-bit buffer offsets", name);
  if (K % mp::ROWB == 0)
    hipLaunchKernelGGL((i8_gemm_kernel<T, E, false>), dim3((unsigned)grid), dim3(T::NT), 0,
                       (hipStream_t)stream, a, a_ld, (int)M, w, w_ld, (int)N, (int)K, sa, sw, bias, out, out_ld, mblocks);
  else
    hipLaunchKernelGGL((i8_gemm_kernel<T, E, true>), dim3((unsigned)grid), dim3(T::NT), 0,
                       (hipStream_t)stream, a, a_ld, (int)M, w, w_ld, (int)N, (int)K, sa, sw, bias, out, out_ld, mblocks);
  return intent::launch_status(name);
}

// 256 x 256 tiles once the problem has enough of them to fill the chip.
template <Epi E>
int launch_i8(const int8_t* a, int64_t M, int64_t K, int64_t a_ld, const float* sa, const int8_t* w, int64_t N,
              int64_t w_ld, const float* sw, const int32_t* bias, void* out, int64_t out_ld, void* stream,
              const char* name) {
  const int64_t big = ((M + 255) / 256) * ((N + 255) / 256);
  if (big >= 256)
    return launch_tile<T256, E>(a, M, K, a_ld, sa, w, N, w_ld, sw, bias, out, out_ld, stream, name);
  return launch_tile<T128, E>(a, M, K, a_ld, sa, w, N, w_ld, sw, bias, out, out_ld, stream, name);
}

}  // namespace

extern "C" int intent_w8a8_gemm(const int8_t* a, int64_t M, int64_t K, int64_t a_ld, const float* a_scales,
                                const int8_t* w, int64_t N, int64_t w_ld, const float* w_scales, void* out,
                                int64_t out_ld, void* stream) {
  intent::clear_error();
  int st = check_i8(a, M, K, a_ld, w, N, w_ld, out, out_ld);
  if (st != INTENT_OK || M == 0 || N == 0) return st;
  INTENT_REQUIRE(a_scales && w_scales, INTENT_ERR_INVALID_ARGUMENT, "null scale pointer");
  if (!i8_fast(a, K, a_ld, w, w_ld))
    return intent::i8_generic_launch(a, M, K, a_ld, w, N, w_ld, a_scales, w_scales, nullptr, out, out_ld, true,
                                     stream);
  return launch_i8<Epi::kBf16Scaled>(a, M, K, a_ld, a_scales, w, N, w_ld, w_scales, nullptr, out, out_ld, stream,
                                     "w8a8_gemm");
}

extern "C" int intent_i8_gemm_i32(const int8_t* a, int64_t M, int64_t K, int64_t a_ld, const int8_t* w, int64_t N,
                                  int64_t w_ld, const int32_t* bias, int32_t* c, int64_t c_ld, void* stream) {
  intent::clear_error();
  int st = check_i8(a, M, K, a_ld, w, N, w_ld, c, c_ld);
  if (st != INTENT_OK || M == 0 || N == 0) return st;
  if (!i8_fast(a, K, a_ld, w, w_ld))
    return intent::i8_generic_launch(a, M, K, a_ld, w, N, w_ld, nullptr, nullptr, bias, c, c_ld, false, stream);
  return launch_i8<Epi::kI32Bias>(a, M, K, a_ld, nullptr, w, N, w_ld, nullptr, bias, c, c_ld, stream, "i8_gemm_i32");
}

namespace {

template <class T, bool kBitNet>
int launch_lowbit(const int8_t* a, int64_t M, int64_t K, int64_t a_ld, const uint8_t* w, int64_t N, int64_t w_ld,
                  int32_t* out, int64_t out_ld, void* stream, const char* name) {
  const int64_t rows = kBitNet ? M : N, cols = kBitNet ? N : M;
  const int mblocks = (int)((rows + T::BM - 1) / T::BM);
  const int64_t grid = (int64_t)mblocks * ((cols + T::BN - 1) / T::BN);
  INTENT_REQUIRE(grid < (1ll << 31), INTENT_ERR_UNSUPPORTED, "%s: grid too large", name);
  if (!kBitNet && K <= mp::kX16MaxK)
    hipLaunchKernelGGL((lowbit_gemm_kernel<T, kBitNet, true>), dim3((unsigned)grid), dim3(T::NT), 0,
                       (hipStream_t)stream, a, a_ld, (int)M, w, w_ld, (int)N, (int)K, out, out_ld, mblocks);
  else
    hipLaunchKernelGGL((lowbit_gemm_kernel<T, kBitNet>), dim3((unsigned)grid), dim3(T::NT), 0, (hipStream_t)stream,
                       a, a_ld, (int)M, w, w_ld, (int)N, (int)K, out, out_ld, mblocks);
  return intent::launch_status(name);
}

template <bool kBitNet>
int lowbit_entry(const int8_t* a, int64_t M, int64_t K, int64_t a_ld, const uint8_t* w, int64_t N, int64_t w_ld,
                 int32_t* out, int64_t out_ld, void* stream, const char* name) {
  intent::clear_error();
  const int per_byte = kBitNet ? 4 : 2;
  const int align = kBitNet ? 4 : 8;
  INTENT_REQUIRE(M >= 0 && N >= 0 && K >= 0 && M <= INT32_MAX && N <= INT32_MAX && K <= INT32_MAX,
                 INTENT_ERR_INVALID_ARGUMENT, "%s: bad extents", name);
  INTENT_REQUIRE(K % 128 == 0, INTENT_ERR_UNSUPPORTED, "%s: K must be a multiple of 128, got %lld", name,
                 (long long)K);
  if (M == 0 || N == 0) return INTENT_OK;
  INTENT_REQUIRE(out, INTENT_ERR_INVALID_ARGUMENT, "%s: null output", name);
  INTENT_REQUIRE(a_ld >= K && w_ld >= K / per_byte && out_ld >= (kBitNet ? N : M), INTENT_ERR_INVALID_ARGUMENT,
                 "%s: leading stride smaller than the row", name);
  // empty K: int32 zeros ([N, M] for W4A8, [M, N] for BitNet)
  if (K == 0) return intent::fill_launch(out, kBitNet ? M : N, kBitNet ? N : M, out_ld, 4, 0u, stream);
  INTENT_REQUIRE(a && w, INTENT_ERR_INVALID_ARGUMENT, "%s: null pointer argument", name);
  INTENT_REQUIRE(intent::aligned16(a) && a_ld % 16 == 0 && (reinterpret_cast<uintptr_t>(w) % align) == 0 &&
                     w_ld % align == 0,
                 INTENT_ERR_ALIGNMENT, "%s: activations 16-byte aligned rows, packed weights %d-byte aligned rows",
                 name, align);
  INTENT_REQUIRE(intent::fits_offset(M, a_ld) && intent::fits_offset(N, w_ld), INTENT_ERR_UNSUPPORTED,
                 "%s: operand too large for 31-bit buffer offsets", name);
  const int64_t big = ((M + 255) / 256) * ((N + 255) / 256);
  if (big >= 256) {
    const int mblocks = (int)((M + TWs::BM - 1) / TWs::BM);
    const int64_t grid = (int64_t)mblocks * ((N + TWs::BN - 1) / TWs::BN);
    INTENT_REQUIRE(grid < (1ll << 31), INTENT_ERR_UNSUPPORTED, "%s: grid too large", name);
    if (!kBitNet && K <= mp::kX16MaxK)
      hipLaunchKernelGGL((lowbit_ws_kernel<TWs, kBitNet, true>), dim3((unsigned)grid), dim3(TWs::NT_WS), 0,
                         (hipStream_t)stream, a, a_ld, (int)M, w, w_ld, (int)N, (int)K, out, out_ld, mblocks);
    else
      hipLaunchKernelGGL((lowbit_ws_kernel<TWs, kBitNet>), dim3((unsigned)grid), dim3(TWs::NT_WS), 0,
                         (hipStream_t)stream, a, a_ld, (int)M, w, w_ld, (int)N, (int)K, out, out_ld, mblocks);
    return intent::launch_status(name);
  }
  return launch_lowbit<T128, kBitNet>(a, M, K, a_ld, w, N, w_ld, out, out_ld, stream, name);
}

}  // namespace

extern "C" int intent_w4a8_gemm(const int8_t* a, int64_t M, int64_t K, int64_t a_ld, const uint8_t* w_packed,
                                int64_t N, int64_t w_ld, int32_t* out, int64_t out_ld, void* stream) {
  return lowbit_entry<false>(a, M, K, a_ld, w_packed, N, w_ld, out, out_ld, stream, "w4a8_gemm");
}

extern "C" int intent_bitnet_int2_gemm(const int8_t* a, int64_t M, int64_t K, int64_t a_ld, const uint8_t* w_packed,
                                       int64_t N, int64_t w_ld, int32_t* out, int64_t out_ld, void* stream) {
  return lowbit_entry<true>(a, M, K, a_ld, w_packed, N, w_ld, out, out_ld, stream, "bitnet_int2_gemm");
}
