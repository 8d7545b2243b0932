// Grouped f16 / bf16 GEMMs with [G][K][N] weights read in place (no
// transposed copy): the kernel shared by the ragged grouped GEMMs
// (grouped_kn.hip) and the reference's f16 MoE expert FFN (moe_ffn.hip).
// The two live in separate translation units: with both sets of kernel
// instances in one, hipcc's host pass failed to match mainloop_kn for the
// last one.
//
// Row groups: group g owns rows offsets[g] .. offsets[g+1] (of x, or of the
// member list of a ragged routing). The grid holds ceil(rows / BM) + G row
// tiles (an upper bound of sum_g ceil(count_g / BM)) times the column tiles;
// a workgroup finds its (group, first row) by walking the offsets and exits
// if its index is past the last tile, so no launch is sized for the worst
// case of every row in every group.
#pragma once

#include <type_traits>

#include "common.h"
#include "internal.h"
#include "mfma_pipe.h"

namespace gkn {

using GTile = mp::Tile<256, 256, 2, 4>;  // the dense [K, N] tile (eight waves of 128 x 64)

// Row tile x of the grouped problem: group and first row, or g = -1 past the last tile.
struct GroupTile {
  int g;
  int start;
  int end;
};

// Offsets are clamped to [0, rows]: malformed routing never reaches memory
// outside the operands.
INTENT_DEVICE int clampi(int v, int lo, int hi) { return v < lo ? lo : v > hi ? hi : v; }

INTENT_DEVICE GroupTile find_tile(const int32_t* __restrict__ offsets, int G, int rows, int x, int BM) {
  int lo = clampi(offsets[0], 0, rows);
  for (int g = 0; g < G; ++g) {
    const int hi = clampi(offsets[g + 1], lo, rows);
    const int nb = hi > lo ? (hi - lo + BM - 1) / BM : 0;
    if (x < nb) return GroupTile{g, lo + x * BM, hi};
    x -= nb;
    lo = hi;
  }
  return GroupTile{-1, 0, 0};
}

// Tile rows of the MoE FFN's first projection: member index i = m0 + p is
// route member_routes[i], which reads token route_token[route] of x. Rows
// past the group repeat its last member (never stored).
struct MemberTokenRows {
  const void* base;
  int64_t ld_bytes;
  const int32_t* members;
  const int32_t* route_token;
  int end;
  int nroutes;
  int ntokens;
  INTENT_DEVICE const void* tile_base(int) const { return base; }
  INTENT_DEVICE uint32_t off(int m0, int p) const {
    const int i = m0 + p < end ? m0 + p : end - 1;
    const int r = clampi(members[i], 0, nroutes - 1);
    return (uint32_t)(clampi(route_token[r], 0, ntokens - 1) * ld_bytes);
  }
};

enum class GEpi {
  kStore16,      // out16[row] = f16 / bf16(acc)                         (ragged_grouped_gemm)
  kReluF16,      // out16[row] = f16(max(acc, 0))                        (MoE first projection)
  kRouteWeight,  // out32[row] = route_weights[members[row]] * acc (f32) (MoE second projection)
};

// The epilogue through LDS: after a workgroup barrier (the stage buffers are
// then free) each wave passes its 32-row blocks one at a time through a
// private LDS block (rows of WTN outputs plus 16 bytes of padding, so the
// writes of 16 rows fall in distinct bank groups) and stores whole row
// segments (WTN outputs) per row, where the register layout would store 8 or
// 16 bytes of each of 32 rows per instruction. lds0 / lds1: the two stage
// buffers; waves NW/2.. use lds1 when one buffer cannot hold all waves.
template <class T, GEpi E, bool kBf16>
INTENT_DEVICE void grouped_store_lds(const f32x16 (&acc)[T::TI][T::TJ], char* lds0, char* lds1,
                                     const GroupTile& tile, int n0, int N, const int32_t* __restrict__ members,
                                     int nroutes, const float* __restrict__ route_weights, void* __restrict__ out,
                                     int64_t ldo) {
  constexpr int EB = E == GEpi::kRouteWeight ? 4 : 2;  // output bytes
  constexpr int RS = T::WTN * EB + 16;                  // LDS row bytes
  constexpr int CH = T::WTN * EB / 16;                  // 16-byte pieces per row
  constexpr int PE = 16 / EB;                           // outputs per piece
  constexpr int NP = 32 * CH / 64;                      // pieces per lane and block
  static_assert(NP * 64 == 32 * CH, "whole pieces per lane");
  constexpr bool kOne = T::NW * 32 * RS <= T::STAGE_BYTES;
  static_assert(kOne || (T::NW / 2) * 32 * RS <= T::STAGE_BYTES, "wave blocks fit the stage buffers");
  const int lane = threadIdx.x & 63;
  const int wv = T::wave();
  char* blk = kOne ? lds0 + wv * 32 * RS : (wv < T::NW / 2 ? lds0 + wv * 32 * RS : lds1 + (wv - T::NW / 2) * 32 * RS);
  const int wn = n0 + T::wave_n() * T::WTN;
  const bool vec = ((ldo * EB) & 15) == 0 && (((uintptr_t)out) & 15) == 0;
  __syncthreads();  // every wave is done with the stage buffers
#pragma unroll
  for (int i = 0; i < T::TI; ++i) {
    const int rb = tile.start + T::wave_m() * T::WTM + i * 32;
    if (rb >= tile.end) break;  // wave-uniform
    const int row = rb + (lane & 31);
    float rw = 1.f;
    if constexpr (E == GEpi::kRouteWeight)
      rw = row < tile.end ? route_weights[clampi(members[row], 0, nroutes - 1)] : 0.f;
#pragma unroll
    for (int j = 0; j < T::TJ; ++j)
#pragma unroll
      for (int gq = 0; gq < 4; ++gq) {
        char* dst = blk + (lane & 31) * RS + (T::col(j, gq) - T::wave_n() * T::WTN) * EB;
        if constexpr (E == GEpi::kRouteWeight) {
          *reinterpret_cast<f32x4*>(dst) =
              f32x4{__fmul_rn(rw, acc[i][j][4 * gq]), __fmul_rn(rw, acc[i][j][4 * gq + 1]),
                    __fmul_rn(rw, acc[i][j][4 * gq + 2]), __fmul_rn(rw, acc[i][j][4 * gq + 3])};
        } else {
          uint32_t h[4];
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            float v = acc[i][j][4 * gq + c];
            if constexpr (E == GEpi::kReluF16) v = v < 0.f ? 0.f : v;  // NaN stays NaN
            h[c] = kBf16 ? f32_to_bf16_rne(v) : bit_cast<uint16_t>((f16)v);
          }
          *reinterpret_cast<u32x2*>(dst) = u32x2{h[0] | (h[1] << 16), h[2] | (h[3] << 16)};
        }
      }
#pragma unroll
    for (int q = 0; q < NP; ++q) {
      const int p = q * 64 + lane, r = p / CH, c = (p % CH) * PE;
      const u32x4 v = *reinterpret_cast<const u32x4*>(blk + r * RS + c * EB);
      const int gm = rb + r;
      if (gm >= tile.end) continue;
      const int n = wn + c;
      char* o = reinterpret_cast<char*>(out) + ((int64_t)gm * ldo + n) * EB;
      if (vec && n + PE - 1 < N) {
        *reinterpret_cast<u32x4*>(o) = v;
      } else {
#pragma unroll
        for (int e = 0; e < PE; ++e) {
          if (n + e >= N) continue;
          if constexpr (EB == 4)
            reinterpret_cast<uint32_t*>(o)[e] = v[e];
          else
            reinterpret_cast<uint16_t*>(o)[e] = (uint16_t)(v[e >> 1] >> (16 * (e & 1)));
        }
      }
    }
  }
}

template <class T, class Math, bool kGather, GEpi E>
__global__ __launch_bounds__(T::NT, 1) void grouped_kn_kernel(
    const uint16_t* __restrict__ x, int64_t ldx, const int32_t* __restrict__ offsets, int G, int rows,
    const int32_t* __restrict__ members, const int32_t* __restrict__ route_token, int nroutes, int ntokens,
    const float* __restrict__ route_weights, const uint16_t* __restrict__ w, int64_t ldw, int64_t gstride, int N, int K,
    int ntiles, void* __restrict__ out, int64_t ldo) {
  __shared__ __attribute__((aligned(16))) char buf0[T::STAGE_BYTES];
  __shared__ __attribute__((aligned(16))) char buf1[T::STAGE_BYTES];
  const int bid = xcd_swizzle(blockIdx.x, gridDim.x);
  const GroupTile tile = find_tile(offsets, G, rows, bid % ntiles, T::BM);
  if (tile.g < 0) return;  // workgroup-uniform
  const int n0 = (bid / ntiles) * T::BN;
  const int wave = T::wave();
  mp::DmaKNOperand<T::BN, T::NW> bop;
  bop.init(w + tile.g * gstride + n0, ldw, N - n0, wave);
  using Rows = typename std::conditional<kGather, MemberTokenRows, mp::DenseRows>::type;
  Rows rows_src;
  if constexpr (kGather)
    rows_src = MemberTokenRows{x, ldx * 2, members, route_token, tile.end, nroutes, ntokens};
  else
    rows_src = mp::DenseRows{x, ldx * 2, tile.end};
  mp::DmaRowsOperand<T::BM, Rows, T::NW> aop;
  aop.init(rows_src, tile.start, wave);
  f32x16 acc[T::TI][T::TJ];
  mp::mainloop_kn<T, Math, mp::DmaRowsOperand<T::BM, Rows, T::NW>, mp::DmaKNOperand<T::BN, T::NW>, true>(
      aop, bop, K / 64, buf0, buf1, acc);
  constexpr bool kBf16 = std::is_same<Math, mp::BF16Math>::value;
  grouped_store_lds<T, E, kBf16>(acc, buf0, buf1, tile, n0, N, members, nroutes, route_weights, out, ldo);
}

inline int kn_shape_check(int64_t K, int64_t N, int64_t w_ld, const void* w, const char* what) {
  INTENT_REQUIRE(K % 64 == 0 && K > 0, INTENT_ERR_UNSUPPORTED, "%s: K must be a positive multiple of 64, got %lld",
                 what, (long long)K);
  INTENT_REQUIRE(N % 8 == 0 && w_ld % 8 == 0, INTENT_ERR_UNSUPPORTED,
                 "%s: N and the weight row stride must be multiples of 8 (N=%lld, ld=%lld)", what, (long long)N,
                 (long long)w_ld);
  INTENT_REQUIRE(w_ld >= N, INTENT_ERR_INVALID_ARGUMENT, "%s: weight row stride smaller than N", what);
  INTENT_REQUIRE(intent::aligned16(w), INTENT_ERR_ALIGNMENT, "%s: weights must be 16-byte aligned", what);
  INTENT_REQUIRE(intent::fits_offset(K, w_ld * 2), INTENT_ERR_UNSUPPORTED,
                 "%s: one group's weights exceed 31-bit buffer offsets", what);
  return INTENT_OK;
}

template <class Math, bool kGather, GEpi E>
inline void launch_grouped(const void* x, int64_t x_ld, const int32_t* offsets, int64_t G, int64_t rows,
                    const int32_t* members, const int32_t* route_token, int64_t nroutes, int64_t ntokens,
                    const float* route_weights, const void* w, int64_t w_ld, int64_t gstride, int64_t N, int64_t K,
                    int ntiles, void* out, int64_t out_ld, hipStream_t st) {
  using T = GTile;
  const int64_t grid = (int64_t)ntiles * ((N + T::BN - 1) / T::BN);
  hipLaunchKernelGGL((grouped_kn_kernel<T, Math, kGather, E>), dim3((unsigned)grid), dim3(T::NT), 0, st,
                     (const uint16_t*)x, x_ld, offsets, (int)G, (int)rows, members, route_token, (int)nroutes,
                     (int)ntokens, route_weights, (const uint16_t*)w, w_ld, gstride, (int)N, (int)K, ntiles, out,
                     out_ld);
}

}  // namespace gkn
