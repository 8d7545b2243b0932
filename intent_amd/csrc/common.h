// Shared device helpers for the gfx950 quantized-contraction kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

typedef _Float16 f16;
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

#define INTENT_DEVICE __device__ __forceinline__

template <typename To, typename From>
INTENT_DEVICE To bit_cast(From v) {
  static_assert(sizeof(To) == sizeof(From), "bit_cast size");
  return __builtin_bit_cast(To, v);
}

// Buffer resource over [base, base + 2 GiB): raw buffer loads then take a
// 32-bit lane offset plus a wave-uniform offset.
INTENT_DEVICE __amdgpu_buffer_rsrc_t make_rsrc(const void* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, 0x7fffffff, 0x00020000);
}

// 16-byte global load (global_load_dwordx4).
INTENT_DEVICE u32x4 load16(const void* p) { return *reinterpret_cast<const u32x4*>(p); }
INTENT_DEVICE void store16(void* p, u32x4 v) { *reinterpret_cast<u32x4*>(p) = v; }

// v_bfi_b32: (mask & a) | (~mask & b).
// The compiler matches this pattern (no inline asm, so no hazard padding).
INTENT_DEVICE uint32_t bfi(uint32_t mask, uint32_t a, uint32_t b) { return (mask & a) | (~mask & b); }

// f16 value with bit pattern 0x6400 | q equals 1024 + q for q in 0..1023.
// Subtracting (1024 + z) is exact for nibbles, so (q - z) comes out exact in
// f16 and one packed multiply applies the group scale.
//
// dequant8: one dword holds 8 nibbles (byte b: k = 2b low, k = 2b+1 high);
// returns the 8 dequantized weights in natural k order as f16x8.
INTENT_DEVICE f16x8 dequant8(uint32_t w, f16x2 zoff, f16x2 scale) {
  const uint32_t w4 = w >> 4;
  // v_perm_b32: selector bytes 0-3 pick bytes of the second operand, 4-7 of
  // the first, 0x0c yields zero. Pair b = (low nibble of byte b, high nibble).
  uint32_t p0 = __builtin_amdgcn_perm(w4, w, 0x0c040c00u);
  uint32_t p1 = __builtin_amdgcn_perm(w4, w, 0x0c050c01u);
  uint32_t p2 = __builtin_amdgcn_perm(w4, w, 0x0c060c02u);
  uint32_t p3 = __builtin_amdgcn_perm(w4, w, 0x0c070c03u);
  // (p & 0x000F000F) | 0x64006400 as one v_bfi_b32 (bitfield select); the
  // magic word sits in a register the compiler cannot fold back into a literal.
  uint32_t magic = 0x64006400u;
  asm("" : "+v"(magic));
  p0 = bfi(0x000F000Fu, p0, magic);
  p1 = bfi(0x000F000Fu, p1, magic);
  p2 = bfi(0x000F000Fu, p2, magic);
  p3 = bfi(0x000F000Fu, p3, magic);
  f16x2 h0 = (bit_cast<f16x2>(p0) - zoff) * scale;
  f16x2 h1 = (bit_cast<f16x2>(p1) - zoff) * scale;
  f16x2 h2 = (bit_cast<f16x2>(p2) - zoff) * scale;
  f16x2 h3 = (bit_cast<f16x2>(p3) - zoff) * scale;
  f16x8 r;
  r[0] = h0[0]; r[1] = h0[1]; r[2] = h1[0]; r[3] = h1[1];
  r[4] = h2[0]; r[5] = h2[1]; r[6] = h3[0]; r[7] = h3[1];
  return r;
}

// Four signed int8 lanes of a dword -> f16 (exact), times a per-row scale of 1.
INTENT_DEVICE f16x8 int8x8_to_f16(uint32_t lo, uint32_t hi) {
  f16x8 r;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    r[i] = (f16)(float)(int8_t)(lo >> (8 * i));
    r[4 + i] = (f16)(float)(int8_t)(hi >> (8 * i));
  }
  return r;
}

INTENT_DEVICE f16x2 splat2(f16 v) {
  f16x2 r;
  r[0] = v;
  r[1] = v;
  return r;
}

// fp32 -> bf16, round to nearest even; NaN -> quiet NaN.
INTENT_DEVICE uint16_t f32_to_bf16_rne(float f) {
  uint32_t u = bit_cast<uint32_t>(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

// Two f32 -> bf16 conversions in one v_cvt_pk_bf16_f32 (round to nearest
// even; a NaN stays a NaN): lo in bits 0..15, hi in 16..31. Pinned against
// f32_to_bf16_rne bit for bit by the W8A8 special-value test.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
INTENT_DEVICE uint32_t bf16x2_rne(float lo, float hi) {
  return bit_cast<uint32_t>(__builtin_convertvector(f32x2{lo, hi}, bf16x2_t));
}

// Workgroups are dispatched round-robin over the 8 XCDs (blockIdx % 8 picks
// the XCD). Renumber so that consecutive logical tiles land on one XCD and
// share its L2. Tiles beyond the last full group of 8 keep their id.
INTENT_DEVICE int xcd_swizzle(int bid, int nblocks) {
  const int full = nblocks & ~7;
  if (bid >= full) return bid;
  const int per_xcd = full >> 3;
  return (bid & 7) * per_xcd + (bid >> 3);
}

// Tile (row block, column block) of logical tile id bid, in groups of gm row
// blocks: inside a group the row block varies fastest. After xcd_swizzle an
// XCD's co-resident workgroups hold consecutive ids, so with gm = 4 the 32 of
// a round cover 4 row blocks x 8 column blocks, and the operand blocks they
// stream at one time fit its L2 (row-block-fastest over 16 row blocks would
// stream a column block's whole left operand through every XCD).
INTENT_DEVICE void grouped_tile(int bid, int mblocks, int nblocks, int gm, int& mb, int& nb) {
  const int group = bid / (gm * nblocks);
  const int first = group * gm;
  const int rows = mblocks - first < gm ? mblocks - first : gm;
  const int local = bid - group * gm * nblocks;
  mb = first + local % rows;
  nb = local / rows;
}

// This workgroup's tile in a grid of mblocks x (gridDim.x / mblocks) tiles:
// xcd_swizzle, then groups of gm row blocks (grouped_tile).
INTENT_DEVICE void grid_tile(int mblocks, int gm, int& mb, int& nb) {
  grouped_tile(xcd_swizzle(blockIdx.x, gridDim.x), mblocks, (int)gridDim.x / mblocks, gm, mb, nb);
}

// f32 -> E4M3FN bits, round half to even; |f| >= 448 saturates to 448 (inputs
// past the format's range are outside the cast's contract), NaN -> NaN.
INTENT_DEVICE uint32_t f32_to_e4m3fn(float f) {
  const uint32_t u = bit_cast<uint32_t>(f);
  const uint32_t sign = (u >> 24) & 0x80u;
  const uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return sign | 0x7fu;
  const float mag = bit_cast<float>(a);
  if (mag >= 448.0f) return sign | 0x7eu;
  if (mag < 0.015625f) return sign | (uint32_t)rintf(mag * 512.0f);  // subnormal step 2^-9
  const uint32_t r = a + 0x7ffffu + ((a >> 20) & 1u);
  return sign | ((((r >> 23) - 120u) << 3) | ((r >> 20) & 7u));
}

// f32 -> E5M2 bits, round half to even; finite overflow gives infinity
// (0x7C), NaN -> 0x7F. Subnormal step 2^-16, smallest normal 2^-14.
INTENT_DEVICE uint32_t f32_to_e5m2(float f) {
  const uint32_t u = bit_cast<uint32_t>(f);
  const uint32_t sign = (u >> 24) & 0x80u;
  const uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return sign | 0x7fu;
  if (a == 0x7f800000u) return sign | 0x7cu;
  const float mag = bit_cast<float>(a);
  if (mag < 6.103515625e-05f) return sign | (uint32_t)rintf(mag * 65536.0f);
  const uint32_t r = a + 0xfffffu + ((a >> 21) & 1u);
  const uint32_t e = (r >> 23) - 112u;
  return e >= 31u ? sign | 0x7cu : sign | (e << 2) | ((r >> 21) & 3u);
}

// ---- wave-wide reduction of V per-lane partial sums (no LDS) -----------------
// Reduce-scatter over the 64 lanes: v_permlane32_swap pairs value i with
// value i + V/2 across the two half-waves, v_permlane16_swap does the same
// across 16-lane rows, DPP row rotations finish inside each row. Afterwards
// every lane of row R (lanes 16R..16R+15) holds the wave totals of the values
// listed by wave_reduce_index(R, j), j < V / 4 (for V < 4 a row holds all V).
// The summation order is fixed, so results are deterministic.
template <int CTRL>
INTENT_DEVICE float dpp_f32(float v) {
  return bit_cast<float>(__builtin_amdgcn_update_dpp(0u, bit_cast<uint32_t>(v), CTRL, 0xf, 0xf, false));
}
template <int V>
struct WaveReduce {
  static constexpr int S32 = V >= 2 && V % 2 == 0;           // stage 1 scatters
  static constexpr int V1 = S32 ? V / 2 : V;
  static constexpr int S16 = V1 >= 2 && V1 % 2 == 0;         // stage 2 scatters
  static constexpr int OUT = S16 ? V1 / 2 : V1;              // values left per lane
  // Original index of output j in row R.
  INTENT_DEVICE static constexpr int index(int R, int j) {
    const int h = R >> 1, rr = R & 1;
    const int j1 = S16 ? j + rr * OUT : j;
    return S32 ? j1 + h * V1 : j1;
  }
  INTENT_DEVICE static void run(const float (&in)[V], float (&out)[OUT]) {
    float a[V1];
#pragma unroll
    for (int i = 0; i < V1; ++i) {
      const uint32_t x = bit_cast<uint32_t>(in[i]);
      const uint32_t y = bit_cast<uint32_t>(S32 ? in[i + V1] : in[i]);
      const auto r = __builtin_amdgcn_permlane32_swap(x, y, false, false);
      a[i] = bit_cast<float>(r[0]) + bit_cast<float>(r[1]);
    }
#pragma unroll
    for (int i = 0; i < OUT; ++i) {
      const uint32_t x = bit_cast<uint32_t>(a[i]);
      const uint32_t y = bit_cast<uint32_t>(S16 ? a[i + OUT] : a[i]);
      const auto r = __builtin_amdgcn_permlane16_swap(x, y, false, false);
      float s = bit_cast<float>(r[0]) + bit_cast<float>(r[1]);
      s += dpp_f32<0x128>(s);  // row_ror:8
      s += dpp_f32<0x124>(s);  // row_ror:4
      s += dpp_f32<0x4E>(s);   // quad_perm [2,3,0,1]
      s += dpp_f32<0xB1>(s);   // quad_perm [1,0,3,2]
      out[i] = s;
    }
  }
};
