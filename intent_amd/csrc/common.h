// Shared device helpers for the gfx950 quantized-contraction kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

typedef _Float16 f16;
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
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

// 16-byte global load (global_load_dwordx4).
INTENT_DEVICE u32x4 load16(const void* p) { return *reinterpret_cast<const u32x4*>(p); }
INTENT_DEVICE void store16(void* p, u32x4 v) { *reinterpret_cast<u32x4*>(p) = v; }

// v_bfi_b32: (mask & a) | (~mask & b).
INTENT_DEVICE uint32_t bfi(uint32_t mask, uint32_t a, uint32_t b) {
  uint32_t r;
  asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(r) : "s"(mask), "v"(a), "v"(b));
  return r;
}

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

// Workgroups are dispatched round-robin over the 8 XCDs (blockIdx % 8 picks
// the XCD). Renumber so that consecutive logical tiles land on one XCD and
// share its L2. Tiles beyond the last full group of 8 keep their id.
INTENT_DEVICE int xcd_swizzle(int bid, int nblocks) {
  const int full = nblocks & ~7;
  if (bid >= full) return bid;
  const int per_xcd = full >> 3;
  return (bid & 7) * per_xcd + (bid >> 3);
}
