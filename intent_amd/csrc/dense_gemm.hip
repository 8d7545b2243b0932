// Dense weight-only contractions on the shared f16 MFMA tile GEMM:
//   W4A16 (asymmetric group-quant nibbles) and W8A16 (per-channel int8).

#include "common.h"
#include "internal.h"
#include "mfma_pipe.h"

#include <type_traits>

namespace {

// Weight row of B-tile row c; tail rows read the last valid row and their
// outputs are dropped.
struct ClampRows {
  int n0;
  int N;
  INTENT_DEVICE int operator()(int c) const {
    const int n = n0 + c;
    return n < N ? n : N - 1;
  }
};

struct W4Args {
  const uint8_t* q;
  int64_t ldq;
  const f16* s;
  const uint8_t* z;
  int64_t ldp;
  int gs;
};
struct W8Args {
  const int8_t* q;
  int64_t ldq;
};

template <class T, class WArgs>
struct WeightOp;
template <class T>
struct WeightOp<T, W4Args> {
  using Op = mp::W4Operand<T::BN, T::NT>;  // staged by the NT producer threads
  INTENT_DEVICE static void init(Op& op, const W4Args& w, int n0, int N) {
    op.init(w.q, w.ldq, w.s, w.z, w.ldp, w.gs, ClampRows{n0, N});
  }
};
// W4 with windowed group parameters (W4Operand kWin): group sizes that are
// multiples of 64, scale and zero rows in whole dwords.
struct W4WinArgs : W4Args {};
template <class T>
struct WeightOp<T, W4WinArgs> {
  using Op = mp::W4Operand<T::BN, T::NT, true>;
  INTENT_DEVICE static void init(Op& op, const W4WinArgs& w, int n0, int N) {
    op.init(w.q, w.ldq, w.s, w.z, w.ldp, w.gs, ClampRows{n0, N});
  }
};
// The reference's own W4 layout (int32 [K/8, N] words, f16 [K/64, N] scales).
struct W4SymArgs {
  const int32_t* q;
  int64_t ldq;
  const f16* s;
  int64_t lds;
};
template <class T>
struct WeightOp<T, W4SymArgs> {
  using Op = mp::W4SymOperand<T::BN, T::NT>;
  INTENT_DEVICE static void init(Op& op, const W4SymArgs& w, int n0, int N) { op.init(w.q, w.ldq, w.s, w.lds, n0, N); }
};
template <class T>
struct WeightOp<T, W8Args> {
  using Op = mp::W8Operand<T::BN, T::NT>;
  INTENT_DEVICE static void init(Op& op, const W8Args& w, int n0, int N) { op.init(w.q, w.ldq, ClampRows{n0, N}); }
};

// ---- FP4 (E2M1) weights, bf16 activations: dequant_bf16_fp4_matmul --------------
// weight_only_int4.py:127-175 (CPU baseline cpu_runtime.py:117-124). Row n of
// the packed weights holds K/4 big-endian 16-bit words, word w = (p[2w] << 8) |
// p[2w+1] carrying k = 4w .. 4w+3 at the bit masks below; each 4-bit code
// becomes the bf16 pattern (bits & 0x81C0), and bf16(f32(pattern) * 2^126) is
// the E2M1 value (0, ±0.5, ±1, ±1.5, ±2, ±3, ±4, ±6), exactly: a normal
// pattern gains 126 in its exponent field, the one subnormal pattern is 0.5.
//
// gfx950 converts standard E2M1 nibbles (sign, e1, e0, m0) to bf16 in hardware,
// two per v_cvt_scalef32_pk_bf16_fp4 (low nibble to the low half, scale 1.0, so
// exact). The words' bit order is not that one, so nine rotate-and-mask terms
// first gather the eight codes of a dword into nibbles: term (r, m) moves word
// bits left by r (mod 32) into the nibble bits m. The k-pairs (0,1) (2,3) (4,5)
// (6,7) land in bytes 2, 1, 0, 3. About 2.5 VALU per value, against ~8 for the
// bit-pattern arithmetic it replaces (pinned against it on every 16-bit word).
INTENT_DEVICE uint32_t rotl32(uint32_t x, int r) { return r ? __builtin_amdgcn_alignbit(x, x, 32 - r) : x; }
// Eight bf16 (k = 8c .. 8c+7) from packed dword d (memory bytes b0 b1 b2 b3).
INTENT_DEVICE u32x4 fp4x8_to_bf16(uint32_t d) {
  if constexpr ((INTENT_ABLATE & 8) != 0) return u32x4{d, d, d, d};  // measurement build: no decode
  const uint32_t n = (d & 0x07000700u) | (rotl32(d, 2) & 0x00030003u) | (rotl32(d, 7) & 0x10001000u) |
                     (rotl32(d, 9) & 0x80708070u) | (rotl32(d, 10) & 0x08000800u) |
                     (rotl32(d, 11) & 0x60006000u) | (rotl32(d, 12) & 0x00080008u) |
                     (rotl32(d, 18) & 0x00040004u) | (rotl32(d, 19) & 0x00800080u);
  u32x4 out;
  out[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(n, 1.0f, 2));
  out[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(n, 1.0f, 1));
  out[2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(n, 1.0f, 0));
  out[3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(n, 1.0f, 3));
  return out;
}

// Packed FP4 weight rows decoded to bf16 on the way to LDS (same staging
// contract as mp::W8Operand: a stage is 64 k = 32 packed bytes per row).
template <int ROWS, int NT>
struct Fp4Operand {
  static constexpr int PIECE = (ROWS * 2) % NT == 0 ? 16 : (ROWS * 4) % NT == 0 ? 8 : 4;  // bytes per load
  static constexpr int P = 32 / PIECE;
  static constexpr int NS = ROWS * P / NT;
  static_assert(NS * NT == ROWS * P, "FP4 staging must divide evenly");
  static constexpr int NVM = NS;
  mp::Rsrc rq;
  uint32_t qoff[NS];
  int lrow[NS], part[NS];
  struct Regs {
    u32x4 w[NS];
  };
  template <class RowMap>
  INTENT_DEVICE void init(const uint8_t* q, int64_t ldq, const RowMap& wrow) {
    rq = make_rsrc(q);
#pragma unroll
    for (int i = 0; i < NS; ++i) {
      const int c = (int)(threadIdx.x % NT) + i * NT;
      lrow[i] = c / P;
      part[i] = c % P;
      qoff[i] = (uint32_t)((int64_t)wrow(lrow[i]) * ldq + part[i] * PIECE);
    }
  }
  INTENT_DEVICE void load(int kt, Regs& r) const {
#pragma unroll
    for (int i = 0; i < NS; ++i) {
      if constexpr (PIECE == 16) {
        r.w[i] = __builtin_amdgcn_raw_buffer_load_b128(rq, qoff[i], (uint32_t)kt * 32, 0);
      } else if constexpr (PIECE == 8) {
        const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(rq, qoff[i], (uint32_t)kt * 32, 0);
        r.w[i] = u32x4{v[0], v[1], 0u, 0u};
      } else {
        r.w[i] = u32x4{__builtin_amdgcn_raw_buffer_load_b32(rq, qoff[i], (uint32_t)kt * 32, 0), 0u, 0u, 0u};
      }
    }
  }
  template <bool kAsm = false>
  INTENT_DEVICE void store(const Regs& r, char* lds_b) const {
#pragma unroll
    for (int i = 0; i < NS; ++i) {
      char* row = lds_b + lrow[i] * mp::ROWB;
      const int sw = mp::swz(lrow[i]);
#pragma unroll
      for (int d = 0; d < PIECE / 4; ++d) {
        const int chunk = part[i] * (PIECE / 4) + d;  // each dword = 8 k = one 16-byte bf16 chunk
        const u32x4 v = fp4x8_to_bf16(r.w[i][d]);
        if constexpr (kAsm)
          mp::lds_store16(row + ((chunk ^ sw) << 4), v);
        else
          *reinterpret_cast<u32x4*>(row + ((chunk ^ sw) << 4)) = v;
      }
    }
  }
};


// ---- the reference's own W4 layout -> the asymmetric nibble layout --------------
// weight_only_int4_matmul (weight_only_int4.py:18-51) packs eight signed nibbles
// of consecutive k into an int32 of [K/8, N] (nibble k % 8 at bits 4(k % 8)),
// with f16 scales [K/64, N]. Flipping each nibble's top bit gives u = n ^ 8 with
// u - 8 = the two's-complement value, so (u - z) * s with z = 8 is the same f16
// product; the int32's bytes already hold nibble pairs low = even k. Repacking
// is a transpose of the int32 words (xor 0x88888888) and of the scales.
template <class E, uint32_t kXor>
__global__ __launch_bounds__(256) void transpose32_kernel(const E* __restrict__ src, int R, int C, int64_t sld,
                                                          E* __restrict__ dst, int64_t dld, int64_t sbatch = 0,
                                                          int64_t dbatch = 0) {
  __shared__ E t[32][33];
  src += blockIdx.z * sbatch;  // one matrix per blockIdx.z
  dst += blockIdx.z * dbatch;
  const int r0 = blockIdx.y * 32, c0 = blockIdx.x * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
#pragma unroll
  for (int i = ty; i < 32; i += 8)
    if (r0 + i < R && c0 + tx < C) t[i][tx] = src[(int64_t)(r0 + i) * sld + c0 + tx];
  __syncthreads();
#pragma unroll
  for (int i = ty; i < 32; i += 8)
    if (c0 + i < C && r0 + tx < R) dst[(int64_t)(c0 + i) * dld + r0 + tx] = (E)(t[tx][i] ^ (E)kXor);
}

// f16 / bf16 transpose through a 64 x 64 LDS tile with 16-byte accesses:
// thread t moves 8 elements of row t / 8 (twice: rows and rows + 32), then
// writes 8 elements of one output row. dst[c][r] = src[r][c]; blockIdx.z
// selects a matrix of a batch.
__global__ __launch_bounds__(256) void transpose16_kernel(const uint16_t* __restrict__ src, int R, int C, int64_t sld,
                                                          uint16_t* __restrict__ dst, int64_t dld, int64_t sbatch,
                                                          int64_t dbatch) {
  __shared__ uint16_t t[64][72];
  src += blockIdx.z * sbatch;
  dst += blockIdx.z * dbatch;
  const int r0 = blockIdx.y * 64, c0 = blockIdx.x * 64;
  const int row = threadIdx.x >> 3, seg = (threadIdx.x & 7) * 8;
  const bool full = r0 + 64 <= R && c0 + 64 <= C;
  const bool svec = full && ((sld | (int64_t)(uintptr_t)src) & 7) == 0;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int r = row + 32 * h;
    if (svec) {
      *reinterpret_cast<u32x4*>(&t[r][seg]) = *reinterpret_cast<const u32x4*>(src + (int64_t)(r0 + r) * sld + c0 + seg);
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i)
        t[r][seg + i] = (r0 + r < R && c0 + seg + i < C) ? src[(int64_t)(r0 + r) * sld + c0 + seg + i] : 0;
    }
  }
  __syncthreads();
  const bool dvec = full && ((dld | (int64_t)(uintptr_t)dst) & 7) == 0;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int c = row + 32 * h;  // output row c0 + c, elements r0 + seg .. +7
    uint16_t v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = t[seg + i][c];
    if (dvec) {
      u32x4 w;
#pragma unroll
      for (int d = 0; d < 4; ++d) w[d] = (uint32_t)v[2 * d] | ((uint32_t)v[2 * d + 1] << 16);
      *reinterpret_cast<u32x4*>(dst + (int64_t)(c0 + c) * dld + r0 + seg) = w;
    } else if (c0 + c < C) {
#pragma unroll
      for (int i = 0; i < 8; ++i)
        if (r0 + seg + i < R) dst[(int64_t)(c0 + c) * dld + r0 + seg + i] = v[i];
    }
  }
}

__global__ void fill_u8_kernel(uint8_t* __restrict__ z, int rows, int cols, int64_t ld, uint8_t v) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < (int64_t)rows * cols) z[(i / cols) * ld + i % cols] = v;
}

// ---- quantized_gemm (gemm.py:83-106): f16 GEMM with a fused int8 epilogue ---------
//   out = i8(trunc(clamp((relu(acc + bias[n]) + f32(residual)) / output_scale[n],
//                        -128, 127)))
// (CPU baseline cpu_runtime.py:91-94; relu keeps NaN, the division is IEEE and
// the float -> integer cast truncates toward zero). Both operands are f16 rows
// with K contiguous (the right operand transposed beforehand), on producer/
// consumer workgroups (mainloop_ws): activations by LDS DMA, weight rows
// staged by the producer waves.
// The plain float GEMMs share this kernel (gemm.py:42-80): f16 outputs
// c = f16(acc) or f16(max(acc, 0)) (NaN kept) through the run-time f16_epi of
// the kQuantI8 instances, and kGemmBf16: c = bf16(acc) with bf16 operands.
enum class DenseEpi { kQuantI8, kGemmBf16 };

// quantized_gemm's epilogue of one element (gemm.py:83-106): relu(acc + bias)
// plus the residual, divided by the output scale, clamped to [-128, 127] and
// truncated to int8; each step rounds to f32 (NaN clamps to -128).
INTENT_DEVICE uint32_t quant_i8_epilogue(float acc, float bias, f16 res, float scale) {
  float v = __fadd_rn(acc, bias);
  v = v < 0.f ? 0.f : v;
  v = __fadd_rn(v, (float)res);
  v = __fdiv_rn(v, scale);
  v = fminf(fmaxf(v, -128.f), 127.f);
  return (uint32_t)(int32_t)v & 255u;
}

// Epilogues of the dense f16 / bf16 GEMMs (lane holds m = row(i), n = col(j, g) + 0..3).
template <class T, DenseEpi E>
INTENT_DEVICE void dense_epilogue(const f32x16 (&acc)[T::TI][T::TJ], int m0, int n0, int M, int N,
                                  const float* __restrict__ bias, const f16* __restrict__ residual, int64_t ldr,
                                  const float* __restrict__ oscale, int8_t* __restrict__ out, int64_t ldo,
                                  int f16_epi) {
  // kQuantI8 instances also serve the f16 GEMM epilogues, chosen at run time
  // (f16_epi 1: f16(acc), 2: f16(max(acc, 0))).
  if (E != DenseEpi::kQuantI8 || f16_epi != 0) {
    uint16_t* y = reinterpret_cast<uint16_t*>(out);
    const bool relu = f16_epi == 2;
    auto cvt = [relu](float v) -> uint32_t {
      if constexpr (E == DenseEpi::kGemmBf16) {
        (void)relu;
        return f32_to_bf16_rne(v);
      } else {
        if (relu) v = v < 0.f ? 0.f : v;
        return bit_cast<uint16_t>((f16)v);
      }
    };
    const bool vec = (ldo & 3) == 0 && (((uintptr_t)y) & 7) == 0;
#pragma unroll
    for (int i = 0; i < T::TI; ++i) {
      const int m = m0 + T::row(i);
      if (m >= M) continue;
#pragma unroll
      for (int j = 0; j < T::TJ; ++j)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int n = n0 + T::col(j, g);
          uint16_t* o = y + (int64_t)m * ldo + n;
          if (vec && n + 3 < N) {
            const uint32_t lo = cvt(acc[i][j][4 * g]) | (cvt(acc[i][j][4 * g + 1]) << 16);
            const uint32_t hi = cvt(acc[i][j][4 * g + 2]) | (cvt(acc[i][j][4 * g + 3]) << 16);
            *reinterpret_cast<u32x2*>(o) = u32x2{lo, hi};
          } else {
#pragma unroll
            for (int c = 0; c < 4; ++c)
              if (n + c < N) o[c] = (uint16_t)cvt(acc[i][j][4 * g + c]);
          }
        }
    }
    return;
  }
  // A lane's outputs are 4 consecutive columns per (j, g). Per (i, j) the
  // residual, bias and scale vectors of its four groups are all loaded before
  // any of them is used, so the epilogue pays one memory round trip per 16
  // outputs instead of per 4. Registers allow no larger batch beside the
  // accumulators: preloading all bias and scale columns, or loading block
  // t + 1 during block t, both spill. Edge columns (n + 3 >= N) and unaligned
  // operands take guarded element loads; the arithmetic per element is the
  // same either way.
  const bool vec = (ldo & 3) == 0 && (((uintptr_t)out) & 3) == 0 && (ldr & 3) == 0 &&
                   (((uintptr_t)residual) & 7) == 0 && ((((uintptr_t)bias) | ((uintptr_t)oscale)) & 15) == 0;
#pragma unroll
  for (int i = 0; i < T::TI; ++i) {
    const int m = m0 + T::row(i);
    if (m >= M) continue;
#pragma unroll
    for (int j = 0; j < T::TJ; ++j) {
      f32x4 bv[4], sv[4];
      u32x2 rv[4];
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int n = n0 + T::col(j, g);
        const f16* r = residual + (int64_t)m * ldr + n;
        if (vec && n + 3 < N) {
          rv[g] = *reinterpret_cast<const u32x2*>(r);
          bv[g] = *reinterpret_cast<const f32x4*>(bias + n);
          sv[g] = *reinterpret_cast<const f32x4*>(oscale + n);
        } else {
          uint16_t e[4];
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            e[c] = n + c < N ? bit_cast<uint16_t>(r[c]) : (uint16_t)0;
            bv[g][c] = n + c < N ? bias[n + c] : 0.f;
            sv[g][c] = n + c < N ? oscale[n + c] : 1.f;
          }
          rv[g] = u32x2{(uint32_t)e[0] | ((uint32_t)e[1] << 16), (uint32_t)e[2] | ((uint32_t)e[3] << 16)};
        }
      }
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int n = n0 + T::col(j, g);
        int8_t* o = out + (int64_t)m * ldo + n;
        uint32_t packed = 0;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const f16 res = bit_cast<f16>((uint16_t)(rv[g][c >> 1] >> (16 * (c & 1))));
          packed |= quant_i8_epilogue(acc[i][j][4 * g + c], bv[g][c], res, sv[g][c]) << (8 * c);
        }
        if (vec && n + 3 < N) {
          *reinterpret_cast<uint32_t*>(o) = packed;
        } else {
#pragma unroll
          for (int c = 0; c < 4; ++c)
            if (n + c < N) o[c] = (int8_t)((packed >> (8 * c)) & 255u);
        }
      }
    }
  }
}

// quantized_gemm's int8 epilogue through LDS for the 8-wave [K, N] kernel
// (T::NW = 8 waves of 128 x 64): after a barrier the two stage buffers are
// free; wave w stages one 32-row block of f32 sums at a time in its own
// 32 x (64 * 4 + 16)-byte block (waves 0-3 in buf0, 4-7 in buf1), then lane
// l takes 8 consecutive columns (l % 8) of rows l / 8 + 8 q: 16-byte residual
// loads and 8-byte int8 stores, eight lanes per 128-byte row segment, instead
// of 8-byte residual pieces of 32 rows. Bias and scale are per column: each
// lane loads its 8 once. Same arithmetic per element as dense_epilogue.
template <class T>
INTENT_DEVICE void quant_epilogue_lds(const f32x16 (&acc)[T::TI][T::TJ], char* buf0, char* buf1, int m0, int n0,
                                      int M, int N, const float* __restrict__ bias, const f16* __restrict__ residual,
                                      int64_t ldr, const float* __restrict__ oscale, int8_t* __restrict__ out,
                                      int64_t ldo) {
  static_assert(T::NW == 8 && T::WTN == 64, "eight waves of 64 columns");
  constexpr int RS = T::WTN * 4 + 16;
  static_assert(4 * 32 * RS <= T::STAGE_BYTES, "four wave blocks per stage buffer");
  __syncthreads();  // every wave's DMA has drained (mainloop_kn) and its last fragments are read
  const int lane = threadIdx.x & 63;
  const int w = T::wave();
  char* blk = (w < 4 ? buf0 : buf1) + (w & 3) * 32 * RS;
  const int wm = m0 + T::wave_m() * T::WTM, wn = n0 + T::wave_n() * T::WTN;
  const int c8 = (lane & 7) * 8;
  const int gn = wn + c8;
  const bool full = gn + 7 < N;
  const bool vec = full && (ldr & 7) == 0 && (((uintptr_t)residual) & 15) == 0 && (ldo & 7) == 0 &&
                   (((uintptr_t)out) & 7) == 0 && ((((uintptr_t)bias) | ((uintptr_t)oscale)) & 15) == 0;
  float bv[8], sv[8];
  if (vec) {
    const f32x4 b0 = *reinterpret_cast<const f32x4*>(bias + gn), b1 = *reinterpret_cast<const f32x4*>(bias + gn + 4);
    const f32x4 s0 = *reinterpret_cast<const f32x4*>(oscale + gn), s1 = *reinterpret_cast<const f32x4*>(oscale + gn + 4);
#pragma unroll
    for (int c = 0; c < 4; ++c) bv[c] = b0[c], bv[4 + c] = b1[c], sv[c] = s0[c], sv[4 + c] = s1[c];
  } else {
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      bv[c] = gn + c < N ? bias[gn + c] : 0.f;
      sv[c] = gn + c < N ? oscale[gn + c] : 1.f;
    }
  }
#pragma unroll
  for (int i = 0; i < T::TI; ++i) {
#pragma unroll
    for (int j = 0; j < T::TJ; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g)
        *reinterpret_cast<f32x4*>(blk + (lane & 31) * RS + (j * 32 + g * 8 + (lane >> 5) * 4) * 4) =
            f32x4{acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int r = (lane >> 3) + 8 * q;
      const int gm = wm + i * 32 + r;
      const f32x4 a0 = *reinterpret_cast<const f32x4*>(blk + r * RS + c8 * 4);
      const f32x4 a1 = *reinterpret_cast<const f32x4*>(blk + r * RS + c8 * 4 + 16);
      if (gm >= M) continue;
      const f16* rp = residual + (int64_t)gm * ldr + gn;
      uint16_t e[8];
      if (vec) {
        const u32x4 rv = *reinterpret_cast<const u32x4*>(rp);
#pragma unroll
        for (int c = 0; c < 8; ++c) e[c] = (uint16_t)(rv[c >> 1] >> (16 * (c & 1)));
      } else {
#pragma unroll
        for (int c = 0; c < 8; ++c) e[c] = gn + c < N ? bit_cast<uint16_t>(rp[c]) : (uint16_t)0;
      }
      uint32_t lo = 0, hi = 0;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        lo |= quant_i8_epilogue(a0[c], bv[c], bit_cast<f16>(e[c]), sv[c]) << (8 * c);
        hi |= quant_i8_epilogue(a1[c], bv[4 + c], bit_cast<f16>(e[4 + c]), sv[4 + c]) << (8 * c);
      }
      int8_t* o = out + (int64_t)gm * ldo + gn;
      if (vec) {
        *reinterpret_cast<u32x2*>(o) = u32x2{lo, hi};
      } else {
#pragma unroll
        for (int c = 0; c < 8; ++c)
          if (gn + c < N) o[c] = (int8_t)(((c < 4 ? lo : hi) >> (8 * (c & 3))) & 255u);
      }
    }
  }
}

// The f16 / bf16 outputs of the same kernel (gemm, bf16_gemm) staged the
// same way: lane l converts 8 consecutive columns of a row (f16, optionally
// max(v, 0) with NaN kept, or bf16 round-to-nearest-even) and stores them as
// one 16-byte piece.
template <class T, DenseEpi E>
INTENT_DEVICE void half_epilogue_lds(const f32x16 (&acc)[T::TI][T::TJ], char* buf0, char* buf1, int m0, int n0,
                                     int M, int N, uint16_t* __restrict__ y, int64_t ldy, bool relu) {
  static_assert(T::NW == 8 && T::WTN == 64, "eight waves of 64 columns");
  constexpr int RS = T::WTN * 4 + 16;
  static_assert(4 * 32 * RS <= T::STAGE_BYTES, "four wave blocks per stage buffer");
  __syncthreads();  // every wave's DMA has drained (mainloop_kn) and its last fragments are read
  const int lane = threadIdx.x & 63;
  const int w = T::wave();
  char* blk = (w < 4 ? buf0 : buf1) + (w & 3) * 32 * RS;
  const int wm = m0 + T::wave_m() * T::WTM, wn = n0 + T::wave_n() * T::WTN;
  const int c8 = (lane & 7) * 8;
  const int gn = wn + c8;
  const bool vec = gn + 7 < N && (ldy & 7) == 0 && (((uintptr_t)y) & 15) == 0;
  auto cvt = [relu](float v) -> uint32_t {
    if constexpr (E == DenseEpi::kGemmBf16) {
      (void)relu;
      return f32_to_bf16_rne(v);
    } else {
      if (relu) v = v < 0.f ? 0.f : v;
      return bit_cast<uint16_t>((f16)v);
    }
  };
#pragma unroll
  for (int i = 0; i < T::TI; ++i) {
#pragma unroll
    for (int j = 0; j < T::TJ; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g)
        *reinterpret_cast<f32x4*>(blk + (lane & 31) * RS + (j * 32 + g * 8 + (lane >> 5) * 4) * 4) =
            f32x4{acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int r = (lane >> 3) + 8 * q;
      const int gm = wm + i * 32 + r;
      const f32x4 a0 = *reinterpret_cast<const f32x4*>(blk + r * RS + c8 * 4);
      const f32x4 a1 = *reinterpret_cast<const f32x4*>(blk + r * RS + c8 * 4 + 16);
      if (gm >= M) continue;
      const u32x4 v{cvt(a0[0]) | (cvt(a0[1]) << 16), cvt(a0[2]) | (cvt(a0[3]) << 16), cvt(a1[0]) | (cvt(a1[1]) << 16),
                    cvt(a1[2]) | (cvt(a1[3]) << 16)};
      uint16_t* o = y + (int64_t)gm * ldy + gn;
      if (vec) {
        *reinterpret_cast<u32x4*>(o) = v;
      } else {
#pragma unroll
        for (int c = 0; c < 8; ++c)
          if (gn + c < N) o[c] = (uint16_t)(v[c >> 1] >> (16 * (c & 1)));
      }
    }
  }
}

template <class T, DenseEpi E = DenseEpi::kQuantI8, class Math = mp::F16Math>
__global__ __launch_bounds__(T::NT_WS, 1) void quantized_gemm_kernel(
    const f16* __restrict__ a, int64_t lda, int M, const f16* __restrict__ bt, int64_t ldb, int N, int K,
    const float* __restrict__ bias, const f16* __restrict__ residual, int64_t ldr, const float* __restrict__ oscale,
    int8_t* __restrict__ out, int64_t ldo, int mblocks, int f16_epi = 0) {
  __shared__ __attribute__((aligned(16))) char buf0[T::STAGE_BYTES];
  __shared__ __attribute__((aligned(16))) char buf1[T::STAGE_BYTES];
  char* const bufs[2] = {buf0, buf1};
  int tmb, tnb;
  grid_tile(mblocks, 4, tmb, tnb);
  const int m0 = tmb * T::BM;
  const int n0 = tnb * T::BN;
  const int pw = T::wave() % T::NW;
  mp::RegRowsOperand<T::BN, mp::DenseRows, false, T::NW> bop;
  bop.init(mp::DenseRows{bt, ldb * 2, N}, n0, pw);
  mp::DmaRowsOperand<T::BM, mp::DenseRows, T::NW> aop;
  aop.init(mp::DenseRows{a, lda * 2, M}, m0, pw);
  f32x16 acc[T::TI][T::TJ];
  if (!mp::mainloop_ws<T, Math, 2>(aop, bop, K / 64, bufs, acc)) return;
  dense_epilogue<T, E>(acc, m0, n0, M, N, bias, residual, ldr, oscale, out, ldo, f16_epi);
}

// The same GEMMs with the right operand as the reference passes it, b [K, N]
// (N contiguous): both operands reach LDS by DMA and the B fragments come
// out of LDS through transpose reads (mfma_pipe.h, DmaKNOperand), so no
// transposed copy of b is made. 256 x 256 tiles (KNTile), a ring of two
// 64-KB stages.
template <class T, DenseEpi E = DenseEpi::kQuantI8, class Math = mp::F16Math, bool kSched = false>
__global__ __launch_bounds__(T::NT, 1) void gemm_kn_kernel(
    const f16* __restrict__ a, int64_t lda, int M, const f16* __restrict__ b, int64_t ldb, int N, int K,
    const float* __restrict__ bias, const f16* __restrict__ residual, int64_t ldr, const float* __restrict__ oscale,
    int8_t* __restrict__ out, int64_t ldo, int mblocks, int f16_epi = 0) {
  __shared__ __attribute__((aligned(16))) char buf0[T::STAGE_BYTES];
  __shared__ __attribute__((aligned(16))) char buf1[T::STAGE_BYTES];
  int tmb, tnb;
  grid_tile(mblocks, 4, tmb, tnb);
  const int m0 = tmb * T::BM;
  const int n0 = tnb * T::BN;
  const int wave = T::wave();
  mp::DmaRowsOperand<T::BM, mp::DenseRows, T::NW> aop;
  aop.init(mp::DenseRows{a, lda * 2, M}, m0, wave);
  mp::DmaKNOperand<T::BN, T::NW> bop;
  bop.init(b + n0, ldb, N - n0, wave);
  f32x16 acc[T::TI][T::TJ];
  mp::mainloop_kn<T, Math, mp::DmaRowsOperand<T::BM, mp::DenseRows, T::NW>, mp::DmaKNOperand<T::BN, T::NW>, kSched>(
      aop, bop, K / 64, buf0, buf1, acc);
  if constexpr (T::NW == 8 && T::WTN == 64) {
    if (E == DenseEpi::kQuantI8 && f16_epi == 0)  // workgroup-uniform
      quant_epilogue_lds<T>(acc, buf0, buf1, m0, n0, M, N, bias, residual, ldr, oscale, out, ldo);
    else
      half_epilogue_lds<T, E>(acc, buf0, buf1, m0, n0, M, N, reinterpret_cast<uint16_t*>(out), ldo, f16_epi == 2);
    return;
  }
  dense_epilogue<T, E>(acc, m0, n0, M, N, bias, residual, ldr, oscale, out, ldo, f16_epi);
}

// ---- f16 / bf16 grouped GEMMs over row groups -----------------------------------
// ragged_grouped_gemm(_bf16) (grouped_gemm.py:11-70): group g owns rows
// offsets[g] .. offsets[g+1] of x and y; y[rows] = x[rows] @ W[g].
// routed_expert_projection_bf16 (grouped_gemm.py:101-138): expert e owns
// entries offsets[e] .. offsets[e+1] of member_routes; route r reads token
// r / TOP_K and writes row r of the [T * TOP_K, N] output.
// Weights arrive as [G][N][K] rows (K contiguous). A workgroup owns one
// 256 x 256 tile of one group; the grid covers every group's worst case
// (all rows) and workgroups past their group's rows exit at once.
struct RoutedRows {  // tile row p = route routes[m0 + p]; rows past the group repeat the last
  const void* base;
  int64_t ld_bytes;
  const int32_t* routes;
  int end;
  int top_k;
  INTENT_DEVICE const void* tile_base(int) const { return base; }
  INTENT_DEVICE uint32_t off(int m0, int p) const {
    const int i = m0 + p < end ? m0 + p : end - 1;
    return (uint32_t)((routes[i] / top_k) * ld_bytes);
  }
};

template <class T, class Math, bool kRouted>
__global__ __launch_bounds__(T::NT, 1) void grouped_gemm_kernel(
    const uint16_t* __restrict__ x, int64_t ldx, const int32_t* __restrict__ offsets,
    const int32_t* __restrict__ routes, int top_k, const uint16_t* __restrict__ w, int64_t ldw, int64_t gstride,
    int N, int K, int mbmax, int nblocks, uint16_t* __restrict__ out, int64_t ldo) {
  __shared__ __attribute__((aligned(16))) char buf0[T::STAGE_BYTES];
  __shared__ __attribute__((aligned(16))) char buf1[T::STAGE_BYTES];
  const int nb = blockIdx.x % nblocks;
  const int rest = blockIdx.x / nblocks;
  const int mb = rest % mbmax;
  const int g = rest / mbmax;
  const int start = offsets[g] + mb * T::BM;
  const int end = offsets[g + 1];
  if (start >= end) return;  // workgroup-uniform
  const int n0 = nb * T::BN;
  const int wave = T::wave();
  mp::RegRowsOperand<T::BN, mp::DenseRows, false, T::NW> bop;
  bop.init(mp::DenseRows{w + g * gstride, ldw * 2, N}, n0, wave);
  f32x16 acc[T::TI][T::TJ];
  if constexpr (kRouted) {
    mp::RegRowsOperand<T::BM, RoutedRows, false, T::NW> aop;
    aop.init(RoutedRows{x, ldx * 2, routes, end, top_k}, start, wave);
    mp::mainloop<T, Math>(aop, bop, K / 64, buf0, buf1, acc);
  } else {
    mp::RegRowsOperand<T::BM, mp::DenseRows, false, T::NW> aop;
    aop.init(mp::DenseRows{x, ldx * 2, end}, start, wave);
    mp::mainloop<T, Math>(aop, bop, K / 64, buf0, buf1, acc);
  }
  constexpr bool kBf16 = std::is_same<Math, mp::BF16Math>::value;
  auto cvt = [](float v) -> uint32_t { return kBf16 ? f32_to_bf16_rne(v) : bit_cast<uint16_t>((f16)v); };
  const bool vec = (ldo & 3) == 0 && (((uintptr_t)out) & 7) == 0;
#pragma unroll
  for (int i = 0; i < T::TI; ++i) {
    const int idx = start + T::row(i);
    if (idx >= end) continue;
    const int64_t orow = kRouted ? routes[idx] : idx;
#pragma unroll
    for (int j = 0; j < T::TJ; ++j)
#pragma unroll
      for (int gq = 0; gq < 4; ++gq) {
        const int n = n0 + T::col(j, gq);
        uint16_t* o = out + orow * ldo + n;
        if (vec && n + 3 < N) {
          const uint32_t lo = cvt(acc[i][j][4 * gq]) | (cvt(acc[i][j][4 * gq + 1]) << 16);
          const uint32_t hi = cvt(acc[i][j][4 * gq + 2]) | (cvt(acc[i][j][4 * gq + 3]) << 16);
          *reinterpret_cast<u32x2*>(o) = u32x2{lo, hi};
        } else {
#pragma unroll
          for (int c = 0; c < 4; ++c)
            if (n + c < N) o[c] = (uint16_t)cvt(acc[i][j][4 * gq + c]);
        }
      }
  }
}

// Lane holds m = row(i) and n = col(j, g) + 0..3 in acc[i][j][4g..4g+3].
template <class T, bool kColScale>
INTENT_DEVICE void store_dense(const f32x16 (&acc)[T::TI][T::TJ], int m0, int n0, int M, int N, f16* __restrict__ y,
                               int64_t ldy, const f16* __restrict__ colscale) {
  const bool vec = (ldy & 3) == 0 && (((uintptr_t)y) & 7) == 0;
#pragma unroll
  for (int i = 0; i < T::TI; ++i) {
    const int m = m0 + T::row(i);
    if (m >= M) continue;
#pragma unroll
    for (int j = 0; j < T::TJ; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int n = n0 + T::col(j, g);
        f16* o = y + (int64_t)m * ldy + n;
        float v[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          v[c] = acc[i][j][4 * g + c];
          if (kColScale && n + c < N) v[c] *= (float)colscale[n + c];
        }
        if (vec && n + 3 < N) {
          f16x2 lo, hi;
          lo[0] = (f16)v[0];
          lo[1] = (f16)v[1];
          hi[0] = (f16)v[2];
          hi[1] = (f16)v[3];
          *reinterpret_cast<u32x2*>(o) = u32x2{bit_cast<uint32_t>(lo), bit_cast<uint32_t>(hi)};
        } else {
#pragma unroll
          for (int c = 0; c < 4; ++c)
            if (n + c < N) o[c] = (f16)v[c];
        }
      }
  }

}

// store_dense through LDS: each consumer wave converts one 32-row block of
// its tile at a time into a private block of 32 rows (WTN f16 + 16 bytes of
// padding each: the 8-byte writes of 16 rows fall in distinct bank groups),
// reads it back as 16-byte row pieces and stores whole row segments, where the
// register layout would store 8 bytes in each of 32 rows per instruction.
// lds: NC * 32 * (2 * WTN + 16) bytes that no wave reads or writes any more.
template <class T, bool kColScale, bool kBf16 = false>
INTENT_DEVICE void store_dense_lds(const f32x16 (&acc)[T::TI][T::TJ], char* lds, int m0, int n0, int M, int N,
                                   f16* __restrict__ y, int64_t ldy, const f16* __restrict__ colscale) {
  constexpr int RS = 2 * T::WTN + 16;  // LDS row bytes
  constexpr int CH = T::WTN / 8;       // 16-byte pieces per row
  constexpr int NP = 32 * CH / 64;     // pieces per lane and block
  static_assert(NP * 64 == 32 * CH, "whole pieces per lane");
  const int lane = threadIdx.x & 63;
  char* blk = lds + T::wave() * 32 * RS;
  const int wm = m0 + T::wave_m() * T::WTM, wn = n0 + T::wave_n() * T::WTN;
  const bool vec = (ldy & 7) == 0 && (((uintptr_t)y) & 15) == 0;
#pragma unroll
  for (int i = 0; i < T::TI; ++i) {
#pragma unroll
    for (int j = 0; j < T::TJ; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int n = n0 + T::col(j, g);
        float v[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          v[c] = acc[i][j][4 * g + c];
          if (kColScale) v[c] *= n + c < N ? (float)colscale[n + c] : 0.f;
        }
        u32x2 pk;
        if constexpr (kBf16) {
          pk = u32x2{bf16x2_rne(v[0], v[1]), bf16x2_rne(v[2], v[3])};
        } else {
          pk = u32x2{bit_cast<uint32_t>(__builtin_convertvector(f32x2{v[0], v[1]}, f16x2)),
                     bit_cast<uint32_t>(__builtin_convertvector(f32x2{v[2], v[3]}, f16x2))};
        }
        *reinterpret_cast<u32x2*>(blk + (lane & 31) * RS + (n - wn) * 2) = pk;
      }
#pragma unroll
    for (int q = 0; q < NP; ++q) {
      const int p = q * 64 + lane, r = p / CH, c8 = (p % CH) * 8;
      const u32x4 v = *reinterpret_cast<const u32x4*>(blk + r * RS + c8 * 2);
      const int gm = wm + i * 32 + r, gn = wn + c8;
      if (gm >= M) continue;
      f16* dst = y + (int64_t)gm * ldy + gn;
      if (vec && gn + 7 < N) {
        *reinterpret_cast<u32x4*>(dst) = v;
      } else {
#pragma unroll
        for (int c = 0; c < 8; ++c)
          if (gn + c < N) reinterpret_cast<uint16_t*>(dst)[c] = (uint16_t)(v[c >> 1] >> (16 * (c & 1)));
      }
    }
  }
}

// y[m, n] = bf16(sum_k x[m, k] * fp4(W)[n, k]), bf16 activations, f32 accumulation.
template <class T>
__global__ __launch_bounds__(T::NT_WS, 1) void fp4_bf16_gemm_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                                    int M, const uint8_t* __restrict__ wq,
                                                                    int64_t ldw, int N, int K,
                                                                    uint16_t* __restrict__ y, int64_t ldy,
                                                                    int mblocks) {
  __shared__ __attribute__((aligned(16))) char buf0[T::STAGE_BYTES];
  __shared__ __attribute__((aligned(16))) char buf1[T::STAGE_BYTES];
  char* const bufs[2] = {buf0, buf1};
  int tmb, tnb;
  grid_tile(mblocks, 4, tmb, tnb);
  const int m0 = tmb * T::BM;
  const int n0 = tnb * T::BN;
  Fp4Operand<T::BN, T::NT> bop;
  bop.init(wq, ldw, ClampRows{n0, N});
  f32x16 acc[T::TI][T::TJ];
  mp::DmaRowsOperand<T::BM, mp::DenseRows, T::NW> aop;
  aop.init(mp::DenseRows{x, ldx * 2, M}, m0, T::wave() % T::NW);
  if (!mp::mainloop_ws<T, mp::BF16Math, 2>(aop, bop, K / 64, bufs, acc)) return;
  // The stage buffer of stage nk - 2 is free after the main loop, as in dense_gemm_kernel.
  static_assert(T::NW * 32 * (2 * T::WTN + 16) <= T::STAGE_BYTES, "FP4 tiles stage their epilogue in LDS");
  store_dense_lds<T, false, true>(acc, ((K / 64) & 1) ? buf1 : buf0, m0, n0, M, N, reinterpret_cast<f16*>(y), ldy,
                                  nullptr);
}

// y[m, n] = f16(sum_k x[m, k] * deq(W)[n, k] (* colscale[n])).
template <class T, class WArgs, bool kColScale>
__global__ __launch_bounds__(T::NT_WS, 1) void dense_gemm_kernel(const f16* __restrict__ x, int64_t ldx, int M,
                                                                   WArgs w, int N, int K, f16* __restrict__ y,
                                                                   int64_t ldy, const f16* __restrict__ colscale,
                                                                   int mblocks) {
  __shared__ __attribute__((aligned(16))) char buf0[T::STAGE_BYTES];
  __shared__ __attribute__((aligned(16))) char buf1[T::STAGE_BYTES];
  char* const bufs[2] = {buf0, buf1};
  int tmb, tnb;
  grid_tile(mblocks, 4, tmb, tnb);
  const int m0 = tmb * T::BM;
  const int n0 = tnb * T::BN;
  typename WeightOp<T, WArgs>::Op bop;
  WeightOp<T, WArgs>::init(bop, w, n0, N);
  f32x16 acc[T::TI][T::TJ];
  mp::DmaRowsOperand<T::BM, mp::DenseRows, T::NW> aop;
  aop.init(mp::DenseRows{x, ldx * 2, M}, m0, T::wave() % T::NW);
  if (!mp::mainloop_ws<T, mp::F16Math, 2>(aop, bop, K / 64, bufs, acc)) return;

  // After the main loop's last barrier the stage buffer of stage nk - 2 (of
  // none, for nk = 1) is neither read nor written again: the producers drained
  // their DMA before that barrier and issue nothing after it.
  if constexpr (T::NW * 32 * (2 * T::WTN + 16) <= T::STAGE_BYTES) {
    store_dense_lds<T, kColScale>(acc, ((K / 64) & 1) ? buf1 : buf0, m0, n0, M, N, y, ldy, colscale);
    return;
  }
  store_dense<T, kColScale>(acc, m0, n0, M, N, y, ldy, colscale);
}

template <class T, class WArgs, bool kColScale>
int launch_tile(const f16* x, int64_t ldx, int M, int N, int K, const WArgs& w, f16* y, int64_t ldy,
                const f16* colscale, hipStream_t st, const char* name) {
  const int mblocks = (M + T::BM - 1) / T::BM;
  const int nblocks = (N + T::BN - 1) / T::BN;
  const int64_t grid = (int64_t)mblocks * nblocks;
  INTENT_REQUIRE(grid < (1ll << 31), INTENT_ERR_UNSUPPORTED, "%s: grid too large", name);
  INTENT_REQUIRE(intent::fits_offset(M, ldx * 2), INTENT_ERR_UNSUPPORTED,
                 "%s: activations too large for 31-bit buffer offsets", name);
  hipLaunchKernelGGL((dense_gemm_kernel<T, WArgs, kColScale>), dim3((unsigned)grid), dim3(T::NT_WS), 0, st, x, ldx,
                     M, w, N, K, y, ldy, colscale, mblocks);
  return intent::launch_status(name);
}

// Tiles: 256 x 192 (4 consumer waves of 128 x 96) once M fills it, else
// 128 x 128 (consumers of 64 x 64); each with 4 producer waves that copy the
// activations by LDS DMA and decode the weights (mainloop_ws). 192 columns:
// N = 11008 gives 58 column tiles; with 8 row tiles that is 464 workgroups,
// 1.8 rounds of 256 CUs (256-wide tiles would give 344, 1.34).
template <class WArgs, bool kColScale>
int launch_dense(const f16* x, int64_t ldx, int M, int N, int K, const WArgs& w, f16* y, int64_t ldy,
                 const f16* colscale, hipStream_t st, const char* name) {
  if (M > 128)
    return launch_tile<mp::Tile<256, 192, 2, 2>, WArgs, kColScale>(x, ldx, M, N, K, w, y, ldy, colscale, st, name);
  return launch_tile<mp::Tile<128, 128, 2, 2>, WArgs, kColScale>(x, ldx, M, N, K, w, y, ldy, colscale, st, name);
}

}  // namespace

namespace intent {

int w4a16_check(const void* x, int64_t M, int64_t K, int64_t x_ld, const uint8_t* packed, int64_t N,
                int64_t packed_ld, const void* scales, const uint8_t* zeros, int64_t qparam_ld, int64_t gs,
                const void* y, int64_t y_ld);
bool w4a16_fast(const void* x, int64_t K, int64_t x_ld, const uint8_t* packed, int64_t packed_ld, int64_t gs);
int w4a16_generic_launch(const void* x, int64_t M, int64_t K, int64_t x_ld, const uint8_t* packed, int64_t N,
                         int64_t packed_ld, const void* scales, const uint8_t* zeros, int64_t qparam_ld, int64_t gs,
                         void* y, int64_t y_ld, void* stream);
int w8a16_generic_launch(const void* x, int64_t M, int64_t K, int64_t x_ld, const int8_t* w, int64_t N, int64_t w_ld,
                         const void* scales, void* y, int64_t y_ld, void* stream);
int w4a16_gemv_launch(const void* x, int64_t M, int64_t K, int64_t x_ld, const uint8_t* packed, int64_t N,
                      int64_t packed_ld, const void* scales, const uint8_t* zeros, int64_t qparam_ld, int64_t gs,
                      void* y, int64_t y_ld, void* stream);

int w8a16_gemv_launch(const void* x, int64_t M, int64_t K, int64_t x_ld, const int8_t* w, int64_t N, int64_t w_ld,
                      const void* scales, void* y, int64_t y_ld, void* stream);

int w4a16_gemm_launch(const void* x, int64_t M, int64_t K, int64_t x_ld, const uint8_t* packed, int64_t N,
                      int64_t packed_ld, const void* scales, const uint8_t* zeros, int64_t qparam_ld, int64_t gs,
                      void* y, int64_t y_ld, void* stream) {
  if (M == 0 || N == 0) return INTENT_OK;
  if (!w4a16_fast(x, K, x_ld, packed, packed_ld, gs) || !(gs == 32 || gs % 64 == 0))
    return w4a16_generic_launch(x, M, K, x_ld, packed, N, packed_ld, scales, zeros, qparam_ld, gs, y, y_ld, stream);
  INTENT_REQUIRE(intent::fits_offset(N, packed_ld) && intent::fits_offset(N, qparam_ld * 2) &&
                     intent::fits_offset(256 + 1, x_ld * 2),
                 INTENT_ERR_UNSUPPORTED, "w4a16_gemm: operand too large for 31-bit buffer offsets");
  W4Args w{packed, packed_ld, (const f16*)scales, zeros, qparam_ld, (int)gs};
  if (gs % 64 == 0 && qparam_ld % 4 == 0 && intent::aligned4(scales) && intent::aligned4(zeros) && M > 128)
    return launch_dense<W4WinArgs, false>((const f16*)x, x_ld, (int)M, (int)N, (int)K, W4WinArgs{w}, (f16*)y, y_ld,
                                          nullptr, (hipStream_t)stream, "w4a16_gemm");
  return launch_dense<W4Args, false>((const f16*)x, x_ld, (int)M, (int)N, (int)K, w, (f16*)y, y_ld, nullptr,
                                       (hipStream_t)stream, "w4a16_gemm");
}

}  // namespace intent

namespace {

// quantized_gemm over an empty K: every element is the epilogue of a zero sum.
__global__ __launch_bounds__(256) void quantized_empty_k_kernel(const float* __restrict__ bias,
                                                                const f16* __restrict__ residual, int64_t ldr,
                                                                const float* __restrict__ oscale,
                                                                int8_t* __restrict__ out, int64_t ldo, int64_t M,
                                                                int64_t N) {
  const int64_t n = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (n >= N) return;
  for (int64_t m = blockIdx.y; m < M; m += gridDim.y)
    out[m * ldo + n] = (int8_t)quant_i8_epilogue(0.f, bias[n], residual[m * ldr + n], oscale[n]);
}

// Grouped GEMMs over an empty K: zeros in the rows the groups cover (output
// row idx, or routes[idx] for routed rows, for offsets[g] <= idx < offsets[g + 1]).
__global__ __launch_bounds__(256) void grouped_empty_k_kernel(const int32_t* __restrict__ offsets, int64_t G,
                                                              const int32_t* __restrict__ routes, int64_t rows,
                                                              uint16_t* __restrict__ out, int64_t ldo, int64_t N) {
  const int64_t n = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (n >= N) return;
  for (int64_t g = blockIdx.y; g < G; g += gridDim.y) {
    const int64_t lo = offsets[g] > 0 ? offsets[g] : 0;
    const int64_t hi = offsets[g + 1] < rows ? offsets[g + 1] : rows;
    for (int64_t idx = lo; idx < hi; ++idx) out[(routes ? (int64_t)routes[idx] : idx) * ldo + n] = 0;
  }
}

int quantized_empty_k(const float* bias, const void* residual, int64_t residual_ld, const float* oscale, int8_t* out,
                      int64_t out_ld, int64_t M, int64_t N, void* stream) {
  INTENT_REQUIRE(bias && residual && oscale && out, INTENT_ERR_INVALID_ARGUMENT, "null pointer argument");
  INTENT_REQUIRE(residual_ld >= N && out_ld >= N, INTENT_ERR_INVALID_ARGUMENT, "leading stride smaller than the row");
  const dim3 grid((unsigned)((N + 255) / 256), (unsigned)(M < 65535 ? M : 65535));
  hipLaunchKernelGGL(quantized_empty_k_kernel, grid, dim3(256), 0, (hipStream_t)stream, bias, (const f16*)residual,
                     residual_ld, oscale, out, out_ld, M, N);
  return intent::launch_status("quantized_empty_k_kernel");
}

}  // namespace

namespace intent {

int grouped_empty_k(const int32_t* offsets, int64_t G, const int32_t* routes, int64_t rows, void* out, int64_t out_ld,
                    int64_t N, void* stream) {
  INTENT_REQUIRE(offsets && out && out_ld >= N, INTENT_ERR_INVALID_ARGUMENT, "null pointer or short output stride");
  const dim3 grid((unsigned)((N + 255) / 256), (unsigned)(G < 4096 ? G : 4096));
  hipLaunchKernelGGL(grouped_empty_k_kernel, grid, dim3(256), 0, (hipStream_t)stream, offsets, G, routes, rows,
                     (uint16_t*)out, out_ld, N);
  return launch_status("grouped_empty_k_kernel");
}

}  // namespace intent

extern "C" int intent_w4a16_matmul(const void* x, int64_t M, int64_t K, int64_t x_ld, const uint8_t* packed, int64_t N,
                                   int64_t packed_ld, const void* scales, const uint8_t* zeros, int64_t qparam_ld,
                                   int64_t group_size, void* y, int64_t y_ld, void* stream) {
  intent::clear_error();
  int st = intent::w4a16_check(x, M, K, x_ld, packed, N, packed_ld, scales, zeros, qparam_ld, group_size, y, y_ld);
  if (st != INTENT_OK) return st;
  if (M <= 16 && intent::w4a16_fast(x, K, x_ld, packed, packed_ld, group_size))
    return intent::w4a16_gemv_launch(x, M, K, x_ld, packed, N, packed_ld, scales, zeros, qparam_ld, group_size, y,
                                     y_ld, stream);
  return intent::w4a16_gemm_launch(x, M, K, x_ld, packed, N, packed_ld, scales, zeros, qparam_ld, group_size, y, y_ld,
                                   stream);
}

extern "C" int intent_w4a16_gemv(const void* x, int64_t M, int64_t K, int64_t x_ld, const uint8_t* packed, int64_t N,
                                 int64_t packed_ld, const void* scales, const uint8_t* zeros, int64_t qparam_ld,
                                 int64_t group_size, void* y, int64_t y_ld, void* stream) {
  intent::clear_error();
  int st = intent::w4a16_check(x, M, K, x_ld, packed, N, packed_ld, scales, zeros, qparam_ld, group_size, y, y_ld);
  if (st != INTENT_OK) return st;
  INTENT_REQUIRE(M <= 16, INTENT_ERR_UNSUPPORTED, "the GEMV covers M <= 16, got M=%lld", (long long)M);
  if (M == 0 || N == 0) return INTENT_OK;
  if (!intent::w4a16_fast(x, K, x_ld, packed, packed_ld, group_size))
    return intent::w4a16_generic_launch(x, M, K, x_ld, packed, N, packed_ld, scales, zeros, qparam_ld, group_size, y,
                                        y_ld, stream);
  return intent::w4a16_gemv_launch(x, M, K, x_ld, packed, N, packed_ld, scales, zeros, qparam_ld, group_size, y, y_ld,
                                   stream);
}

extern "C" int intent_w4a16_gemm(const void* x, int64_t M, int64_t K, int64_t x_ld, const uint8_t* packed, int64_t N,
                                 int64_t packed_ld, const void* scales, const uint8_t* zeros, int64_t qparam_ld,
                                 int64_t group_size, void* y, int64_t y_ld, void* stream) {
  intent::clear_error();
  int st = intent::w4a16_check(x, M, K, x_ld, packed, N, packed_ld, scales, zeros, qparam_ld, group_size, y, y_ld);
  if (st != INTENT_OK) return st;
  return intent::w4a16_gemm_launch(x, M, K, x_ld, packed, N, packed_ld, scales, zeros, qparam_ld, group_size, y, y_ld,
                                   stream);
}

extern "C" int intent_w8a16_matmul(const void* x, int64_t M, int64_t K, int64_t x_ld, const int8_t* w, int64_t N,
                                   int64_t w_ld, const void* scales, void* y, int64_t y_ld, void* stream) {
  intent::clear_error();
  INTENT_REQUIRE(M >= 0 && N >= 0 && K >= 0, INTENT_ERR_INVALID_ARGUMENT, "negative extent");
  INTENT_REQUIRE(M <= INT32_MAX && N <= INT32_MAX && K <= INT32_MAX, INTENT_ERR_UNSUPPORTED, "extent exceeds int32");
  if (M == 0 || N == 0) return INTENT_OK;
  INTENT_REQUIRE(scales && y && (K == 0 || (x && w)), INTENT_ERR_INVALID_ARGUMENT, "null pointer argument");
  INTENT_REQUIRE(x_ld >= K && w_ld >= K && y_ld >= N, INTENT_ERR_INVALID_ARGUMENT, "leading stride smaller than the row");
  // the tiled kernels take whole 64-k stages of 16-byte aligned rows; other shapes (and an empty K,
  // y = f16(0 * scale)) run the generic kernel
  if (K == 0 || K % 64 != 0 || !intent::aligned16(x) || !intent::aligned16(w) || x_ld % 8 != 0 || w_ld % 16 != 0)
    return intent::w8a16_generic_launch(x, M, K, x_ld, w, N, w_ld, scales, y, y_ld, stream);
  if (M <= 16) return intent::w8a16_gemv_launch(x, M, K, x_ld, w, N, w_ld, scales, y, y_ld, stream);
  INTENT_REQUIRE(intent::fits_offset(N, w_ld) && intent::fits_offset(256 + 1, x_ld * 2), INTENT_ERR_UNSUPPORTED,
                 "w8a16_matmul: operand too large for 31-bit buffer offsets");
  W8Args ws{w, w_ld};
  return launch_dense<W8Args, true>((const f16*)x, x_ld, (int)M, (int)N, (int)K, ws, (f16*)y, y_ld,
                                      (const f16*)scales, (hipStream_t)stream, "w8a16_matmul");
}

extern "C" int intent_fp4_bf16_matmul(const void* x, int64_t M, int64_t K, int64_t x_ld, const uint8_t* packed,
                                      int64_t N, int64_t packed_ld, void* y, int64_t y_ld, void* stream) {
  intent::clear_error();
  INTENT_REQUIRE(M >= 0 && N >= 0 && K >= 0 && M <= INT32_MAX && N <= INT32_MAX && K <= INT32_MAX,
                 INTENT_ERR_INVALID_ARGUMENT, "bad extents");
  INTENT_REQUIRE(K % 64 == 0, INTENT_ERR_UNSUPPORTED, "K must be a multiple of 64, got %lld", (long long)K);
  if (M == 0 || N == 0) return INTENT_OK;
  if (K == 0) return intent::fill_launch(y, M, N, y_ld, 2, 0u, stream);  // bf16(0)
  INTENT_REQUIRE(x && packed && y, INTENT_ERR_INVALID_ARGUMENT, "null pointer argument");
  INTENT_REQUIRE(x_ld >= K && packed_ld >= K / 2 && y_ld >= N, INTENT_ERR_INVALID_ARGUMENT,
                 "leading stride smaller than the row");
  INTENT_REQUIRE(intent::aligned16(x) && x_ld % 8 == 0 && intent::aligned16(packed) && packed_ld % 16 == 0,
                 INTENT_ERR_ALIGNMENT, "x and packed must be 16-byte aligned with 16-byte row strides");
  INTENT_REQUIRE(intent::fits_offset(N, packed_ld) && intent::fits_offset(M, x_ld * 2), INTENT_ERR_UNSUPPORTED,
                 "fp4_bf16_matmul: operand too large for 31-bit buffer offsets");
  auto launch = [&](auto tile) -> int {
    using T = decltype(tile);
    const int mblocks = (int)((M + T::BM - 1) / T::BM);
    const int64_t grid = (int64_t)mblocks * ((N + T::BN - 1) / T::BN);
    INTENT_REQUIRE(grid < (1ll << 31), INTENT_ERR_UNSUPPORTED, "fp4_bf16_matmul: grid too large");
    hipLaunchKernelGGL((fp4_bf16_gemm_kernel<T>), dim3((unsigned)grid), dim3(T::NT_WS), 0, (hipStream_t)stream,
                       (const uint16_t*)x, x_ld, (int)M, packed, packed_ld, (int)N, (int)K, (uint16_t*)y, y_ld,
                       mblocks);
    return intent::launch_status("fp4_bf16_matmul");
  };
  // 256 x 128 tiles (consumers of 128 x 64) once M fills them: at 4096 x 4096
  // that is 512 workgroups, two full rounds of 256 CUs (256 x 192 gives 1.38).
  if (M > 128) return launch(mp::Tile<256, 128, 2, 2>{});
  return launch(mp::Tile<128, 128, 2, 2>{});
}

extern "C" int intent_w4_sym_repack(const int32_t* packed, int64_t P, int64_t N, int64_t packed_ld,
                                    const void* scales, int64_t G, int64_t scales_ld, uint8_t* q_out, int64_t q_ld,
                                    void* s_out, uint8_t* z_out, int64_t sz_ld, void* stream) {
  intent::clear_error();
  INTENT_REQUIRE(P >= 0 && N >= 0 && G >= 0 && P <= INT32_MAX && N <= INT32_MAX && G <= INT32_MAX,
                 INTENT_ERR_INVALID_ARGUMENT, "bad extents");
  if (N == 0) return INTENT_OK;
  INTENT_REQUIRE(packed_ld >= N && scales_ld >= N && q_ld >= 4 * P && sz_ld >= G, INTENT_ERR_INVALID_ARGUMENT,
                 "leading stride smaller than the row");
  INTENT_REQUIRE((P == 0 || (packed && q_out)) && (G == 0 || (scales && s_out && z_out)), INTENT_ERR_INVALID_ARGUMENT,
                 "null pointer argument");
  INTENT_REQUIRE(q_ld % 4 == 0 && intent::aligned4(q_out), INTENT_ERR_ALIGNMENT, "q_out rows must be 4-byte aligned");
  hipStream_t st = (hipStream_t)stream;
  if (P > 0) {
    hipLaunchKernelGGL((transpose32_kernel<uint32_t, 0x88888888u>), dim3((unsigned)((N + 31) / 32), (unsigned)((P + 31) / 32)),
                       dim3(256), 0, st, (const uint32_t*)packed, (int)P, (int)N, packed_ld, (uint32_t*)q_out, q_ld / 4);
    int rc = intent::launch_status("w4_sym_repack");
    if (rc != INTENT_OK) return rc;
  }
  if (G > 0) {
    hipLaunchKernelGGL((transpose32_kernel<uint16_t, 0u>), dim3((unsigned)((N + 31) / 32), (unsigned)((G + 31) / 32)),
                       dim3(256), 0, st, (const uint16_t*)scales, (int)G, (int)N, scales_ld, (uint16_t*)s_out, sz_ld);
    int rc = intent::launch_status("w4_sym_repack");
    if (rc != INTENT_OK) return rc;
    hipLaunchKernelGGL(fill_u8_kernel, dim3((unsigned)((N * G + 255) / 256)), dim3(256), 0, st, z_out, (int)N, (int)G,
                       sz_ld, (uint8_t)8);
  }
  return intent::launch_status("w4_sym_repack");
}

extern "C" int intent_f16_transpose(const void* src, int64_t rows, int64_t cols, int64_t src_ld, void* dst,
                                    int64_t dst_ld, void* stream) {
  intent::clear_error();
  INTENT_REQUIRE(rows >= 0 && cols >= 0 && rows <= INT32_MAX && cols <= INT32_MAX, INTENT_ERR_INVALID_ARGUMENT,
                 "bad extents");
  if (rows == 0 || cols == 0) return INTENT_OK;
  INTENT_REQUIRE(src && dst, INTENT_ERR_INVALID_ARGUMENT, "null pointer argument");
  INTENT_REQUIRE(src_ld >= cols && dst_ld >= rows, INTENT_ERR_INVALID_ARGUMENT, "leading stride smaller than the row");
  INTENT_REQUIRE((rows + 63) / 64 < 65536, INTENT_ERR_UNSUPPORTED, "f16_transpose: grid too large");
  hipLaunchKernelGGL(transpose16_kernel, dim3((unsigned)((cols + 63) / 64), (unsigned)((rows + 63) / 64)), dim3(256), 0,
                     (hipStream_t)stream, (const uint16_t*)src, (int)rows, (int)cols, src_ld, (uint16_t*)dst, dst_ld,
                     (int64_t)0, (int64_t)0);
  return intent::launch_status("f16_transpose");
}

extern "C" int intent_quantized_gemm(const void* a, int64_t M, int64_t K, int64_t a_ld, const void* bt, int64_t N,
                                     int64_t bt_ld, const float* bias, const void* residual, int64_t residual_ld,
                                     const float* output_scale, int8_t* out, int64_t out_ld, void* stream) {
  intent::clear_error();
  INTENT_REQUIRE(M >= 0 && N >= 0 && K >= 0 && M <= INT32_MAX && N <= INT32_MAX && K <= INT32_MAX,
                 INTENT_ERR_INVALID_ARGUMENT, "bad extents");
  INTENT_REQUIRE(K % 64 == 0, INTENT_ERR_UNSUPPORTED, "K must be a multiple of 64, got %lld", (long long)K);
  if (M == 0 || N == 0) return INTENT_OK;
  if (K == 0) return quantized_empty_k(bias, residual, residual_ld, output_scale, out, out_ld, M, N, stream);
  INTENT_REQUIRE(a && bt && bias && residual && output_scale && out, INTENT_ERR_INVALID_ARGUMENT,
                 "null pointer argument");
  INTENT_REQUIRE(a_ld >= K && bt_ld >= K && residual_ld >= N && out_ld >= N, INTENT_ERR_INVALID_ARGUMENT,
                 "leading stride smaller than the row");
  INTENT_REQUIRE(intent::aligned16(a) && intent::aligned16(bt) && a_ld % 8 == 0 && bt_ld % 8 == 0,
                 INTENT_ERR_ALIGNMENT, "operands must be 16-byte aligned with 16-byte row strides");
  INTENT_REQUIRE(intent::fits_offset(M, a_ld * 2) && intent::fits_offset(N, bt_ld * 2), INTENT_ERR_UNSUPPORTED,
                 "quantized_gemm: operand too large for 31-bit buffer offsets");
  using T = mp::Tile<256, 192, 2, 2>;  // producer/consumer: 4 consumers of 128 x 96 + 4 producers
  const int mblocks = (int)((M + T::BM - 1) / T::BM);
  const int64_t grid = (int64_t)mblocks * ((N + T::BN - 1) / T::BN);
  INTENT_REQUIRE(grid < (1ll << 31), INTENT_ERR_UNSUPPORTED, "quantized_gemm: grid too large");
  hipLaunchKernelGGL((quantized_gemm_kernel<T>), dim3((unsigned)grid), dim3(T::NT_WS), 0, (hipStream_t)stream,
                     (const f16*)a, a_ld, (int)M, (const f16*)bt, bt_ld, (int)N, (int)K, bias, (const f16*)residual,
                     residual_ld, output_scale, out, out_ld, mblocks);
  return intent::launch_status("quantized_gemm");
}

extern "C" int intent_f16_transpose_batched(const void* src, int64_t batch, int64_t rows, int64_t cols,
                                            int64_t src_ld, int64_t src_batch, void* dst, int64_t dst_ld,
                                            int64_t dst_batch, void* stream) {
  intent::clear_error();
  INTENT_REQUIRE(batch >= 0 && rows >= 0 && cols >= 0 && rows <= INT32_MAX && cols <= INT32_MAX && batch < 65536,
                 INTENT_ERR_INVALID_ARGUMENT, "bad extents");
  if (batch == 0 || rows == 0 || cols == 0) return INTENT_OK;
  INTENT_REQUIRE(src && dst, INTENT_ERR_INVALID_ARGUMENT, "null pointer argument");
  INTENT_REQUIRE(src_ld >= cols && dst_ld >= rows, INTENT_ERR_INVALID_ARGUMENT, "leading stride smaller than the row");
  INTENT_REQUIRE((rows + 63) / 64 < 65536, INTENT_ERR_UNSUPPORTED, "f16_transpose: grid too large");
  hipLaunchKernelGGL(transpose16_kernel, dim3((unsigned)((cols + 63) / 64), (unsigned)((rows + 63) / 64), (unsigned)batch),
                     dim3(256), 0, (hipStream_t)stream, (const uint16_t*)src, (int)rows, (int)cols, src_ld,
                     (uint16_t*)dst, dst_ld, src_batch, dst_batch);
  return intent::launch_status("f16_transpose_batched");
}

extern "C" int intent_grouped_gemm(const void* x, int64_t rows, int64_t K, int64_t x_ld, const int32_t* offsets,
                                   int64_t G, const int32_t* routes, int64_t top_k, const void* w, int64_t N,
                                   int64_t w_ld, int64_t w_group_stride, int bf16, void* out, int64_t out_ld,
                                   void* stream) {
  intent::clear_error();
  INTENT_REQUIRE(rows >= 0 && K >= 0 && N >= 0 && G >= 0 && rows <= INT32_MAX && K <= INT32_MAX && N <= INT32_MAX,
                 INTENT_ERR_INVALID_ARGUMENT, "bad extents");
  INTENT_REQUIRE(K % 64 == 0, INTENT_ERR_UNSUPPORTED, "K must be a multiple of 64, got %lld", (long long)K);
  if (rows == 0 || N == 0 || G == 0) return INTENT_OK;
  INTENT_REQUIRE(!routes || top_k >= 1, INTENT_ERR_INVALID_ARGUMENT, "bad top_k");
  if (K == 0) return intent::grouped_empty_k(offsets, G, routes, rows, out, out_ld, N, stream);
  INTENT_REQUIRE(x && offsets && w && out, INTENT_ERR_INVALID_ARGUMENT, "null pointer argument");
  INTENT_REQUIRE(x_ld >= K && w_ld >= K && out_ld >= N && w_group_stride >= N * w_ld, INTENT_ERR_INVALID_ARGUMENT,
                 "leading stride smaller than the row");
  INTENT_REQUIRE(intent::aligned16(x) && intent::aligned16(w) && x_ld % 8 == 0 && w_ld % 8 == 0 &&
                     w_group_stride % 8 == 0,
                 INTENT_ERR_ALIGNMENT, "operands must be 16-byte aligned with 16-byte row strides");
  INTENT_REQUIRE(intent::fits_offset(N, w_ld * 2) && intent::fits_offset(rows, x_ld * 2), INTENT_ERR_UNSUPPORTED,
                 "grouped_gemm: operand too large for 31-bit buffer offsets");
  using T = mp::Tile<256, 256, 2, 2>;
  // Worst case per group: every row (or route) in one group.
  const int mbmax = (int)((rows + T::BM - 1) / T::BM);
  const int nblocks = (int)((N + T::BN - 1) / T::BN);
  const int64_t grid = G * mbmax * (int64_t)nblocks;
  INTENT_REQUIRE(grid < (1ll << 31), INTENT_ERR_UNSUPPORTED, "grouped_gemm: grid too large");
  const uint16_t* xx = (const uint16_t*)x;
  const uint16_t* ww = (const uint16_t*)w;
  uint16_t* oo = (uint16_t*)out;
  hipStream_t st = (hipStream_t)stream;
  if (routes && bf16)
    hipLaunchKernelGGL((grouped_gemm_kernel<T, mp::BF16Math, true>), dim3((unsigned)grid), dim3(T::NT), 0, st, xx,
                       x_ld, offsets, routes, (int)top_k, ww, w_ld, w_group_stride, (int)N, (int)K, mbmax, nblocks, oo,
                       out_ld);
  else if (routes)
    hipLaunchKernelGGL((grouped_gemm_kernel<T, mp::F16Math, true>), dim3((unsigned)grid), dim3(T::NT), 0, st, xx,
                       x_ld, offsets, routes, (int)top_k, ww, w_ld, w_group_stride, (int)N, (int)K, mbmax, nblocks, oo,
                       out_ld);
  else if (bf16)
    hipLaunchKernelGGL((grouped_gemm_kernel<T, mp::BF16Math, false>), dim3((unsigned)grid), dim3(T::NT), 0, st, xx,
                       x_ld, offsets, routes, 1, ww, w_ld, w_group_stride, (int)N, (int)K, mbmax, nblocks, oo, out_ld);
  else
    hipLaunchKernelGGL((grouped_gemm_kernel<T, mp::F16Math, false>), dim3((unsigned)grid), dim3(T::NT), 0, st, xx,
                       x_ld, offsets, routes, 1, ww, w_ld, w_group_stride, (int)N, (int)K, mbmax, nblocks, oo, out_ld);
  return intent::launch_status("grouped_gemm");
}

extern "C" int intent_f16_gemm(const void* a, int64_t M, int64_t K, int64_t a_ld, const void* bt, int64_t N,
                               int64_t bt_ld, int epilogue, void* c, int64_t c_ld, void* stream) {
  intent::clear_error();
  INTENT_REQUIRE(M >= 0 && N >= 0 && K >= 0 && M <= INT32_MAX && N <= INT32_MAX && K <= INT32_MAX,
                 INTENT_ERR_INVALID_ARGUMENT, "bad extents");
  INTENT_REQUIRE(epilogue >= 0 && epilogue <= 2, INTENT_ERR_INVALID_ARGUMENT,
                 "epilogue must be 0 (f16), 1 (f16 relu) or 2 (bf16)");
  INTENT_REQUIRE(K % 64 == 0, INTENT_ERR_UNSUPPORTED, "K must be a multiple of 64, got %lld", (long long)K);
  if (M == 0 || N == 0) return INTENT_OK;
  if (K == 0) return intent::fill_launch(c, M, N, c_ld, 2, 0u, stream);  // f16 / bf16 zero (relu(0) = 0)
  INTENT_REQUIRE(a && bt && c, INTENT_ERR_INVALID_ARGUMENT, "null pointer argument");
  INTENT_REQUIRE(a_ld >= K && bt_ld >= K && c_ld >= N, INTENT_ERR_INVALID_ARGUMENT,
                 "leading stride smaller than the row");
  INTENT_REQUIRE(intent::aligned16(a) && intent::aligned16(bt) && a_ld % 8 == 0 && bt_ld % 8 == 0,
                 INTENT_ERR_ALIGNMENT, "operands must be 16-byte aligned with 16-byte row strides");
  INTENT_REQUIRE(intent::fits_offset(M, a_ld * 2) && intent::fits_offset(N, bt_ld * 2), INTENT_ERR_UNSUPPORTED,
                 "f16_gemm: operand too large for 31-bit buffer offsets");
  using T = mp::Tile<256, 192, 2, 2>;
  const int mblocks = (int)((M + T::BM - 1) / T::BM);
  const int64_t grid = (int64_t)mblocks * ((N + T::BN - 1) / T::BN);
  INTENT_REQUIRE(grid < (1ll << 31), INTENT_ERR_UNSUPPORTED, "f16_gemm: grid too large");
  if (epilogue == 2)
    hipLaunchKernelGGL((quantized_gemm_kernel<T, DenseEpi::kGemmBf16, mp::BF16Math>), dim3((unsigned)grid),
                       dim3(T::NT_WS), 0, (hipStream_t)stream, (const f16*)a, a_ld, (int)M, (const f16*)bt, bt_ld,
                       (int)N, (int)K, nullptr, nullptr, 0, nullptr, (int8_t*)c, c_ld, mblocks, 0);
  else
    hipLaunchKernelGGL((quantized_gemm_kernel<T>), dim3((unsigned)grid), dim3(T::NT_WS), 0, (hipStream_t)stream,
                       (const f16*)a, a_ld, (int)M, (const f16*)bt, bt_ld, (int)N, (int)K, nullptr, nullptr, 0,
                       nullptr, (int8_t*)c, c_ld, mblocks, epilogue + 1);
  return intent::launch_status("f16_gemm");
}

namespace {

int gemm_kn_check(const void* a, int64_t M, int64_t K, int64_t a_ld, const void* b, int64_t N, int64_t b_ld,
                  int64_t c_ld, const char* what) {
  INTENT_REQUIRE(M >= 0 && N >= 0 && K >= 0 && M <= INT32_MAX && N <= INT32_MAX && K <= INT32_MAX,
                 INTENT_ERR_INVALID_ARGUMENT, "%s: bad extents", what);
  INTENT_REQUIRE(K % 64 == 0, INTENT_ERR_UNSUPPORTED, "%s: K must be a multiple of 64, got %lld", what, (long long)K);
  INTENT_REQUIRE(N % 8 == 0, INTENT_ERR_UNSUPPORTED, "%s: N must be a multiple of 8 for the [K, N] operand, got %lld",
                 what, (long long)N);
  if (M == 0 || N == 0 || K == 0) return INTENT_OK;  // an empty K reads no operand
  INTENT_REQUIRE(a && b, INTENT_ERR_INVALID_ARGUMENT, "%s: null pointer argument", what);
  INTENT_REQUIRE(a_ld >= K && b_ld >= N && c_ld >= N, INTENT_ERR_INVALID_ARGUMENT,
                 "%s: leading stride smaller than the row", what);
  INTENT_REQUIRE(intent::aligned16(a) && intent::aligned16(b) && a_ld % 8 == 0 && b_ld % 8 == 0,
                 INTENT_ERR_ALIGNMENT, "%s: operands must be 16-byte aligned with 16-byte row strides", what);
  INTENT_REQUIRE(intent::fits_offset(M, a_ld * 2) && intent::fits_offset(K, b_ld * 2), INTENT_ERR_UNSUPPORTED,
                 "%s: operand too large for 31-bit buffer offsets", what);
  return INTENT_OK;
}

// Eight waves (two per SIMD) of 128 x 64: measured at 4096 x 4096 x 14336
// (quantized_gemm) 525 us against 710 us for four waves of 128 x 128 (which
// spill) and 576 us without the MFMA / LDS-read interleaving schedule.
using KNTile = mp::Tile<256, 256, 2, 4>;

}  // namespace

extern "C" int intent_quantized_gemm_kn(const void* a, int64_t M, int64_t K, int64_t a_ld, const void* b, int64_t N,
                                        int64_t b_ld, const float* bias, const void* residual, int64_t residual_ld,
                                        const float* output_scale, int8_t* out, int64_t out_ld, void* stream) {
  intent::clear_error();
  int st = gemm_kn_check(a, M, K, a_ld, b, N, b_ld, out_ld, "quantized_gemm_kn");
  if (st != INTENT_OK || M == 0 || N == 0) return st;
  if (K == 0) return quantized_empty_k(bias, residual, residual_ld, output_scale, out, out_ld, M, N, stream);
  INTENT_REQUIRE(bias && residual && output_scale && out, INTENT_ERR_INVALID_ARGUMENT, "null pointer argument");
  INTENT_REQUIRE(residual_ld >= N, INTENT_ERR_INVALID_ARGUMENT, "leading stride smaller than the row");
  using T = KNTile;
  const int mblocks = (int)((M + T::BM - 1) / T::BM);
  const int64_t grid = (int64_t)mblocks * ((N + T::BN - 1) / T::BN);
  INTENT_REQUIRE(grid < (1ll << 31), INTENT_ERR_UNSUPPORTED, "quantized_gemm_kn: grid too large");
  hipLaunchKernelGGL((gemm_kn_kernel<T, DenseEpi::kQuantI8, mp::F16Math, true>), dim3((unsigned)grid), dim3(T::NT), 0,
                     (hipStream_t)stream, (const f16*)a, a_ld, (int)M, (const f16*)b, b_ld, (int)N, (int)K, bias,
                     (const f16*)residual, residual_ld, output_scale, out, out_ld, mblocks, 0);
  return intent::launch_status("gemm_kn_kernel<quantized_gemm>");
}

extern "C" int intent_f16_gemm_kn(const void* a, int64_t M, int64_t K, int64_t a_ld, const void* b, int64_t N,
                                  int64_t b_ld, int epilogue, void* c, int64_t c_ld, void* stream) {
  intent::clear_error();
  INTENT_REQUIRE(epilogue >= 0 && epilogue <= 2, INTENT_ERR_INVALID_ARGUMENT,
                 "epilogue must be 0 (f16), 1 (f16 relu) or 2 (bf16)");
  int st = gemm_kn_check(a, M, K, a_ld, b, N, b_ld, c_ld, "f16_gemm_kn");
  if (st != INTENT_OK || M == 0 || N == 0) return st;
  if (K == 0) return intent::fill_launch(c, M, N, c_ld, 2, 0u, stream);  // f16 / bf16 zero (relu(0) = 0)
  INTENT_REQUIRE(c, INTENT_ERR_INVALID_ARGUMENT, "null pointer argument");
  using T = KNTile;
  const int mblocks = (int)((M + T::BM - 1) / T::BM);
  const int64_t grid = (int64_t)mblocks * ((N + T::BN - 1) / T::BN);
  INTENT_REQUIRE(grid < (1ll << 31), INTENT_ERR_UNSUPPORTED, "f16_gemm_kn: grid too large");
  if (epilogue == 2)
    hipLaunchKernelGGL((gemm_kn_kernel<T, DenseEpi::kGemmBf16, mp::BF16Math, true>), dim3((unsigned)grid), dim3(T::NT), 0,
                       (hipStream_t)stream, (const f16*)a, a_ld, (int)M, (const f16*)b, b_ld, (int)N, (int)K, nullptr,
                       nullptr, 0, nullptr, (int8_t*)c, c_ld, mblocks, 0);
  else
    hipLaunchKernelGGL((gemm_kn_kernel<T, DenseEpi::kQuantI8, mp::F16Math, true>), dim3((unsigned)grid), dim3(T::NT),
                       0, (hipStream_t)stream, (const f16*)a, a_ld, (int)M, (const f16*)b, b_ld, (int)N, (int)K,
                       nullptr, nullptr, 0, nullptr, (int8_t*)c, c_ld, mblocks, epilogue + 1);
  return intent::launch_status(epilogue == 2 ? "gemm_kn_kernel<bf16>" : "gemm_kn_kernel<f16>");
}

extern "C" int intent_w4a16_sym_gemm(const void* x, int64_t M, int64_t K, int64_t x_ld, const int32_t* packed,
                                     int64_t N, int64_t packed_ld, const void* scales, int64_t scales_ld, void* y,
                                     int64_t y_ld, void* stream) {
  intent::clear_error();
  INTENT_REQUIRE(M >= 0 && N >= 0 && K >= 0 && M <= INT32_MAX && N <= INT32_MAX && K <= INT32_MAX,
                 INTENT_ERR_INVALID_ARGUMENT, "bad extents");
  INTENT_REQUIRE(K % 64 == 0, INTENT_ERR_UNSUPPORTED, "w4a16_sym_gemm: K must be a multiple of 64, got %lld",
                 (long long)K);
  if (M == 0 || N == 0) return INTENT_OK;
  INTENT_REQUIRE(K > 0, INTENT_ERR_UNSUPPORTED, "w4a16_sym_gemm: K must be positive");
  INTENT_REQUIRE(x && packed && scales && y, INTENT_ERR_INVALID_ARGUMENT, "null pointer argument");
  INTENT_REQUIRE(x_ld >= K && packed_ld >= N && scales_ld >= N && y_ld >= N, INTENT_ERR_INVALID_ARGUMENT,
                 "leading stride smaller than the row");
  INTENT_REQUIRE(intent::aligned16(x) && x_ld % 8 == 0 && intent::aligned4(packed) &&
                     (reinterpret_cast<uintptr_t>(scales) & 1) == 0,
                 INTENT_ERR_ALIGNMENT, "w4a16_sym_gemm: 16-byte aligned activation rows, aligned words and scales");
  INTENT_REQUIRE(intent::fits_offset(K / 8, packed_ld * 4) && intent::fits_offset(K / 64, scales_ld * 2) &&
                     intent::fits_offset(256 + 1, x_ld * 2),
                 INTENT_ERR_UNSUPPORTED, "w4a16_sym_gemm: operand too large for 31-bit buffer offsets");
  W4SymArgs w{packed, packed_ld, (const f16*)scales, scales_ld};
  return launch_dense<W4SymArgs, false>((const f16*)x, x_ld, (int)M, (int)N, (int)K, w, (f16*)y, y_ld, nullptr,
                                        (hipStream_t)stream, "w4a16_sym_gemm");
}
