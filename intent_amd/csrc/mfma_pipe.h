// Software-pipelined MFMA GEMM core for gfx950 (f16 and int8 operands).
//
//   acc[m, n] = sum_k A[m, k] * B[n, k]          (A rows: activations, B rows: weights)
//
// Both operands are staged through LDS one k-stage at a time. A stage holds
// 128 bytes of every tile row: 64 k of f16 or 128 k of int8. Operands go
// global -> VGPR (buffer loads) -> LDS (ds_write_b128); quantized weights are
// decoded to f16 on the way. Two register sets and two LDS buffers keep two
// stages in flight per workgroup (128 KB for a 256 x 256 int8 tile), which is
// what the L2/MALL latency under a full-chip load needs to stay hidden.
//
// LDS layout of a stage row: eight 16-byte chunks; chunk c of row r sits in
// slot c ^ ((r >> 1) & 7). Sixteen consecutive rows reading the same chunk then
// hit sixteen distinct (bank half, slot) pairs, so the 32-row fragment reads of
// v_mfma_*_32x32x* are conflict-free.
//
// Pipeline, one barrier per stage (step kt computes on LDS buffer kt % 2):
//   top:    buffer loads of stage kt+2 into register set kt % 2;
//   middle: MFMAs of stage kt, fragment reads of step kk+1 interleaved with
//           the MFMAs of step kk;
//   end:    stage kt+1 (register set (kt+1) % 2, loaded one step earlier)
//           written to the other LDS buffer; lgkmcnt wait; barrier.
//
// Each wave owns a (BM/WM) x (BN/WN) block of 32 x 32 MFMA tiles. The MFMA
// is issued as mfma(Bfrag, Afrag), so a lane's accumulator holds one m and
// four consecutive n per 4-register group:
//   m = wave_m*(BM/WM) + i*32 + lane%32
//   n = wave_n*(BN/WN) + j*32 + (v/4)*8 + (lane/32)*4 + v%4
// which lets epilogues store 4 (f16/bf16) or 4 (f32/i32) adjacent outputs.
#pragma once

// Measurement-only switches, 0 in the product build. `python -m intent_amd.build
// --ablations` links separate libraries with them set, which `bench.py --probe
// ablation` times beside the product library to split a kernel's time:
//   bit 0: the int8/f16 main loop (mainloop) issues no global loads after its
//          first two stages (later stages compute on stale register data);
//   bit 1: ... and writes nothing to its LDS stage buffers after the first;
//   bit 2: the W8A8 epilogue stores nothing (the accumulators stay live);
//   bit 3: the FP4 x bf16 producers copy the packed words instead of decoding.
// Results are meaningless with any bit set; only the timing is of interest.
#ifndef INTENT_ABLATE
#define INTENT_ABLATE 0
#endif

#include <type_traits>

#include "common.h"

namespace mp {

constexpr int ROWB = 128;  // bytes per tile row per stage
constexpr int NTHREADS = 256;  // default workgroup: 4 waves

typedef __attribute__((address_space(3))) void lds_t;

INTENT_DEVICE constexpr int swz(int row) { return (row >> 1) & 7; }

// f(std::integral_constant<int, S>) for S = B .. E-1.
template <int B, int E, class F>
INTENT_DEVICE void static_for_mp(F&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    static_for_mp<B + 1, E>(f);
  }
}

using Rsrc = __amdgpu_buffer_rsrc_t;

// Buffer load of BYTES (4 or 16) per lane straight into LDS: lane l's bytes
// land at lds + l * BYTES (M0 holds the workgroup-relative LDS byte address)
// and come from buffer base + voff + soff.
//
// kAsm = false: the compiler builtin. The compiler's wait insertion then makes
// LDS reads that follow such a DMA wait for all outstanding loads (vmcnt 0),
// the next stages' DMA included, whenever it cannot tell which LDS bytes the
// DMA writes. kAsm = true: the same instructions as assembly, which that pass
// does not track; a pipeline using it orders every read of DMA-written LDS
// with its own vmcnt waits and barriers, and keeps the compiler's own vector
// loads (spill reloads included) out of its loop, since their waits would
// drain the DMA too. Which form is faster depends on the kernel's schedule,
// so each pipeline picks the one measured faster.
template <int BYTES, bool kAsm>
INTENT_DEVICE void lds_dma(Rsrc rs, lds_t* lds, uint32_t voff, uint32_t soff) {
  static_assert(BYTES == 4 || BYTES == 16, "dword or dwordx4");
  if constexpr (!kAsm) {
    if constexpr (BYTES == 16)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, lds, 16, voff, soff, 0, 0);
    else
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, lds, 4, voff, soff, 0, 0);
  } else {
    // M0 is an input operand ("{m0}"), so the compiler writes it and knows it
    // is overwritten; the s_nop is the one wait state gfx9 needs between an
    // SALU write of M0 and an LDS DMA that reads it (inline assembly gets no
    // hazard padding). The resource and offset SGPRs must not be VALU results
    // of the last 5 wait states; intent_amd/codeobj_check.py rejects a build
    // where they are, or where such a kernel uses scratch.
    const uint32_t m = (uint32_t)(uintptr_t)lds;
    if constexpr (BYTES == 16)
      asm volatile("s_nop 0\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds"
                   :
                   : "v"(voff), "s"(rs), "s"(soff), "{m0}"(m)
                   : "memory");
    else
      asm volatile("s_nop 0\n\tbuffer_load_dword %0, %1, %2 offen lds"
                   :
                   : "v"(voff), "s"(rs), "s"(soff), "{m0}"(m)
                   : "memory");
  }
}

// s_waitcnt with only vmcnt constrained (expcnt 7, lgkmcnt 15 = no wait).
template <int N>
INTENT_DEVICE void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}
// s_waitcnt vmcnt(N) lgkmcnt(0), then a workgroup barrier.
template <int N>
INTENT_DEVICE void wait_vm_lgkm_barrier() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (0 << 8));
  __builtin_amdgcn_s_barrier();
}

// ds_write_b128 that the compiler does not see as an LDS access. Producer
// waves write decoded weights into a stage buffer while LDS DMAs into other
// buffers are in flight; a visible LDS store there would make the compiler's
// wait-count pass wait for those DMAs. The caller waits lgkmcnt before the
// barrier that publishes the stage.
INTENT_DEVICE void lds_store16(char* p, u32x4 v) {
  const uint32_t a = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)p;
  asm volatile("ds_write_b128 %0, %1" : : "v"(a), "v"(v) : "memory");
}

template <int BM_, int BN_, int WM_, int WN_>
struct Tile {
  static constexpr int BM = BM_;
  static constexpr int BN = BN_;
  static constexpr int WM = WM_;
  static constexpr int WN = WN_;
  static constexpr int NW = WM * WN;  // waves: 4 (one per SIMD) or 8 (two per SIMD)
  static constexpr int NT = NW * 64;
  static_assert(NW == 4 || NW == 8, "four or eight waves");
  // Producer/consumer workgroups (mainloop_ws): NW consumer waves plus NW
  // producer waves, one of each per SIMD.
  static constexpr int NT_WS = 2 * NT;
  static constexpr int WTM = BM / WM;
  static constexpr int WTN = BN / WN;
  static constexpr int TI = WTM / 32;
  static constexpr int TJ = WTN / 32;
  static_assert(TI * 32 * WM == BM && TJ * 32 * WN == BN, "tile shape");
  static constexpr int A_BYTES = BM * ROWB;
  static constexpr int STAGE_BYTES = (BM + BN) * ROWB;

  INTENT_DEVICE static int wave() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }
  INTENT_DEVICE static int wave_m() { return wave() % WM; }
  INTENT_DEVICE static int wave_n() { return wave() / WM; }
  // Tile-local output coordinates of accumulator acc[i][j], register group g (0..3).
  INTENT_DEVICE static int row(int i) { return wave_m() * WTM + i * 32 + (threadIdx.x & 31); }
  INTENT_DEVICE static int col(int j, int g) { return wave_n() * WTN + j * 32 + g * 8 + ((threadIdx.x >> 5) & 1) * 4; }
};

struct F16Math {
  using Acc = f32x16;
  using Frag = f16x8;
  INTENT_DEVICE static Acc mfma(Frag b, Frag a, Acc c) { return __builtin_amdgcn_mfma_f32_32x32x16_f16(b, a, c, 0, 0, 0); }
};
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
struct BF16Math {
  using Acc = f32x16;
  using Frag = bf16x8;
  INTENT_DEVICE static Acc mfma(Frag b, Frag a, Acc c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(b, a, c, 0, 0, 0);
  }
};
struct I8Math {
  using Acc = i32x16;
  using Frag = i32x4;
  INTENT_DEVICE static Acc mfma(Frag b, Frag a, Acc c) { return __builtin_amdgcn_mfma_i32_32x32x32_i8(b, a, c, 0, 0, 0); }
};
// E4M3 x E4M3 -> f32 on the f8f6f4 MFMA (32 x 32 x 64, block scales 2^0).
// Its operands are 32 bytes per lane, so the main loops feed it pairs of the
// 16-byte fragments the other maths use (kPairs): steps 2s and 2s + 1 of a
// stage together. A and B take the same k positions, so only the summation
// order within an MFMA differs from the row order.
typedef int i32x8 __attribute__((ext_vector_type(8)));
struct F8Math {
  using Acc = f32x16;
  using Frag = i32x4;
  static constexpr bool kPairs = true;
  INTENT_DEVICE static Acc mfma2(Frag b0, Frag b1, Frag a0, Frag a1, Acc c) {
    const i32x8 b{b0[0], b0[1], b0[2], b0[3], b1[0], b1[1], b1[2], b1[3]};
    const i32x8 a{a0[0], a0[1], a0[2], a0[3], a1[0], a1[1], a1[2], a1[3]};
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(b, a, c, 0, 0, 0, 127, 0, 127);
  }
};
template <class Math, class = void>
struct PairedFrags : std::false_type {};
template <class Math>
struct PairedFrags<Math, std::void_t<decltype(Math::kPairs)>> : std::bool_constant<Math::kPairs> {};

// ---- row sources: byte offset of tile row p from a per-tile base --------------
// Rows that hold no data map to some valid row; loads stay unpredicated and
// epilogues never store those rows.

struct DenseRows {  // rows m0.. of a row-major matrix; rows >= M clamp to M-1
  const void* base;
  int64_t ld_bytes;
  int M;
  INTENT_DEVICE const void* tile_base(int m0) const { return (const char*)base + (int64_t)m0 * ld_bytes; }
  INTENT_DEVICE uint32_t off(int m0, int p) const {
    const int m = m0 + p;
    return (uint32_t)((m < M ? p : M - 1 - m0) * ld_bytes);
  }
};

// Rows m0.. of a row-major matrix whose tile rows all exist (no clamp): row p
// sits p * ld_bytes after the tile base, so the DMA of consecutive row groups
// differs by a uniform offset.
struct LinearRows {
  static constexpr bool kLinear = true;
  const void* base;
  int64_t ld_bytes;
  INTENT_DEVICE const void* tile_base(int m0) const { return (const char*)base + (int64_t)m0 * ld_bytes; }
  INTENT_DEVICE uint32_t off(int, int p) const { return (uint32_t)(p * ld_bytes); }
};

template <class R, class = void>
struct IsLinearRows : std::false_type {};
template <class R>
struct IsLinearRows<R, std::void_t<decltype(R::kLinear)>> : std::bool_constant<R::kLinear> {};

struct GatherRows {  // MoE gate/up: padded row p holds route sorted[p]; token = route / top_k
  const void* base;
  int64_t ld_bytes;
  const int32_t* sorted;
  int R;
  int top_k;
  INTENT_DEVICE const void* tile_base(int) const { return base; }
  INTENT_DEVICE uint32_t off(int m0, int p) const {
    const int r = sorted[m0 + p];
    return (uint32_t)(((r >= 0 && r < R) ? r / top_k : 0) * ld_bytes);
  }
};

// ---- operand staging ----------------------------------------------------------

// Raw rows (f16 activations, int8 operands): lane i of instruction j holds
// 16 bytes of tile row (NW*j + wave) * 8 + i/8 and writes LDS slot i % 8 of that
// row, so it fetches chunk (i % 8) ^ swz(row). A half stage (64 bytes, int8
// with K % 128 == 64) re-reads chunks 0..3 instead of running past the row.
template <int ROWS, class Rows, bool kHalf = false, int NW = 4>
struct RegRowsOperand {
  static constexpr int N_INST = ROWS / (8 * NW);
  static_assert(N_INST * 8 * NW == ROWS, "tile rows must be a multiple of 8 per wave");
  static constexpr int NVM = N_INST;
  static constexpr int NDS = N_INST;  // LDS writes per stage
  Rsrc rs;
  uint32_t voff[N_INST];
  uint32_t lds_off[N_INST];
  int half_kt;        // stage index that is a half stage, or -1
  uint32_t half_adj;  // 64 if this lane fetches a chunk in 4..7, else 0
  struct Regs {
    u32x4 v[N_INST];
  };
  INTENT_DEVICE void init(const Rows& rows, int m0, int wave, int half_stage = -1) {
    rs = make_rsrc(rows.tile_base(m0));
    half_kt = half_stage;
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int j = 0; j < N_INST; ++j) {
      const int r = (j * NW + wave) * 8 + (lane >> 3);
      const int chunk = (lane & 7) ^ swz(r);
      voff[j] = rows.off(m0, r) + chunk * 16;
      lds_off[j] = (uint32_t)(r * ROWB + (lane & 7) * 16);
    }
    // swz(row) does not depend on j, so neither does the fetched chunk.
    half_adj = (((lane & 7) ^ swz((wave * 8) + (lane >> 3))) >= 4) ? 64u : 0u;
  }
  INTENT_DEVICE void load(int kt, Regs& r) const {
    const uint32_t adj = (kHalf && kt == half_kt) ? half_adj : 0u;
#pragma unroll
    for (int j = 0; j < N_INST; ++j) r.v[j] = __builtin_amdgcn_raw_buffer_load_b128(rs, voff[j] - adj, (uint32_t)kt * ROWB, 0);
  }
  template <bool kAsm = false>  // kAsm: see lds_store16
  INTENT_DEVICE void store(const Regs& r, char* lds_region) const {
#pragma unroll
    for (int j = 0; j < N_INST; ++j) {
      if constexpr (kAsm)
        lds_store16(lds_region + lds_off[j], r.v[j]);
      else
        *reinterpret_cast<u32x4*>(lds_region + lds_off[j]) = r.v[j];
    }
  }
};

// Packed low-bit weight rows decoded to int8 on the way to LDS, for the int8
// MFMA path. Same row / slot assignment as RegRowsOperand (lane i of
// instruction j: tile row (NW*j + wave)*8 + i/8, LDS slot i%8 holding 16-k
// chunk (i%8) ^ swz(row)); a lane loads only the packed bytes of its chunk.
//   kSignedNibble: two 4-bit values per byte, low nibble = even k, decoded
//     as two's complement (n - 2*(n & 8)) (weight_only_int4.py:54-91);
//   kInt2: four 2-bit values (0..3) per byte, interleaved: k lives in byte
//     (k/16)*4 + k%4 at bit 2*((k/4)%4) (weight_only_int4.py:94-124), so the
//     16-k chunk c is packed dword c and output dword a is (d >> 2a) & 3s;
//   kSignedNibbleX16: the signed nibbles of kSignedNibble placed in the high
//     half of their bytes, i.e. decoded as 16 * value: no sign extension, and
//     the int32 products are exact multiples of 16, so the accumulator shifted
//     right by 4 is kSignedNibble's as long as it does not wrap
//     (16 * 128 * 8 * K < 2^31, K <= kX16MaxK).
enum class LowBit { kSignedNibble, kInt2, kSignedNibbleX16 };
constexpr int64_t kX16MaxK = 131071;

template <int ROWS, LowBit F, int NW = 4>
struct LowBitRowsOperand {
  static constexpr int N_INST = ROWS / (8 * NW);
  static_assert(N_INST * 8 * NW == ROWS, "tile rows must be a multiple of 8 per wave");
  static constexpr int NVM = N_INST;
  static constexpr int NDS = N_INST;
  static constexpr int CHUNK_BYTES = F == LowBit::kInt2 ? 4 : 8;  // packed bytes per 16 k
  static constexpr int STAGE_BYTES = 8 * CHUNK_BYTES;                     // per row per 128-k stage
  Rsrc rs;
  uint32_t voff[N_INST];
  uint32_t lds_off[N_INST];
  struct Regs {
    u32x2 v[N_INST];
  };
  // rows: packed rows (row stride ld_bytes); tile rows past M read row M-1.
  INTENT_DEVICE void init(const uint8_t* base, int64_t ld_bytes, int M, int m0, int wave) {
    rs = make_rsrc(base + (int64_t)m0 * ld_bytes);
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int j = 0; j < N_INST; ++j) {
      const int r = (j * NW + wave) * 8 + (lane >> 3);
      const int chunk = (lane & 7) ^ swz(r);
      const int rr = m0 + r < M ? r : M - 1 - m0;
      voff[j] = (uint32_t)(rr * ld_bytes + chunk * CHUNK_BYTES);
      lds_off[j] = (uint32_t)(r * ROWB + (lane & 7) * 16);
    }
  }
  INTENT_DEVICE void load(int kt, Regs& r) const {
#pragma unroll
    for (int j = 0; j < N_INST; ++j) {
      if constexpr (F != LowBit::kInt2) {
        r.v[j] = __builtin_amdgcn_raw_buffer_load_b64(rs, voff[j], (uint32_t)kt * STAGE_BYTES, 0);
      } else {
        r.v[j][0] = __builtin_amdgcn_raw_buffer_load_b32(rs, voff[j], (uint32_t)kt * STAGE_BYTES, 0);
        r.v[j][1] = 0u;
      }
    }
  }
  INTENT_DEVICE static u32x4 decode(u32x2 v) {
    if constexpr (F == LowBit::kSignedNibble) {
      u32x4 out;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        uint32_t lo = v[h] & 0x0F0F0F0Fu, hi = (v[h] >> 4) & 0x0F0F0F0Fu;
        lo |= ((lo >> 3) & 0x01010101u) * 0xF0u;  // sign-extend each nibble into its byte
        hi |= ((hi >> 3) & 0x01010101u) * 0xF0u;
        out[2 * h] = __builtin_amdgcn_perm(hi, lo, 0x05010400u);      // k = 0, 1, 2, 3 of the dword
        out[2 * h + 1] = __builtin_amdgcn_perm(hi, lo, 0x07030602u);  // k = 4, 5, 6, 7
      }
      return out;
    } else if constexpr (F == LowBit::kSignedNibbleX16) {
      u32x4 out;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const uint32_t lo = (v[h] << 4) & 0xF0F0F0F0u, hi = v[h] & 0xF0F0F0F0u;
        out[2 * h] = __builtin_amdgcn_perm(hi, lo, 0x05010400u);
        out[2 * h + 1] = __builtin_amdgcn_perm(hi, lo, 0x07030602u);
      }
      return out;
    } else {
      const uint32_t d = v[0];
      return u32x4{d & 0x03030303u, (d >> 2) & 0x03030303u, (d >> 4) & 0x03030303u, (d >> 6) & 0x03030303u};
    }
  }
  template <bool kAsm = false>  // kAsm: see lds_store16
  INTENT_DEVICE void store(const Regs& r, char* lds_region) const {
#pragma unroll
    for (int j = 0; j < N_INST; ++j) {
      if constexpr (kAsm)
        lds_store16(lds_region + lds_off[j], decode(r.v[j]));
      else
        *reinterpret_cast<u32x4*>(lds_region + lds_off[j]) = decode(r.v[j]);
    }
  }
};

// Raw rows copied global -> LDS by DMA (buffer_load ... lds): no VGPRs and
// no ds_write issue slots. Each wave instruction moves 8 rows x 128 bytes;
// lane i writes slot i%8 of row i/8, fetching chunk slot ^ swz(row).
// LinearRows: instruction j's rows sit j * NW * 8 rows after instruction 0's
// with the same swizzle (NW even), so one offset register serves all and the
// row step goes into the uniform offset.
template <int ROWS, class Rows, int NW = 4, bool kAsm = false>
struct DmaRowsOperand {
  static constexpr int N_INST = ROWS / (8 * NW);
  static_assert(N_INST * 8 * NW == ROWS, "tile rows must be a multiple of 8 per wave");
  static constexpr int NVM = N_INST;
  static constexpr bool kLin = IsLinearRows<Rows>::value;
  static_assert(!kLin || NW % 2 == 0, "linear rows keep one swizzle per lane only for an even wave count");
  Rsrc rs;
  uint32_t voff[kLin ? 1 : N_INST];
  uint32_t jstep = 0;  // LinearRows: bytes between the rows of instructions j and j + 1
  int lds_row0[N_INST];
  INTENT_DEVICE void init(const Rows& rows, int m0, int wave) {
    rs = make_rsrc(rows.tile_base(m0));
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int j = 0; j < N_INST; ++j) {
      const int r0 = (j * NW + wave) * 8;
      const int r = r0 + (lane >> 3);
      if (!kLin || j == 0) voff[kLin ? 0 : j] = rows.off(m0, r) + (((lane & 7) ^ swz(r)) << 4);
      lds_row0[j] = r0;
    }
    if constexpr (kLin) jstep = rows.off(m0, NW * 8);
  }
  INTENT_DEVICE void issue(char* lds_region, int kt) const {
#pragma unroll
    for (int j = 0; j < N_INST; ++j)
      lds_dma<16, kAsm>(rs, (lds_t*)(lds_region + lds_row0[j] * ROWB), voff[kLin ? 0 : j],
                        (uint32_t)kt * ROWB + (kLin ? j * jstep : 0u));
  }
};

// Asymmetric group-quantized 4-bit weight rows (packed two per byte, low nibble
// = even k), decoded to f16 (q - z) * s. A stage is 64 k = 32 packed bytes per
// row, read as P = 2 pieces of 16 bytes (32 k each) or 4 pieces of 8 bytes.
// kWin (group sizes that are multiples of 64, scale and zero rows in whole
// dwords): the scale dword of groups 2d, 2d + 1 and the zero dword of groups
// 4e .. 4e + 3 are loaded only by the stage that opens a pair of groups, and
// the decode keeps them in registers (ps, pz) for the stages that follow; the
// per-stage form loads a 2-byte scale and a 1-byte zero per piece and stage,
// one cache line per row each time. params_at(kt) says whether stage kt's
// load carries them (vm_ops = NS or 3 * NS instructions).
template <int ROWS, int NT = NTHREADS, bool kWin = false>
struct W4Operand {
  static constexpr bool kWinParams = kWin;
  static constexpr int PIECE = (ROWS * 2) % NT == 0 ? 16 : (ROWS * 4) % NT == 0 ? 8 : 4;  // bytes per load
  static constexpr int P = 32 / PIECE;                                                     // pieces per row per stage
  static constexpr int NS = ROWS * P / NT;                                                 // loads per thread per stage
  static_assert(NS * NT == ROWS * P, "W4 staging must divide evenly");
  static_assert(P <= 8 && ROWS % (2 * (8 / P)) == 0 && NT % 16 == 0, "8-lane write blocks pair up over whole rows");
  static constexpr int NVM = 3 * NS;            // vector memory instructions per stage (at most)
  static constexpr int NVM_W = NS;              // ... of a windowed stage without group parameters
  static constexpr int NDS = NS * (PIECE / 4);  // LDS writes per stage
  typedef uint32_t Piece __attribute__((ext_vector_type(PIECE / 4 > 1 ? PIECE / 4 : 2)));

  Rsrc rq, rs, rz;
  uint32_t qoff[NS], soff[NS], zoff[NS];
  int lrow[NS], part[NS];
  int gs;   // 32 or a multiple of 64
  int spg;  // kWin: stages per group (gs / 64)
  mutable uint32_t ps[NS], pz[NS];  // kWin: the parameter dwords in use

  // Scales and zeros stay in 32-bit registers: packing two 16-bit loads
  // into one VGPR would force a wait right after they are issued.
  struct Regs {
    Piece w[NS];
    uint32_t s[NS];
    uint32_t z[NS];
  };

  // wrow(c): weight row of B-tile row c; ldq bytes per packed row; ldp groups per row.
  template <class RowMap>
  INTENT_DEVICE void init(const uint8_t* q, int64_t ldq, const f16* s, const uint8_t* z, int64_t ldp, int gsize,
                          const RowMap& wrow) {
    rq = make_rsrc(q);
    rs = make_rsrc(s);
    rz = make_rsrc(z);
    gs = gsize;
    spg = gsize / 64;
#pragma unroll
    for (int i = 0; i < NS; ++i) {
      const int c = (int)(threadIdx.x % NT) + i * NT;
      // The 16-byte LDS writes of 8 lanes (128 bytes) go out together; with
      // c / P as the row, those 8 lanes would hold 8 / P consecutive rows, and
      // rows 2m and 2m + 1 share swz, so their chunks would land on the same
      // banks. Lanes are instead grouped so that an 8-lane block holds rows
      // r0, r0 + 2, .. (distinct swz): block b takes rows (b & 1) +
      // 2 * (8 / P) * (b >> 1) + 2k, k = 0 .. 8 / P - 1.
      const int b = c >> 3, t = c & 7;
      lrow[i] = (b & 1) + 2 * (8 / P) * (b >> 1) + 2 * (t / P);
      part[i] = t % P;
      const int64_t w = wrow(lrow[i]);
      // gs == 32: a stage spans two groups; piece p starts at k = p * PIECE * 2.
      const int extra = !kWin && gsize == 32 ? (part[i] * PIECE * 2) / 32 : 0;
      qoff[i] = (uint32_t)(w * ldq + part[i] * PIECE);
      soff[i] = (uint32_t)((w * ldp + extra) * 2);
      zoff[i] = (uint32_t)(w * ldp + extra);
    }
  }
  INTENT_DEVICE bool params_at(int kt) const { return !kWin || kt % (2 * spg) == 0; }
  INTENT_DEVICE void load(int kt, Regs& r) const {
    const uint32_t g = kWin ? (uint32_t)(kt / spg) : gs == 32 ? 2 * kt : (kt * 64) / gs;
    const bool with_params = params_at(kt);
#pragma unroll
    for (int i = 0; i < NS; ++i) {
      if constexpr (PIECE == 16)
        r.w[i] = __builtin_amdgcn_raw_buffer_load_b128(rq, qoff[i], (uint32_t)kt * 32, 0);
      else if constexpr (PIECE == 8)
        r.w[i] = __builtin_amdgcn_raw_buffer_load_b64(rq, qoff[i], (uint32_t)kt * 32, 0);
      else
        r.w[i][0] = __builtin_amdgcn_raw_buffer_load_b32(rq, qoff[i], (uint32_t)kt * 32, 0);
      if constexpr (kWin) {
        if (with_params) {
          r.s[i] = __builtin_amdgcn_raw_buffer_load_b32(rs, soff[i], (g & ~1u) * 2, 0);
          r.z[i] = __builtin_amdgcn_raw_buffer_load_b32(rz, zoff[i], g & ~3u, 0);
        }
      } else {
        r.s[i] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(rs, soff[i], g * 2, 0);
        r.z[i] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b8(rz, zoff[i], g, 0);
      }
    }
  }
  // Decode stage kt into the B region of a stage buffer (kAsm: see lds_store16).
  template <bool kAsm = false>
  INTENT_DEVICE void store(const Regs& r, char* lds_b, int kt = 0) const {
    const int g = kWin ? kt / spg : 0;
    const bool fresh = params_at(kt);
#pragma unroll
    for (int i = 0; i < NS; ++i) {
      uint32_t zq = r.z[i], sq = r.s[i];
      if constexpr (kWin) {
        if (fresh) {
          ps[i] = r.s[i];
          pz[i] = r.z[i];
        }
        zq = (pz[i] >> ((g & 3) * 8)) & 0xFFu;
        sq = (ps[i] >> ((g & 1) * 16)) & 0xFFFFu;
      }
      const f16x2 zo = splat2((f16)(float)(1024 + zq));
      const f16x2 sc = splat2(bit_cast<f16>((uint16_t)sq));
      char* row = lds_b + lrow[i] * ROWB;
      const int sw = swz(lrow[i]);
#pragma unroll
      for (int d = 0; d < PIECE / 4; ++d) {
        const int chunk = part[i] * (PIECE / 4) + d;  // each dword = 8 k = one 16-byte f16 chunk
        const f16x8 v = dequant8(r.w[i][d], zo, sc);
        if constexpr (kAsm)
          lds_store16(row + ((chunk ^ sw) << 4), bit_cast<u32x4>(v));
        else
          *reinterpret_cast<f16x8*>(row + ((chunk ^ sw) << 4)) = v;
      }
    }
  }
};

// The reference's own W4 layout as a B operand (weight_only_int4_matmul,
// examples/kernels/contraction/weight_only_int4.py:18-51): int32 words
// [K/8, N] (word (r, n): k = 8r .. 8r+7 of column n, signed nibble k % 8) and
// f16 scales [K/64, N]. A stage (64 k) is one scale group and eight k-rows of
// words; item i = thread + NT j takes column i % ROWS of k-row i / ROWS, so a
// wave loads 64 consecutive columns (256 bytes) of one k-row per instruction.
// A word has the nibble order of a [N, K/2] dword, so w ^ 0x88888888 (nibble
// + 8) decodes through dequant8 with zero point 8 into 16 bytes of f16: chunk
// r of B row (column) i % ROWS.
template <int ROWS, int NT = NTHREADS>
struct W4SymOperand {
  static constexpr bool kWinParams = false;
  static constexpr int NS = 8 * ROWS / NT;  // words per thread per stage
  static_assert(NS * NT == 8 * ROWS, "W4 word staging must divide evenly");
  static constexpr int NVM = 2 * NS;
  static constexpr int NDS = NS;
  Rsrc rq, rs;
  uint32_t qoff[NS], soff[NS];
  int lcol[NS], krow[NS];
  uint32_t ldq_stage;  // bytes of eight k-rows of words
  uint32_t lds_stage;  // bytes of one scale row
  struct Regs {
    uint32_t w[NS];
    uint32_t s[NS];
  };
  // q: word (0, 0); ldq / lds: words / scales per row; the tile's columns are
  // n0 .. n0 + ROWS - 1, those past N re-read column N - 1.
  INTENT_DEVICE void init(const int32_t* q, int64_t ldq, const f16* s, int64_t lds, int n0, int N) {
    rq = make_rsrc(q);
    rs = make_rsrc(s);
    ldq_stage = (uint32_t)(8 * ldq * 4);
    lds_stage = (uint32_t)(lds * 2);
#pragma unroll
    for (int j = 0; j < NS; ++j) {
      const int i = (int)(threadIdx.x % NT) + NT * j;
      lcol[j] = i % ROWS;
      krow[j] = i / ROWS;
      const int n = n0 + lcol[j] < N ? n0 + lcol[j] : N - 1;
      qoff[j] = (uint32_t)((krow[j] * ldq + n) * 4);
      soff[j] = (uint32_t)(n * 2);
    }
  }
  INTENT_DEVICE bool params_at(int) const { return true; }
  INTENT_DEVICE void load(int kt, Regs& r) const {
#pragma unroll
    for (int j = 0; j < NS; ++j) {
      r.w[j] = __builtin_amdgcn_raw_buffer_load_b32(rq, qoff[j], (uint32_t)kt * ldq_stage, 0);
      r.s[j] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(rs, soff[j], (uint32_t)kt * lds_stage, 0);
    }
  }
  template <bool kAsm = false>
  INTENT_DEVICE void store(const Regs& r, char* lds_b, int = 0) const {
    const f16x2 zo = splat2((f16)1032.0f);
#pragma unroll
    for (int j = 0; j < NS; ++j) {
      const f16x2 sc = splat2(bit_cast<f16>((uint16_t)r.s[j]));
      const f16x8 v = dequant8(r.w[j] ^ 0x88888888u, zo, sc);
      char* dst = lds_b + lcol[j] * ROWB + ((krow[j] ^ swz(lcol[j])) << 4);
      if constexpr (kAsm)
        lds_store16(dst, bit_cast<u32x4>(v));
      else
        *reinterpret_cast<f16x8*>(dst) = v;
    }
  }
};

// WinParams<B>::value: B loads its group parameters only at some stages
// (W4Operand<..., true>); mainloop_ws then picks the wait count per step.
template <class B, class = void>
struct WinParams : std::false_type {};
template <class B>
struct WinParams<B, std::void_t<decltype(B::kWinParams)>> : std::bool_constant<B::kWinParams> {};

// Per-channel int8 weight rows converted exactly to f16 (scale applied in the
// epilogue). A stage is 64 k = 64 bytes per row, loaded as 16-byte pieces
// (two f16 chunks) or 8-byte pieces (one chunk) so that every thread gets the
// same number of pieces.
template <int ROWS, int NT = NTHREADS>
struct W8Operand {
  static constexpr int PIECE = (ROWS * 4) % NT == 0 ? 16 : 8;
  static constexpr int P = 64 / PIECE;
  static constexpr int NS = ROWS * P / NT;
  static_assert(NS * NT == ROWS * P, "W8 staging must divide evenly");
  static constexpr int NVM = NS;
  static constexpr int NDS = NS * PIECE / 8;
  Rsrc rq;
  uint32_t qoff[NS];
  int lrow[NS], part[NS];
  struct Regs {
    u32x4 w[NS];
  };
  template <class RowMap>
  INTENT_DEVICE void init(const int8_t* q, int64_t ldq, const RowMap& wrow) {
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
        r.w[i] = __builtin_amdgcn_raw_buffer_load_b128(rq, qoff[i], (uint32_t)kt * 64, 0);
      } else {
        const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(rq, qoff[i], (uint32_t)kt * 64, 0);
        r.w[i] = u32x4{v[0], v[1], 0u, 0u};
      }
    }
  }
  template <bool kAsm = false>
  INTENT_DEVICE void store(const Regs& r, char* lds_b) const {
#pragma unroll
    for (int i = 0; i < NS; ++i) {
      char* row = lds_b + lrow[i] * ROWB;
      const int sw = swz(lrow[i]);
      const int c0 = part[i] * (PIECE / 8);
      const f16x8 v0 = int8x8_to_f16(r.w[i][0], r.w[i][1]);
      if constexpr (kAsm)
        lds_store16(row + ((c0 ^ sw) << 4), bit_cast<u32x4>(v0));
      else
        *reinterpret_cast<f16x8*>(row + ((c0 ^ sw) << 4)) = v0;
      if constexpr (PIECE == 16) {
        const f16x8 v1 = int8x8_to_f16(r.w[i][2], r.w[i][3]);
        if constexpr (kAsm)
          lds_store16(row + (((c0 + 1) ^ sw) << 4), bit_cast<u32x4>(v1));
        else
          *reinterpret_cast<f16x8*>(row + (((c0 + 1) ^ sw) << 4)) = v1;
      }
    }
  }
};

// ---- main loop ------------------------------------------------------------------

// Fragment reads and MFMAs of one stage (KK steps of 32 bytes of k). The reads
// of step kk+1 are interleaved one-for-one with the MFMAs of step kk.
// kSwap: issue mfma(A, B) instead of mfma(B, A), so that a lane's
// accumulators hold one n and four consecutive m per 4-register group.
template <class T, class Math, int KK = 4, bool kSched = true, bool kSwap = false>
INTENT_DEVICE void compute_stage(const char* buf, const uint32_t (&aaddr)[4], const uint32_t (&baddr)[4],
                                 typename Math::Acc (&acc)[T::TI][T::TJ]) {
  using Frag = typename Math::Frag;
  constexpr int NR = T::TI + T::TJ;
  constexpr int NM = T::TI * T::TJ;
  Frag af[2][T::TI], bf[2][T::TJ];
  const char* a = buf;
  const char* b = buf + T::A_BYTES;
#pragma unroll
  for (int i = 0; i < T::TI; ++i) af[0][i] = *reinterpret_cast<const Frag*>(a + aaddr[0] + i * 32 * ROWB);
#pragma unroll
  for (int j = 0; j < T::TJ; ++j) bf[0][j] = *reinterpret_cast<const Frag*>(b + baddr[0] + j * 32 * ROWB);
#pragma unroll
  for (int kk = 0; kk < KK; ++kk) {
    const int cb = kk & 1;
    if (kk + 1 < KK) {
#pragma unroll
      for (int i = 0; i < T::TI; ++i)
        af[cb ^ 1][i] = *reinterpret_cast<const Frag*>(a + aaddr[kk + 1] + i * 32 * ROWB);
#pragma unroll
      for (int j = 0; j < T::TJ; ++j)
        bf[cb ^ 1][j] = *reinterpret_cast<const Frag*>(b + baddr[kk + 1] + j * 32 * ROWB);
    }
#pragma unroll
    for (int i = 0; i < T::TI; ++i)
#pragma unroll
      for (int j = 0; j < T::TJ; ++j)
        acc[i][j] = kSwap ? Math::mfma(af[cb][i], bf[cb][j], acc[i][j]) : Math::mfma(bf[cb][j], af[cb][i], acc[i][j]);
  }
  if constexpr (kSched) {
    // Standalone stage (no loads or stores around it): the first step's
    // reads, then MFMA/read pairs while reads of the next step remain.
    __builtin_amdgcn_sched_group_barrier(0x100, NR, 0);
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      if (kk + 1 < KK) {
        constexpr int PAIRS = NR < NM ? NR : NM;
#pragma unroll
        for (int x = 0; x < PAIRS; ++x) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
        if (NR > NM) __builtin_amdgcn_sched_group_barrier(0x100, NR - NM, 0);
        if (NM > NR) __builtin_amdgcn_sched_group_barrier(0x008, NM - NR, 0);
      } else {
        __builtin_amdgcn_sched_group_barrier(0x008, NM, 0);
      }
    }
  }
}

// compute_stage for a Math with paired fragments (PairedFrags): two MFMA
// steps per 128-byte stage, step s on the fragments of steps 2s and 2s + 1;
// the reads of step 1 are interleaved with the MFMAs of step 0.
template <class T, class Math>
INTENT_DEVICE void compute_stage_pairs(const char* buf, const uint32_t (&aaddr)[4], const uint32_t (&baddr)[4],
                                       typename Math::Acc (&acc)[T::TI][T::TJ]) {
  using Frag = typename Math::Frag;
  constexpr int NR = 2 * (T::TI + T::TJ);
  constexpr int NM = T::TI * T::TJ;
  Frag af[2][2][T::TI], bf[2][2][T::TJ];
  const char* a = buf;
  const char* b = buf + T::A_BYTES;
#pragma unroll
  for (int s = 0; s < 2; ++s)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
#pragma unroll
      for (int i = 0; i < T::TI; ++i)
        af[s][h][i] = *reinterpret_cast<const Frag*>(a + aaddr[2 * s + h] + i * 32 * ROWB);
#pragma unroll
      for (int j = 0; j < T::TJ; ++j)
        bf[s][h][j] = *reinterpret_cast<const Frag*>(b + baddr[2 * s + h] + j * 32 * ROWB);
    }
#pragma unroll
  for (int s = 0; s < 2; ++s)
#pragma unroll
    for (int i = 0; i < T::TI; ++i)
#pragma unroll
      for (int j = 0; j < T::TJ; ++j)
        acc[i][j] = Math::mfma2(bf[s][0][j], bf[s][1][j], af[s][0][i], af[s][1][i], acc[i][j]);
  __builtin_amdgcn_sched_group_barrier(0x100, NR, 0);
  constexpr int PAIRS = NR < NM ? NR : NM;
  static_for_mp<0, PAIRS>([&](auto X) {
    constexpr int x = decltype(X)::value;
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x100, (x + 1) * NR / PAIRS - x * NR / PAIRS, 0);
  });
  if (NM > PAIRS) __builtin_amdgcn_sched_group_barrier(0x008, NM - PAIRS, 0);
  __builtin_amdgcn_sched_group_barrier(0x008, NM, 0);
}

// Instruction schedule of one pipelined step: 4*NM MFMA slots. The fragment
// reads of step kk+1 ride on the first NR slots of step kk; NV buffer loads
// are spread over the first half of the slots and NW LDS writes over the
// second half (sched_group_barrier masks: 0x008 MFMA, 0x020 VMEM read,
// 0x100 DS read, 0x200 DS write). Decode VALU is left to the compiler.
constexpr int spread(int s, int n, int slots) { return (s + 1) * n / slots - s * n / slots; }

template <int NM, int NR, int NV, int NW, int S>
INTENT_DEVICE void sched_slots() {
  if constexpr (S < 4 * NM) {
    constexpr int kk = S / NM;
    constexpr int x = S % NM;
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    if constexpr (kk < 3 && x < NR) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    if constexpr (S < 2 * NM && spread(S, NV, 2 * NM) > 0)
      __builtin_amdgcn_sched_group_barrier(0x020, spread(S, NV, 2 * NM), 0);
    if constexpr (S >= 2 * NM && spread(S - 2 * NM, NW, 2 * NM) > 0)
      __builtin_amdgcn_sched_group_barrier(0x200, spread(S - 2 * NM, NW, 2 * NM), 0);
    sched_slots<NM, NR, NV, NW, S + 1>();
  }
}
template <int NM, int NR, int NV, int NW>
INTENT_DEVICE void sched_step() {
  __builtin_amdgcn_sched_group_barrier(0x100, NR, 0);
  sched_slots<NM, NR, NV, NW, 0>();
}

// buf0/buf1: the two LDS stage buffers, each STAGE_BYTES: A rows then B rows.
// nk: number of stages; half_last: the last stage carries 64 bytes of k
// (its loads must already re-read chunks 0..3, see RegRowsOperand).
template <class T, class Math, class AOp, class BOp>
INTENT_DEVICE void mainloop(const AOp& aop, const BOp& bop, int nk, char* buf0, char* buf1,
                            typename Math::Acc (&acc)[T::TI][T::TJ], bool half_last = false, int k_rot = 0) {
  // Stage order: full stages start at k_rot and wrap; a half stage stays last.
  const int nfull = half_last ? nk - 1 : nk;
  const int rot = nfull > 0 ? k_rot % nfull : 0;
  auto kidx = [&](int kt) {
    if (kt >= nfull) return kt;
    const int r = kt + rot;
    return r >= nfull ? r - nfull : r;
  };
  const int lane = threadIdx.x & 63;
  // Fragment addresses: row (lane % 32) of each 32-row tile, chunk 2*kk + lane/32.
  uint32_t aaddr[4], baddr[4];
  {
    const int r = lane & 31;
    const int x = (lane >> 5) ^ swz(r);
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const uint32_t s = (uint32_t)(((2 * kk) ^ x) << 4);
      aaddr[kk] = (uint32_t)((T::wave_m() * T::WTM + r) * ROWB) + s;
      baddr[kk] = (uint32_t)((T::wave_n() * T::WTN + r) * ROWB) + s;
    }
  }
#pragma unroll
  for (int i = 0; i < T::TI; ++i)
#pragma unroll
    for (int j = 0; j < T::TJ; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0;
  if (nk <= 0) return;

  typename AOp::Regs ra0, ra1;
  typename BOp::Regs rb0, rb1;
  aop.load(kidx(0), ra0);
  bop.load(kidx(0), rb0);
  if (nk > 1) {
    aop.load(kidx(1), ra1);
    bop.load(kidx(1), rb1);
  }
  aop.store(ra0, buf0);
  bop.store(rb0, buf0 + T::A_BYTES);
  wait_vm_lgkm_barrier<AOp::NVM + BOp::NVM>();

  // Step kt: rn holds stage kt+1, rf receives stage kt+2.
  // The step body is one basic block: the stage-kt+2 load is clamped to the
  // last stage (the last step re-loads it and never stores it), so the whole
  // step can be scheduled as one interleaved stream.
  auto step = [&](int kt, char* cur, char* nxt, typename AOp::Regs& ran, typename BOp::Regs& rbn,
                  typename AOp::Regs& raf, typename BOp::Regs& rbf) {
    const int kn = kidx(kt + 2 < nk ? kt + 2 : nk - 1);
    if constexpr (!(INTENT_ABLATE & 1)) {
      aop.load(kn, raf);
      bop.load(kn, rbf);
    }
    compute_stage<T, Math, 4, false>(cur, aaddr, baddr, acc);
    if constexpr (!(INTENT_ABLATE & 2)) {
      aop.store(ran, nxt);
      bop.store(rbn, nxt + T::A_BYTES);
    }
    sched_step<T::TI * T::TJ, T::TI + T::TJ, AOp::NVM + BOp::NVM, AOp::NDS + BOp::NDS>();
    wait_vm_lgkm_barrier<AOp::NVM + BOp::NVM>();
  };
  // Every stage but the last runs a full step; the last stage is peeled so
  // that it can be a half stage and issues no loads or stores.
  int kt = 0;
  for (; kt + 2 < nk; kt += 2) {
    step(kt, buf0, buf1, ra1, rb1, ra0, rb0);
    step(kt + 1, buf1, buf0, ra0, rb0, ra1, rb1);
  }
  if (kt + 1 < nk) {
    step(kt, buf0, buf1, ra1, rb1, ra0, rb0);
    ++kt;
  }
  char* last = (kt & 1) ? buf1 : buf0;
  if (half_last)
    compute_stage<T, Math, 2>(last, aaddr, baddr, acc);
  else
    compute_stage<T, Math, 4>(last, aaddr, baddr, acc);
}

// ---- right operand as [K][N] rows (N contiguous), no transpose pass ---------------
//
// A stage holds 64 k-rows of BN columns (BN * 2 bytes each) copied global ->
// LDS by DMA: the stage is one linear block and DMA instruction j fills its
// kilobyte j, lane i moving 16-byte slot q = 64j + i (k-row q / CH, slot
// q % CH). Slot s of k-row r holds column chunk s ^ kn_swz(r). MFMA B
// fragments (8 consecutive k of one column per lane) are read with
// ds_read_b64_tr_b16: inside a group of 16 lanes, output lane t element e is
// element t % 4 of the 8 bytes addressed by lane 4e + t / 4. Lane j of a
// group therefore addresses k-row k0 + j / 4, columns n0 + 4 (j % 4) .. + 3,
// and lane t receives column n0 + t at k-rows k0 .. k0 + 3; two such reads
// (k0 and k0 + 4) make a fragment. The four k-rows of one read then fall
// into four distinct 32-byte bank windows thanks to kn_swz.
INTENT_DEVICE constexpr int kn_swz(int krow) { return 2 * (krow & 3); }

template <int BN, int NW>
struct DmaKNOperand {
  static constexpr int CH = BN / 8;      // 16-byte column chunks per k-row
  static constexpr int RB = BN * 2;      // bytes per k-row in LDS
  static constexpr int TOTAL = BN / 8;   // kilobyte DMA instructions per stage (64 * RB / 1024)
  static constexpr int N_INST = (TOTAL + NW - 1) / NW;
  static constexpr int NVM = N_INST;
  static_assert(BN % 64 == 0, "KN tiles need a multiple of 64 columns");
  Rsrc rs;
  uint32_t voff[N_INST];
  int lds_kb[N_INST];  // destination kilobyte of instruction j
  uint32_t kstep;      // bytes per stage (64 k-rows)
  // b: element (0, n0) of the [K][N] matrix; ldb elements per k-row; ncols:
  // valid columns from n0 (chunks past them re-read a valid chunk; their
  // products land in output columns that are never stored).
  INTENT_DEVICE void init(const void* b, int64_t ldb, int ncols, int wave) {
    rs = make_rsrc(b);
    kstep = (uint32_t)(64 * ldb * 2);
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int j = 0; j < N_INST; ++j) {
      const int t = j * NW + wave < TOTAL ? j * NW + wave : TOTAL - 1;
      const int q = t * 64 + lane;
      const int r = q / CH;
      const int c = (q % CH) ^ kn_swz(r);
      int col = c * 8;
      col = col + 8 <= ncols ? col : ((ncols - 8) > 0 ? ((ncols - 8) & ~7) : 0);
      voff[j] = (uint32_t)(r * ldb * 2 + col * 2);
      lds_kb[j] = t;
    }
  }
  INTENT_DEVICE void issue(char* lds_b, int kt) const {
#pragma unroll
    for (int j = 0; j < N_INST; ++j)
      lds_dma<16, false>(rs, (lds_t*)(lds_b + lds_kb[j] * 1024), voff[j], (uint32_t)kt * kstep);
  }
};

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4_t;

// B fragment of 32x32x16 step kk for column block n (wave-tile relative n0 +
// 32 * j): lane l takes column n + l % 32, k-rows 16kk + 8(l / 32) .. + 7.
template <class Frag>
INTENT_DEVICE Frag kn_frag(const char* b, uint32_t addr0, uint32_t addr1) {
  const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)(__attribute__((address_space(3))) char*)(b + addr0));
  const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)(__attribute__((address_space(3))) char*)(b + addr1));
  typedef short s16x8 __attribute__((ext_vector_type(8)));
  const s16x8 v = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  return bit_cast<Frag>(v);
}

// LDS byte offset (within the B region) of a lane's transpose read for step
// kk, column block j and half hh (k-rows +0 / +4). The lane addresses k-row
// krow = 16kk + 8(g / 2) + 4hh + t / 4 and column col = wave_n * WTN + 32j +
// 16(g % 2) + 4(t % 4) (g = lane / 16, t = lane % 16), i.e. 32-byte window
// w = col / 16 = wave_n * WTN / 16 + 2j + g % 2 stored at w ^ (krow & 3),
// where krow & 3 = t / 4 for every kk, hh. Only bit 0 of j meets the swizzle,
// so two per-lane bases (even / odd j) plus constant offsets cover all reads.
template <class T>
struct KNAddr {
  static constexpr int RB = T::BN * 2;
  static_assert(T::WTN % 32 == 0, "column blocks of 32");
  uint32_t base[2];
  INTENT_DEVICE void init() {
    const int lane = threadIdx.x & 63;
    const int g = lane >> 4, t = lane & 15;
    const int r = t >> 2;  // krow & 3
    const int w0 = (g & 1) ^ (r & 1);  // bit 0 of the stored window
    const uint32_t row = (uint32_t)((8 * (g >> 1) + r) * RB);
    const uint32_t in = (uint32_t)(T::wave_n() * T::WTN * 2 + w0 * 32 + (t & 3) * 8);
    // stored window bit 1 = (j & 1) ^ (r >> 1): +64 for even j when r >> 1,
    // -64 for odd j
    base[0] = row + in + ((r >> 1) ? 64u : 0u);
    base[1] = row + in - ((r >> 1) ? 64u : 0u);
  }
  INTENT_DEVICE uint32_t at(int kk, int j, int hh) const {
    return base[j & 1] + (uint32_t)(j * 64 + kk * 16 * RB + hh * 4 * RB);
  }
};

// One stage: A fragments as compute_stage, B fragments by transpose reads.
template <class T, class Math, bool kSched = false>
INTENT_DEVICE void compute_stage_kn(const char* buf, const uint32_t (&aaddr)[4], const KNAddr<T>& ka,
                                    typename Math::Acc (&acc)[T::TI][T::TJ]) {
  using Frag = typename Math::Frag;
  const char* a = buf;
  const char* b = buf + T::A_BYTES;
  Frag af[2][T::TI], bf[2][T::TJ];
#pragma unroll
  for (int i = 0; i < T::TI; ++i) af[0][i] = *reinterpret_cast<const Frag*>(a + aaddr[0] + i * 32 * ROWB);
#pragma unroll
  for (int j = 0; j < T::TJ; ++j) bf[0][j] = kn_frag<Frag>(b, ka.at(0, j, 0), ka.at(0, j, 1));
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) {
    const int cb = kk & 1;
    if (kk + 1 < 4) {
#pragma unroll
      for (int i = 0; i < T::TI; ++i)
        af[cb ^ 1][i] = *reinterpret_cast<const Frag*>(a + aaddr[kk + 1] + i * 32 * ROWB);
#pragma unroll
      for (int j = 0; j < T::TJ; ++j) bf[cb ^ 1][j] = kn_frag<Frag>(b, ka.at(kk + 1, j, 0), ka.at(kk + 1, j, 1));
    }
#pragma unroll
    for (int i = 0; i < T::TI; ++i)
#pragma unroll
      for (int j = 0; j < T::TJ; ++j) acc[i][j] = Math::mfma(bf[cb][j], af[cb][i], acc[i][j]);
  }
  if constexpr (kSched) {
    // the first step's reads, then the next step's reads paired with MFMAs
    // (a B fragment is two transpose reads)
    constexpr int NR = T::TI + 2 * T::TJ;
    constexpr int NM = T::TI * T::TJ;
    __builtin_amdgcn_sched_group_barrier(0x100, NR, 0);
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      if (kk + 1 < 4) {
        constexpr int PAIRS = NR < NM ? NR : NM;
#pragma unroll
        for (int x = 0; x < PAIRS; ++x) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
        if (NR > NM) __builtin_amdgcn_sched_group_barrier(0x100, NR - NM, 0);
        if (NM > NR) __builtin_amdgcn_sched_group_barrier(0x008, NM - NR, 0);
      } else {
        __builtin_amdgcn_sched_group_barrier(0x008, NM, 0);
      }
    }
  }
}

// All-consumer main loop over two stage buffers, both operands by DMA (A rows
// as DmaRowsOperand, B as DmaKNOperand): stage kt + 1 is issued into the
// other buffer while stage kt computes; one barrier per stage. Stage indices
// past the end clamp to the last stage (a copy into a buffer nobody reads
// again), so every step issues the same DMA count and vmcnt(0) before the
// barrier is exact.
template <class T, class Math, class ADma, class BDma, bool kSched>
INTENT_DEVICE void mainloop_kn(const ADma& aop, const BDma& bop, int nk, char* buf0, char* buf1,
                               typename Math::Acc (&acc)[T::TI][T::TJ]) {
#pragma unroll
  for (int i = 0; i < T::TI; ++i)
#pragma unroll
    for (int j = 0; j < T::TJ; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0;
  if (nk <= 0) return;
  const int lane = threadIdx.x & 63;
  uint32_t aaddr[4];
  {
    const int r = lane & 31;
    const int x = (lane >> 5) ^ swz(r);
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) aaddr[kk] = (uint32_t)((T::wave_m() * T::WTM + r) * ROWB) + (((2 * kk) ^ x) << 4);
  }
  KNAddr<T> ka;
  ka.init();
  aop.issue(buf0, 0);
  bop.issue(buf0 + T::A_BYTES, 0);
  wait_vm_lgkm_barrier<0>();
  for (int kt = 0; kt < nk; kt += 2) {
    {
      const int nx = kt + 1 < nk ? kt + 1 : nk - 1;
      aop.issue(buf1, nx);
      bop.issue(buf1 + T::A_BYTES, nx);
      compute_stage_kn<T, Math, kSched>(buf0, aaddr, ka, acc);
      if (kt + 1 >= nk) break;
      wait_vm_lgkm_barrier<0>();
    }
    {
      const int nx = kt + 2 < nk ? kt + 2 : nk - 1;
      aop.issue(buf0, nx);
      bop.issue(buf0 + T::A_BYTES, nx);
      compute_stage_kn<T, Math, kSched>(buf1, aaddr, ka, acc);
      if (kt + 2 >= nk) break;
      wait_vm_lgkm_barrier<0>();
    }
  }
  wait_vm<0>();  // no DMA may land in LDS that an epilogue reuses
}

// Producer/consumer variant. Waves 0..NW-1 (consumers) only read fragments
// and issue MFMAs; waves NW..2NW-1 (producers, one per SIMD beside a
// consumer) copy the A rows by LDS DMA NB-1 stages ahead, load the weights NB
// stages ahead into a ring of NB register sets and decode them into LDS one
// stage ahead. A wave's MFMAs do not co-issue with its own VALU decode, but
// they do with the other wave of the SIMD. Both roles meet at one barrier per
// stage. bufs: NB stage buffers (distinct __shared__ objects, STAGE_BYTES
// each). Operands must be built with NT = T::NT (producer thread index =
// threadIdx.x % NT) and the producer wave index. Returns true in consumer
// waves, which then hold acc.
// kmap: the k block (128 bytes of each A row) that stage kt reads, the same
// for A and B (identity: stage kt reads block kt). hook(acc, kt) runs in the
// consumer waves after stage kt's MFMAs.
struct StageIdentity {
  INTENT_DEVICE int operator()(int kt) const { return kt; }
};
struct StageNoHook {
  template <class A>
  INTENT_DEVICE void operator()(A&, int) const {}
};
template <class T, class Math, int NB, class Rows, class BOp, bool kSwap = false, class KMap = StageIdentity,
          class Hook = StageNoHook>
INTENT_DEVICE bool mainloop_ws(const DmaRowsOperand<T::BM, Rows, T::NW>& aop, const BOp& bop, int nk,
                               char* const (&bufs)[NB], typename Math::Acc (&acc)[T::TI][T::TJ], KMap kmap = {},
                               Hook&& hook = {}) {
  static_assert(NB == 2 || NB == 3, "two or three stage buffers");
  using ADma = DmaRowsOperand<T::BM, Rows, T::NW>;
  const bool consumer = T::wave() < T::NW;
#pragma unroll
  for (int i = 0; i < T::TI; ++i)
#pragma unroll
    for (int j = 0; j < T::TJ; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0;
  if (nk <= 0) return consumer;
  if (!consumer) {
    typename BOp::Regs rb[NB];
#pragma unroll
    for (int s = 0; s < NB - 1; ++s)
      if (s < nk) aop.issue(bufs[s], kmap(s));
#pragma unroll
    for (int s = 0; s < NB; ++s)
      if (s < nk) bop.load(kmap(s), rb[s]);
    constexpr bool kWinB = WinParams<BOp>::value;
    static_assert(!kWinB || NB == 2, "windowed group parameters: two stage buffers");
    static_assert(!kWinB || std::is_same_v<KMap, StageIdentity>, "windowed group parameters: stages in order");
    if constexpr (kWinB)
      bop.template store<true>(rb[0], bufs[0] + T::A_BYTES, 0);
    else
      bop.template store<true>(rb[0], bufs[0] + T::A_BYTES);
    wait_vm_lgkm_barrier<0>();
    // Step kt publishes stage kt+1. Its DMA was issued NB-2 steps earlier;
    // vmcnt counts in issue order, so the wait leaves exactly the operations
    // issued after it in flight (sched_barrier pins the DMA ahead of the
    // loads). Near the end some are skipped and the wait drains everything.
    // The DMA and the loads are unconditional, with stage indices clamped to
    // the last stage (a conditional load would make the compiler wait for it
    // where the paths join); near the end the extra copies land in buffers
    // and registers that nobody reads any more, and those steps drain.
    constexpr int kAfter = (NB - 2) * (ADma::NVM + BOp::NVM) + BOp::NVM;
    auto step = [&](auto J, int kt) {
      constexpr int j = decltype(J)::value;  // kt % NB
      const bool full = kt + NB < nk;
      aop.issue(bufs[(j + NB - 1) % NB], kmap(kt + NB - 1 < nk ? kt + NB - 1 : nk - 1));
      __builtin_amdgcn_sched_barrier(0);
      bop.load(kmap(full ? kt + NB : nk - 1), rb[j]);
      if constexpr (kWinB) {
        bop.template store<true>(rb[(j + 1) % NB], bufs[(j + 1) % NB] + T::A_BYTES, kt + 1);
        // in flight: stage kt + 2's loads, with or without its group parameters
        if (full && bop.params_at(kt + NB))
          wait_vm_lgkm_barrier<kAfter>();
        else if (full)
          wait_vm_lgkm_barrier<kAfter - (BOp::NVM - BOp::NVM_W)>();
        else
          wait_vm_lgkm_barrier<0>();
      } else {
        bop.template store<true>(rb[(j + 1) % NB], bufs[(j + 1) % NB] + T::A_BYTES);
        if (full)
          wait_vm_lgkm_barrier<kAfter>();
        else
          wait_vm_lgkm_barrier<0>();
      }
    };
    for (int kt = 0; kt < nk - 1; kt += NB) {
      step(std::integral_constant<int, 0>{}, kt);
      if (kt + 1 < nk - 1) step(std::integral_constant<int, 1>{}, kt + 1);
      if constexpr (NB > 2)
        if (kt + 2 < nk - 1) step(std::integral_constant<int, 2 % NB>{}, kt + 2);
    }
    return false;
  }
  const int lane = threadIdx.x & 63;
  uint32_t aaddr[4], baddr[4];
  {
    const int r = lane & 31;
    const int x = (lane >> 5) ^ swz(r);
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const uint32_t s = (uint32_t)(((2 * kk) ^ x) << 4);
      aaddr[kk] = (uint32_t)((T::wave_m() * T::WTM + r) * ROWB) + s;
      baddr[kk] = (uint32_t)((T::wave_n() * T::WTN + r) * ROWB) + s;
    }
  }
  wait_vm_lgkm_barrier<0>();
  for (int kt = 0; kt < nk; kt += NB) {
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      if (kt + j < nk) {
        if constexpr (PairedFrags<Math>::value)
          compute_stage_pairs<T, Math>(bufs[j], aaddr, baddr, acc);
        else
          compute_stage<T, Math, 4, true, kSwap>(bufs[j], aaddr, baddr, acc);
        hook(acc, kt + j);
        if (kt + j < nk - 1) wait_vm_lgkm_barrier<0>();
      }
    }
  }
  return true;
}

}  // namespace mp
