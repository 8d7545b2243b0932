// MX block-scaled FP8 GEMM on gfx950's scaled MFMA (v_mfma_scale_f32_32x32x64_f8f6f4):
//   out[m, n] = sum_k (A[m, k] * 2^(sa[m, k/32] - 127)) * (B[n, k] * 2^(sb[n, k/32] - 127))
// with A, B OCP E4M3FN bytes (K contiguous), E8M0 scales per 32 k, f32 output.
// Replaces block_scaled_matmul (examples/kernels/contraction/block_scaled.py:11-39;
// CPU semantics lib/Conversion/KIRToCPU/Contractions.cpp:177-259: decode each
// operand to f32 = value * 2^(s-127), E8M0 255 = NaN, then an f32 contraction).
//
// Two kernels share the stage layout: 128 k per LDS stage in XOR-swizzled
// 128-byte rows, plus one dword of scales per tile row (the four E8M0 bytes
// of its four 32-k groups). Problems with at least 256 tiles of 256 x 256 use
// four waves of 128 x 128 fed by LDS DMA (mxfp8_gemm_dma_kernel); smaller
// ones use 128 x 128 tiles on the int8 pipeline (mfma_pipe.h: operands
// through VGPRs, two stages in flight) for more workgroups. One scaled MFMA covers 64 k (step s). The
// instruction reads a lane's 32 operand bytes as two 16-k halves, k 16h..16h+15
// and 32+16h..32+16h+15 of the step (h = lane / 32), and applies lane half
// b's scale to k 32b..32b+31; so lane half h takes LDS chunks 4s+h and
// 4s+2+h, and its scale byte is that of group 2s+h. (Measured: with the two
// halves read as one contiguous 32-k run, groups with different scales mix.)
#include "common.h"
#include "internal.h"
#include "w4pk.h"

namespace {

typedef int i32x8 __attribute__((ext_vector_type(8)));

// Data rows plus their per-stage scale dword. Lanes 8q (one per tile row of
// an instruction) store the scale; every lane loads it (same address).
template <int ROWS, int NW>
struct ScaledRows {
  using Data = mp::RegRowsOperand<ROWS, mp::DenseRows, false, NW>;
  static constexpr int N_INST = Data::N_INST;
  static constexpr int NVM = 2 * N_INST;
  Data data;
  mp::Rsrc rsc;
  uint32_t soff[N_INST];
  uint32_t slds[N_INST];
  struct Regs {
    typename Data::Regs d;
    uint32_t s[N_INST];
  };
  INTENT_DEVICE void init(const uint8_t* rows, int64_t ld, int M, const uint8_t* scales, int64_t ld_scale, int m0,
                          int wave) {
    data.init(mp::DenseRows{rows, ld, M}, m0, wave);
    rsc = make_rsrc(scales);
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int j = 0; j < N_INST; ++j) {
      const int r = (j * NW + wave) * 8 + (lane >> 3);
      const int m = m0 + r < M ? m0 + r : M - 1;
      soff[j] = (uint32_t)(m * ld_scale);
      slds[j] = (uint32_t)(r * 4);
    }
  }
  INTENT_DEVICE void load(int kt, Regs& r) const {
    data.load(kt, r.d);
#pragma unroll
    for (int j = 0; j < N_INST; ++j) r.s[j] = __builtin_amdgcn_raw_buffer_load_b32(rsc, soff[j], (uint32_t)kt * 4, 0);
  }
  INTENT_DEVICE void store(const Regs& r, char* lds_rows, char* lds_scales) const {
    data.store(r.d, lds_rows);
    if ((threadIdx.x & 7) == 0) {
#pragma unroll
      for (int j = 0; j < N_INST; ++j) *reinterpret_cast<uint32_t*>(lds_scales + slds[j]) = r.s[j];
    }
  }
};

template <class T>
struct MxLayout {
  static constexpr int A_SCALES = (T::BM + T::BN) * mp::ROWB;  // after A rows then B rows
  static constexpr int B_SCALES = A_SCALES + T::BM * 4;
  static constexpr int STAGE = B_SCALES + T::BN * 4;
};

// 32 bytes of row r: chunks c0 and c0 + 2 of a swizzled 128-byte LDS row.
INTENT_DEVICE i32x8 read_frag(const char* rows, int r, int c0) {
  const i32x4 lo = *reinterpret_cast<const i32x4*>(rows + r * mp::ROWB + ((c0 ^ mp::swz(r)) << 4));
  const i32x4 hi = *reinterpret_cast<const i32x4*>(rows + r * mp::ROWB + (((c0 + 2) ^ mp::swz(r)) << 4));
  return i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

template <class T>
INTENT_DEVICE void compute_stage_mx(const char* buf, i32x16 (&acc)[T::TI][T::TJ]) {
  using L = MxLayout<T>;
  const int lane = threadIdx.x & 63;
  const int h = lane >> 5;
  const int ra = T::wave_m() * T::WTM + (lane & 31);
  const int rb = T::wave_n() * T::WTN + (lane & 31);
  uint32_t sa[T::TI], sb[T::TJ];
#pragma unroll
  for (int i = 0; i < T::TI; ++i) sa[i] = *reinterpret_cast<const uint32_t*>(buf + L::A_SCALES + (ra + 32 * i) * 4);
#pragma unroll
  for (int j = 0; j < T::TJ; ++j) sb[j] = *reinterpret_cast<const uint32_t*>(buf + L::B_SCALES + (rb + 32 * j) * 4);
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    const int c0 = 4 * s + h;
    const int sh = 8 * (2 * s + h);
    i32x8 af[T::TI], bf[T::TJ];
#pragma unroll
    for (int i = 0; i < T::TI; ++i) af[i] = read_frag(buf, ra + 32 * i, c0);
#pragma unroll
    for (int j = 0; j < T::TJ; ++j) bf[j] = read_frag(buf + T::A_BYTES, rb + 32 * j, c0);
#pragma unroll
    for (int i = 0; i < T::TI; ++i)
#pragma unroll
      for (int j = 0; j < T::TJ; ++j) {
        // (B, A) order: the lane's accumulators hold one m and four adjacent n.
        f32x16 c = bit_cast<f32x16>(acc[i][j]);
        c = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(bf[j], af[i], c, 0, 0, 0, (int)((sb[j] >> sh) & 255u), 0,
                                                             (int)((sa[i] >> sh) & 255u));
        acc[i][j] = bit_cast<i32x16>(c);
      }
  }
}

// Lane holds m = row(i) and n = col(j, g) + 0..3 in acc[i][j][4g..4g+3].
template <class T>
INTENT_DEVICE void store_mx(const i32x16 (&acc)[T::TI][T::TJ], int m0, int n0, int M, int N, float* __restrict__ out,
                            int64_t ldo) {
  const bool vec = (ldo & 3) == 0 && (((uintptr_t)out) & 15) == 0;
#pragma unroll
  for (int i = 0; i < T::TI; ++i) {
    const int m = m0 + T::row(i);
    if (m >= M) continue;
#pragma unroll
    for (int j = 0; j < T::TJ; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int n = n0 + T::col(j, g);
        const f32x16 c = bit_cast<f32x16>(acc[i][j]);
        float* o = out + (int64_t)m * ldo + n;
        if (vec && n + 3 < N) {
          *reinterpret_cast<f32x4*>(o) = f32x4{c[4 * g], c[4 * g + 1], c[4 * g + 2], c[4 * g + 3]};
        } else {
#pragma unroll
          for (int q = 0; q < 4; ++q)
            if (n + q < N) o[q] = c[4 * g + q];
        }
      }
  }
}

template <class T>
__global__ __launch_bounds__(T::NT, 1) void mxfp8_gemm_kernel(const uint8_t* __restrict__ a, int64_t lda, int M,
                                                              const uint8_t* __restrict__ sa, int64_t ld_sa,
                                                              const uint8_t* __restrict__ b, int64_t ldb, int N,
                                                              const uint8_t* __restrict__ sb, int64_t ld_sb, int K,
                                                              float* __restrict__ out, int64_t ldo, int mblocks) {
  using L = MxLayout<T>;
  __shared__ __attribute__((aligned(16))) char buf0[L::STAGE];
  __shared__ __attribute__((aligned(16))) char buf1[L::STAGE];
  int tmb, tnb;
  grid_tile(mblocks, 4, tmb, tnb);
  const int m0 = tmb * T::BM;
  const int n0 = tnb * T::BN;
  const int wave = T::wave();
  const int nk = K / mp::ROWB;
  ScaledRows<T::BM, T::NW> aop;
  aop.init(a, lda, M, sa, ld_sa, m0, wave);
  ScaledRows<T::BN, T::NW> bop;
  bop.init(b, ldb, N, sb, ld_sb, n0, wave);
  i32x16 acc[T::TI][T::TJ];
#pragma unroll
  for (int i = 0; i < T::TI; ++i)
#pragma unroll
    for (int j = 0; j < T::TJ; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0;  // the bits of +0.0f

  constexpr int NV = ScaledRows<T::BM, T::NW>::NVM + ScaledRows<T::BN, T::NW>::NVM;
  typename ScaledRows<T::BM, T::NW>::Regs ra0, ra1;
  typename ScaledRows<T::BN, T::NW>::Regs rb0, rb1;
  auto stage_store = [&](const auto& rra, const auto& rrb, char* buf) {
    aop.store(rra, buf, buf + L::A_SCALES);
    bop.store(rrb, buf + T::A_BYTES, buf + L::B_SCALES);
  };
  aop.load(0, ra0);
  bop.load(0, rb0);
  if (nk > 1) {
    aop.load(1, ra1);
    bop.load(1, rb1);
  }
  stage_store(ra0, rb0, buf0);
  mp::wait_vm_lgkm_barrier<NV>();
  // Step kt computes on one buffer while stage kt+1 (loaded a step earlier)
  // goes to the other and stage kt+2 is loaded; the last step only computes.
  auto step = [&](int kt, char* cur, char* nxt, auto& ran, auto& rbn, auto& raf, auto& rbf) {
    const int kn = kt + 2 < nk ? kt + 2 : nk - 1;
    aop.load(kn, raf);
    bop.load(kn, rbf);
    compute_stage_mx<T>(cur, acc);
    stage_store(ran, rbn, nxt);
    mp::wait_vm_lgkm_barrier<NV>();
  };
  int kt = 0;
  for (; kt + 2 < nk; kt += 2) {
    step(kt, buf0, buf1, ra1, rb1, ra0, rb0);
    step(kt + 1, buf1, buf0, ra0, rb0, ra1, rb1);
  }
  if (kt + 1 < nk) {
    step(kt, buf0, buf1, ra1, rb1, ra0, rb0);
    ++kt;
  }
  compute_stage_mx<T>((kt & 1) ? buf1 : buf0, acc);

  store_mx<T>(acc, m0, n0, M, N, out, ldo);
}

// ---- 256 x 256 tiles, four waves, operands and scales by LDS DMA --------------
// Four waves of 128 x 128 (one per SIMD; the 256 accumulators live in AGPRs).
// Operand rows and scale dwords are copied global -> LDS by DMA
// (buffer_load ... lds), so no staging registers are needed and the 32-byte
// fragments of both steps of a stage fit beside the accumulators. A stage is
// 128 k: 128 bytes of every tile row (8 rows per DMA instruction, chunk c of
// row r in slot c ^ swz(r)) plus one scale dword per row (64 rows per DMA
// instruction). Two stage buffers; the refill of a buffer is issued right
// after the stage's barrier, which sits after the stage's last fragment
// reads, so the next stage's first reads overlap the last step's MFMAs.
namespace mxdma {

using Tile = mp::Tile<256, 256, 2, 2>;
constexpr int kRowBytes = (Tile::BM + Tile::BN) * mp::ROWB;
constexpr int kStage = kRowBytes + (Tile::BM + Tile::BN) * 4;

// Byte offset of stage kt (128 k) inside a row. With SP splits of 256-k
// chunks interleaved along k (the [.., IT, SP, 256] layout of a split-K
// contraction), split s reads chunks it*SP + s; SP = 1 is the plain order.
struct SplitK {
  int sp, s;
  INTENT_DEVICE uint32_t operator()(int kt) const { return (uint32_t)(((kt >> 1) * sp + s) * 256 + (kt & 1) * 128); }
};

template <int ROWS, int NW, bool kScales>
struct Rows {
  static constexpr bool kKN = false;
  static constexpr int N_INST = ROWS / 8 / NW;  // data instructions per wave
  static_assert(N_INST * 8 * NW == ROWS && ROWS % 64 == 0, "tile rows must split evenly");
  // Scale dwords: 64 rows per instruction; a wave with none left repeats the
  // last one (same data, same place), so that every wave issues S_INST.
  static constexpr int S_TOTAL = ROWS / 64;
  static constexpr int S_INST = kScales ? (S_TOTAL + NW - 1) / NW : 0;
  static constexpr int NVM = N_INST + S_INST;
  mp::Rsrc rd, rs;
  uint32_t voff[N_INST], soff[S_INST > 0 ? S_INST : 1];
  int srow0[S_INST > 0 ? S_INST : 1];
  int wave;
  // Row r's scale dwords start at scales + (r / sdiv) * ld_scale bytes.
  INTENT_DEVICE void init(const uint8_t* rows, int64_t ld, int M, const uint8_t* scales, int64_t ld_scale, int m0,
                          int w, int sdiv = 1) {
    wave = w;
    rd = make_rsrc(rows + (int64_t)m0 * ld);
    rs = make_rsrc(kScales ? scales : rows);
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int j = 0; j < N_INST; ++j) {
      const int r = (j * NW + w) * 8 + (lane >> 3);
      const int rr = m0 + r < M ? r : M - 1 - m0;
      voff[j] = (uint32_t)(rr * ld + (((lane & 7) ^ mp::swz(r)) << 4));
    }
#pragma unroll
    for (int j = 0; j < S_INST; ++j) {
      const int t = j * NW + w < S_TOTAL ? j * NW + w : S_TOTAL - 1;
      srow0[j] = t * 64;
      const int r = t * 64 + lane;
      const int m = m0 + r < M ? m0 + r : M - 1;
      soff[j] = (uint32_t)((m / sdiv) * ld_scale);
    }
  }
  // rows: this operand's row region of a stage; scl: its scale region;
  // koff: the stage's byte offset in a row; kt: its index (scale dword).
  INTENT_DEVICE void issue(char* rows, char* scl, uint32_t koff, int kt) const {
#pragma unroll
    for (int j = 0; j < N_INST; ++j)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rd, (mp::lds_t*)(rows + (j * NW + wave) * 8 * mp::ROWB), 16, voff[j],
                                               koff, 0, 0);
#pragma unroll
    for (int j = 0; j < S_INST; ++j)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (mp::lds_t*)(scl + srow0[j] * 4), 4, soff[j], (uint32_t)kt * 4, 0,
                                               0);
  }
};

// The right operand as [K][N] bytes (N contiguous), read in place: no
// transposed copy. A stage is 128 k-rows of the tile's 128 columns, 128 bytes
// each (the size of the row form's stage). DMA instruction t fills LDS
// kilobyte t, k-rows 8t..8t+7: lane i moves 16-byte slot i % 8 of k-row
// 8t + i / 8, which holds column chunk (i % 8) ^ kn8_swz(k-row). Fragments
// are read with ds_read_b64_tr_b8: inside a group of 16 lanes, lane j
// addresses k-row k0 + j / 2, columns c0 + 8 (j % 2) .. + 7, and lane t
// receives column c0 + t at k-rows k0 .. k0 + 7. Four such reads give a lane
// the 32 k of one column that read_frag gives a row (chunks c and c + 2 of
// the stage). One read touches, per half wave, 8 k-rows x 32 bytes; with the
// swizzle the four k-rows of each parity hit four distinct 32-byte windows,
// so those 16 pieces cover the 64 banks once.
INTENT_DEVICE constexpr int kn8_swz(int krow) { return 2 * ((krow >> 1) & 3); }

template <int COLS, int NW>
struct KNBytes {
  static constexpr bool kKN = true;
  static_assert(COLS == 128, "128 columns: one 128-byte LDS row per k-row");
  static constexpr int TOTAL = 16;  // kilobyte DMA instructions per stage
  static constexpr int N_INST = TOTAL / NW;
  static constexpr int NVM = N_INST;
  static_assert(N_INST * NW == TOTAL, "stage instructions split evenly over the waves");
  mp::Rsrc rd;
  uint32_t voff[N_INST];
  uint32_t ld;  // bytes per k-row
  int wave;
  // b: element (0, 0) of [K][N]; ldb bytes per k-row; n0: first column of the
  // tile. Requires N % 16 == 0: column chunks past N re-read the last valid
  // chunk (their products land in output columns that are never stored).
  INTENT_DEVICE void init(const uint8_t* b, int64_t ldb, int N, int n0, int w) {
    wave = w;
    ld = (uint32_t)ldb;
    rd = make_rsrc(b + n0);
    const int lane = threadIdx.x & 63;
    const int valid = N - n0;
#pragma unroll
    for (int j = 0; j < N_INST; ++j) {
      const int r = (j * NW + w) * 8 + (lane >> 3);
      int col = ((lane & 7) ^ kn8_swz(r)) * 16;
      col = col + 16 <= valid ? col : valid - 16;
      voff[j] = (uint32_t)(r * ldb + col);
    }
  }
  // koff: the stage's first k (the row form's byte offset inside a row).
  INTENT_DEVICE void issue(char* rows, char*, uint32_t koff, int) const {
#pragma unroll
    for (int j = 0; j < N_INST; ++j)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rd, (mp::lds_t*)(rows + (j * NW + wave) * 1024), 16, voff[j],
                                               koff * ld, 0, 0);
  }
};

typedef int i32x2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) i32x2 lds_i32x2_t;

INTENT_DEVICE i32x2 read_tr8(const char* p) {
  return __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_i32x2_t*)(__attribute__((address_space(3))) char*)p);
}

// Per-lane base of the transpose reads of column block j (wave-tile column
// wn0 + 32 j): the lane's k-row inside an 8-row group is t / 2 (t = lane %
// 16), so its swizzle is the same for every read.
INTENT_DEVICE uint32_t kn8_base(int wn0, int j) {
  const int lane = threadIdx.x & 63;
  const int g = lane >> 4, t = lane & 15;
  const int cc = wn0 / 16 + 2 * j + (g & 1);
  const int kr = t >> 1;
  return (uint32_t)(kr * 128 + ((cc ^ kn8_swz(kr)) << 4) + 8 * (t & 1) + (g >> 1) * 16 * 128);
}

// The lane's 32 bytes of step s (chunks 4s + h and 4s + 2 + h in k units of
// 16, h = lane / 32, already in base): k-rows 64 s + {0, 8, 32, 40} + ...
INTENT_DEVICE i32x8 read_frag_kn(const char* b, uint32_t base, int s) {
  const char* p = b + base + s * 64 * 128;
  const i32x2 q0 = read_tr8(p), q1 = read_tr8(p + 8 * 128), q2 = read_tr8(p + 32 * 128), q3 = read_tr8(p + 40 * 128);
  return i32x8{q0[0], q0[1], q1[0], q1[1], q2[0], q2[1], q3[0], q3[1]};
}

// How a stage's per-row scale dwords are used.
enum class ScaleMode {
  kNone,     // no scales: every block scale is E8M0 127 (2^0)
  kE8M0,     // four E8M0 block scales (32 k each) feed the scaled MFMA
  kPromote,  // one f32 scale per row and 128-k stage: each stage is summed into
             // a fresh accumulator, then hook(acc, row scales of A, of B, kt)
             // folds it into the caller's own accumulators
  kHook,     // no scales; hook(acc, -, -, kt) runs after every stage (and may
             // consume and clear acc)
  kInt8,     // no scales; int8 operands, exact int32 sums: each 64-k step is
             // two v_mfma_i32_32x32x32_i8 over the two 16-byte halves
};

// acc += A·B over nk stages (stage kt at byte offset koff(kt) of every row).
// T: a 4-wave tile whose rows are multiples of 64. Starts with a barrier, so
// that it can run again on the same LDS, and ends with no DMA in flight.
// kFmt: the operands' format code for the f8f6f4 MFMA (0 E4M3, 1 E5M2).
// BOp: Rows (B as [N][K] rows) or KNBytes (B as [K][N], no scales).
template <class T, ScaleMode kMode, class KOff, class Hook, int kFmt = 0,
          class BOp = Rows<T::BN, T::NW, kMode == ScaleMode::kE8M0 || kMode == ScaleMode::kPromote>>
INTENT_DEVICE void dma_mainloop(char* smem,
                                const Rows<T::BM, T::NW, kMode == ScaleMode::kE8M0 || kMode == ScaleMode::kPromote>& aop,
                                const BOp& bop, int nk, KOff koff,
                                i32x16 (&acc)[T::TI][T::TJ], Hook&& hook) {
  constexpr bool kScales = kMode == ScaleMode::kE8M0 || kMode == ScaleMode::kPromote;
  constexpr bool kHooked = kMode == ScaleMode::kPromote || kMode == ScaleMode::kHook;
  constexpr int ROWBYTES = (T::BM + T::BN) * mp::ROWB;
  constexpr int SB = ROWBYTES + (T::BM + T::BN) * 4;
  constexpr int A_SC = ROWBYTES;
  constexpr int B_SC = A_SC + T::BM * 4;
  constexpr int NV = Rows<T::BM, T::NW, kScales>::NVM + BOp::NVM;
  static_assert(!(BOp::kKN && kScales), "the [K][N] operand carries no scales");
  static_assert(2 * NV < 64, "vmcnt range");
  const int lane = threadIdx.x & 63;
  const int h = lane >> 5;
  const int ra = T::wave_m() * T::WTM + (lane & 31);
  const int rb = T::wave_n() * T::WTN + (lane & 31);
  auto issue = [&](int slot, int kt) {
    char* base = smem + slot * SB;
    const int st = kt < nk ? kt : nk - 1;  // past the end: the last stage again, into a buffer nobody reads
    aop.issue(base, base + A_SC, koff(st), st);
    bop.issue(base + T::A_BYTES, base + B_SC, koff(st), st);
  };
  // Fragments of step s: lane half h reads chunks 4s+h and 4s+2+h; two
  // register sets (step parity). Scales: one dword per fragment row and
  // stage; the next stage's are read into nsa / nsb and become current at the
  // stage's end.
  i32x8 af[2][T::TI], bf[2][T::TJ];
  uint32_t csa[T::TI], csb[T::TJ], nsa[T::TI], nsb[T::TJ];
  // kPromote: hook(i, j, fresh, xa, xb) folds one tile's stage sum. Stage
  // kt's sums are folded tile by tile just before stage kt + 1's first MFMA
  // of the tile overwrites them, with stage kt's scale dwords kept in psa /
  // psb, so each fold's VALU work overlaps the MFMAs in flight; the first
  // fold adds zeros, the last stage is folded after the loop.
  uint32_t psa[T::TI], psb[T::TJ];
  if constexpr (kMode == ScaleMode::kPromote) {
#pragma unroll
    for (int i = 0; i < T::TI; ++i) psa[i] = 0u;
#pragma unroll
    for (int j = 0; j < T::TJ; ++j) psb[j] = 0u;
#pragma unroll
    for (int i = 0; i < T::TI; ++i)
#pragma unroll
      for (int j = 0; j < T::TJ; ++j) acc[i][j] = i32x16{};
  }
  uint32_t knb[T::TJ];
  if constexpr (BOp::kKN) {
#pragma unroll
    for (int j = 0; j < T::TJ; ++j) knb[j] = kn8_base(T::wave_n() * T::WTN, j);
  }
  auto read = [&](const char* base, int s, int set) {
#pragma unroll
    for (int i = 0; i < T::TI; ++i) af[set][i] = read_frag(base, ra + 32 * i, 4 * s + h);
#pragma unroll
    for (int j = 0; j < T::TJ; ++j)
      bf[set][j] = BOp::kKN ? read_frag_kn(base + T::A_BYTES, knb[j], s)
                            : read_frag(base + T::A_BYTES, rb + 32 * j, 4 * s + h);
  };
  // E8M0 scale dwords are shifted right by 8h as they are read: lane half h
  // then finds group 2s + h's byte at byte 2s, which the MFMA's scale byte
  // select picks (no byte extraction per MFMA).
  const uint32_t sc_shift = kMode == ScaleMode::kE8M0 ? 8u * (uint32_t)h : 0u;
  auto read_scales = [&](const char* base, uint32_t (&xa)[T::TI], uint32_t (&xb)[T::TJ]) {
#pragma unroll
    for (int i = 0; i < T::TI; ++i)
      xa[i] = kScales ? *reinterpret_cast<const uint32_t*>(base + A_SC + (ra + 32 * i) * 4) >> sc_shift : 0x7F7F7F7Fu;
#pragma unroll
    for (int j = 0; j < T::TJ; ++j)
      xb[j] = kScales ? *reinterpret_cast<const uint32_t*>(base + B_SC + (rb + 32 * j) * 4) >> sc_shift : 0x7F7F7F7Fu;
  };
  auto mfmas = [&](auto S) {
    constexpr int s = decltype(S)::value;
#pragma unroll
    for (int i = 0; i < T::TI; ++i)
#pragma unroll
      for (int j = 0; j < T::TJ; ++j) {
        if constexpr (kMode == ScaleMode::kInt8) {
          const i32x8 x = bf[s][j], y = af[s][i];
          acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(i32x4{x[0], x[1], x[2], x[3]}, i32x4{y[0], y[1], y[2], y[3]},
                                                           acc[i][j], 0, 0, 0);
          acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(i32x4{x[4], x[5], x[6], x[7]}, i32x4{y[4], y[5], y[6], y[7]},
                                                           acc[i][j], 0, 0, 0);
          continue;
        }
        if constexpr (kMode == ScaleMode::kPromote)
          if (s == 0) hook(i, j, acc[i][j], psa, psb);  // fold the previous stage's sum of this tile
        f32x16 c = bit_cast<f32x16>(acc[i][j]);
        if (kMode == ScaleMode::kPromote && s == 0) c = f32x16{};  // a fresh sum per stage
        if constexpr (kMode == ScaleMode::kE8M0)
          c = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(bf[s][j], af[s][i], c, kFmt, kFmt, 2 * s, (int)csb[j],
                                                              2 * s, (int)csa[i]);
        else
          c = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(bf[s][j], af[s][i], c, kFmt, kFmt, 0, 127, 0, 127);
        acc[i][j] = bit_cast<i32x16>(c);
      }
  };
  // Schedule hint: each MFMA followed by its share of NR LDS reads (0x100).
  constexpr int NMF = T::TI * T::TJ * (kMode == ScaleMode::kInt8 ? 2 : 1);  // MFMAs per step
  auto interleave = [&](auto NR) {
    mp::static_for<0, NMF>([&](auto X) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      constexpr int x = decltype(X)::value;
      constexpr int nr = decltype(NR)::value;
      constexpr int r = (x + 1) * nr / NMF - x * nr / NMF;
      if constexpr (r > 0) __builtin_amdgcn_sched_group_barrier(0x100, r, 0);
    });
  };
  constexpr int NR = 2 * T::TI + (BOp::kKN ? 4 : 2) * T::TJ;  // LDS reads per step

  __syncthreads();  // a previous pass over this LDS is fully read
  issue(0, 0);
  issue(1, 1);
  mp::wait_vm_lgkm_barrier<NV>();
  read_scales(smem, csa, csb);
  read(smem, 0, 0);

  // The last stage is peeled off so that the loop body has no branch.
  auto stage = [&](int kt, auto more) {
    const int slot = kt & 1;
    const char* base = smem + slot * SB;
    read(base, 1, 1);
    mfmas(std::integral_constant<int, 0>{});
    interleave(std::integral_constant<int, NR>{});
    if constexpr (decltype(more)::value) {
      mp::wait_vm_lgkm_barrier<0>();  // stage kt+1 landed everywhere; stage kt fully read
      issue(slot, kt + 2);
      const char* nb = smem + (slot ^ 1) * SB;
      read_scales(nb, nsa, nsb);
      read(nb, 0, 0);
      mfmas(std::integral_constant<int, 1>{});
      interleave(std::integral_constant<int, NR + (kScales ? 4 : 0)>{});
      if constexpr (kMode == ScaleMode::kPromote) {
#pragma unroll
        for (int i = 0; i < T::TI; ++i) psa[i] = csa[i];
#pragma unroll
        for (int j = 0; j < T::TJ; ++j) psb[j] = csb[j];
      } else if constexpr (kHooked) {
        hook(acc, csa, csb, kt);
      }
#pragma unroll
      for (int i = 0; i < T::TI; ++i) csa[i] = nsa[i];
#pragma unroll
      for (int j = 0; j < T::TJ; ++j) csb[j] = nsb[j];
    } else {
      mfmas(std::integral_constant<int, 1>{});
      if constexpr (kMode == ScaleMode::kPromote) {
#pragma unroll
        for (int i = 0; i < T::TI; ++i)
#pragma unroll
          for (int j = 0; j < T::TJ; ++j) hook(i, j, acc[i][j], csa, csb);
      } else if constexpr (kHooked) {
        hook(acc, csa, csb, kt);
      }
    }
  };
  for (int kt = 0; kt < nk - 1; ++kt) stage(kt, std::true_type{});
  stage(nk - 1, std::false_type{});
  mp::wait_vm<0>();  // no DMA may still be writing LDS when the workgroup ends
}

struct NoHook {
  template <class... A>
  INTENT_DEVICE void operator()(A&&...) const {}
};

template <int TI, int TJ>
INTENT_DEVICE void zero(i32x16 (&acc)[TI][TJ]) {
#pragma unroll
  for (int i = 0; i < TI; ++i)
#pragma unroll
    for (int j = 0; j < TJ; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0;  // the bits of +0.0f
}


// Output staging through LDS for the kernels fed by dma_mainloop. After its
// last stage every wave has waited for its own DMA, so one workgroup barrier
// leaves the whole stage ring free. Each wave then owns 32 x (WTN * EB + 16)
// bytes and moves its WTM x WTN tile 32 rows at a time: lanes write their
// accumulator layout (row lane % 32, four consecutive columns, packed by
// pack(i, j, g) into EB dwords: one output element is EB bytes), then read
// back whole 16-byte row pieces, so a store instruction covers whole row
// segments instead of 4 * EB bytes in each of 32 rows. Rows past M are
// skipped; pieces past N, or an output without 16-byte aligned rows, store
// element by element.
template <int EB>
struct Piece {
  uint32_t w[EB];
};
template <class T, int EB, class Pack>
INTENT_DEVICE void store_rows_lds(char* smem, int m0, int n0, int M, int N, char* __restrict__ out, int64_t ldo_bytes,
                                  Pack&& pack) {
  constexpr int RS = T::WTN * EB + 16;  // LDS row bytes
  constexpr int CH = T::WTN * EB / 16;  // 16-byte pieces per row
  constexpr int NP = 32 * CH / 64;      // pieces per lane and block
  constexpr int EPP = 16 / EB;          // elements per piece
  static_assert(NP * 64 == 32 * CH, "whole pieces per lane");
  static_assert(T::NW * 32 * RS <= 2 * ((T::BM + T::BN) * mp::ROWB), "staging fits the stage ring");
  __syncthreads();
  const int lane = threadIdx.x & 63;
  char* blk = smem + T::wave() * 32 * RS;
  const int wm = m0 + T::wave_m() * T::WTM, wn = n0 + T::wave_n() * T::WTN;
  const bool vec = (ldo_bytes & 15) == 0 && (((uintptr_t)out) & 15) == 0;
#pragma unroll
  for (int i = 0; i < T::TI; ++i) {
#pragma unroll
    for (int j = 0; j < T::TJ; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const Piece<EB> v = pack(i, j, g);
        char* d = blk + (lane & 31) * RS + (n0 + T::col(j, g) - wn) * EB;
        if constexpr (EB == 4)
          *reinterpret_cast<u32x4*>(d) = u32x4{v.w[0], v.w[1], v.w[2], v.w[3]};
        else if constexpr (EB == 2)
          *reinterpret_cast<u32x2*>(d) = u32x2{v.w[0], v.w[1]};
        else
          *reinterpret_cast<uint32_t*>(d) = v.w[0];
      }
#pragma unroll
    for (int q = 0; q < NP; ++q) {
      const int p = q * 64 + lane, r = p / CH, cb = (p % CH) * 16;
      const u32x4 v = *reinterpret_cast<const u32x4*>(blk + r * RS + cb);
      const int gm = wm + i * 32 + r, gn = wn + cb / EB;
      if (gm >= M) continue;
      char* dst = out + (int64_t)gm * ldo_bytes + (int64_t)gn * EB;
      if (vec && gn + EPP <= N) {
        *reinterpret_cast<u32x4*>(dst) = v;
      } else {
        uint8_t b[16];
        __builtin_memcpy(b, &v, 16);
#pragma unroll
        for (int e = 0; e < EPP; ++e)
          if (gn + e < N) __builtin_memcpy(dst + e * EB, b + e * EB, EB);
      }
    }
  }
}
}  // namespace mxdma

// One output tile of the MX product on dma_mainloop (four waves).
template <class T>
INTENT_DEVICE void mx_dma_tile(char* smem, const uint8_t* __restrict__ a, int64_t lda, int M,
                               const uint8_t* __restrict__ sa, int64_t ld_sa, const uint8_t* __restrict__ b,
                               int64_t ldb, int N, const uint8_t* __restrict__ sb, int64_t ld_sb, int K,
                               float* __restrict__ out, int64_t ldo, int m0, int n0) {
  mxdma::Rows<T::BM, T::NW, true> aop;
  mxdma::Rows<T::BN, T::NW, true> bop;
  aop.init(a, lda, M, sa, ld_sa, m0, T::wave());
  bop.init(b, ldb, N, sb, ld_sb, n0, T::wave());
  i32x16 acc[T::TI][T::TJ];
  mxdma::zero(acc);
  mxdma::dma_mainloop<T, mxdma::ScaleMode::kE8M0>(smem, aop, bop, K / mp::ROWB, mxdma::SplitK{1, 0}, acc,
                                                  mxdma::NoHook{});
  mxdma::store_rows_lds<T, 4>(smem, m0, n0, M, N, reinterpret_cast<char*>(out), ldo * 4, [&](int i, int j, int g) {
    return mxdma::Piece<4>{{(uint32_t)acc[i][j][4 * g], (uint32_t)acc[i][j][4 * g + 1], (uint32_t)acc[i][j][4 * g + 2],
                            (uint32_t)acc[i][j][4 * g + 3]}};
  });
}

// Workgroups 0 .. nbig-1 take the 256 x 256 tiles of columns [0, n_split)
// (XCD-grouped order); the rest, dispatched last, take 256 x 128 tiles of
// columns [n_split, N). The launch picks n_split so that the half-size tiles
// fill what would otherwise be a partial last round of 256 x 256 tiles.
using TMxHalf = mp::Tile<256, 128, 2, 2>;
__global__ __launch_bounds__(256, 1) void mxfp8_gemm_dma_kernel(const uint8_t* __restrict__ a, int64_t lda, int M,
                                                                const uint8_t* __restrict__ sa, int64_t ld_sa,
                                                                const uint8_t* __restrict__ b, int64_t ldb, int N,
                                                                const uint8_t* __restrict__ sb, int64_t ld_sb, int K,
                                                                float* __restrict__ out, int64_t ldo, int mblocks,
                                                                int nbig, int n_split) {
  using T = mxdma::Tile;
  __shared__ __attribute__((aligned(1024))) char smem[2 * mxdma::kStage];
  const int bid = blockIdx.x;
  if (bid < nbig) {
    int tmb, tnb;
    grouped_tile(xcd_swizzle(bid, nbig), mblocks, nbig / mblocks, 4, tmb, tnb);
    mx_dma_tile<T>(smem, a, lda, M, sa, ld_sa, b, ldb, N, sb, ld_sb, K, out, ldo, tmb * T::BM, tnb * T::BN);
  } else {
    const int t = bid - nbig;
    mx_dma_tile<TMxHalf>(smem, a, lda, M, sa, ld_sa, b, ldb, N, sb, ld_sb, K, out, ldo, (t % mblocks) * TMxHalf::BM,
                         n_split + (t / mblocks) * TMxHalf::BN);
  }
}

// Per-tensor scaled FP8 GEMM with an f16 result (block_scaled.py:42-63 and,
// with splits > 1, the split-K form :66-98): for each split s in order,
//   p = f16((acc_s * lhs_scale) * rhs_scale)   (acc_s: the f32 sum over split s)
// and out = p (kAccum false, one split) or out = f16(out + p) (kAccum).
// bt: the right operand as [N, K] rows (K contiguous). K % (256 * splits) == 0
// when splits > 1, K % 128 == 0 otherwise. One pipelined pass over all
// splits' stages (split s, stage t at mxdma::SplitK order); at the end of each
// split the hook folds the split's f32 sum into the f16 output tile, which
// stays in registers: read once (kAccum) and written once.
using TSk = mp::Tile<256, 128, 2, 2>;  // four waves of 128 x 64

// The same output for an empty K: p = f16((0 * lhs_scale) * rhs_scale) (zero,
// or NaN for a non-finite scale); splits == 0 stores p, else out = f16(out + p)
// once per split.
__global__ __launch_bounds__(256) void fp8_scaled_empty_k_kernel(f16* __restrict__ out, int64_t rows, int64_t cols,
                                                                 int64_t ldo, float lhs_scale, float rhs_scale,
                                                                 int splits) {
  const int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (c >= cols) return;
  const float acc = 0.f;
  const f16 p = (f16)((acc * lhs_scale) * rhs_scale);
  for (int64_t r = blockIdx.y; r < rows; r += gridDim.y) {
    f16* o = out + r * ldo + c;
    if (splits == 0) {
      *o = p;
    } else {
      f16 v = *o;
      for (int s = 0; s < splits; ++s) v = v + p;
      *o = v;
    }
  }
}

// b: the right operand's [N][K] rows (the [K][N] form goes to fp8_scaled_ws_kernel).
template <bool kAccum>
__global__ __launch_bounds__(256, 1) void fp8_scaled_gemm_kernel(const uint8_t* __restrict__ a, int64_t lda, int M,
                                                                 const uint8_t* __restrict__ b, int64_t ldb, int N,
                                                                 int K, int splits, float ls, float rs,
                                                                 f16* __restrict__ out, int64_t ldo, int mblocks) {
  using T = TSk;
  constexpr int SB = (T::BM + T::BN) * (mp::ROWB + 4);
  __shared__ __attribute__((aligned(1024))) char smem[2 * SB];
  int tmb, tnb;
  grid_tile(mblocks, 4, tmb, tnb);
  const int m0 = tmb * T::BM;
  const int n0 = tnb * T::BN;
  mxdma::Rows<T::BM, T::NW, false> aop;
  mxdma::Rows<T::BN, T::NW, false> bop;
  aop.init(a, lda, M, nullptr, 0, m0, T::wave());
  bop.init(b, ldb, N, nullptr, 0, n0, T::wave());
  const int nks = K / mp::ROWB / splits;
  // The lane's outputs: m = row(i), n = col(j, g) + q, as packed f16 pairs
  // o[i][j][2g + q/2] (64 registers).
  f16x2 o[T::TI][T::TJ][8];
  const bool vec = (ldo & 3) == 0 && (((uintptr_t)out) & 7) == 0;
#pragma unroll
  for (int i = 0; i < T::TI; ++i) {
    const int m = m0 + T::row(i);
#pragma unroll
    for (int j = 0; j < T::TJ; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int n = n0 + T::col(j, g);
        const f16* src = out + (int64_t)m * ldo + n;
        f16x2 lo = splat2((f16)0.f), hi = splat2((f16)0.f);
        if (kAccum && m < M) {
          if (vec && n + 3 < N) {
            const u32x2 w = *reinterpret_cast<const u32x2*>(src);
            lo = bit_cast<f16x2>(w[0]);
            hi = bit_cast<f16x2>(w[1]);
          } else {
            if (n < N) lo[0] = src[0];
            if (n + 1 < N) lo[1] = src[1];
            if (n + 2 < N) hi[0] = src[2];
            if (n + 3 < N) hi[1] = src[3];
          }
        }
        o[i][j][2 * g] = lo;
        o[i][j][2 * g + 1] = hi;
      }
  }
  i32x16 acc[T::TI][T::TJ];
  mxdma::zero(acc);
  auto fold = [&](i32x16 (&f)[T::TI][T::TJ], const uint32_t (&)[T::TI], const uint32_t (&)[T::TJ], int kt) {
    if ((kt + 1) % nks) return;  // wave-uniform: only at the end of a split
#pragma unroll
    for (int i = 0; i < T::TI; ++i)
#pragma unroll
      for (int j = 0; j < T::TJ; ++j) {
        const f32x16 v = bit_cast<f32x16>(f[i][j]);
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const f16 p = (f16)__fmul_rn(__fmul_rn(v[e], ls), rs);
          o[i][j][e >> 1][e & 1] = kAccum ? (f16)__fadd_rn((float)o[i][j][e >> 1][e & 1], (float)p) : p;
        }
        f[i][j] = i32x16{};
      }
  };
  const auto koff = [nks, splits](int kt) { return mxdma::SplitK{splits, kt / nks}(kt % nks); };
  mxdma::dma_mainloop<T, mxdma::ScaleMode::kHook>(smem, aop, bop, nks * splits, koff, acc, fold);
  mxdma::store_rows_lds<T, 2>(smem, m0, n0, M, N, reinterpret_cast<char*>(out), ldo * 2, [&](int i, int j, int g) {
    return mxdma::Piece<2>{{bit_cast<uint32_t>(o[i][j][2 * g]), bit_cast<uint32_t>(o[i][j][2 * g + 1])}};
  });
}

// [K][N] bytes (N contiguous: the reference's right operand, block_scaled.py
// :62-93) read in place by producer waves and transposed on the way to LDS:
// k block kb (128 bytes of k) of columns n0 .. n0 + 127 becomes 128 LDS rows,
// one per column, of 128 k-bytes in the row form's chunk order (chunk c of
// row n at c ^ swz(n)), so that the consumers read it like an [N][K] operand.
// Producer thread t of NT: column quad q = t % 32 (columns 4q .. 4q + 3),
// k-rows 16 (t / 32) .. + 15. Per stage it issues 16 dword loads (a wave
// reads two 128-byte row segments per load), transposes each 4 x 4 byte
// block with v_perm_b32 and writes one 16-byte chunk per column. Lanes whose
// bit 2 of q is set write their columns in the order 2 3 0 1, so that any 8
// consecutive lanes write 8 distinct chunk positions (no bank conflicts).
// Columns past N re-read the last valid quad (their products land in output
// columns that are never stored): N % 4 == 0.
template <int NT>
struct KNTransposeOperand {
  static_assert(NT == 256, "eight k-row groups of 32 column quads");
  static constexpr bool kWinParams = false;
  static constexpr int NVM = 16;  // loads per stage
  struct Regs {
    uint32_t d[16];
  };
  mp::Rsrc rb;
  uint32_t voff;
  uint32_t ld;
  int kb, q;
  uint32_t sel_lo, sel_hi;  // first-level perm selectors (swapped for the rotated lanes)
  INTENT_DEVICE void init(const uint8_t* b, int64_t ldb, int N, int n0) {
    const int t = (int)(threadIdx.x % NT);
    q = t & 31;
    kb = t >> 5;
    const int valid = N - n0;
    const int col = 4 * q + 4 <= valid ? 4 * q : valid - 4;
    rb = make_rsrc(b + n0);
    ld = (uint32_t)ldb;
    voff = (uint32_t)(kb * 16 * ldb + col);
    const bool rot = (q >> 2) & 1;
    // (d_even, d_odd) -> {e.b0, o.b0, e.b1, o.b1} and {e.b2, o.b2, e.b3, o.b3}
    sel_lo = rot ? 0x07030602u : 0x05010400u;
    sel_hi = rot ? 0x05010400u : 0x07030602u;
  }
  // blk: the k block of the stage (128 k-rows of [K][N]).
  INTENT_DEVICE void load(int blk, Regs& r) const {
    const uint32_t base = (uint32_t)blk * 128u * ld;
#pragma unroll
    for (int i = 0; i < 16; ++i) r.d[i] = __builtin_amdgcn_raw_buffer_load_b32(rb, voff, base + (uint32_t)i * ld, 0);
  }
  template <bool kAsm = false>
  INTENT_DEVICE void store(const Regs& r, char* lds_b) const {
    // col[c][g]: k-bytes 4g .. 4g + 3 of column slot c (slot c holds column c
    // for unrotated lanes, c ^ 2 for rotated ones).
    uint32_t col[4][4];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const uint32_t d0 = r.d[4 * g], d1 = r.d[4 * g + 1], d2 = r.d[4 * g + 2], d3 = r.d[4 * g + 3];
      const uint32_t lo01 = __builtin_amdgcn_perm(d1, d0, sel_lo), hi01 = __builtin_amdgcn_perm(d1, d0, sel_hi);
      const uint32_t lo23 = __builtin_amdgcn_perm(d3, d2, sel_lo), hi23 = __builtin_amdgcn_perm(d3, d2, sel_hi);
      col[0][g] = __builtin_amdgcn_perm(lo23, lo01, 0x05040100u);
      col[1][g] = __builtin_amdgcn_perm(lo23, lo01, 0x07060302u);
      col[2][g] = __builtin_amdgcn_perm(hi23, hi01, 0x05040100u);
      col[3][g] = __builtin_amdgcn_perm(hi23, hi01, 0x07060302u);
    }
    const int rot = ((q >> 2) & 1) << 1;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int n = 4 * q + (c ^ rot);
      char* dst = lds_b + n * mp::ROWB + ((kb ^ mp::swz(n)) << 4);
      const u32x4 v{col[c][0], col[c][1], col[c][2], col[c][3]};
      if constexpr (kAsm)
        mp::lds_store16(dst, v);
      else
        *reinterpret_cast<u32x4*>(dst) = v;
    }
  }
};

// The per-tensor scaled FP8 GEMM (and split-K) with the [K][N] operand read in
// place, on the producer/consumer core (mp::mainloop_ws): four consumer waves
// of 128 x 64 and four producer waves per 256 x 128 tile; producers copy the
// A rows by LDS DMA and transpose the B bytes into LDS. Split s's stages run
// in order, and at the end of each the consumers fold the split's f32 sum
// into the f16 output tile, which lives in LDS (64 KB beside the two 48 KB
// stage buffers: the registers of two waves per SIMD do not hold it beside
// the accumulators and fragments): o = f16(o + f16((acc * ls) * rs)), o read
// from out first (kAccum), else o = the one split's product.
// Consumer wave c's region: 128 rows of 128 bytes (its 64 columns); 16-byte
// unit u (columns 8u .. 8u + 7) of row r sits at unit u ^ (r & 7). With
// 16-byte aligned output rows, producer wave c fills region c from out by LDS
// DMA before the main loop (the prologue's wait covers it); otherwise the
// consumer loads it.
INTENT_DEVICE int ounit(int r, int u) { return u ^ (r & 7); }

template <bool kAccum>
__global__ __launch_bounds__(TSk::NT_WS, 1) void fp8_scaled_ws_kernel(const uint8_t* __restrict__ a, int64_t lda,
                                                                      int M, const uint8_t* __restrict__ b,
                                                                      int64_t ldb, int N, int K, int splits, float ls,
                                                                      float rs, f16* __restrict__ out, int64_t ldo,
                                                                      int mblocks) {
  using T = TSk;
  constexpr int ORB = T::WTN * 2;  // bytes per row of an output region
  static_assert(ORB == 128 && T::WTM == 128, "output regions of 128 x 64");
  __shared__ __attribute__((aligned(16))) char buf0[T::STAGE_BYTES];
  __shared__ __attribute__((aligned(16))) char buf1[T::STAGE_BYTES];
  __shared__ __attribute__((aligned(16))) char otile[T::NW * T::WTM * ORB];
  char* const bufs[2] = {buf0, buf1};
  int mb, nb;
  grouped_tile(xcd_swizzle(blockIdx.x, gridDim.x), mblocks, (int)gridDim.x / mblocks, 4, mb, nb);
  const int m0 = mb * T::BM;
  const int n0 = nb * T::BN;
  const int nks = K / mp::ROWB / splits;
  const int lane = threadIdx.x & 63;
  const bool consumer = T::wave() < T::NW;
  const int region = T::wave() % T::NW;  // consumer: its own; producer: the one it fills
  char* const ot = otile + region * T::WTM * ORB;
  const int wm = m0 + (region % T::WM) * T::WTM, wn = n0 + (region / T::WM) * T::WTN;
  const bool dma_out = (ldo & 7) == 0 && (((uintptr_t)out) & 15) == 0 && (int64_t)M * ldo * 2 < (1ll << 31);
  if (kAccum && !consumer && dma_out) {
    // 16 DMA instructions of 8 rows x 128 bytes; lane l fills unit l % 8 of
    // row 8 j + l / 8, i.e. logical unit (l % 8) ^ (row & 7). Rows past M
    // re-read row M - 1 and units past N the last valid one (never stored).
    const mp::Rsrc ro = make_rsrc(out);
#pragma unroll
    for (int j = 0; j < T::WTM / 8; ++j) {
      const int r = 8 * j + (lane >> 3);
      const int gm = wm + r < M ? wm + r : M - 1;
      const int gn0 = wn + 8 * ounit(r, lane & 7);
      const int gn = gn0 + 8 <= N ? gn0 : N - 8;
      mp::lds_dma<16, false>(ro, (mp::lds_t*)(ot + j * 8 * ORB), (uint32_t)(((int64_t)gm * ldo + gn) * 2), 0u);
    }
  }
  if (kAccum && consumer && !dma_out) {
#pragma unroll 4
    for (int p = lane; p < T::WTM * 16; p += 64) {  // 8-byte pieces: row p / 16, columns 4 (p % 16) ..
      const int r = p >> 4, sl = p & 15, gm = wm + r, gn = wn + 4 * sl;
      uint16_t e[4] = {0, 0, 0, 0};
      if (gm < M) {
        const uint16_t* src = reinterpret_cast<const uint16_t*>(out + (int64_t)gm * ldo + gn);
#pragma unroll
        for (int c = 0; c < 4; ++c)
          if (gn + c < N) e[c] = src[c];
      }
      *reinterpret_cast<u32x2*>(ot + r * ORB + (ounit(r, sl >> 1) << 4) + ((sl & 1) << 3)) =
          u32x2{e[0] | ((uint32_t)e[1] << 16), e[2] | ((uint32_t)e[3] << 16)};
    }
  }
  KNTransposeOperand<T::NT> bop;
  bop.init(b, ldb, N, n0);
  mp::DmaRowsOperand<T::BM, mp::DenseRows, T::NW> aop;
  aop.init(mp::DenseRows{a, lda, M}, m0, T::wave() % T::NW);
  f32x16 acc[T::TI][T::TJ];
  auto fold = [&](f32x16 (&c)[T::TI][T::TJ], int kt) {
    if ((kt + 1) % nks) return;  // wave-uniform: only at the end of a split
    const int h = lane >> 5;
#pragma unroll
    for (int i = 0; i < T::TI; ++i) {
      const int r = i * 32 + (lane & 31);
      char* row = ot + r * ORB + (h << 3);
      // The lane's 4 columns of group (j, g) are unit 4 j + g, half h.
      u32x2 o[T::TJ][4];
      if constexpr (kAccum) {
#pragma unroll
        for (int j = 0; j < T::TJ; ++j)
#pragma unroll
          for (int g = 0; g < 4; ++g) o[j][g] = *reinterpret_cast<const u32x2*>(row + (ounit(r, 4 * j + g) << 4));
      }
#pragma unroll
      for (int j = 0; j < T::TJ; ++j) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          f16 p[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) p[e] = (f16)__fmul_rn(__fmul_rn(c[i][j][4 * g + e], ls), rs);
          f16x2 lo{p[0], p[1]}, hi{p[2], p[3]};
          if constexpr (kAccum) {
            const f16x2 olo = bit_cast<f16x2>(o[j][g][0]), ohi = bit_cast<f16x2>(o[j][g][1]);
            lo = f16x2{(f16)__fadd_rn((float)olo[0], (float)p[0]), (f16)__fadd_rn((float)olo[1], (float)p[1])};
            hi = f16x2{(f16)__fadd_rn((float)ohi[0], (float)p[2]), (f16)__fadd_rn((float)ohi[1], (float)p[3])};
          }
          *reinterpret_cast<u32x2*>(row + (ounit(r, 4 * j + g) << 4)) =
              u32x2{bit_cast<uint32_t>(lo), bit_cast<uint32_t>(hi)};
        }
        c[i][j] = f32x16{};
      }
    }
  };
  const auto kmap = [nks, splits](int kt) { return (int)(mxdma::SplitK{splits, kt / nks}(kt % nks) / mp::ROWB); };
  if (!mp::mainloop_ws<T, mp::F8Math, 2>(aop, bop, nks * splits, bufs, acc, kmap, fold)) return;
  // The wave's region -> out: 8 lanes (128 bytes) per row segment.
  const bool vec = (ldo & 7) == 0 && (((uintptr_t)out) & 15) == 0;
#pragma unroll 4
  for (int p = lane; p < T::WTM * 8; p += 64) {
    const int r = p >> 3, u = p & 7, gm = wm + r, gn = wn + 8 * u;
    if (gm >= M) continue;
    const u32x4 v = *reinterpret_cast<const u32x4*>(ot + r * ORB + (ounit(r, u) << 4));
    f16* dst = out + (int64_t)gm * ldo + gn;
    if (vec && gn + 7 < N) {
      *reinterpret_cast<u32x4*>(dst) = v;
    } else {
#pragma unroll
      for (int c = 0; c < 8; ++c)
        if (gn + c < N) reinterpret_cast<uint16_t*>(dst)[c] = (uint16_t)(v[c >> 1] >> (16 * (c & 1)));
    }
  }
}

// int8 GEMM with b [K][N] read in place (gemm_i8, examples/kernels/contraction/
// gemm.py:29-39): c[m, n] = sum_k a[m, k] * b[k, n] + bias[n], int32 modulo
// 2^32. The scaled-FP8 tiles (TSk) and DMA main loop with the int8 MFMA;
// K % 128 == 0, N % 16 == 0.
__global__ __launch_bounds__(256, 1) void i8_gemm_kn_kernel(const uint8_t* __restrict__ a, int64_t lda, int M,
                                                            const uint8_t* __restrict__ b, int64_t ldb, int N, int K,
                                                            const int32_t* __restrict__ bias, int32_t* __restrict__ c,
                                                            int64_t ldc, int mblocks) {
  using T = TSk;
  constexpr int SB = (T::BM + T::BN) * (mp::ROWB + 4);
  __shared__ __attribute__((aligned(1024))) char smem[2 * SB];
  int tmb, tnb;
  grid_tile(mblocks, 4, tmb, tnb);
  const int m0 = tmb * T::BM;
  const int n0 = tnb * T::BN;
  mxdma::Rows<T::BM, T::NW, false> aop;
  mxdma::KNBytes<T::BN, T::NW> bop;
  aop.init(a, lda, M, nullptr, 0, m0, T::wave());
  bop.init(b, ldb, N, n0, T::wave());
  i32x16 acc[T::TI][T::TJ];
  mxdma::zero(acc);
  mxdma::dma_mainloop<T, mxdma::ScaleMode::kInt8>(smem, aop, bop, K / mp::ROWB, mxdma::SplitK{1, 0}, acc,
                                                  mxdma::NoHook{});
  mxdma::store_rows_lds<T, 4>(smem, m0, n0, M, N, reinterpret_cast<char*>(c), ldc * 4, [&](int i, int j, int g) {
    mxdma::Piece<4> v;
    const int n = n0 + T::col(j, g);
#pragma unroll
    for (int q = 0; q < 4; ++q)
      v.w[q] = (uint32_t)acc[i][j][4 * g + q] + (uint32_t)(bias && n + q < N ? bias[n + q] : 0);
    return v;
  });
}

// DeepGEMM-style FP8 GEMM with f32 block scales (deepgemm_fp8_2xacc,
// block_scaled.py:101-122): lhs [M, KB, 128] with one f32 scale per (row, kb),
// rhs [N, KB, 128] with one per (128-row block, kb); out = bf16(sum_kb
// (sum_k lhs*rhs) * lhs_scale * rhs_scale). The f32 scales cannot ride the
// MFMA's E8M0 scale operand, so each 128-k stage is summed into a fresh
// accumulator and folded into the main one with one fma per element
// ("2xacc"): main += fresh * (lhs_scale * rhs_scale). Tiles of 256 x 128, four
// waves of 128 x 64; the per-row scales of a stage travel with it by DMA.
using TDg = mp::Tile<256, 128, 2, 2>;

__global__ __launch_bounds__(256, 1) void deepgemm_fp8_kernel(const uint8_t* __restrict__ a, int64_t lda, int M,
                                                              const float* __restrict__ sa, int64_t ld_sa,
                                                              const uint8_t* __restrict__ b, int64_t ldb, int N,
                                                              const float* __restrict__ sb, int64_t ld_sb, int K,
                                                              uint16_t* __restrict__ out, int64_t ldo, int mblocks) {
  using T = TDg;
  constexpr int SB = (T::BM + T::BN) * (mp::ROWB + 4);
  __shared__ __attribute__((aligned(1024))) char smem[2 * SB];
  int tmb, tnb;
  grid_tile(mblocks, 4, tmb, tnb);
  const int m0 = tmb * T::BM;
  const int n0 = tnb * T::BN;
  mxdma::Rows<T::BM, T::NW, true> aop;
  mxdma::Rows<T::BN, T::NW, true> bop;
  aop.init(a, lda, M, reinterpret_cast<const uint8_t*>(sa), ld_sa * 4, m0, T::wave(), 1);
  bop.init(b, ldb, N, reinterpret_cast<const uint8_t*>(sb), ld_sb * 4, n0, T::wave(), 128);
  i32x16 fresh[T::TI][T::TJ];
  f32x16 acc[T::TI][T::TJ];
#pragma unroll
  for (int i = 0; i < T::TI; ++i)
#pragma unroll
    for (int j = 0; j < T::TJ; ++j) acc[i][j] = f32x16{};
  // The wave's B rows all lie in one 128-row block (BN = 128), so one rhs
  // scale serves the stage.
  auto promote = [&](int i, int j, const i32x16& f, const uint32_t (&xa)[T::TI], const uint32_t (&xb)[T::TJ]) {
    const float w = __fmul_rn(bit_cast<float>(xa[i]), bit_cast<float>(xb[0]));
    const f32x16 v = bit_cast<f32x16>(f);
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[i][j][e] = __builtin_fmaf(v[e], w, acc[i][j][e]);
  };
  mxdma::dma_mainloop<T, mxdma::ScaleMode::kPromote>(smem, aop, bop, K / mp::ROWB, mxdma::SplitK{1, 0}, fresh,
                                                     promote);
  mxdma::store_rows_lds<T, 2>(smem, m0, n0, M, N, reinterpret_cast<char*>(out), ldo * 2, [&](int i, int j, int g) {
    const f32x16& v = acc[i][j];
    return mxdma::Piece<2>{{f32_to_bf16_rne(v[4 * g]) | ((uint32_t)f32_to_bf16_rne(v[4 * g + 1]) << 16),
                            f32_to_bf16_rne(v[4 * g + 2]) | ((uint32_t)f32_to_bf16_rne(v[4 * g + 3]) << 16)}};
  });
}

// FP8 x FP8 -> FP8 GEMM (fp8_e4m3_matmul, fp8_e5m2_matmul,
// weight_only_int4.py:178-215): out = cast(f32 sum over k, format), both
// operands [rows, K] with K contiguous. kFmt 0: E4M3FN (nearest-even; the
// cast's contract requires results within +-448), 1: E5M2 (nearest-even,
// finite overflow to infinity).
template <int kFmt>
__global__ __launch_bounds__(256, 1) void fp8_gemm_kernel(const uint8_t* __restrict__ a, int64_t lda, int M,
                                                          const uint8_t* __restrict__ bt, int64_t ldb, int N, int K,
                                                          uint8_t* __restrict__ out, int64_t ldo, int mblocks) {
  using T = mxdma::Tile;
  __shared__ __attribute__((aligned(1024))) char smem[2 * mxdma::kStage];
  int tmb, tnb;
  grid_tile(mblocks, 4, tmb, tnb);
  const int m0 = tmb * T::BM;
  const int n0 = tnb * T::BN;
  mxdma::Rows<T::BM, T::NW, false> aop;
  mxdma::Rows<T::BN, T::NW, false> bop;
  aop.init(a, lda, M, nullptr, 0, m0, T::wave());
  bop.init(bt, ldb, N, nullptr, 0, n0, T::wave());
  i32x16 acc[T::TI][T::TJ];
  mxdma::zero(acc);
  mxdma::dma_mainloop<T, mxdma::ScaleMode::kNone, mxdma::SplitK, mxdma::NoHook, kFmt>(
      smem, aop, bop, K / mp::ROWB, mxdma::SplitK{1, 0}, acc, mxdma::NoHook{});
  mxdma::store_rows_lds<T, 1>(smem, m0, n0, M, N, reinterpret_cast<char*>(out), ldo, [&](int i, int j, int g) {
    const f32x16 c = bit_cast<f32x16>(acc[i][j]);
    uint32_t q[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) q[e] = kFmt == 0 ? f32_to_e4m3fn(c[4 * g + e]) : f32_to_e5m2(c[4 * g + e]);
    return mxdma::Piece<1>{{q[0] | (q[1] << 8) | (q[2] << 16) | (q[3] << 24)}};
  });
}

// Byte-matrix transpose through a 64 x 64 LDS tile: dst[c][r] = src[r][c].
__global__ __launch_bounds__(256) void byte_transpose_kernel(const uint8_t* __restrict__ src, int R, int C,
                                                             int64_t sld, uint8_t* __restrict__ dst, int64_t dld) {
  __shared__ uint8_t t[64][80];
  const int r0 = blockIdx.y * 64, c0 = blockIdx.x * 64;
  const int row = threadIdx.x >> 2, seg = (threadIdx.x & 3) * 16;
  const bool full = r0 + 64 <= R && c0 + 64 <= C;
  if (full && ((sld | (int64_t)(uintptr_t)src) & 15) == 0) {
    const u32x4 v = *reinterpret_cast<const u32x4*>(src + (int64_t)(r0 + row) * sld + c0 + seg);
    *reinterpret_cast<u32x4*>(&t[row][seg]) = v;
  } else {
#pragma unroll
    for (int i = 0; i < 16; ++i)
      t[row][seg + i] = (r0 + row < R && c0 + seg + i < C) ? src[(int64_t)(r0 + row) * sld + c0 + seg + i] : 0;
  }
  __syncthreads();
  uint8_t v[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) v[i] = t[seg + i][row];
  if (full && ((dld | (int64_t)(uintptr_t)dst) & 15) == 0) {
    u32x4 w;
#pragma unroll
    for (int d = 0; d < 4; ++d)
      w[d] = (uint32_t)v[4 * d] | ((uint32_t)v[4 * d + 1] << 8) | ((uint32_t)v[4 * d + 2] << 16) |
             ((uint32_t)v[4 * d + 3] << 24);
    *reinterpret_cast<u32x4*>(dst + (int64_t)(c0 + row) * dld + r0 + seg) = w;
  } else if (c0 + row < C) {
#pragma unroll
    for (int i = 0; i < 16; ++i)
      if (r0 + seg + i < R) dst[(int64_t)(c0 + row) * dld + r0 + seg + i] = v[i];
  }
}

// Byte-matrix transpose of whole 128 x 128 tiles (R, C multiples of 128,
// 16-byte aligned rows): dst[c][r] = src[r][c]. Each thread loads four
// 16-byte row pieces into LDS (128-byte rows, 16-byte slot q of row r holding
// column chunk q ^ tsw(r)), then builds four 16-byte pieces of output rows
// from two ds_read_b64_tr_b8 each: inside a group of 16 lanes, lane j
// addresses row k0 + j / 2, columns 16 cg + 8 (j % 2) .. + 7, and lane t
// receives column 16 cg + t at rows k0 .. k0 + 7. Piece p = 16 w + 4 i + g
// (wave w, step i, lane group g) is output rows 16 cg + t, cg = p / 8, at
// source rows 16 rb .. + 15, rb = p % 8: the four groups of one store cover
// 64 contiguous bytes of 16 output rows. In the 64 banks, the 16 pieces of
// each half wave (8 rows of a group x 2 groups, rows 16 apart) fall on
// distinct (row parity, slot) pairs thanks to the (r >> 4) term.
INTENT_DEVICE constexpr int tsw(int r) { return (r & 7) ^ ((r >> 4) & 1); }

__global__ __launch_bounds__(256) void byte_transpose128_kernel(const uint8_t* __restrict__ src, int64_t sld,
                                                                uint8_t* __restrict__ dst, int64_t dld) {
  __shared__ __attribute__((aligned(16))) uint8_t t[128 * 128];
  const int64_t r0 = (int64_t)blockIdx.y * 128, c0 = (int64_t)blockIdx.x * 128;
  const int tid = threadIdx.x;
  u32x4 v[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = i * 32 + (tid >> 3);
    v[i] = *reinterpret_cast<const u32x4*>(src + (r0 + r) * sld + c0 + (tid & 7) * 16);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = i * 32 + (tid >> 3);
    *reinterpret_cast<u32x4*>(&t[r * 128 + (((tid & 7) ^ tsw(r)) << 4)]) = v[i];
  }
  __syncthreads();
  const int lane = tid & 63, w = tid >> 6, g = lane >> 4, j = lane & 15;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int p = 16 * w + 4 * i + g;
    const int cg = p >> 3, rb = p & 7;
    mxdma::i32x2 q[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int r = 16 * rb + 8 * h + (j >> 1);
      q[h] = mxdma::read_tr8((const char*)t + r * 128 + ((cg ^ tsw(r)) << 4) + 8 * (j & 1));
    }
    *reinterpret_cast<i32x4*>(dst + (c0 + 16 * cg + j) * dld + r0 + 16 * rb) = i32x4{q[0][0], q[0][1], q[1][0], q[1][1]};
  }
}

// 128 x 128 tiles, four waves of 64 x 64 (a 256 x 256 tile does not fit the
// registers of eight waves once the 32-byte scaled-MFMA fragments are counted).
using TMx128 = mp::Tile<128, 128, 2, 2>;

template <class T>
int launch_mx(const uint8_t* a, int64_t M, int64_t K, int64_t a_ld, const uint8_t* sa, int64_t sa_ld,
              const uint8_t* b, int64_t N, int64_t b_ld, const uint8_t* sb, int64_t sb_ld, float* out, int64_t out_ld,
              void* stream) {
  const int mblocks = (int)((M + T::BM - 1) / T::BM);
  const int64_t grid = (int64_t)mblocks * ((N + T::BN - 1) / T::BN);
  INTENT_REQUIRE(grid < (1ll << 31), INTENT_ERR_UNSUPPORTED, "mxfp8_gemm: grid too large");
  hipLaunchKernelGGL((mxfp8_gemm_kernel<T>), dim3((unsigned)grid), dim3(T::NT), 0, (hipStream_t)stream, a, a_ld,
                     (int)M, sa, sa_ld, b, b_ld, (int)N, sb, sb_ld, (int)K, out, out_ld, mblocks);
  return intent::launch_status("mxfp8_gemm");
}

}  // namespace

extern "C" int intent_mxfp8_gemm(const uint8_t* a, int64_t M, int64_t K, int64_t a_ld, const uint8_t* a_scales,
                                 int64_t a_scales_ld, const uint8_t* b, int64_t N, int64_t b_ld,
                                 const uint8_t* b_scales, int64_t b_scales_ld, float* out, int64_t out_ld,
                                 void* stream) {
  intent::clear_error();
  INTENT_REQUIRE(M >= 0 && N >= 0 && K >= 0 && M <= INT32_MAX && N <= INT32_MAX && K <= INT32_MAX,
                 INTENT_ERR_INVALID_ARGUMENT, "bad extents");
  INTENT_REQUIRE(K % 128 == 0, INTENT_ERR_UNSUPPORTED, "K must be a multiple of 128, got %lld", (long long)K);
  if (M == 0 || N == 0) return INTENT_OK;
  if (K == 0) return intent::fill_launch(out, M, N, out_ld, 4, 0u, stream);  // no scale blocks: 0.0f
  INTENT_REQUIRE(a && b && a_scales && b_scales && out, INTENT_ERR_INVALID_ARGUMENT, "null pointer argument");
  INTENT_REQUIRE(a_ld >= K && b_ld >= K && a_scales_ld >= K / 32 && b_scales_ld >= K / 32 && out_ld >= N,
                 INTENT_ERR_INVALID_ARGUMENT, "leading stride smaller than the row");
  INTENT_REQUIRE(intent::aligned16(a) && intent::aligned16(b) && a_ld % 16 == 0 && b_ld % 16 == 0 &&
                     intent::aligned4(a_scales) && intent::aligned4(b_scales) && a_scales_ld % 4 == 0 &&
                     b_scales_ld % 4 == 0,
                 INTENT_ERR_ALIGNMENT, "operand rows 16-byte aligned, scale rows 4-byte aligned");
  INTENT_REQUIRE(intent::fits_offset(M, a_ld) && intent::fits_offset(N, b_ld) &&
                     intent::fits_offset(M, a_scales_ld) && intent::fits_offset(N, b_scales_ld),
                 INTENT_ERR_UNSUPPORTED, "mxfp8_gemm: operand too large for 31-bit buffer offsets");
  const int64_t big = ((M + 255) / 256) * ((N + 255) / 256);
  if (big >= 256) {
    const int mblocks = (int)((M + 255) / 256);
    const int nblocks = (int)((N + 255) / 256);
    INTENT_REQUIRE(big < (1ll << 31), INTENT_ERR_UNSUPPORTED, "mxfp8_gemm: grid too large");
    // One workgroup per CU: a last round of at most half the CUs is covered by
    // half-width tiles instead (whole trailing column blocks of 256).
    int split_cols = 0;
    const int cus = intent::cu_count();
    const int64_t tail = cus > 0 ? big % cus : 0;
    if (tail > 0 && 2 * tail <= cus && tail % mblocks == 0 && tail / mblocks < nblocks)
      split_cols = (int)(tail / mblocks);
    const int nbig = mblocks * (nblocks - split_cols);
    const int n_split = (nblocks - split_cols) * 256;
    const int64_t nsmall = split_cols ? (int64_t)mblocks * ((N - n_split + TMxHalf::BN - 1) / TMxHalf::BN) : 0;
    hipLaunchKernelGGL(mxfp8_gemm_dma_kernel, dim3((unsigned)(nbig + nsmall)), dim3(256), 0, (hipStream_t)stream, a,
                       a_ld, (int)M, a_scales, a_scales_ld, b, b_ld, (int)N, b_scales, b_scales_ld, (int)K, out, out_ld,
                       mblocks, nbig, n_split);
    return intent::launch_status("mxfp8_gemm");
  }
  return launch_mx<TMx128>(a, M, K, a_ld, a_scales, a_scales_ld, b, N, b_ld, b_scales, b_scales_ld, out, out_ld,
                           stream);
}

extern "C" int intent_fp8_transpose(const uint8_t* src, int64_t rows, int64_t cols, int64_t src_ld, uint8_t* dst,
                                    int64_t dst_ld, void* stream) {
  intent::clear_error();
  INTENT_REQUIRE(rows >= 0 && cols >= 0 && rows <= INT32_MAX && cols <= INT32_MAX, INTENT_ERR_INVALID_ARGUMENT,
                 "bad extents");
  if (rows == 0 || cols == 0) return INTENT_OK;
  INTENT_REQUIRE(src && dst, INTENT_ERR_INVALID_ARGUMENT, "null pointer argument");
  INTENT_REQUIRE(src_ld >= cols && dst_ld >= rows, INTENT_ERR_INVALID_ARGUMENT, "leading stride smaller than the row");
  const int64_t gx = (cols + 63) / 64, gy = (rows + 63) / 64;
  INTENT_REQUIRE(gx < (1ll << 31) && gy < 65536, INTENT_ERR_UNSUPPORTED, "fp8_transpose: grid too large");
  if (rows % 128 == 0 && cols % 128 == 0 && intent::aligned16(src) && intent::aligned16(dst) && src_ld % 16 == 0 &&
      dst_ld % 16 == 0) {
    hipLaunchKernelGGL(byte_transpose128_kernel, dim3((unsigned)(cols / 128), (unsigned)(rows / 128)), dim3(256), 0,
                       (hipStream_t)stream, src, src_ld, dst, dst_ld);
    return intent::launch_status("fp8_transpose");
  }
  hipLaunchKernelGGL(byte_transpose_kernel, dim3((unsigned)gx, (unsigned)gy), dim3(256), 0, (hipStream_t)stream, src,
                     (int)rows, (int)cols, src_ld, dst, dst_ld);
  return intent::launch_status("fp8_transpose");
}

// b: [N][K] rows (kn false, K contiguous) or the [K][N] matrix (kn true).
static int scaled_fp8_gemm(const uint8_t* a, int64_t M, int64_t K, int64_t a_ld, const uint8_t* b, int64_t N,
                           int64_t b_ld, bool kn, float a_scale, float b_scale, int64_t splits, int accumulate,
                           void* out, int64_t out_ld, void* stream) {
  intent::clear_error();
  INTENT_REQUIRE(M >= 0 && N >= 0 && K >= 0 && M <= INT32_MAX && N <= INT32_MAX && K <= INT32_MAX,
                 INTENT_ERR_INVALID_ARGUMENT, "bad extents");
  INTENT_REQUIRE(splits >= 1 && splits <= 64, INTENT_ERR_INVALID_ARGUMENT, "splits must be in [1, 64], got %lld",
                 (long long)splits);
  INTENT_REQUIRE(splits == 1 || accumulate, INTENT_ERR_INVALID_ARGUMENT, "split-K accumulates into the output");
  if (splits > 1)
    INTENT_REQUIRE(K % (256 * splits) == 0, INTENT_ERR_UNSUPPORTED, "K must be a multiple of 256 * splits, got %lld",
                   (long long)K);
  else
    INTENT_REQUIRE(K % 128 == 0, INTENT_ERR_UNSUPPORTED, "K must be a multiple of 128, got %lld", (long long)K);
  if (M == 0 || N == 0) return INTENT_OK;
  if (K == 0) {  // every split sums nothing: p = f16((0 * lhs_scale) * rhs_scale)
    INTENT_REQUIRE(out && out_ld >= N, INTENT_ERR_INVALID_ARGUMENT, "null output or short output stride");
    const dim3 grid((unsigned)((N + 255) / 256), (unsigned)(M < 65535 ? M : 65535));
    hipLaunchKernelGGL(fp8_scaled_empty_k_kernel, grid, dim3(256), 0, (hipStream_t)stream, (f16*)out, M, N, out_ld,
                       a_scale, b_scale, accumulate ? (int)splits : 0);
    return intent::launch_status("fp8_scaled_empty_k_kernel");
  }
  INTENT_REQUIRE(a && b && out, INTENT_ERR_INVALID_ARGUMENT, "null pointer argument");
  INTENT_REQUIRE(a_ld >= K && b_ld >= (kn ? N : K) && out_ld >= N, INTENT_ERR_INVALID_ARGUMENT,
                 "leading stride smaller than the row");
  INTENT_REQUIRE(intent::aligned16(a) && intent::aligned16(b) && a_ld % 16 == 0 && b_ld % 16 == 0,
                 INTENT_ERR_ALIGNMENT, "operand rows must be 16-byte aligned");
  if (kn) INTENT_REQUIRE(N % 16 == 0, INTENT_ERR_UNSUPPORTED, "[K, N] operand: N must be a multiple of 16");
  INTENT_REQUIRE(intent::fits_offset(M, a_ld) && intent::fits_offset(kn ? K : N, b_ld), INTENT_ERR_UNSUPPORTED,
                 "scaled_fp8_gemm: operand too large for 31-bit buffer offsets");
  const int mblocks = (int)((M + TSk::BM - 1) / TSk::BM);
  const int64_t grid = (int64_t)mblocks * ((N + TSk::BN - 1) / TSk::BN);
  INTENT_REQUIRE(grid < (1ll << 31), INTENT_ERR_UNSUPPORTED, "scaled_fp8_gemm: grid too large");
  if (kn) {  // producer waves transpose [K][N] on its way to LDS
    hipLaunchKernelGGL(accumulate ? fp8_scaled_ws_kernel<true> : fp8_scaled_ws_kernel<false>, dim3((unsigned)grid),
                       dim3(TSk::NT_WS), 0, (hipStream_t)stream, a, a_ld, (int)M, b, b_ld, (int)N, (int)K,
                       (int)splits, a_scale, b_scale, (f16*)out, out_ld, mblocks);
    return intent::launch_status("scaled_fp8_gemm");
  }
  auto kernel = accumulate ? fp8_scaled_gemm_kernel<true> : fp8_scaled_gemm_kernel<false>;
  hipLaunchKernelGGL(kernel, dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream, a, a_ld, (int)M, b, b_ld,
                     (int)N, (int)K, (int)splits, a_scale, b_scale, (f16*)out, out_ld, mblocks);
  return intent::launch_status("scaled_fp8_gemm");
}

extern "C" int intent_scaled_fp8_gemm(const uint8_t* a, int64_t M, int64_t K, int64_t a_ld, const uint8_t* bt,
                                      int64_t N, int64_t bt_ld, float a_scale, float b_scale, int64_t splits,
                                      int accumulate, void* out, int64_t out_ld, void* stream) {
  return scaled_fp8_gemm(a, M, K, a_ld, bt, N, bt_ld, false, a_scale, b_scale, splits, accumulate, out, out_ld,
                         stream);
}

extern "C" int intent_scaled_fp8_gemm_kn(const uint8_t* a, int64_t M, int64_t K, int64_t a_ld, const uint8_t* b,
                                         int64_t N, int64_t b_ld, float a_scale, float b_scale, int64_t splits,
                                         int accumulate, void* out, int64_t out_ld, void* stream) {
  return scaled_fp8_gemm(a, M, K, a_ld, b, N, b_ld, true, a_scale, b_scale, splits, accumulate, out, out_ld, stream);
}

extern "C" int intent_i8_gemm_i32_kn(const int8_t* a, int64_t M, int64_t K, int64_t a_ld, const int8_t* b,
                                     int64_t N, int64_t b_ld, const int32_t* bias, int32_t* c, int64_t c_ld,
                                     void* stream) {
  intent::clear_error();
  INTENT_REQUIRE(M >= 0 && N >= 0 && K >= 0 && M <= INT32_MAX && N <= INT32_MAX && K <= INT32_MAX,
                 INTENT_ERR_INVALID_ARGUMENT, "bad extents");
  INTENT_REQUIRE(K > 0 && K % 128 == 0, INTENT_ERR_UNSUPPORTED, "K must be a positive multiple of 128, got %lld",
                 (long long)K);
  INTENT_REQUIRE(N % 16 == 0, INTENT_ERR_UNSUPPORTED, "[K, N] operand: N must be a multiple of 16");
  if (M == 0 || N == 0) return INTENT_OK;
  INTENT_REQUIRE(a && b && c, INTENT_ERR_INVALID_ARGUMENT, "null pointer argument");
  INTENT_REQUIRE(a_ld >= K && b_ld >= N && c_ld >= N, INTENT_ERR_INVALID_ARGUMENT,
                 "leading stride smaller than the row");
  INTENT_REQUIRE(intent::aligned16(a) && intent::aligned16(b) && a_ld % 16 == 0 && b_ld % 16 == 0,
                 INTENT_ERR_ALIGNMENT, "operand rows must be 16-byte aligned");
  INTENT_REQUIRE(intent::fits_offset(M, a_ld) && intent::fits_offset(K, b_ld), INTENT_ERR_UNSUPPORTED,
                 "i8_gemm_i32_kn: operand too large for 31-bit buffer offsets");
  const int mblocks = (int)((M + TSk::BM - 1) / TSk::BM);
  const int64_t grid = (int64_t)mblocks * ((N + TSk::BN - 1) / TSk::BN);
  INTENT_REQUIRE(grid < (1ll << 31), INTENT_ERR_UNSUPPORTED, "i8_gemm_i32_kn: grid too large");
  hipLaunchKernelGGL(i8_gemm_kn_kernel, dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream, (const uint8_t*)a,
                     a_ld, (int)M, (const uint8_t*)b, b_ld, (int)N, (int)K, bias, c, c_ld, mblocks);
  return intent::launch_status("i8_gemm_i32_kn");
}

extern "C" int intent_deepgemm_fp8(const uint8_t* a, int64_t M, int64_t K, int64_t a_ld, const float* a_scales,
                                   int64_t a_scales_ld, const uint8_t* b, int64_t N, int64_t b_ld,
                                   const float* b_scales, int64_t b_scales_ld, void* out, int64_t out_ld,
                                   void* stream) {
  intent::clear_error();
  INTENT_REQUIRE(M >= 0 && N >= 0 && K >= 0 && M <= INT32_MAX && N <= INT32_MAX && K <= INT32_MAX,
                 INTENT_ERR_INVALID_ARGUMENT, "bad extents");
  INTENT_REQUIRE(K % 128 == 0, INTENT_ERR_UNSUPPORTED, "K must be a multiple of 128, got %lld", (long long)K);
  if (M == 0 || N == 0) return INTENT_OK;
  if (K == 0) return intent::fill_launch(out, M, N, out_ld, 2, 0u, stream);  // no K blocks: bf16(0)
  INTENT_REQUIRE(a && b && a_scales && b_scales && out, INTENT_ERR_INVALID_ARGUMENT, "null pointer argument");
  INTENT_REQUIRE(a_ld >= K && b_ld >= K && a_scales_ld >= K / 128 && b_scales_ld >= K / 128 && out_ld >= N,
                 INTENT_ERR_INVALID_ARGUMENT, "leading stride smaller than the row");
  INTENT_REQUIRE(intent::aligned16(a) && intent::aligned16(b) && a_ld % 16 == 0 && b_ld % 16 == 0 &&
                     intent::aligned4(a_scales) && intent::aligned4(b_scales),
                 INTENT_ERR_ALIGNMENT, "operand rows 16-byte aligned, scales 4-byte aligned");
  INTENT_REQUIRE(intent::fits_offset(M, a_ld) && intent::fits_offset(N, b_ld) &&
                     intent::fits_offset(M, a_scales_ld * 4) && intent::fits_offset(N / 128 + 1, b_scales_ld * 4),
                 INTENT_ERR_UNSUPPORTED, "deepgemm_fp8: operand too large for 31-bit buffer offsets");
  const int mblocks = (int)((M + TDg::BM - 1) / TDg::BM);
  const int64_t grid = (int64_t)mblocks * ((N + TDg::BN - 1) / TDg::BN);
  INTENT_REQUIRE(grid < (1ll << 31), INTENT_ERR_UNSUPPORTED, "deepgemm_fp8: grid too large");
  hipLaunchKernelGGL(deepgemm_fp8_kernel, dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream, a, a_ld, (int)M,
                     a_scales, a_scales_ld, b, b_ld, (int)N, b_scales, b_scales_ld, (int)K, (uint16_t*)out, out_ld,
                     mblocks);
  return intent::launch_status("deepgemm_fp8");
}

extern "C" int intent_fp8_gemm(const uint8_t* a, int64_t M, int64_t K, int64_t a_ld, const uint8_t* bt, int64_t N,
                               int64_t bt_ld, int format, uint8_t* out, int64_t out_ld, void* stream) {
  intent::clear_error();
  INTENT_REQUIRE(M >= 0 && N >= 0 && K >= 0 && M <= INT32_MAX && N <= INT32_MAX && K <= INT32_MAX,
                 INTENT_ERR_INVALID_ARGUMENT, "bad extents");
  INTENT_REQUIRE(format == 0 || format == 1, INTENT_ERR_INVALID_ARGUMENT, "format must be 0 (E4M3FN) or 1 (E5M2)");
  INTENT_REQUIRE(K % 128 == 0, INTENT_ERR_UNSUPPORTED, "K must be a multiple of 128, got %lld", (long long)K);
  if (M == 0 || N == 0) return INTENT_OK;
  if (K == 0) return intent::fill_launch(out, M, N, out_ld, 1, 0u, stream);  // the FP8 code of +0
  INTENT_REQUIRE(a && bt && out, INTENT_ERR_INVALID_ARGUMENT, "null pointer argument");
  INTENT_REQUIRE(a_ld >= K && bt_ld >= K && out_ld >= N, INTENT_ERR_INVALID_ARGUMENT,
                 "leading stride smaller than the row");
  INTENT_REQUIRE(intent::aligned16(a) && intent::aligned16(bt) && a_ld % 16 == 0 && bt_ld % 16 == 0,
                 INTENT_ERR_ALIGNMENT, "operand rows must be 16-byte aligned");
  INTENT_REQUIRE(intent::fits_offset(M, a_ld) && intent::fits_offset(N, bt_ld), INTENT_ERR_UNSUPPORTED,
                 "fp8_gemm: operand too large for 31-bit buffer offsets");
  const int mblocks = (int)((M + 255) / 256);
  const int64_t grid = (int64_t)mblocks * ((N + 255) / 256);
  INTENT_REQUIRE(grid < (1ll << 31), INTENT_ERR_UNSUPPORTED, "fp8_gemm: grid too large");
  if (format == 0)
    hipLaunchKernelGGL(fp8_gemm_kernel<0>, dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream, a, a_ld, (int)M,
                       bt, bt_ld, (int)N, (int)K, out, out_ld, mblocks);
  else
    hipLaunchKernelGGL(fp8_gemm_kernel<1>, dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream, a, a_ld, (int)M,
                       bt, bt_ld, (int)N, (int)K, out, out_ld, mblocks);
  return intent::launch_status("fp8_gemm");
}
