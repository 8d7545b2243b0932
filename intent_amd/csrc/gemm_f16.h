// LDS-tiled f16 MFMA GEMM with in-LDS weight dequantization (gfx950).
//
//   C[p, c] = sum_k A[p, k] * B[c, k]      (fp32 accumulation)
//
// A rows come from a RowSource (dense rows, MoE token gather, or padded MoE
// rows); B rows are quantized weight rows decoded by a WeightSource while being
// staged into LDS, so the MFMA loop only ever sees f16 tiles. An epilogue
// consumes the fp32 accumulators.
//
// A Tile<BM, BN, WM, WN> is BM x BN outputs computed by WM x WN waves; each
// wave owns a (BM/WM) x (BN/WN) block of 32 x 32 v_mfma_f32_32x32x16_f16 tiles.
// BK = 64 k per LDS stage. LDS traffic per MFMA falls with the wave block:
// a 64 x 64 wave block reads 1 KB of fragments per MFMA, 128 x 64 reads 0.75 KB.
// Pipeline: global loads of k-tile t+1 are issued into registers before the
// MFMAs of tile t, then decoded and written to LDS after the barrier; the
// fragments of 16-k step kk+1 are read before the MFMAs of step kk.
#pragma once

#include "common.h"

namespace gemm {

constexpr int BK = 64;
constexpr int LDS_LD = BK + 8;  // halfs per LDS row: 144 B breaks bank aliasing of the 32-row fragment reads

template <int BM_, int BN_, int WM_, int WN_>
struct Tile {
  static constexpr int BM = BM_;
  static constexpr int BN = BN_;
  static constexpr int WM = WM_;
  static constexpr int WN = WN_;
  static constexpr int NT = WM * WN * 64;
  static constexpr int TI = BM / WM / 32;  // 32-row MFMA tiles per wave
  static constexpr int TJ = BN / WN / 32;  // 32-col MFMA tiles per wave
  static_assert(TI >= 1 && TJ >= 1 && TI * WM * 32 == BM && TJ * WN * 32 == BN, "tile shape");
  static_assert((BM * 8) % NT == 0, "A staging chunks must divide evenly");

  struct Shared {
    f16 a[BM][LDS_LD];
    f16 b[BN][LDS_LD];
  };

  INTENT_DEVICE static int wave_m() { return (threadIdx.x >> 6) % WM; }
  INTENT_DEVICE static int wave_n() { return (threadIdx.x >> 6) / WM; }
  // Tile-local coordinates of accumulator element v of acc[i][j]; 32x32 layout:
  // lane l holds column l%32, rows (v/4)*8 + (l/32)*4 + v%4 for v = 0..15.
  INTENT_DEVICE static int acc_row(int i, int v) {
    const int lane = threadIdx.x & 63;
    return wave_m() * (BM / WM) + i * 32 + (v >> 2) * 8 + (lane >> 5) * 4 + (v & 3);
  }
  INTENT_DEVICE static int acc_col(int j) {
    const int lane = threadIdx.x & 63;
    return wave_n() * (BN / WN) + j * 32 + (lane & 31);
  }
};

// ---- buffer addressing ----------------------------------------------------
// Operands are read with buffer loads: a per-workgroup resource (base
// pointer), a per-thread 32-bit byte offset fixed for the whole K loop and a
// scalar byte offset that advances with k, so the loop spends no vector
// instructions on addresses. Hosts check that every offset fits 31 bits.

using Rsrc = __amdgpu_buffer_rsrc_t;
INTENT_DEVICE Rsrc make_rsrc(const void* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, 0x7fffffff, 0x00020000);
}
INTENT_DEVICE u32x4 bload16(Rsrc r, uint32_t voff, uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
}

// ---- A row sources ------------------------------------------------------
// base(m0) is the tile's base pointer; off(p) the element offset of tile row
// p from it. Rows that hold no data (past M, MoE padding) map to some valid
// row: loads stay unpredicated and the epilogue never stores those rows.

struct DenseRows {
  const f16* x;
  int64_t ld;
  int M;
  INTENT_DEVICE const f16* base(int m0) const { return x + (int64_t)m0 * ld; }
  INTENT_DEVICE int off(int m0, int p) const { return (int)((p < M ? p - m0 : M - 1 - m0) * ld); }
};

// MoE gate/up: padded row p holds route sorted[p]; token = route / top_k.
struct GatherRows {
  const f16* x;
  int64_t ld;
  const int32_t* sorted;
  int R;
  int top_k;
  INTENT_DEVICE const f16* base(int) const { return x; }
  INTENT_DEVICE int off(int, int p) const {
    const int r = sorted[p];
    return (int)(((r >= 0 && r < R) ? r / top_k : 0) * ld);
  }
};

// MoE down: padded activation rows are stored contiguously.
struct PaddedRows {
  const f16* x;
  int64_t ld;
  INTENT_DEVICE const f16* base(int m0) const { return x + (int64_t)m0 * ld; }
  INTENT_DEVICE int off(int m0, int p) const { return (int)((p - m0) * ld); }
};

// ---- Weight sources -----------------------------------------------------
// Each thread stages a fixed set of 16-byte weight chunks; RowMap maps a
// B-tile row (0..BN-1) to a weight row index. load() fetches k-tile kt into
// registers, store() decodes it into LDS.

// W4 asymmetric group quant: a chunk is one half (32 nibbles) of a row's
// 64-k tile. The group size is 32 or a multiple of 64, so the group of a
// chunk is 2*kt + half or kt*64/gs: a scalar term plus a per-slot constant.
struct W4Source {
  const uint8_t* q;
  int64_t ldq;  // bytes per row
  const f16* s;
  const uint8_t* z;
  int64_t ldp;  // scales/zeros per row
  int gs;

  struct Regs {
    u32x4 w;
    uint16_t s;
    uint8_t z;
  };
  struct Slot {
    uint32_t q;  // byte offsets
    uint32_t s;
    uint32_t z;
    int lds_row;
    int half;
  };
  template <class T>
  static constexpr int slots() {
    static_assert((T::BN * 2) % T::NT == 0, "W4 staging chunks must divide evenly");
    return T::BN * 2 / T::NT;
  }

  template <class T, class RowMap>
  INTENT_DEVICE void slot(int tid, const RowMap& rowmap, Slot* out) const {
#pragma unroll
    for (int i = 0; i < slots<T>(); ++i) {
      const int c = tid + i * T::NT;
      const int lrow = c >> 1;
      const int half = c & 1;
      const int wrow = rowmap(lrow);
      const int extra = gs == 32 ? half : 0;
      out[i].q = (uint32_t)(wrow * ldq + half * 16);
      out[i].s = (uint32_t)((wrow * ldp + extra) * 2);
      out[i].z = (uint32_t)(wrow * ldp + extra);
      out[i].lds_row = lrow;
      out[i].half = half;
    }
  }
  struct Rsrcs {
    Rsrc q, s, z;
  };
  INTENT_DEVICE Rsrcs rsrcs() const { return {make_rsrc(q), make_rsrc(s), make_rsrc(z)}; }
  template <class T>
  INTENT_DEVICE void load(const Rsrcs& rs, const Slot* sl, int kt, Regs* r) const {
    const uint32_t g = gs == 32 ? 2 * kt : (kt * BK) / gs;
#pragma unroll
    for (int i = 0; i < slots<T>(); ++i) {
      r[i].w = bload16(rs.q, sl[i].q, (uint32_t)kt * (BK / 2));
      r[i].s = __builtin_amdgcn_raw_buffer_load_b16(rs.s, sl[i].s, g * 2, 0);
      r[i].z = __builtin_amdgcn_raw_buffer_load_b8(rs.z, sl[i].z, g, 0);
    }
  }
  template <class T>
  INTENT_DEVICE void store(const Slot* sl, const Regs* r, typename T::Shared& t) const {
#pragma unroll
    for (int i = 0; i < slots<T>(); ++i) {
      const f16x2 zoff = splat2((f16)(float)(1024 + r[i].z));
      const f16x2 sc = splat2(bit_cast<f16>(r[i].s));
      f16* dst = &t.b[sl[i].lds_row][sl[i].half * 32];
#pragma unroll
      for (int c = 0; c < 4; ++c) *reinterpret_cast<f16x8*>(dst + 8 * c) = dequant8(r[i].w[c], zoff, sc);
    }
  }
};

// W8 per-channel: int8 rows converted exactly to f16 (the channel scale is
// applied in the epilogue). A chunk is a quarter (16 bytes) of a row's 64-k tile.
struct W8Source {
  const int8_t* q;
  int64_t ldq;

  struct Regs {
    u32x4 w;
  };
  struct Slot {
    uint32_t q;
    int lds_row;
    int quarter;
  };
  template <class T>
  static constexpr int slots() {
    static_assert((T::BN * 4) % T::NT == 0, "W8 staging chunks must divide evenly");
    return T::BN * 4 / T::NT;
  }

  template <class T, class RowMap>
  INTENT_DEVICE void slot(int tid, const RowMap& rowmap, Slot* out) const {
#pragma unroll
    for (int i = 0; i < slots<T>(); ++i) {
      const int c = tid + i * T::NT;
      const int lrow = c >> 2;
      const int quarter = c & 3;
      out[i].q = (uint32_t)(rowmap(lrow) * ldq + quarter * 16);
      out[i].lds_row = lrow;
      out[i].quarter = quarter;
    }
  }
  struct Rsrcs {
    Rsrc q;
  };
  INTENT_DEVICE Rsrcs rsrcs() const { return {make_rsrc(q)}; }
  template <class T>
  INTENT_DEVICE void load(const Rsrcs& rs, const Slot* sl, int kt, Regs* r) const {
#pragma unroll
    for (int i = 0; i < slots<T>(); ++i) r[i].w = bload16(rs.q, sl[i].q, (uint32_t)kt * BK);
  }
  template <class T>
  INTENT_DEVICE void store(const Slot* sl, const Regs* r, typename T::Shared& t) const {
#pragma unroll
    for (int i = 0; i < slots<T>(); ++i) {
      f16* dst = &t.b[sl[i].lds_row][sl[i].quarter * 16];
      *reinterpret_cast<f16x8*>(dst) = int8x8_to_f16(r[i].w[0], r[i].w[1]);
      *reinterpret_cast<f16x8*>(dst + 8) = int8x8_to_f16(r[i].w[2], r[i].w[3]);
    }
  }
};

// ---- Main loop ------------------------------------------------------------
// acc[i][j]: wave block rows wave_m*(BM/WM) + i*32, cols wave_n*(BN/WN) + j*32.

template <class T, class Rows, class WSrc, class RowMap>
INTENT_DEVICE void mainloop(const Rows& rows, int m0, const WSrc& wsrc, const RowMap& rowmap, int K,
                            typename T::Shared& t, f32x16 (&acc)[T::TI][T::TJ]) {
  constexpr int NA = T::BM * 8 / T::NT;  // 16-byte A chunks per thread
  constexpr int NW = WSrc::template slots<T>();
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wm = T::wave_m();
  const int wn = T::wave_n();

  // A staging: chunk c = tid + NT*i covers row c/8, halfs (c%8)*8.
  const Rsrc ars = make_rsrc(rows.base(m0));
  uint32_t aoff[NA];
  int a_r[NA];
  const int acol = (tid & 7) * 8;
#pragma unroll
  for (int i = 0; i < NA; ++i) {
    a_r[i] = (tid + T::NT * i) >> 3;
    aoff[i] = (uint32_t)(rows.off(m0, m0 + a_r[i]) + acol) * 2;
  }
  typename WSrc::Slot slots[NW];
  wsrc.template slot<T>(tid, rowmap, slots);
  const typename WSrc::Rsrcs wrs = wsrc.rsrcs();

#pragma unroll
  for (int i = 0; i < T::TI; ++i)
#pragma unroll
    for (int j = 0; j < T::TJ; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  const int nk = K / BK;
  u32x4 areg[NA];
  typename WSrc::Regs wreg[NW];
#pragma unroll
  for (int i = 0; i < NA; ++i) areg[i] = bload16(ars, aoff[i], 0);
  wsrc.template load<T>(wrs, slots, 0, wreg);

  for (int kt = 0; kt < nk; ++kt) {
#pragma unroll
    for (int i = 0; i < NA; ++i) *reinterpret_cast<u32x4*>(&t.a[a_r[i]][acol]) = areg[i];
    wsrc.template store<T>(slots, wreg, t);
    __syncthreads();
    if (kt + 1 < nk) {
#pragma unroll
      for (int i = 0; i < NA; ++i) areg[i] = bload16(ars, aoff[i], (uint32_t)(kt + 1) * BK * 2);
      wsrc.template load<T>(wrs, slots, kt + 1, wreg);
    }
    // Fragments of 16-k step kk+1 are read before the MFMAs of step kk.
    f16x8 af[2][T::TI], bf[2][T::TJ];
    const int arow0 = wm * (T::BM / T::WM) + (lane & 31);
    const int brow0 = wn * (T::BN / T::WN) + (lane & 31);
    const int khalf = (lane >> 5) * 8;
#pragma unroll
    for (int i = 0; i < T::TI; ++i) af[0][i] = *reinterpret_cast<const f16x8*>(&t.a[arow0 + i * 32][khalf]);
#pragma unroll
    for (int j = 0; j < T::TJ; ++j) bf[0][j] = *reinterpret_cast<const f16x8*>(&t.b[brow0 + j * 32][khalf]);
#pragma unroll
    for (int kk = 0; kk < BK / 16; ++kk) {
      const int cb = kk & 1;
      if (kk + 1 < BK / 16) {
        const int kof = (kk + 1) * 16 + khalf;
#pragma unroll
        for (int i = 0; i < T::TI; ++i) af[cb ^ 1][i] = *reinterpret_cast<const f16x8*>(&t.a[arow0 + i * 32][kof]);
#pragma unroll
        for (int j = 0; j < T::TJ; ++j) bf[cb ^ 1][j] = *reinterpret_cast<const f16x8*>(&t.b[brow0 + j * 32][kof]);
      }
#pragma unroll
      for (int i = 0; i < T::TI; ++i)
#pragma unroll
        for (int j = 0; j < T::TJ; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[cb][i], bf[cb][j], acc[i][j], 0, 0, 0);
    }
    __syncthreads();
  }
}

}  // namespace gemm
