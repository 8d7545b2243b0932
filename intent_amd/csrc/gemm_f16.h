// LDS-tiled f16 MFMA GEMM with in-LDS weight dequantization (gfx950).
//
//   C[p, c] = sum_k A[p, k] * B[c, k]      (fp32 accumulation)
//
// A rows come from a RowSource (dense rows, MoE token gather, or padded MoE
// rows); B rows are quantized weight rows decoded by a WeightSource while being
// staged into LDS, so the MFMA loop only ever sees f16 tiles. An Epilogue
// consumes the fp32 accumulators.
//
// Tile: BM x BN = 128 x 128, BK = 64, 256 threads = 4 waves in a 2 x 2 grid,
// each wave 64 x 64 = 2 x 2 tiles of v_mfma_f32_32x32x16_f16.
// Pipeline: global loads of k-tile t+1 are issued into registers before the
// MFMAs of tile t, then decoded and written to LDS after the barrier.
#pragma once

#include "common.h"

namespace gemm {

constexpr int BM = 128;
constexpr int BN = 128;
constexpr int BK = 64;
constexpr int NTHREADS = 256;
constexpr int LDS_LD = BK + 8;  // halfs per LDS row: 144 B breaks bank aliasing of the 32-row fragment reads

struct SharedTile {
  f16 a[BM][LDS_LD];
  f16 b[BN][LDS_LD];
};

// ---- A row sources ------------------------------------------------------
// row(p) returns the f16 row pointer of tile row p or nullptr for a zero row.

struct DenseRows {
  const f16* x;
  int64_t ld;
  int M;
  INTENT_DEVICE const f16* row(int p) const { return p < M ? x + (int64_t)p * ld : nullptr; }
};

// MoE gate/up: padded row p holds route sorted[p]; token = route / top_k.
struct GatherRows {
  const f16* x;
  int64_t ld;
  const int32_t* sorted;
  int R;
  int top_k;
  INTENT_DEVICE const f16* row(int p) const {
    const int r = sorted[p];
    return (r >= 0 && r < R) ? x + (int64_t)(r / top_k) * ld : nullptr;
  }
};

// MoE down: padded activation rows are stored contiguously.
struct PaddedRows {
  const f16* x;
  int64_t ld;
  INTENT_DEVICE const f16* row(int p) const { return x + (int64_t)p * ld; }
};

// ---- Weight sources -----------------------------------------------------
// Each thread stages a fixed set of weight rows; RowMap maps a B-tile row
// (0..BN-1) to a weight row index. load() fetches k-tile kt into registers,
// store() decodes it into LDS row(s).

// W4 asymmetric group quant; a thread owns one weight row and one half
// (32 nibbles) of the 64-k tile.
struct W4Source {
  const uint8_t* q;
  int64_t ldq;  // bytes per row
  const f16* s;
  const uint8_t* z;
  int64_t ldp;  // scales/zeros per row
  int gs;

  struct Regs {
    u32x4 w;
    f16 s;
    uint8_t z;
  };
  struct Slot {
    const uint8_t* q;
    const f16* s;
    const uint8_t* z;
    int lds_row;
    int half;
  };
  static constexpr int kSlots = 1;

  template <class RowMap>
  INTENT_DEVICE void slot(int tid, const RowMap& rowmap, Slot* out) const {
    const int lrow = tid >> 1;
    const int half = tid & 1;
    const int wrow = rowmap(lrow);
    out[0].q = q + (int64_t)wrow * ldq + half * 16;
    out[0].s = s + (int64_t)wrow * ldp;
    out[0].z = z + (int64_t)wrow * ldp;
    out[0].lds_row = lrow;
    out[0].half = half;
  }
  INTENT_DEVICE void load(const Slot* sl, int kt, Regs* r) const {
    const int g = (kt * BK + sl[0].half * 32) / gs;
    r[0].w = load16(sl[0].q + (int64_t)kt * (BK / 2));
    r[0].s = sl[0].s[g];
    r[0].z = sl[0].z[g];
  }
  INTENT_DEVICE void store(const Slot* sl, const Regs* r, SharedTile& t) const {
    const f16x2 zoff = splat2((f16)(float)(1024 + r[0].z));
    const f16x2 sc = splat2(r[0].s);
    f16* dst = &t.b[sl[0].lds_row][sl[0].half * 32];
#pragma unroll
    for (int i = 0; i < 4; ++i) *reinterpret_cast<f16x8*>(dst + 8 * i) = dequant8(r[0].w[i], zoff, sc);
  }
};

// W8 per-channel: int8 rows converted exactly to f16 (the channel scale is
// applied in the epilogue). A thread owns two 16-byte chunks.
struct W8Source {
  const int8_t* q;
  int64_t ldq;

  struct Regs {
    u32x4 w;
  };
  struct Slot {
    const int8_t* q;
    int lds_row;
    int quarter;
  };
  static constexpr int kSlots = 2;

  template <class RowMap>
  INTENT_DEVICE void slot(int tid, const RowMap& rowmap, Slot* out) const {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int c = tid + i * NTHREADS;
      const int lrow = c >> 2;
      const int quarter = c & 3;
      out[i].q = q + (int64_t)rowmap(lrow) * ldq + quarter * 16;
      out[i].lds_row = lrow;
      out[i].quarter = quarter;
    }
  }
  INTENT_DEVICE void load(const Slot* sl, int kt, Regs* r) const {
#pragma unroll
    for (int i = 0; i < 2; ++i) r[i].w = load16(sl[i].q + (int64_t)kt * BK);
  }
  INTENT_DEVICE void store(const Slot* sl, const Regs* r, SharedTile& t) const {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      f16* dst = &t.b[sl[i].lds_row][sl[i].quarter * 16];
      *reinterpret_cast<f16x8*>(dst) = int8x8_to_f16(r[i].w[0], r[i].w[1]);
      *reinterpret_cast<f16x8*>(dst + 8) = int8x8_to_f16(r[i].w[2], r[i].w[3]);
    }
  }
};

// ---- Main loop ------------------------------------------------------------
// acc[i][j]: wave tile rows wm*64 + i*32, cols wn*64 + j*32; 32x32 layout:
// lane l holds column l%32, rows (v/4)*8 + (l/32)*4 + v%4 for v = 0..15.

template <class Rows, class WSrc, class RowMap>
INTENT_DEVICE void mainloop(const Rows& rows, int m0, const WSrc& wsrc, const RowMap& rowmap, int K, SharedTile& t,
                            f32x16 (&acc)[2][2]) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave & 1;
  const int wn = wave >> 1;

  // A staging: thread owns rows tid/8 + 32*i, column chunk (tid%8)*8.
  const f16* arow[4];
  const int acol = (tid & 7) * 8;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const f16* p = rows.row(m0 + (tid >> 3) + 32 * i);
    arow[i] = p ? p + acol : nullptr;
  }
  typename WSrc::Slot slots[WSrc::kSlots];
  wsrc.slot(tid, rowmap, slots);

#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  const int nk = K / BK;
  u32x4 areg[4];
  typename WSrc::Regs wreg[WSrc::kSlots];
#pragma unroll
  for (int i = 0; i < 4; ++i) areg[i] = arow[i] ? load16(arow[i]) : u32x4{0, 0, 0, 0};
  wsrc.load(slots, 0, wreg);

  for (int kt = 0; kt < nk; ++kt) {
#pragma unroll
    for (int i = 0; i < 4; ++i) *reinterpret_cast<u32x4*>(&t.a[(tid >> 3) + 32 * i][acol]) = areg[i];
    wsrc.store(slots, wreg, t);
    __syncthreads();
    if (kt + 1 < nk) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        areg[i] = arow[i] ? load16(arow[i] + (int64_t)(kt + 1) * BK) : u32x4{0, 0, 0, 0};
      wsrc.load(slots, kt + 1, wreg);
    }
#pragma unroll
    for (int kk = 0; kk < BK / 16; ++kk) {
      f16x8 af[2], bf[2];
      const int kof = kk * 16 + (lane >> 5) * 8;
#pragma unroll
      for (int i = 0; i < 2; ++i) af[i] = *reinterpret_cast<const f16x8*>(&t.a[wm * 64 + i * 32 + (lane & 31)][kof]);
#pragma unroll
      for (int j = 0; j < 2; ++j) bf[j] = *reinterpret_cast<const f16x8*>(&t.b[wn * 64 + j * 32 + (lane & 31)][kof]);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
    }
    __syncthreads();
  }
}

// Tile-local coordinates of accumulator element v of acc[i][j].
INTENT_DEVICE int acc_row(int i, int v) {
  const int lane = threadIdx.x & 63;
  const int wm = (threadIdx.x >> 6) & 1;
  return wm * 64 + i * 32 + (v >> 2) * 8 + (lane >> 5) * 4 + (v & 3);
}
INTENT_DEVICE int acc_col(int j) {
  const int lane = threadIdx.x & 63;
  const int wn = threadIdx.x >> 7;
  return wn * 64 + j * 32 + (lane & 31);
}

}  // namespace gemm
