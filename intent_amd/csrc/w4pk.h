// W4 GEMM core with the weights kept packed in LDS (gfx950).
//
//   acc[m, n] = sum_k A[m, k] * deq(W)[n, k],   deq(W) = (q - z) * s per group
//
// Every wave is a consumer. A stage is 64 k: A rows (f16, 128 bytes each) and
// packed weight rows (32 bytes each) are copied global -> LDS by DMA
// (buffer_load ... lds), NB - 1 stages ahead through a ring of NB stage
// buffers, so no operand passes through VGPRs on its way to LDS and the LDS
// holds 4-bit weights (a quarter of their f16 size). Each wave reads its
// weight fragments as packed dwords and decodes them in registers right
// before the MFMA; the decode of one fragment is amortised over the wave's
// TI = 4 row blocks (128 rows of A), which keeps VALU time near half of the
// MFMA time.
//
// k order inside a stage. v_mfma_f32_32x32x16_f16 step kk (0..3) takes, in
// lane half h = lane / 32, 8 consecutive k of row lane % 32 from each operand.
// Here half h of step kk holds k-chunk 4h + kk (8 k per chunk), so over the
// four steps a lane walks 32 contiguous k: one 16-byte read covers its
// packed weights for the whole stage. A and B agree on the assignment, so the
// sum is unchanged.
//
// LDS layout of a stage: A rows as in mfma_pipe.h (chunk c of row r in slot
// c ^ swz(r)); then weight rows of 32 bytes, half h of row r in slot
// h ^ ((r >> 3) & 1), which keeps sixteen lanes reading sixteen rows
// conflict-free.
#pragma once

#include <type_traits>

#include "mfma_pipe.h"

namespace mp {

INTENT_DEVICE constexpr int bswz(int row) { return (row >> 3) & 1; }

// f(std::integral_constant<int, S>) for S = B .. E-1.
template <int B, int E, class F>
INTENT_DEVICE void static_for(F&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    static_for<B + 1, E>(f);
  }
}

// Packed 4-bit weight rows by DMA. One instruction moves 32 rows x 32 bytes;
// lane i fills slot i % 2 of row i / 2. Instructions are spread over the NW
// waves; a wave with no instruction left repeats the last one (same data,
// same place), so every wave issues N_INST.
template <int ROWS, int NW>
struct PackedRowsDma {
  static constexpr int TOTAL = ROWS / 32;
  static constexpr int N_INST = (TOTAL + NW - 1) / NW;
  static constexpr int NVM = N_INST;
  static_assert(TOTAL * 32 == ROWS, "weight tile rows must be a multiple of 32");
  Rsrc rq;
  uint32_t voff[N_INST];
  int lds_row0[N_INST];
  // wrow(c): weight row of tile row c (relative to q); ldq bytes per packed row.
  template <class RowMap>
  INTENT_DEVICE void init(const uint8_t* q, int64_t ldq, const RowMap& wrow, int wave) {
    rq = make_rsrc(q);
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int j = 0; j < N_INST; ++j) {
      const int t = j * NW + wave < TOTAL ? j * NW + wave : TOTAL - 1;
      const int r0 = t * 32;
      const int r = r0 + (lane >> 1);
      const int h = (lane & 1) ^ bswz(r);
      voff[j] = (uint32_t)((int64_t)wrow(r) * ldq + h * 16);
      lds_row0[j] = r0;
    }
  }
  INTENT_DEVICE void issue(char* lds_b, int kt) const {
#pragma unroll
    for (int j = 0; j < N_INST; ++j)
      lds_dma<16, true>(rq, (lds_t*)(lds_b + lds_row0[j] * 32), voff[j], (uint32_t)kt * 32);
  }
};

// Group scales (f16) and zero points (u8), also by DMA: per stage and tile
// row one dword of each, the aligned dword that holds the row's entry for the
// stage's first group (and for gs == 32 the second one too, which sits in
// the same dword). Lane i of instruction t fills dword i of rows 64t..64t+63.
// Requires 4-byte aligned rows of scales and zeros (checked by the caller).
template <int ROWS, int NW>
struct GroupParamsDma {
  static constexpr bool kWindowed = false;
  static constexpr int TOTAL = ROWS / 64;
  static_assert(ROWS % 64 == 0, "weight tile rows must be a multiple of 64");
  static constexpr int N_INST = (TOTAL + NW - 1) / NW;  // per array
  static constexpr int NVM = 2 * N_INST;
  static constexpr int BYTES = 8 * ROWS;  // scale dwords, then zero dwords
  Rsrc rs, rz;
  uint32_t soff[N_INST], zoff[N_INST];
  int row0[N_INST];
  int gs;
  template <class RowMap>
  INTENT_DEVICE void init(const f16* s, const uint8_t* z, int64_t ldp, int gsize, const RowMap& wrow, int wave) {
    rs = make_rsrc(s);
    rz = make_rsrc(z);
    gs = gsize;
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int j = 0; j < N_INST; ++j) {
      const int t = j * NW + wave < TOTAL ? j * NW + wave : TOTAL - 1;
      row0[j] = t * 64;
      const int r = t * 64 + lane;
      const int64_t w = wrow(r);
      soff[j] = (uint32_t)(w * ldp * 2);
      zoff[j] = (uint32_t)(w * ldp);
    }
  }
  // First group of stage kt.
  INTENT_DEVICE int group(int kt) const { return gs == 32 ? 2 * kt : (kt * 64) / gs; }
  INTENT_DEVICE void issue(char* lds_p, int kt) const {
    const uint32_t g = (uint32_t)group(kt);
#pragma unroll
    for (int j = 0; j < N_INST; ++j) {
      lds_dma<4, true>(rs, (lds_t*)(lds_p + row0[j] * 4), soff[j], (2 * g) & ~3u);
      lds_dma<4, true>(rz, (lds_t*)(lds_p + 4 * ROWS + row0[j] * 4), zoff[j], g & ~3u);
    }
  }
};

// Group scales and zero points of a window of four groups, for group sizes
// that are multiples of 64 (a window then spans gs / 16 >= 4 stages). A
// window is loaded once into one of two LDS buffers outside the stage ring:
// per tile row the two scale dwords (8 bytes) and the zero dword (4 bytes)
// of groups 4w .. 4w + 3. The per-stage form above touches one cache line
// per row and array in every stage; this one does so once per window.
// Scale instruction t: lane i fills dword i % 2 of row 32t + i / 2; zero
// instruction t: lane i fills row 64t + i. Requires ldp % 4 == 0, 4-byte
// aligned rows, and K ranges that start on a window (checked by the caller).
template <int ROWS, int NW>
struct GroupWindowDma {
  static constexpr bool kWindowed = true;
  static_assert(ROWS % 64 == 0, "weight tile rows must be a multiple of 64");
  static constexpr int S_TOTAL = ROWS / 32;
  static constexpr int Z_TOTAL = ROWS / 64;
  static constexpr int S_INST = (S_TOTAL + NW - 1) / NW;
  static constexpr int Z_INST = (Z_TOTAL + NW - 1) / NW;
  static constexpr int NVM = S_INST + Z_INST;
  static constexpr int BYTES = 12 * ROWS;  // scale dword pairs, then zero dwords
  Rsrc rs, rz;
  uint32_t soff[S_INST], zoff[Z_INST];
  int srow0[S_INST], zrow0[Z_INST];
  int spg;  // stages per group: gs / 64
  template <class RowMap>
  INTENT_DEVICE void init(const f16* s, const uint8_t* z, int64_t ldp, int gsize, const RowMap& wrow, int wave) {
    rs = make_rsrc(s);
    rz = make_rsrc(z);
    spg = gsize / 64;
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int j = 0; j < S_INST; ++j) {
      const int t = j * NW + wave < S_TOTAL ? j * NW + wave : S_TOTAL - 1;
      srow0[j] = t * 32;
      soff[j] = (uint32_t)(wrow(t * 32 + (lane >> 1)) * ldp * 2 + (lane & 1) * 4);
    }
#pragma unroll
    for (int j = 0; j < Z_INST; ++j) {
      const int t = j * NW + wave < Z_TOTAL ? j * NW + wave : Z_TOTAL - 1;
      zrow0[j] = t * 64;
      zoff[j] = (uint32_t)(wrow(t * 64 + lane) * ldp);
    }
  }
  INTENT_DEVICE void issue(char* lds_p, int w) const {
#pragma unroll
    for (int j = 0; j < S_INST; ++j)
      lds_dma<4, true>(rs, (lds_t*)(lds_p + srow0[j] * 8), soff[j], (uint32_t)w * 8);
#pragma unroll
    for (int j = 0; j < Z_INST; ++j)
      lds_dma<4, true>(rz, (lds_t*)(lds_p + 8 * ROWS + zrow0[j] * 4), zoff[j], (uint32_t)w * 4);
  }
};

// Per-stage register state: the stage's packed weight fragments with their
// group parameters, and the A fragments and decoded weights of step 0.
template <class T>
struct StagePk {
  u32x4 bq[T::TJ];
  f16x2 zo[T::TJ], sc[T::TJ];
  f16x8 af[T::TI], bf[T::TJ];
};

// Reads of a stage that the first MFMA needs. sshift / zshift select the
// lane's scale half and zero byte inside the staged dwords.
// ps / pz: the lane's scale and zero dwords for accumulator column block 0;
// for block j they sit j * SJ and j * 128 bytes further.
template <class T, int TA, int SJ>
INTENT_DEVICE void stage_prologue(const char* buf, const uint32_t (&aaddr)[4], uint32_t baddr, const char* ps,
                                  const char* pz, int sshift, int zshift, StagePk<T>& st) {
  const char* a = buf;
  const char* b = buf + T::A_BYTES;
#pragma unroll
  for (int j = 0; j < T::TJ; ++j) {
    st.bq[j] = *reinterpret_cast<const u32x4*>(b + baddr + j * 32 * 32);
    const uint32_t sw = *reinterpret_cast<const uint32_t*>(ps + j * SJ);
    const uint32_t zw = *reinterpret_cast<const uint32_t*>(pz + j * 32 * 4);
    st.zo[j] = splat2((f16)(float)(1024 + ((zw >> zshift) & 0xFFu)));
    st.sc[j] = splat2(bit_cast<f16>((uint16_t)(sw >> sshift)));
  }
#pragma unroll
  for (int i = 0; i < TA; ++i) st.af[i] = *reinterpret_cast<const f16x8*>(a + aaddr[0] + i * 32 * ROWB);
#pragma unroll
  for (int j = 0; j < T::TJ; ++j) st.bf[j] = dequant8(st.bq[j][0], st.zo[j], st.sc[j]);
}

// The four MFMA steps of a stage; the A reads and weight decodes of step
// kk + 1 are interleaved with the MFMAs of step kk. With five row blocks
// (kSingleA) each row block's A fragment is reread right after its last MFMA
// of the step, into the same registers: double-buffering all of them would
// need 20 more VGPRs than the 256 that two workgroups per CU allow.
template <class T, int TA>
INTENT_DEVICE void stage_body(const char* buf, const uint32_t (&aaddr)[4], const StagePk<T>& st,
                              f32x16 (&acc)[T::TI][T::TJ]) {
  constexpr bool kSingleA = T::TI >= 5;
  constexpr int NAB = kSingleA ? 1 : 2;
  const char* a = buf;
  f16x8 af[NAB][T::TI], bf[2][T::TJ];
#pragma unroll
  for (int i = 0; i < TA; ++i) af[0][i] = st.af[i];
#pragma unroll
  for (int j = 0; j < T::TJ; ++j) bf[0][j] = st.bf[j];
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) {
    const int cb = kk & 1;
    const int ca = kSingleA ? 0 : cb;
    if (kk + 1 < 4) {
      if constexpr (!kSingleA) {
#pragma unroll
        for (int i = 0; i < TA; ++i)
          af[ca ^ 1][i] = *reinterpret_cast<const f16x8*>(a + aaddr[kk + 1] + i * 32 * ROWB);
      }
#pragma unroll
      for (int j = 0; j < T::TJ; ++j) bf[cb ^ 1][j] = dequant8(st.bq[j][kk + 1], st.zo[j], st.sc[j]);
    }
#pragma unroll
    for (int i = 0; i < TA; ++i) {
#pragma unroll
      for (int j = 0; j < T::TJ; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(bf[cb][j], af[ca][i], acc[i][j], 0, 0, 0);
      if constexpr (kSingleA)
        if (kk + 1 < 4) af[0][i] = *reinterpret_cast<const f16x8*>(a + aaddr[kk + 1] + i * 32 * ROWB);
    }
  }
  // Schedule (masks: 0x008 MFMA, 0x002 VALU, 0x100 DS read): per step one
  // MFMA followed by its share of the next step's reads and decode VALU
  // (kSingleA: a row block's read after its last MFMA).
  constexpr int NM = TA * T::TJ;
  constexpr int VALU_STEP = T::TJ * 17;  // decode of one step (dequant8)
  static_for<0, 4>([&](auto KK) {
    constexpr int kk = decltype(KK)::value;
    static_for<0, NM>([&](auto X) {
      constexpr int x = decltype(X)::value;
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      if constexpr (kk < 3) {
        constexpr bool rd = kSingleA ? x % T::TJ == T::TJ - 1 : x < TA;
        if constexpr (rd) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        constexpr int v = (x + 1) * VALU_STEP / NM - x * VALU_STEP / NM;
        if constexpr (v > 0) __builtin_amdgcn_sched_group_barrier(0x002, v, 0);
      }
    });
  });
}

// Main loop. bufs: NB distinct stage buffers of stage_bytes_pk<T>() bytes.
// All NB buffers are filled before the loop. Step kt runs the MFMAs of stage
// kt; then, while the last of them are still executing, the wave waits for
// its own DMA of stage kt + 1 (vmcnt counts in issue order and every step
// issues exactly one group), meets the other waves at the barrier (stage
// kt + 1 complete everywhere, stage kt no longer read), refills stage kt's
// buffer with stage kt + NB (indices past the end clamp to the last stage:
// same data into a buffer nobody reads again) and reads the first fragments
// of stage kt + 1. Only DMA is in flight across steps, so the compiler's own
// wait-count pass has nothing to wait for.
template <class T, bool kWindowed = false>
constexpr int stage_bytes_pk() {
  return T::A_BYTES + T::BN * 32 + (kWindowed ? 0 : GroupParamsDma<T::BN, T::NW>::BYTES);
}

// TA <= T::TI: only the first TA 32-row blocks of the tile are computed (the
// others are padding); their accumulators stay zero.
//
// With a windowed PDma (GroupWindowDma), pwin holds two window buffers of
// PDma::BYTES. Windows 0 and 1 are loaded before the loop; the step whose
// next stage opens window w loads window w + 1 into the buffer window w - 1
// used, right after that step's stage group. Such a load sits between stage
// groups in the vmcnt order, so the wait of each of the next NB - 1 steps
// (whose target stage group was issued before it) allows its NVM
// instructions on top of NB - 2 stage groups; a window is read
// at least three steps after its load was issued (a window spans >= 4
// stages), by which time the stage group issued after it has been waited for.
template <class T, int NB, class ADma, class BDma, class PDma, int TA = T::TI>
INTENT_DEVICE void mainloop_pk(const ADma& aop, const BDma& bop, const PDma& pop, int nk, char* const (&bufs)[NB],
                               f32x16 (&acc)[T::TI][T::TJ], char* pwin = nullptr) {
  static_assert(NB >= 2 && NB <= 8, "stage ring");
  constexpr bool kWin = PDma::kWindowed;
  constexpr int NV = ADma::NVM + BDma::NVM + (kWin ? 0 : PDma::NVM);
  constexpr int NVP = kWin ? PDma::NVM : 0;
  static_assert(NB * NV + NVP < 64, "vmcnt range");
#pragma unroll
  for (int i = 0; i < T::TI; ++i)
#pragma unroll
    for (int j = 0; j < T::TJ; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0;
  if (nk <= 0) return;

  const int lane = threadIdx.x & 63;
  const int h = lane >> 5;
  uint32_t aaddr[4];
  {
    const int r = T::wave_m() * T::WTM + (lane & 31);
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) aaddr[kk] = (uint32_t)(r * ROWB + (((4 * h + kk) ^ swz(r)) << 4));
  }
  const int brow = T::wave_n() * T::WTN + (lane & 31);
  const uint32_t baddr = (uint32_t)(brow * 32 + ((h ^ bswz(brow)) << 4));

  auto issue = [&](auto J, int kt) {
    constexpr int j = decltype(J)::value;
    const int st = kt < nk ? kt : nk - 1;
    aop.issue(bufs[j], st);
    bop.issue(bufs[j] + T::A_BYTES, st);
    if constexpr (!kWin) pop.issue(bufs[j] + T::A_BYTES + T::BN * 32, st);
  };
  // Windowed: group pg and stage psg inside it of the next stage read.
  int pg = 0, psg = 0, nwin = 0, pmask = 0;
  if constexpr (kWin) nwin = (nk / pop.spg + 3) >> 2;
  // Per-stage params: the lane's group is g0 + h for gs == 32, else g0; its
  // scale is half (group & 1) of the dword at 2*(g0 & ~1), its zero byte
  // (group & 3). Windowed: group gi = pg & 3 of the window, scale dword
  // gi / 2, half gi & 1, zero byte gi.
  auto prologue = [&](auto J, int kt, StagePk<T>& st) {
    constexpr int j = decltype(J)::value;
    if constexpr (kWin) {
      const int gi = pg & 3;
      const char* pw = pwin + ((pg >> 2) & 1) * PDma::BYTES;
      stage_prologue<T, TA, 32 * 8>(bufs[j], aaddr, baddr, pw + brow * 8 + (gi >> 1) * 4, pw + 8 * T::BN + brow * 4,
                                    (gi & 1) * 16, gi * 8, st);
      if (++psg == pop.spg) {
        psg = 0;
        ++pg;
      }
    } else {
      const int g0 = pop.group(kt);
      const int g = pop.gs == 32 ? g0 + h : g0;
      const char* p = bufs[j] + T::A_BYTES + T::BN * 32 + brow * 4;
      stage_prologue<T, TA, 32 * 4>(bufs[j], aaddr, baddr, p, p + 4 * T::BN, (g & 1) * 16, (g & 3) * 8, st);
    }
  };
  if constexpr (kWin) {
    pop.issue(pwin, 0);
    if (nwin > 1) pop.issue(pwin + PDma::BYTES, 1);
  }
  static_for<0, NB>([&](auto S) { issue(S, decltype(S)::value); });
  StagePk<T> st;
  wait_vm_lgkm_barrier<(NB - 1) * NV>();
  prologue(std::integral_constant<int, 0>{}, 0, st);

  auto step = [&](auto J, int kt) {
    constexpr int j = decltype(J)::value;
    stage_body<T, TA>(bufs[j], aaddr, st, acc);
    if (kt + 1 < nk) {
      if constexpr (kWin) {
        if (pmask)
          wait_vm_lgkm_barrier<(NB - 2) * NV + NVP>();
        else
          wait_vm_lgkm_barrier<(NB - 2) * NV>();
      } else {
        wait_vm_lgkm_barrier<(NB - 2) * NV>();
      }
      issue(J, kt + NB);
      if constexpr (kWin) {
        pmask = (pmask << 1) & ((1 << (NB - 1)) - 1);  // loads issued in the last NB - 1 steps
        const int w1 = (pg >> 2) + 1;
        if ((pg & 3) == 0 && psg == 0 && w1 < nwin) {
          pop.issue(pwin + (w1 & 1) * PDma::BYTES, w1);
          pmask |= 1;
        }
      }
      prologue(std::integral_constant<int, (j + 1) % NB>{}, kt + 1, st);
    }
  };
  for (int kt = 0; kt < nk; kt += NB) {
    static_for<0, NB>([&](auto S) {
      if (kt + decltype(S)::value < nk) step(S, kt + decltype(S)::value);
    });
  }
  wait_vm<0>();  // no DMA may land in LDS that an epilogue reuses
}

}  // namespace mp
