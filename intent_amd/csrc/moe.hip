// Quantized MoE on gfx950: router top-k, deterministic alignment, grouped W4
// gate/up (+SiLU) and down projections, fixed-order weighted combine.
#include <math.h>

#include "common.h"
#include "internal.h"
#include "mfma_pipe.h"
#include "w4pk.h"

#include <type_traits>

namespace {

constexpr int kMaxTopK = 8;
constexpr int kMaxRouteExperts = 256;
constexpr int kAlignThreads = 1024;
constexpr int kAlignWaves = kAlignThreads / 64;
constexpr int kMaxAlignExperts = 2048;  // LDS: (3E + 1 + 16E) ints

// ---- router ---------------------------------------------------------------
// One wave per token; lane L holds the logits of experts 4L .. 4L+3. Every
// selection reproduces the sequential scan "best = first untaken expert, then
// any later one strictly greater replaces it": a NaN wins only as the first
// untaken expert, otherwise the largest non-NaN logit wins and ties keep the
// lower index (softmax is monotonic, so raw logits are compared). A run of
// consecutive experts is summarised by its first untaken candidate and its
// best non-NaN one, and two adjacent runs merge exactly, so a butterfly over
// the lanes gives the scan's answer. The max for the softmax is the same
// selection over all experts; the softmax denominator is a lane-tree sum.
struct RouteSel {
  float fv;  // first untaken candidate of the run (fi < 0: none)
  int fi;
  float mv;  // best non-NaN candidate of the run (mi < 0: none)
  int mi;
};

INTENT_DEVICE RouteSel route_merge(const RouteSel& a, const RouteSel& b) {  // run a precedes run b
  RouteSel r;
  r.fv = a.fi >= 0 ? a.fv : b.fv;
  r.fi = a.fi >= 0 ? a.fi : b.fi;
  const bool take_b = a.mi < 0 || (b.mi >= 0 && b.mv > a.mv);
  r.mv = take_b ? b.mv : a.mv;
  r.mi = take_b ? b.mi : a.mi;
  return r;
}

// Selection over the untaken experts of the wave (bit i of `taken`: expert 4L + i).
INTENT_DEVICE int route_select(const float (&v)[4], int e0, int E, uint32_t taken, float& value) {
  RouteSel s{0.f, -1, 0.f, -1};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int e = e0 + i;
    if (e < E && !(taken & (1u << i))) {
      const RouteSel one{v[i], e, v[i], v[i] == v[i] ? e : -1};
      s = route_merge(s, one);
    }
  }
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    RouteSel o;
    o.fv = __shfl_xor(s.fv, d);
    o.fi = __shfl_xor(s.fi, d);
    o.mv = __shfl_xor(s.mv, d);
    o.mi = __shfl_xor(s.mi, d);
    s = (lane & d) ? route_merge(o, s) : route_merge(s, o);
  }
  const bool first_nan = s.fi >= 0 && !(s.fv == s.fv);
  value = first_nan ? s.fv : s.mv;
  return first_nan ? s.fi : s.mi;
}

__global__ __launch_bounds__(256) void moe_route_kernel(const float* __restrict__ logits, int T, int E, int top_k,
                                                        int renorm, int32_t* __restrict__ ids,
                                                        float* __restrict__ weights) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;  // whole waves
  const float* l = logits + (int64_t)t * E;
  const int e0 = 4 * lane;
  float v[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] = e0 + i < E ? l[e0 + i] : 0.f;
  float mx;
  route_select(v, e0, E, 0u, mx);
  float part = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    if (e0 + i < E) part += expf(v[i] - mx);
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) part += __shfl_xor(part, d);
  const float sum = part;
  uint32_t taken = 0;
  float p[kMaxTopK];
  float psum = 0.f;
#pragma unroll
  for (int j = 0; j < kMaxTopK; ++j) {  // unrolled: p stays in registers
    if (j >= top_k) break;
    float bv;
    const int best = route_select(v, e0, E, taken, bv);
    if ((best >> 2) == lane) taken |= 1u << (best & 3);
    p[j] = expf(bv - mx) / sum;
    psum += p[j];
    if (lane == 0) ids[(int64_t)t * top_k + j] = best;
  }
  if (lane == 0) {
#pragma unroll
    for (int j = 0; j < kMaxTopK; ++j)
      if (j < top_k) weights[(int64_t)t * top_k + j] = renorm ? p[j] / psum : p[j];
  }
}

// Any E above the wave kernel's 256: one thread per token runs the scan itself
// (the chosen experts, at most kMaxTopK, kept in registers).
__global__ __launch_bounds__(256) void moe_route_seq_kernel(const float* __restrict__ logits, int T, int E, int top_k,
                                                            int renorm, int32_t* __restrict__ ids,
                                                            float* __restrict__ weights) {
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= T) return;
  const float* l = logits + (int64_t)t * E;
  float mx = l[0];
  for (int e = 1; e < E; ++e) mx = l[e] > mx ? l[e] : mx;
  float sum = 0.f;
  for (int e = 0; e < E; ++e) sum += expf(l[e] - mx);
  int chosen[kMaxTopK];
  float p[kMaxTopK];
  float psum = 0.f;
#pragma unroll
  for (int j = 0; j < kMaxTopK; ++j) {
    chosen[j] = -1;
    p[j] = 0.f;
  }
#pragma unroll
  for (int j = 0; j < kMaxTopK; ++j) {
    if (j >= top_k) break;
    int best = -1;
    float bv = 0.f;
    for (int e = 0; e < E; ++e) {
      bool taken = false;
#pragma unroll
      for (int i = 0; i < kMaxTopK; ++i) taken |= chosen[i] == e;
      if (taken) continue;
      if (best < 0 || l[e] > bv) {
        best = e;
        bv = l[e];
      }
    }
    chosen[j] = best;
    ids[(int64_t)t * top_k + j] = best;
    p[j] = expf(bv - mx) / sum;
    psum += p[j];
  }
#pragma unroll
  for (int j = 0; j < kMaxTopK; ++j)
    if (j < top_k) weights[(int64_t)t * top_k + j] = renorm ? p[j] / psum : p[j];
}

// ---- alignment --------------------------------------------------------------
// One workgroup. Counts use LDS atomics (order-free). The scatter is stable:
// routes are processed in chunks of 1024 in route order; inside a wave the rank
// of a route among same-expert lanes comes from ballots, across waves from a
// prefix over per-wave counts, across chunks from a running base per expert.
// The result equals a stable argsort of the expert ids.
__global__ __launch_bounds__(kAlignThreads) void moe_align_kernel(const int32_t* __restrict__ ids, int R, int E, int B,
                                                                  int32_t* __restrict__ sorted, int capacity,
                                                                  int32_t* __restrict__ blocks, int nblocks,
                                                                  int32_t* __restrict__ offsets,
                                                                  int32_t* __restrict__ total) {
  // LDS sized by E at launch: counts, offsets (E + 1), bases, then the
  // per-wave counts of a chunk (kAlignWaves x E)
  extern __shared__ int align_lds[];
  int* cnt = align_lds;
  int* off = cnt + E;
  int* base = off + E + 1;
  int* wcnt_flat = base + E;
  auto wcnt = [&](int w, int e) -> int& { return wcnt_flat[w * E + e]; };
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;

  for (int e = tid; e < E; e += kAlignThreads) {
    cnt[e] = 0;
    base[e] = 0;
  }
  __syncthreads();
  for (int r = tid; r < R; r += kAlignThreads) {
    const int e = ids[r];
    if (e >= 0 && e < E) atomicAdd(&cnt[e], 1);
  }
  __syncthreads();
  if (tid == 0) {
    int acc = 0;
    off[0] = 0;
    for (int e = 0; e < E; ++e) {
      acc += (cnt[e] + B - 1) / B * B;
      off[e + 1] = acc;
    }
    total[0] = acc;
  }
  __syncthreads();
  for (int e = tid; e <= E; e += kAlignThreads) offsets[e] = off[e];
  for (int i = tid; i < capacity; i += kAlignThreads) sorted[i] = R;
  for (int b = tid; b < nblocks; b += kAlignThreads) {
    const int pos = b * B;
    int owner = -1;
    if (pos < off[E]) {
      int lo = 0, hi = E;  // largest e with off[e] <= pos
      while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (off[mid] <= pos) lo = mid; else hi = mid;
      }
      owner = lo;
    }
    blocks[b] = owner;
  }
  __syncthreads();  // sentinel fill is complete before any scatter store

  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  for (int c = 0; c < R; c += kAlignThreads) {
    for (int i = tid; i < kAlignWaves * E; i += kAlignThreads) wcnt(i / E, i % E) = 0;
    const int r = c + tid;
    int e = r < R ? ids[r] : -1;
    const bool valid = e >= 0 && e < E;
    if (!valid) e = -1;
    __syncthreads();
    int rank = 0;
    uint64_t remaining = __ballot(valid);
    while (remaining) {
      const int leader = __ffsll((unsigned long long)remaining) - 1;
      const int le = __shfl(e, leader);
      const uint64_t same = __ballot(e == le) & remaining;
      if (e == le) rank = __popcll(same & lt_mask);
      if (lane == leader) wcnt(wave, le) = __popcll(same);
      remaining &= ~same;
    }
    __syncthreads();
    for (int x = tid; x < E; x += kAlignThreads) {
      int run = base[x];
      for (int w = 0; w < kAlignWaves; ++w) {
        const int n = wcnt(w, x);
        wcnt(w, x) = run;
        run += n;
      }
      base[x] = run;
    }
    __syncthreads();
    if (valid) sorted[off[e] + wcnt(wave, e) + rank] = r;
    __syncthreads();
  }
}

// ---- grouped projections ------------------------------------------------------
// Tile GEMMs on the pipelined core (mfma_pipe.h) over 128- or 64-row blocks
// of the aligned route order; the block's expert comes from the block map
// and selects the weight base pointers. Token rows reach LDS by DMA through
// the route ids; weights go through VGPRs with the W4 decode.

// XCD-aware tile order. Workgroup b runs on XCD b % 8, and each XCD takes
// the column tiles [x * ct / 8, (x + 1) * ct / 8) of every row block, row
// block outer: the workgroups an XCD runs back to back share their token
// rows in its L2 instead of re-reading them from MALL for every column tile,
// and no weight tile is read by two XCDs. Plain order when ct % 8 != 0.
INTENT_DEVICE void moe_tile_order(int bid, int mblocks, int ctiles, int& mb, int& ct) {
  if ((ctiles & 7) != 0) {
    mb = bid % mblocks;
    ct = bid / mblocks;
    return;
  }
  const int per = ctiles >> 3;
  const int local = bid >> 3;
  mb = local / per;
  ct = (bid & 7) * per + local % per;
}

// Tiles per alignment block size B: gate/up covers 256 weight rows (128
// features, gate and up), down 128 output columns. Producer/consumer
// workgroups (mainloop_ws): 4 consumer waves + 4 producer waves.
template <int B>
struct MoeTiles;
template <>
struct MoeTiles<128> {
  using GateUp = mp::Tile<128, 256, 2, 2>;  // consumers of 64 x 128
  using Down = mp::Tile<128, 128, 2, 2>;    // consumers of 64 x 64
};
template <>
struct MoeTiles<64> {
  using GateUp = mp::Tile<64, 256, 2, 2>;  // consumers of 32 x 128
  using Down = mp::Tile<64, 128, 2, 2>;    // consumers of 32 x 64
};

// B-tile row c of a gate/up tile. Wave column block w (BN/WN rows) holds
// WTN/2 gate rows then the WTN/2 up rows of the same features, so a lane's
// accumulators j and j + TJ/2 hold gate and up of one output element.
// Features past F read row F-1 and are never stored.
template <class T>
struct GateUpRowMap {
  int f0;
  int F;
  static constexpr int kHalf = T::WTN / 2;
  INTENT_DEVICE static int feature(int w, int u) { return w * kHalf + u; }
  INTENT_DEVICE int operator()(int c) const {
    const int w = c / T::WTN;
    const int u = c % T::WTN;
    int f = f0 + feature(w, u % kHalf);
    f = f < F ? f : F - 1;
    return u >= kHalf ? F + f : f;
  }
};

struct ClampRows {
  int n0;
  int N;
  INTENT_DEVICE int operator()(int c) const {
    const int n = n0 + c;
    return n < N ? n : N - 1;
  }
};

// acc[i][j][4g + c]: row(i), feature f0 + feature(wave_n, j*32 + g*8 + h*4 + c);
// j < TJ/2 are gate columns, j + TJ/2 the up columns of the same features.
// silu(g) * u = g / (1 + e^-g) * u with v_exp_f32 and v_rcp_f32 (about one
// ulp each, so a few f32 ulps in all, far below the f16 rounding of the
// result; g = -inf gives NaN and g = +inf gives inf, as the quotient does,
// and a large negative g gives -0).
INTENT_DEVICE float silu_mul(float g, float u) {
  const float e = __builtin_amdgcn_exp2f(g * -1.44269504088896341f);
  return g * __builtin_amdgcn_rcpf(1.0f + e) * u;
}

template <class T>
INTENT_DEVICE void store_gate_up(const f32x16 (&acc)[T::TI][T::TJ], int m0, int f0, int F,
                                 const int32_t* __restrict__ sorted, int R, f16* __restrict__ act, int64_t ld_act) {
  const bool vec = (ld_act & 3) == 0 && (F & 3) == 0;
#pragma unroll
  for (int i = 0; i < T::TI; ++i) {
    const int row = m0 + T::row(i);
    const int r = sorted[row];
    const bool valid = r >= 0 && r < R;
#pragma unroll
    for (int j = 0; j < T::TJ / 2; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int f = f0 + GateUpRowMap<T>::feature(T::wave_n(), T::col(j, g) - T::wave_n() * T::WTN);
        f16 o[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const float gt = acc[i][j][4 * g + c];
          const float up = acc[i][j + T::TJ / 2][4 * g + c];
          o[c] = valid ? (f16)silu_mul(gt, up) : (f16)0.f;
        }
        f16* dst = act + (int64_t)row * ld_act + f;
        if (vec && f + 3 < F) {
          f16x2 lo, hi;
          lo[0] = o[0];
          lo[1] = o[1];
          hi[0] = o[2];
          hi[1] = o[3];
          *reinterpret_cast<u32x2*>(dst) = u32x2{bit_cast<uint32_t>(lo), bit_cast<uint32_t>(hi)};
        } else {
#pragma unroll
          for (int c = 0; c < 4; ++c)
            if (f + c < F) dst[c] = o[c];
        }
      }
  }

}

// store_gate_up through LDS for the packed-weight tiles (one wave row, NW
// waves of WTN / 2 features each): the tile's BM rows x NW * WTN / 2 features
// are gathered in LDS (rows padded by 16 bytes, so the 8-byte writes of 16
// rows fall in distinct bank groups), then stored as 16-byte pieces of whole
// row segments. lds: BM * (NW * WTN + 16) bytes that no wave reads any more
// once the workgroup barrier inside has passed.
template <class T>
INTENT_DEVICE void store_gate_up_lds(const f32x16 (&acc)[T::TI][T::TJ], char* lds, int m0, int f0, int F,
                                     const int32_t* __restrict__ sorted, int R, f16* __restrict__ act,
                                     int64_t ld_act) {
  static_assert(T::WM == 1, "one wave row");
  constexpr int FW = T::WTN / 2;   // features per wave
  constexpr int FT = T::NW * FW;   // features per tile
  constexpr int RS = 2 * FT + 16;  // LDS row bytes
  constexpr int NP = T::BM * (FT / 8) / T::NT;  // 16-byte pieces per thread
  static_assert(NP * T::NT == T::BM * (FT / 8), "whole pieces per thread");
  const int lane = threadIdx.x & 63;
  const int w = T::wave_n();
  __syncthreads();  // every wave is done with the stage buffers
#pragma unroll
  for (int i = 0; i < T::TI; ++i) {
    const int row = T::row(i);
    const int r = sorted[m0 + row];
    const bool valid = r >= 0 && r < R;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      float o[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) o[c] = valid ? silu_mul(acc[i][0][4 * g + c], acc[i][T::TJ / 2][4 * g + c]) : 0.f;
      const f16x2 lo = __builtin_convertvector(f32x2{o[0], o[1]}, f16x2);
      const f16x2 hi = __builtin_convertvector(f32x2{o[2], o[3]}, f16x2);
      const int fl = w * FW + (T::col(0, g) - w * T::WTN);
      *reinterpret_cast<u32x2*>(lds + row * RS + fl * 2) = u32x2{bit_cast<uint32_t>(lo), bit_cast<uint32_t>(hi)};
    }
  }
  __syncthreads();
  const bool vec = (ld_act & 7) == 0 && (((uintptr_t)act) & 15) == 0;
#pragma unroll
  for (int q = 0; q < NP; ++q) {
    const int p = q * T::NT + (int)threadIdx.x;
    const int row = p / (FT / 8), c8 = (p % (FT / 8)) * 8;
    const u32x4 v = *reinterpret_cast<const u32x4*>(lds + row * RS + c8 * 2);
    const int f = f0 + c8;
    f16* dst = act + (int64_t)(m0 + row) * ld_act + f;
    if (vec && f + 7 < F) {
      *reinterpret_cast<u32x4*>(dst) = v;
    } else {
#pragma unroll
      for (int c = 0; c < 8; ++c)
        if (f + c < F) reinterpret_cast<uint16_t*>(dst)[c] = (uint16_t)(v[c >> 1] >> (16 * (c & 1)));
    }
  }
}

template <int B>
__global__ __launch_bounds__(MoeTiles<B>::GateUp::NT_WS, 1) void moe_gate_up_kernel(
    const f16* __restrict__ x, int64_t ldx, int H, const int32_t* __restrict__ sorted,
    const int32_t* __restrict__ blocks, int mblocks, int R, int top_k, const uint8_t* __restrict__ wq,
    const f16* __restrict__ ws, const uint8_t* __restrict__ wz, int F, int gs, f16* __restrict__ act,
    int64_t ld_act) {
  using T = typename MoeTiles<B>::GateUp;
  __shared__ __attribute__((aligned(16))) char buf0[T::STAGE_BYTES];
  __shared__ __attribute__((aligned(16))) char buf1[T::STAGE_BYTES];
  __shared__ __attribute__((aligned(16))) char buf2[T::STAGE_BYTES];
  char* const bufs[3] = {buf0, buf1, buf2};
  int mb, ct;
  moe_tile_order(blockIdx.x, mblocks, gridDim.x / mblocks, mb, ct);
  const int f0 = ct * (T::BN / 2);
  const int e = blocks[mb];
  if (e < 0) return;
  const int64_t ldq = H / 2;
  const int64_t ldp = H / gs;
  const int m0 = mb * B;
  mp::DmaRowsOperand<T::BM, mp::GatherRows, T::NW> aop;
  aop.init(mp::GatherRows{x, ldx * 2, sorted, R, top_k}, m0, T::wave() % T::NW);
  mp::W4Operand<T::BN, T::NT> bop;
  bop.init(wq + (int64_t)e * 2 * F * ldq, ldq, ws + (int64_t)e * 2 * F * ldp, wz + (int64_t)e * 2 * F * ldp, ldp, gs,
           GateUpRowMap<T>{f0, F});
  f32x16 acc[T::TI][T::TJ];
  if (!mp::mainloop_ws<T, mp::F16Math, 3>(aop, bop, H / 64, bufs, acc)) return;

  store_gate_up<T>(acc, m0, f0, F, sorted, R, act, ld_act);
}

// Gate/up on the packed-weight core (w4pk.h): 128-row blocks x 128 features
// (256 weight rows), four waves of 128 x 64 (32 gate + 32 up columns), each
// decoding its own weight fragments; a three-stage DMA ring (78 KB of LDS)
// leaves room for two workgroups per CU, whose independent barriers hide
// each other's stalls. Measured on config 4: 613 us with the producer/
// consumer kernel below, 618 us with this core at one 8-wave workgroup per
// CU, 519 us at two 4-wave workgroups per CU.
using GateUpPk = mp::Tile<128, 256, 1, 4>;
constexpr int kGateUpPkStages = 3;
// 160-row blocks (five row blocks per wave): an expert with 129..160 routes
// is one block, not a full block plus a light one that streams and decodes
// the expert's weights a second time. 160 x 128 B token rows make a 28 KB
// stage, so two workgroups per CU hold a ring of two stages (a two-stage ring
// measured the same as three on the 128-row tile); 15-17 VGPRs spill. Config
// 4 (experts of 112..143 routes): gate/up 348 -> 334 us, down 213 -> 207 us.
using Pk160 = mp::Tile<160, 256, 1, 4>;
constexpr int kPk160Stages = 2;

// Group parameters per stage (gs == 32) or per window of four groups.
template <bool kWin>
using PkParams = std::conditional_t<kWin, mp::GroupWindowDma<GateUpPk::BN, GateUpPk::NW>,
                                    mp::GroupParamsDma<GateUpPk::BN, GateUpPk::NW>>;

template <bool kWin, class T = GateUpPk, int NB = kGateUpPkStages>
__global__ __launch_bounds__(GateUpPk::NT, 2) void moe_gate_up_pk_kernel(
    const f16* __restrict__ x, int64_t ldx, int H, const int32_t* __restrict__ sorted,
    const int32_t* __restrict__ blocks, int mblocks, int R, int top_k, const uint8_t* __restrict__ wq,
    const f16* __restrict__ ws, const uint8_t* __restrict__ wz, int F, int gs, f16* __restrict__ act,
    int64_t ld_act) {
  __shared__ __attribute__((aligned(16))) char smem[NB][mp::stage_bytes_pk<T, kWin>()];
  __shared__ __attribute__((aligned(16))) char pwin[kWin ? 2 * PkParams<true>::BYTES : 16];
  char* bufs[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) bufs[b] = smem[b];
  int mb, ct;
  moe_tile_order(blockIdx.x, mblocks, gridDim.x / mblocks, mb, ct);
  const int f0 = ct * (T::BN / 2);
  const int e = blocks[mb];
  if (e < 0) return;
  const int64_t ldq = H / 2;
  const int64_t ldp = H / gs;
  const int m0 = mb * T::BM;
  const int wave = T::wave();
  const GateUpRowMap<T> rows{f0, F};
  mp::DmaRowsOperand<T::BM, mp::GatherRows, T::NW, true> aop;
  aop.init(mp::GatherRows{x, ldx * 2, sorted, R, top_k}, m0, wave);
  mp::PackedRowsDma<T::BN, T::NW> bop;
  bop.init(wq + (int64_t)e * 2 * F * ldq, ldq, rows, wave);
  PkParams<kWin> pop;
  pop.init(ws + (int64_t)e * 2 * F * ldp, wz + (int64_t)e * 2 * F * ldp, ldp, gs, rows, wave);
  f32x16 acc[T::TI][T::TJ];
  // An expert's padding rows (sentinel route R) sit at the end of its last
  // block: only the 32-row blocks holding a route are computed.
  int ta = 0;
#pragma unroll
  for (int i = 0; i < T::TI; ++i) ta += sorted[m0 + 32 * i] < R ? 1 : 0;
  ta = __builtin_amdgcn_readfirstlane(ta);
  using ADma = decltype(aop);
  using BDma = decltype(bop);
  using PDma = decltype(pop);
  if (ta <= 1)
    mp::mainloop_pk<T, NB, ADma, BDma, PDma, 1>(aop, bop, pop, H / 64, bufs, acc, pwin);
  else if (ta == 2)
    mp::mainloop_pk<T, NB, ADma, BDma, PDma, 2>(aop, bop, pop, H / 64, bufs, acc, pwin);
  else if (ta == 3)
    mp::mainloop_pk<T, NB, ADma, BDma, PDma, 3>(aop, bop, pop, H / 64, bufs, acc, pwin);
  else if (ta == 4 || T::TI == 4)
    mp::mainloop_pk<T, NB, ADma, BDma, PDma, 4>(aop, bop, pop, H / 64, bufs, acc, pwin);
  else
    mp::mainloop_pk<T, NB, ADma, BDma, PDma, T::TI>(aop, bop, pop, H / 64, bufs, acc, pwin);
  if constexpr (T::WM == 1 && T::BM * (T::NW * T::WTN + 16) <= (int)sizeof(smem)) {
    store_gate_up_lds<T>(acc, &smem[0][0], m0, f0, F, sorted, R, act, ld_act);
    return;
  }
  store_gate_up<T>(acc, m0, f0, F, sorted, R, act, ld_act);
}

// fp32 rows of the down projection scattered to their routes.
template <class T>
INTENT_DEVICE void store_down(const f32x16 (&acc)[T::TI][T::TJ], int m0, int n0, int H,
                              const int32_t* __restrict__ sorted, int R, float* __restrict__ out, int64_t ldo) {
  const bool vec = (ldo & 3) == 0 && (((uintptr_t)out) & 15) == 0;
#pragma unroll
  for (int i = 0; i < T::TI; ++i) {
    const int r = sorted[m0 + T::row(i)];
    if (r < 0 || r >= R) continue;
#pragma unroll
    for (int j = 0; j < T::TJ; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int col = n0 + T::col(j, g);
        float* dst = out + (int64_t)r * ldo + col;
        if (vec && col + 3 < H) {
          *reinterpret_cast<f32x4*>(dst) =
              f32x4{acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]};
        } else {
#pragma unroll
          for (int c = 0; c < 4; ++c)
            if (col + c < H) dst[c] = acc[i][j][4 * g + c];
        }
      }
  }

}

// Down projection: grid = mblocks x ntiles; fp32 rows scattered to routes.
template <int B>
__global__ __launch_bounds__(MoeTiles<B>::Down::NT_WS, 1) void moe_down_kernel(
    const f16* __restrict__ act, int64_t ld_act, const int32_t* __restrict__ sorted,
    const int32_t* __restrict__ blocks, int mblocks, int ntiles, int R, const uint8_t* __restrict__ wq,
    const f16* __restrict__ ws, const uint8_t* __restrict__ wz, int H, int F, int gs, float* __restrict__ out,
    int64_t ldo) {
  using T = typename MoeTiles<B>::Down;
  __shared__ __attribute__((aligned(16))) char buf0[T::STAGE_BYTES];
  __shared__ __attribute__((aligned(16))) char buf1[T::STAGE_BYTES];
  __shared__ __attribute__((aligned(16))) char buf2[T::STAGE_BYTES];
  char* const bufs[3] = {buf0, buf1, buf2};
  int mb, ct;
  moe_tile_order(blockIdx.x, mblocks, ntiles, mb, ct);
  const int n0 = ct * T::BN;
  const int e = blocks[mb];
  if (e < 0) return;
  const int64_t ldq = F / 2;
  const int64_t ldp = F / gs;
  const int m0 = mb * B;
  mp::DmaRowsOperand<T::BM, mp::DenseRows, T::NW> aop;
  aop.init(mp::DenseRows{act, ld_act * 2, m0 + T::BM}, m0, T::wave() % T::NW);
  mp::W4Operand<T::BN, T::NT> bop;
  bop.init(wq + (int64_t)e * H * ldq, ldq, ws + (int64_t)e * H * ldp, wz + (int64_t)e * H * ldp, ldp, gs,
           ClampRows{n0, H});
  f32x16 acc[T::TI][T::TJ];
  if (!mp::mainloop_ws<T, mp::F16Math, 3>(aop, bop, F / 64, bufs, acc)) return;
  store_down<T>(acc, m0, n0, H, sorted, R, out, ldo);
}

// Down projection on the packed-weight core (the gate/up tile: 128-row blocks
// x 256 output columns, four waves decoding their own weight fragments, two
// workgroups per CU). K (= F) is split into `splits` equal parts, each a
// multiple of four quantisation groups (so a part starts on a group dword),
// and part p writes its f32 partial sums to out + p * part_stride; the
// combine adds the parts in order. Measured on config 4: 328 us for the
// producer/consumer kernel below, which runs 384 workgroups of 128 x 128 with
// the decode in separate waves.
template <bool kWin, class T = GateUpPk, int NB = kGateUpPkStages>
__global__ __launch_bounds__(GateUpPk::NT, 2) void moe_down_pk_kernel(
    const f16* __restrict__ act, int64_t ld_act, const int32_t* __restrict__ sorted,
    const int32_t* __restrict__ blocks, int mblocks, int ntiles, int R, const uint8_t* __restrict__ wq,
    const f16* __restrict__ ws, const uint8_t* __restrict__ wz, int H, int F, int gs, int splits,
    float* __restrict__ out, int64_t ldo, int64_t part_stride) {
  __shared__ __attribute__((aligned(16))) char smem[NB][mp::stage_bytes_pk<T, kWin>()];
  __shared__ __attribute__((aligned(16))) char pwin[kWin ? 2 * PkParams<true>::BYTES : 16];
  char* bufs[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) bufs[b] = smem[b];
  // XCD-owned (row block, K part) pairs: workgroup b runs on XCD b % 8, and
  // an XCD runs every column tile of the pairs it owns (pair p = mb * splits
  // + part goes to XCD p % 8), so each pair's activation rows are fetched
  // into one L2 once, and each weight tile is still read by one workgroup.
  // (Spreading every pair's column tiles over all eight XCDs fetched the
  // activation rows, the larger operand of a down tile, eight times.)
  const int xcd = blockIdx.x & 7, local = blockIdx.x >> 3;
  const int pidx = xcd + 8 * (local / ntiles);
  if (pidx >= mblocks * splits) return;
  const int ct = local % ntiles;
  const int mb = pidx / splits, part = pidx % splits;
  const int n0 = ct * T::BN;
  const int e = blocks[mb];
  if (e < 0) return;
  const int kpart = F / splits;
  const int k0 = part * kpart;
  const int64_t ldq = F / 2;
  const int64_t ldp = F / gs;
  const int m0 = mb * T::BM;
  const int wave = T::wave();
  const ClampRows rows{n0, H};
  mp::DmaRowsOperand<T::BM, mp::LinearRows, T::NW, true> aop;
  aop.init(mp::LinearRows{act + k0, ld_act * 2}, m0, wave);
  mp::PackedRowsDma<T::BN, T::NW> bop;
  bop.init(wq + (int64_t)e * H * ldq + k0 / 2, ldq, rows, wave);
  PkParams<kWin> pop;
  pop.init(ws + (int64_t)e * H * ldp + k0 / gs, wz + (int64_t)e * H * ldp + k0 / gs, ldp, gs, rows, wave);
  f32x16 acc[T::TI][T::TJ];
  int ta = 0;
#pragma unroll
  for (int i = 0; i < T::TI; ++i) ta += sorted[m0 + 32 * i] < R ? 1 : 0;
  ta = __builtin_amdgcn_readfirstlane(ta);
  using ADma = decltype(aop);
  using BDma = decltype(bop);
  using PDma = decltype(pop);
  const int nk = kpart / 64;
  if (ta <= 1)
    mp::mainloop_pk<T, NB, ADma, BDma, PDma, 1>(aop, bop, pop, nk, bufs, acc, pwin);
  else if (ta == 2)
    mp::mainloop_pk<T, NB, ADma, BDma, PDma, 2>(aop, bop, pop, nk, bufs, acc, pwin);
  else if (ta == 3)
    mp::mainloop_pk<T, NB, ADma, BDma, PDma, 3>(aop, bop, pop, nk, bufs, acc, pwin);
  else if (ta == 4 || T::TI == 4)
    mp::mainloop_pk<T, NB, ADma, BDma, PDma, 4>(aop, bop, pop, nk, bufs, acc, pwin);
  else
    mp::mainloop_pk<T, NB, ADma, BDma, PDma, T::TI>(aop, bop, pop, nk, bufs, acc, pwin);
  store_down<T>(acc, m0, n0, H, sorted, R, out + part * part_stride, ldo);
}

// y[t, d] += w[t, s] * out[t*k + s, d], slot by slot (mul then add, no fma).
// With splits > 1 the route's output is the in-order sum of its K parts
// (part p at route_out + p * part_stride).
__global__ void moe_combine_kernel(const float* __restrict__ route_out, int64_t ldo,
                                   const float* __restrict__ weights, int T, int top_k, float* __restrict__ y, int H,
                                   int64_t ldy, int splits = 1, int64_t part_stride = 0) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = (int64_t)T * H;
  if (i >= total) return;
  const int t = (int)(i / H);
  const int d = (int)(i % H);
  float acc = y[(int64_t)t * ldy + d];
  for (int s = 0; s < top_k; ++s) {
    const int64_t o = ((int64_t)t * top_k + s) * ldo + d;
    float v = route_out[o];
    for (int p = 1; p < splits; ++p) v = __fadd_rn(v, route_out[o + p * part_stride]);
    const float prod = __fmul_rn(weights[(int64_t)t * top_k + s], v);
    acc = __fadd_rn(acc, prod);
  }
  y[(int64_t)t * ldy + d] = acc;
}

// The same sums four columns per thread with 16-byte loads (H, the strides
// and the part stride multiples of 4, 16-byte aligned bases).
__global__ void moe_combine4_kernel(const float* __restrict__ route_out, int64_t ldo,
                                    const float* __restrict__ weights, int T, int top_k, float* __restrict__ y, int H,
                                    int64_t ldy, int splits, int64_t part_stride) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int H4 = H >> 2;
  if (i >= (int64_t)T * H4) return;
  const int t = (int)(i / H4);
  const int d = (int)(i % H4) * 4;
  f32x4 acc = *reinterpret_cast<const f32x4*>(y + (int64_t)t * ldy + d);
  for (int s = 0; s < top_k; ++s) {
    const float* o = route_out + ((int64_t)t * top_k + s) * ldo + d;
    f32x4 v = *reinterpret_cast<const f32x4*>(o);
    for (int p = 1; p < splits; ++p) {
      const f32x4 q = *reinterpret_cast<const f32x4*>(o + p * part_stride);
#pragma unroll
      for (int c = 0; c < 4; ++c) v[c] = __fadd_rn(v[c], q[c]);
    }
    const float w = weights[(int64_t)t * top_k + s];
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[c] = __fadd_rn(acc[c], __fmul_rn(w, v[c]));
  }
  *reinterpret_cast<f32x4*>(y + (int64_t)t * ldy + d) = acc;
}

void launch_combine(const float* route_out, int64_t ldo, const float* weights, int64_t T, int64_t top_k, float* y,
                    int64_t H, int64_t ldy, int splits, int64_t part_stride, hipStream_t st) {
  const int threads = 256;
  if (H % 4 == 0 && ldo % 4 == 0 && ldy % 4 == 0 && part_stride % 4 == 0 && intent::aligned16(route_out) &&
      intent::aligned16(y)) {
    const int64_t n = T * (H / 4);
    hipLaunchKernelGGL(moe_combine4_kernel, dim3((unsigned)((n + threads - 1) / threads)), dim3(threads), 0, st,
                       route_out, ldo, weights, (int)T, (int)top_k, y, (int)H, ldy, splits, part_stride);
  } else {
    hipLaunchKernelGGL(moe_combine_kernel, dim3((unsigned)((T * H + threads - 1) / threads)), dim3(threads), 0, st,
                       route_out, ldo, weights, (int)T, (int)top_k, y, (int)H, ldy, splits, part_stride);
  }
}

int64_t align_capacity(int64_t R, int64_t E, int64_t B) { return R + E * (B - 1); }

}  // namespace

extern "C" int intent_moe_route(const float* logits, int64_t T, int64_t E, int64_t top_k, int renormalize,
                                int32_t* topk_ids, float* topk_weights, void* stream) {
  intent::clear_error();
  INTENT_REQUIRE(T >= 0 && T <= INT32_MAX, INTENT_ERR_INVALID_ARGUMENT, "bad token count %lld", (long long)T);
  INTENT_REQUIRE(E >= 1 && E <= INT32_MAX, INTENT_ERR_INVALID_ARGUMENT, "experts must be at least 1, got %lld",
                 (long long)E);
  INTENT_REQUIRE(top_k >= 1 && top_k <= E && top_k <= kMaxTopK, INTENT_ERR_UNSUPPORTED,
                 "top_k must be in [1, min(E, %d)], got %lld", kMaxTopK, (long long)top_k);
  if (T == 0) return INTENT_OK;
  INTENT_REQUIRE(logits && topk_ids && topk_weights, INTENT_ERR_INVALID_ARGUMENT, "null pointer argument");
  if (E > kMaxRouteExperts) {
    hipLaunchKernelGGL(moe_route_seq_kernel, dim3((unsigned)((T + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                       logits, (int)T, (int)E, (int)top_k, renormalize, topk_ids, topk_weights);
    return intent::launch_status("moe_route_seq_kernel");
  }
  hipLaunchKernelGGL(moe_route_kernel, dim3((unsigned)((T + 3) / 4)), dim3(256), 0,
                     (hipStream_t)stream, logits, (int)T, (int)E, (int)top_k, renormalize, topk_ids, topk_weights);
  return intent::launch_status("moe_route");
}

extern "C" int intent_moe_align(const int32_t* topk_ids, int64_t T, int64_t top_k, int64_t E, int64_t block_size,
                                int32_t* sorted_route_ids, int64_t capacity, int32_t* expert_blocks,
                                int64_t num_blocks, int32_t* expert_offsets, int32_t* total_padded, void* stream) {
  intent::clear_error();
  INTENT_REQUIRE(T >= 0 && top_k >= 1 && T * top_k <= (1ll << 30), INTENT_ERR_INVALID_ARGUMENT,
                 "bad route count (T=%lld top_k=%lld)", (long long)T, (long long)top_k);
  INTENT_REQUIRE(E >= 1 && E <= kMaxAlignExperts, INTENT_ERR_UNSUPPORTED, "experts must be in [1, %d], got %lld",
                 kMaxAlignExperts, (long long)E);
  INTENT_REQUIRE(block_size >= 1 && block_size <= (1 << 16), INTENT_ERR_INVALID_ARGUMENT, "bad block size %lld",
                 (long long)block_size);
  const int64_t R = T * top_k;
  const int64_t need = align_capacity(R, E, block_size);
  INTENT_REQUIRE(capacity >= need, INTENT_ERR_INVALID_ARGUMENT, "sorted_route_ids needs %lld entries, got %lld",
                 (long long)need, (long long)capacity);
  INTENT_REQUIRE(num_blocks >= (capacity + block_size - 1) / block_size, INTENT_ERR_INVALID_ARGUMENT,
                 "expert_blocks needs %lld entries, got %lld", (long long)((capacity + block_size - 1) / block_size),
                 (long long)num_blocks);
  INTENT_REQUIRE(capacity <= INT32_MAX && num_blocks <= INT32_MAX, INTENT_ERR_UNSUPPORTED, "capacity exceeds int32");
  INTENT_REQUIRE(sorted_route_ids && expert_blocks && expert_offsets && total_padded && (R == 0 || topk_ids),
                 INTENT_ERR_INVALID_ARGUMENT, "null pointer argument");
  const size_t lds = (size_t)(3 * E + 1 + kAlignWaves * E) * sizeof(int);
  if (lds > 65536) {
    const hipError_t e = hipFuncSetAttribute((const void*)moe_align_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                             (int)lds);
    INTENT_REQUIRE(e == hipSuccess, INTENT_ERR_LAUNCH, "moe_align: %zu bytes of LDS refused (%s)", lds,
                   hipGetErrorString(e));
  }
  hipLaunchKernelGGL(moe_align_kernel, dim3(1), dim3(kAlignThreads), lds, (hipStream_t)stream, topk_ids, (int)R, (int)E,
                     (int)block_size, sorted_route_ids, (int)capacity, expert_blocks, (int)num_blocks,
                     expert_offsets, total_padded);
  return intent::launch_status("moe_align");
}

namespace {


// ---- any block size / shape: one output element per thread -------------------
// The same dequantisation (f16 (q - z) * s, one rounding), f32 sums of the
// f16 products, SiLU gating and route scatter as the tiled kernels; used
// where those do not apply (block sizes other than 64 and 128, dimensions
// off their tiles, unaligned rows).
INTENT_DEVICE float w4_dot_row(const f16* __restrict__ xr, const uint8_t* __restrict__ qr,
                               const f16* __restrict__ sr, const uint8_t* __restrict__ zr, int K, int gs) {
  float acc = 0.f;
  for (int g0 = 0, g = 0; g0 < K; g0 += gs, ++g) {
    const float s = (float)sr[g];
    const float z = (float)zr[g];
    for (int k = g0; k < g0 + gs; ++k) {
      const uint32_t byte = qr[k >> 1];
      const float q = (float)((k & 1) ? (byte >> 4) : (byte & 15u));
      const f16 w = (f16)((float)(f16)(q - z) * s);
      acc = __builtin_fmaf((float)xr[k], (float)w, acc);
    }
  }
  return acc;
}

__global__ __launch_bounds__(256) void moe_gate_up_generic_kernel(
    const f16* __restrict__ x, int64_t ldx, int H, const int32_t* __restrict__ sorted,
    const int32_t* __restrict__ blocks, int B, int R, int top_k, const uint8_t* __restrict__ wq,
    const f16* __restrict__ ws, const uint8_t* __restrict__ wz, int F, int gs, f16* __restrict__ act,
    int64_t ld_act, int fchunks) {
  const int row = blockIdx.x / fchunks;
  const int f = (blockIdx.x % fchunks) * 256 + threadIdx.x;
  if (f >= F) return;
  const int e = blocks[row / B];
  if (e < 0) return;
  const int r = sorted[row];
  f16 o = (f16)0.f;
  if (r >= 0 && r < R) {
    const int64_t ldq = H / 2, ldp = H / gs;
    const int64_t gr = (int64_t)e * 2 * F + f, ur = gr + F;
    const f16* xr = x + (int64_t)(r / top_k) * ldx;
    const float gt = w4_dot_row(xr, wq + gr * ldq, ws + gr * ldp, wz + gr * ldp, H, gs);
    const float up = w4_dot_row(xr, wq + ur * ldq, ws + ur * ldp, wz + ur * ldp, H, gs);
    o = (f16)((gt / (1.0f + expf(-gt))) * up);
  }
  act[(int64_t)row * ld_act + f] = o;
}

__global__ __launch_bounds__(256) void moe_down_generic_kernel(
    const f16* __restrict__ act, int64_t ld_act, const int32_t* __restrict__ sorted,
    const int32_t* __restrict__ blocks, int B, int R, const uint8_t* __restrict__ wq, const f16* __restrict__ ws,
    const uint8_t* __restrict__ wz, int H, int F, int gs, float* __restrict__ out, int64_t ldo, int dchunks) {
  const int row = blockIdx.x / dchunks;
  const int d = (blockIdx.x % dchunks) * 256 + threadIdx.x;
  if (d >= H) return;
  const int e = blocks[row / B];
  const int r = sorted[row];
  if (e < 0 || r < 0 || r >= R) return;
  const int64_t ldq = F / 2, ldp = F / gs;
  const int64_t wr = (int64_t)e * H + d;
  out[(int64_t)r * ldo + d] = w4_dot_row(act + (int64_t)row * ld_act, wq + wr * ldq, ws + wr * ldp, wz + wr * ldp,
                                         F, gs);
}

template <int B>
int gate_up_launch(const void* x, int64_t T, int64_t H, int64_t x_ld, const int32_t* sorted, const int32_t* blocks,
                   int64_t num_blocks, int64_t top_k, const uint8_t* wq, const void* ws, const uint8_t* wz,
                   int64_t F, int64_t gs, void* act, int64_t act_ld, void* stream) {
  const int64_t ldp = H / gs;
  if (B == GateUpPk::BM && ldp % 4 == 0 && intent::aligned4(ws) && intent::aligned4(wz)) {
    const int64_t grid = num_blocks * ((F + GateUpPk::BN / 2 - 1) / (GateUpPk::BN / 2));
    INTENT_REQUIRE(grid < (1ll << 31), INTENT_ERR_UNSUPPORTED, "grid too large");
    auto kernel = gs % 64 == 0 ? moe_gate_up_pk_kernel<true> : moe_gate_up_pk_kernel<false>;
    hipLaunchKernelGGL(kernel, dim3((unsigned)grid), dim3(GateUpPk::NT), 0, (hipStream_t)stream, (const f16*)x, x_ld,
                       (int)H, sorted, blocks, (int)num_blocks, (int)(T * top_k), (int)top_k, wq, (const f16*)ws, wz,
                       (int)F, (int)gs, (f16*)act, act_ld);
    return intent::launch_status("moe_gate_up_w4");
  }
  using Tl = typename MoeTiles<B>::GateUp;
  const int64_t ftile = Tl::BN / 2;
  const int64_t grid = num_blocks * ((F + ftile - 1) / ftile);
  INTENT_REQUIRE(grid < (1ll << 31), INTENT_ERR_UNSUPPORTED, "grid too large");
  hipLaunchKernelGGL((moe_gate_up_kernel<B>), dim3((unsigned)grid), dim3(Tl::NT_WS), 0, (hipStream_t)stream,
                     (const f16*)x, x_ld, (int)H, sorted, blocks, (int)num_blocks, (int)(T * top_k), (int)top_k, wq,
                     (const f16*)ws, wz, (int)F, (int)gs, (f16*)act, act_ld);
  return intent::launch_status("moe_gate_up_w4");
}

template <int B>
int down_launch(const void* act, int64_t act_ld, const int32_t* sorted, const int32_t* blocks, int64_t num_blocks,
                int64_t R, const uint8_t* wq, const void* ws, const uint8_t* wz, int64_t H, int64_t F, int64_t gs,
                float* out, int64_t out_ld, void* stream) {
  using Tl = typename MoeTiles<B>::Down;
  const int64_t ntiles = (H + Tl::BN - 1) / Tl::BN;
  const int64_t grid = num_blocks * ntiles;
  INTENT_REQUIRE(grid < (1ll << 31), INTENT_ERR_UNSUPPORTED, "grid too large");
  hipLaunchKernelGGL((moe_down_kernel<B>), dim3((unsigned)grid), dim3(Tl::NT_WS), 0, (hipStream_t)stream,
                     (const f16*)act, act_ld, sorted, blocks, (int)num_blocks, (int)ntiles, (int)R, wq,
                     (const f16*)ws, wz, (int)H, (int)F, (int)gs, out, out_ld);
  return intent::launch_status("moe_down_w4");
}

int combine_launch(const float* route_out, int64_t out_ld, const float* topk_weights, int64_t T, int64_t top_k,
                   float* y, int64_t H, int64_t y_ld, void* stream) {
  INTENT_REQUIRE((T * H + 255) / 256 < (1ll << 31), INTENT_ERR_UNSUPPORTED, "grid too large");
  launch_combine(route_out, out_ld, topk_weights, T, top_k, y, H, y_ld, 1, 0, (hipStream_t)stream);
  return intent::launch_status("moe_combine");
}

// The 160-row tile takes windowed group parameters only: group sizes that
// are multiples of 64, K / group a multiple of 4, 4-byte aligned parameters.
bool pk160_ok(int64_t K, int64_t gs, const void* scales, const void* zeros) {
  return gs % 64 == 0 && (K / gs) % 4 == 0 && intent::aligned4(scales) && intent::aligned4(zeros);
}

bool supported_block(int64_t b) { return b == 64 || b == 128 || b == Pk160::BM; }

}  // namespace

extern "C" int intent_moe_gate_up_w4(const void* x, int64_t T, int64_t H, int64_t x_ld,
                                     const int32_t* sorted_route_ids, const int32_t* expert_blocks, int64_t num_blocks,
                                     int64_t block_size, int64_t top_k, const uint8_t* w_packed, const void* w_scales,
                                     const uint8_t* w_zeros, int64_t E, int64_t F, int64_t group_size, void* act,
                                     int64_t act_ld, void* stream) {
  intent::clear_error();
  INTENT_REQUIRE(block_size >= 1 && block_size <= (1 << 20), INTENT_ERR_INVALID_ARGUMENT, "bad block_size %lld",
                 (long long)block_size);
  INTENT_REQUIRE(H > 0 && H % 2 == 0 && H <= INT32_MAX && F > 0 && F <= INT32_MAX / 2, INTENT_ERR_INVALID_ARGUMENT,
                 "H must be positive and even, F positive");
  INTENT_REQUIRE(group_size > 0 && H % group_size == 0, INTENT_ERR_INVALID_ARGUMENT,
                 "group_size must divide H (H=%lld group=%lld)", (long long)H, (long long)group_size);
  INTENT_REQUIRE(T >= 0 && top_k >= 1 && E >= 1 && num_blocks >= 0, INTENT_ERR_INVALID_ARGUMENT, "bad extents");
  if (num_blocks == 0 || T == 0) return INTENT_OK;
  INTENT_REQUIRE(x && sorted_route_ids && expert_blocks && w_packed && w_scales && w_zeros && act,
                 INTENT_ERR_INVALID_ARGUMENT, "null pointer argument");
  INTENT_REQUIRE(x_ld >= H && act_ld >= F, INTENT_ERR_INVALID_ARGUMENT, "leading stride smaller than the row");
  const bool fast = supported_block(block_size) && H % 128 == 0 && F % 64 == 0 &&
                    (group_size == 32 || group_size % 64 == 0) && intent::fits_offset(2 * F, H / 2) &&
                    intent::fits_offset(2 * F, H / group_size * 2) && intent::fits_offset(T, x_ld * 2) &&
                    intent::fits_offset(256 + 1, act_ld * 2) && intent::aligned16(x) && x_ld % 8 == 0 &&
                    intent::aligned16(w_packed) &&
                    (block_size != Pk160::BM || pk160_ok(H, group_size, w_scales, w_zeros));
  if (!fast) {
    const int64_t fchunks = (F + 255) / 256;
    const int64_t grid = num_blocks * block_size * fchunks;
    INTENT_REQUIRE(grid < (1ll << 31), INTENT_ERR_UNSUPPORTED, "moe_gate_up_w4: grid too large");
    hipLaunchKernelGGL(moe_gate_up_generic_kernel, dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream,
                       (const f16*)x, x_ld, (int)H, sorted_route_ids, expert_blocks, (int)block_size,
                       (int)(T * top_k), (int)top_k, w_packed, (const f16*)w_scales, w_zeros, (int)F, (int)group_size,
                       (f16*)act, act_ld, (int)fchunks);
    return intent::launch_status("moe_gate_up_generic_kernel");
  }
  if (block_size == Pk160::BM) {
    const int64_t grid = num_blocks * ((F + Pk160::BN / 2 - 1) / (Pk160::BN / 2));
    INTENT_REQUIRE(grid < (1ll << 31), INTENT_ERR_UNSUPPORTED, "grid too large");
    hipLaunchKernelGGL((moe_gate_up_pk_kernel<true, Pk160, kPk160Stages>), dim3((unsigned)grid), dim3(Pk160::NT), 0,
                       (hipStream_t)stream, (const f16*)x, x_ld, (int)H, sorted_route_ids, expert_blocks,
                       (int)num_blocks, (int)(T * top_k), (int)top_k, w_packed, (const f16*)w_scales, w_zeros, (int)F,
                       (int)group_size, (f16*)act, act_ld);
    return intent::launch_status("moe_gate_up_w4");
  }
  if (block_size == 64)
    return gate_up_launch<64>(x, T, H, x_ld, sorted_route_ids, expert_blocks, num_blocks, top_k, w_packed, w_scales,
                              w_zeros, F, group_size, act, act_ld, stream);
  return gate_up_launch<128>(x, T, H, x_ld, sorted_route_ids, expert_blocks, num_blocks, top_k, w_packed, w_scales,
                             w_zeros, F, group_size, act, act_ld, stream);
}

namespace {

int down_check(const void* act, int64_t act_ld, const int32_t* sorted_route_ids, const int32_t* expert_blocks,
               int64_t num_blocks, int64_t block_size, int64_t R, const uint8_t* w_packed, const void* w_scales,
               const uint8_t* w_zeros, int64_t E, int64_t H, int64_t F, int64_t group_size, const float* out,
               int64_t out_ld) {
  INTENT_REQUIRE(block_size >= 1 && block_size <= (1 << 20), INTENT_ERR_INVALID_ARGUMENT, "bad block_size %lld",
                 (long long)block_size);
  INTENT_REQUIRE(F > 0 && F % 2 == 0 && F <= INT32_MAX && H > 0 && H <= INT32_MAX, INTENT_ERR_INVALID_ARGUMENT,
                 "F must be positive and even, H positive");
  INTENT_REQUIRE(group_size > 0 && F % group_size == 0, INTENT_ERR_INVALID_ARGUMENT,
                 "group_size must divide F (F=%lld group=%lld)", (long long)F, (long long)group_size);
  INTENT_REQUIRE(R >= 0 && E >= 1 && num_blocks >= 0, INTENT_ERR_INVALID_ARGUMENT, "bad extents");
  if (num_blocks == 0 || R == 0) return INTENT_OK;
  INTENT_REQUIRE(act && sorted_route_ids && expert_blocks && w_packed && w_scales && w_zeros && out,
                 INTENT_ERR_INVALID_ARGUMENT, "null pointer argument");
  INTENT_REQUIRE(act_ld >= F && out_ld >= H, INTENT_ERR_INVALID_ARGUMENT, "leading stride smaller than the row");
  return INTENT_OK;
}

// Shapes the tiled down projections take.
bool down_fast(const void* act, int64_t act_ld, int64_t block_size, const uint8_t* w_packed, int64_t H, int64_t F,
               int64_t group_size) {
  return supported_block(block_size) && F % 128 == 0 && (group_size == 32 || group_size % 64 == 0) &&
         intent::fits_offset(H, F / 2) && intent::fits_offset(H, F / group_size * 2) &&
         intent::fits_offset(256 + 1, act_ld * 2) && intent::aligned16(act) && act_ld % 8 == 0 &&
         intent::aligned16(w_packed);
}

// Grid of moe_down_pk_kernel: every XCD runs ntiles column tiles for each
// of the (row block, K part) pairs it owns, eight pairs per round of XCDs.
int64_t down_pk_grid(int64_t splits, int64_t num_blocks, int64_t ntiles) {
  return 8 * ntiles * ((splits * num_blocks + 7) / 8);
}

int down_generic(const void* act, int64_t act_ld, const int32_t* sorted, const int32_t* blocks, int64_t num_blocks,
                 int64_t block_size, int64_t R, const uint8_t* wq, const void* ws, const uint8_t* wz, int64_t H,
                 int64_t F, int64_t gs, float* out, int64_t out_ld, void* stream) {
  const int64_t dchunks = (H + 255) / 256;
  const int64_t grid = num_blocks * block_size * dchunks;
  INTENT_REQUIRE(grid < (1ll << 31), INTENT_ERR_UNSUPPORTED, "moe_down_w4: grid too large");
  hipLaunchKernelGGL(moe_down_generic_kernel, dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream,
                     (const f16*)act, act_ld, sorted, blocks, (int)block_size, (int)R, wq, (const f16*)ws, wz, (int)H,
                     (int)F, (int)gs, out, out_ld, (int)dchunks);
  return intent::launch_status("moe_down_generic_kernel");
}

// Down projection on the 160-row packed-weight tile, K split into `splits`
// parts (part p at out + p * part_stride).
int down_pk160_launch(const void* act, int64_t act_ld, const int32_t* sorted, const int32_t* blocks,
                      int64_t num_blocks, int64_t R, const uint8_t* wq, const void* ws, const uint8_t* wz, int64_t H,
                      int64_t F, int64_t gs, int splits, float* out, int64_t out_ld, int64_t part_stride,
                      void* stream) {
  const int64_t ntiles = (H + Pk160::BN - 1) / Pk160::BN;
  const int64_t grid = down_pk_grid(splits, num_blocks, ntiles);
  INTENT_REQUIRE(grid < (1ll << 31), INTENT_ERR_UNSUPPORTED, "grid too large");
  hipLaunchKernelGGL((moe_down_pk_kernel<true, Pk160, kPk160Stages>), dim3((unsigned)grid), dim3(Pk160::NT), 0,
                     (hipStream_t)stream, (const f16*)act, act_ld, sorted, blocks, (int)num_blocks, (int)ntiles, (int)R,
                     wq, (const f16*)ws, wz, (int)H, (int)F, (int)gs, splits, out, out_ld, part_stride);
  return intent::launch_status("moe_down_pk");
}

int down_dispatch(const void* act, int64_t act_ld, const int32_t* sorted, const int32_t* blocks, int64_t num_blocks,
                  int64_t block_size, int64_t R, const uint8_t* wq, const void* ws, const uint8_t* wz, int64_t H,
                  int64_t F, int64_t gs, float* out, int64_t out_ld, void* stream) {
  if (block_size == Pk160::BM)
    return down_pk160_launch(act, act_ld, sorted, blocks, num_blocks, R, wq, ws, wz, H, F, gs, 1, out, out_ld, 0,
                             stream);
  if (block_size == 64)
    return down_launch<64>(act, act_ld, sorted, blocks, num_blocks, R, wq, ws, wz, H, F, gs, out, out_ld, stream);
  return down_launch<128>(act, act_ld, sorted, blocks, num_blocks, R, wq, ws, wz, H, F, gs, out, out_ld, stream);
}

}  // namespace

extern "C" int intent_moe_down_w4(const void* act, int64_t act_ld, const int32_t* sorted_route_ids,
                                  const int32_t* expert_blocks, int64_t num_blocks, int64_t block_size, int64_t R,
                                  const uint8_t* w_packed, const void* w_scales, const uint8_t* w_zeros, int64_t E,
                                  int64_t H, int64_t F, int64_t group_size, float* out, int64_t out_ld, void* stream) {
  intent::clear_error();
  int st = down_check(act, act_ld, sorted_route_ids, expert_blocks, num_blocks, block_size, R, w_packed, w_scales,
                      w_zeros, E, H, F, group_size, out, out_ld);
  if (st != INTENT_OK || num_blocks == 0 || R == 0) return st;
  if (!down_fast(act, act_ld, block_size, w_packed, H, F, group_size) ||
      (block_size == Pk160::BM && !pk160_ok(F, group_size, w_scales, w_zeros)))
    return down_generic(act, act_ld, sorted_route_ids, expert_blocks, num_blocks, block_size, R, w_packed, w_scales,
                        w_zeros, H, F, group_size, out, out_ld, stream);
  return down_dispatch(act, act_ld, sorted_route_ids, expert_blocks, num_blocks, block_size, R, w_packed, w_scales,
                       w_zeros, H, F, group_size, out, out_ld, stream);
}

extern "C" int intent_moe_combine(const float* route_out, int64_t out_ld, const float* topk_weights, int64_t T,
                                  int64_t top_k, float* y, int64_t H, int64_t y_ld, void* stream) {
  intent::clear_error();
  INTENT_REQUIRE(T >= 0 && H >= 0 && top_k >= 1 && T * H < (1ll << 40), INTENT_ERR_INVALID_ARGUMENT, "bad extents");
  if (T == 0 || H == 0) return INTENT_OK;
  INTENT_REQUIRE(route_out && topk_weights && y, INTENT_ERR_INVALID_ARGUMENT, "null pointer argument");
  INTENT_REQUIRE(out_ld >= H && y_ld >= H, INTENT_ERR_INVALID_ARGUMENT, "leading stride smaller than the row");
  return combine_launch(route_out, out_ld, topk_weights, T, top_k, y, H, y_ld, stream);
}

namespace {

// K parts of the composite's down projection (moe_down_pk_kernel).
// At most this many; the composite takes the largest of 4, 2, 1 that splits F
// into whole dwords of groups (measured on config 4: 2 parts 653 us, 4 parts
// 603 us, 7 parts 631 us for the whole layer).
constexpr int kDownSplits = 4;

int down_splits(int64_t F, int64_t gs) {
  for (int s = kDownSplits; s > 1; s /= 2)
    if (F % (s * 4 * gs) == 0 && (F / s) % 64 == 0) return s;
  return 1;
}

struct MoEWorkspace {
  size_t ids, weights, sorted, blocks, offsets, total, act, out, bytes;
  int64_t capacity, nblocks;
};

size_t round256(size_t v) { return (v + 255) & ~(size_t)255; }

MoEWorkspace moe_layout(int64_t T, int64_t top_k, int64_t E, int64_t H, int64_t F, int64_t B) {
  MoEWorkspace w{};
  const int64_t R = T * top_k;
  w.capacity = align_capacity(R, E, B);
  w.nblocks = (w.capacity + B - 1) / B;
  size_t o = 0;
  w.ids = o;     o = round256(o + sizeof(int32_t) * R);
  w.weights = o; o = round256(o + sizeof(float) * R);
  w.sorted = o;  o = round256(o + sizeof(int32_t) * w.capacity);
  w.blocks = o;  o = round256(o + sizeof(int32_t) * w.nblocks);
  w.offsets = o; o = round256(o + sizeof(int32_t) * (E + 1));
  w.total = o;   o = round256(o + sizeof(int32_t));
  w.act = o;     o = round256(o + sizeof(uint16_t) * (size_t)(w.nblocks * B) * F);
  w.out = o;     o = round256(o + sizeof(float) * (size_t)R * H * kDownSplits);
  w.bytes = o;
  return w;
}

// The composite aligns to 128-row blocks: measured on config 4, 64-row
// blocks and 256-row expert segments were both slower (the W4 decode per
// MFMA grows as the tile's row count falls), and a split-K down projection
// did not help either.
constexpr int64_t kCompositeBlock = 128;

// The composite takes 160-row blocks (Pk160) when experts average at least 96
// routes (with fewer, 160-row blocks mostly hold padding) and both
// projections take windowed group parameters; else 128-row blocks.
bool composite_wants_pk160(int64_t T, int64_t top_k, int64_t E) { return T * top_k >= 96 * E; }

// Workspace for either block size the composite may pick.
size_t composite_workspace(int64_t T, int64_t top_k, int64_t E, int64_t H, int64_t F) {
  const size_t base = moe_layout(T, top_k, E, H, F, kCompositeBlock).bytes;
  if (!composite_wants_pk160(T, top_k, E)) return base;
  const size_t big = moe_layout(T, top_k, E, H, F, Pk160::BM).bytes;
  return big > base ? big : base;
}

}  // namespace

extern "C" size_t intent_moe_workspace_size(int64_t T, int64_t top_k, int64_t E, int64_t H, int64_t F,
                                            int64_t block_size) {
  if (T < 0 || top_k < 1 || E < 1 || H < 0 || F < 0) return 0;
  return block_size > 0 ? moe_layout(T, top_k, E, H, F, block_size).bytes : composite_workspace(T, top_k, E, H, F);
}

extern "C" int intent_moe_expert_ffn_w4(const float* router_logits, const void* x, int64_t T, int64_t H, int64_t E,
                                        int64_t top_k, int renormalize, const uint8_t* wgu_packed,
                                        const void* wgu_scales, const uint8_t* wgu_zeros, const uint8_t* wd_packed,
                                        const void* wd_scales, const uint8_t* wd_zeros, int64_t F,
                                        int64_t group_size, float* y, void* workspace, size_t workspace_bytes,
                                        int32_t* topk_ids_out, float* topk_weights_out, void* stream) {
  intent::clear_error();
  INTENT_REQUIRE(T >= 0 && top_k >= 1 && E >= 1 && H > 0 && F > 0, INTENT_ERR_INVALID_ARGUMENT, "bad extents");
  if (T == 0) return INTENT_OK;
  INTENT_REQUIRE(group_size > 0, INTENT_ERR_INVALID_ARGUMENT, "group_size must be positive");
  const bool big = composite_wants_pk160(T, top_k, E) && pk160_ok(H, group_size, wgu_scales, wgu_zeros) &&
                   pk160_ok(F, group_size, wd_scales, wd_zeros) && F % (down_splits(F, group_size) * 4 * group_size) == 0;
  const int64_t B = big ? Pk160::BM : kCompositeBlock;
  const MoEWorkspace L = moe_layout(T, top_k, E, H, F, B);
  const size_t need = composite_workspace(T, top_k, E, H, F);
  INTENT_REQUIRE(workspace && workspace_bytes >= need, INTENT_ERR_WORKSPACE, "workspace needs %zu bytes, got %zu", need,
                 workspace_bytes);
  INTENT_REQUIRE(intent::aligned16(workspace), INTENT_ERR_ALIGNMENT, "workspace must be 16-byte aligned");
  INTENT_REQUIRE(y, INTENT_ERR_INVALID_ARGUMENT, "null output");
  char* ws = (char*)workspace;
  int32_t* ids = topk_ids_out ? topk_ids_out : (int32_t*)(ws + L.ids);
  float* wts = topk_weights_out ? topk_weights_out : (float*)(ws + L.weights);
  int32_t* sorted = (int32_t*)(ws + L.sorted);
  int32_t* blocks = (int32_t*)(ws + L.blocks);
  int32_t* offsets = (int32_t*)(ws + L.offsets);
  int32_t* total = (int32_t*)(ws + L.total);
  void* act = ws + L.act;
  float* out = (float*)(ws + L.out);
  int st = intent_moe_route(router_logits, T, E, top_k, renormalize, ids, wts, stream);
  if (st != INTENT_OK) return st;
  st = intent_moe_align(ids, T, top_k, E, B, sorted, L.capacity, blocks, L.nblocks, offsets, total, stream);
  if (st != INTENT_OK) return st;
  st = intent_moe_gate_up_w4(x, T, H, H, sorted, blocks, L.nblocks, B, top_k, wgu_packed, wgu_scales, wgu_zeros, E, F,
                             group_size, act, F, stream);
  if (st != INTENT_OK) return st;
  const int64_t R = T * top_k;
  const int64_t ldp = F / group_size;
  const int want = down_splits(F, group_size);
  const bool pk = down_fast(act, F, B, wd_packed, H, F, group_size) && ldp % 4 == 0 &&
                  F % (want * 4 * group_size) == 0 && (F / want) % 64 == 0 &&
                  intent::aligned4(wd_scales) && intent::aligned4(wd_zeros);
  int splits = 1;
  if (pk) {
    st = down_check(act, F, sorted, blocks, L.nblocks, B, R, wd_packed, wd_scales, wd_zeros, E, H, F, group_size, out,
                    H);
    if (st != INTENT_OK) return st;
    splits = want;
    if (B == Pk160::BM) {
      st = down_pk160_launch(act, F, sorted, blocks, L.nblocks, R, wd_packed, wd_scales, wd_zeros, H, F, group_size,
                             splits, out, H, R * H, stream);
      if (st != INTENT_OK) return st;
      launch_combine(out, H, wts, T, top_k, y, H, H, splits, R * H, (hipStream_t)stream);
      return intent::launch_status("moe_combine");
    }
    const int64_t ntiles = (H + GateUpPk::BN - 1) / GateUpPk::BN;
    const int64_t grid = down_pk_grid(splits, L.nblocks, ntiles);
    INTENT_REQUIRE(grid < (1ll << 31), INTENT_ERR_UNSUPPORTED, "grid too large");
    auto kernel = group_size % 64 == 0 ? moe_down_pk_kernel<true> : moe_down_pk_kernel<false>;
    hipLaunchKernelGGL(kernel, dim3((unsigned)grid), dim3(GateUpPk::NT), 0, (hipStream_t)stream,
                       (const f16*)act, F, sorted, blocks, (int)L.nblocks, (int)ntiles, (int)R, wd_packed,
                       (const f16*)wd_scales, wd_zeros, (int)H, (int)F, (int)group_size, splits, out, H, R * H);
    st = intent::launch_status("moe_down_pk");
  } else {
    st = intent_moe_down_w4(act, F, sorted, blocks, L.nblocks, B, R, wd_packed, wd_scales, wd_zeros, E, H, F,
                            group_size, out, H, stream);
  }
  if (st != INTENT_OK) return st;
  launch_combine(out, H, wts, T, top_k, y, H, H, splits, R * H, (hipStream_t)stream);
  return intent::launch_status("moe_combine");
}
