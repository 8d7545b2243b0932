// W4A16 decode GEMV (M <= 16) for gfx950.
//
// Work split: one workgroup owns 16*NT output columns (weight rows n) and all
// M <= 16 activation rows. Its KW waves split K in 128-wide steps, interleaved
// (wave w takes steps w, w+KW, ...), so at any moment the waves of a group
// stream KW*64 contiguous bytes of every weight row.
//
// Per step a lane (r = lane%16, quad = lane/16) loads 16 bytes = 32 nibbles of
// weight row n0+r (k = step*128 + quad*32 .. +32) with one 128-bit load, and
// the matching 32 activations of row m = r. Nibbles are dequantized in
// registers ((q - z) * s in packed f16) and fed to v_mfma_f32_16x16x32_f16:
// MFMA t (t = 0..3) consumes k = step*128 + quad*32 + t*8 + [0..7] from both
// operands, so four MFMAs cover the 128 k of the step. Activation rows m >= M
// are zero and never loaded. Partial sums of the KW waves are reduced through
// LDS in a fixed order and rounded to f16 once.

#include "common.h"
#include "internal.h"

namespace {

template <int NT, int KW>
__global__ __launch_bounds__(64 * KW) void w4a16_gemv_kernel(
    const f16* __restrict__ x, int64_t ldx, int M, int K,
    const uint8_t* __restrict__ wq, int64_t ldw,
    const f16* __restrict__ sc, const uint8_t* __restrict__ zp, int64_t ldq, int gs,
    f16* __restrict__ y, int64_t ldy, int N) {
  __shared__ f32x4 red[KW][NT][64];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int r = lane & 15;
  const int quad = lane >> 4;
  const int n_base = blockIdx.x * 16 * NT;
  const int nsteps = K >> 7;

  const uint8_t* wrow[NT];
  const f16* srow[NT];
  const uint8_t* zrow[NT];
#pragma unroll
  for (int j = 0; j < NT; ++j) {
    int n = n_base + j * 16 + r;
    n = n < N ? n : N - 1;  // tail rows compute on a valid row; their outputs are dropped
    wrow[j] = wq + (int64_t)n * ldw + quad * 16;
    srow[j] = sc + (int64_t)n * ldq;
    zrow[j] = zp + (int64_t)n * ldq;
  }
  // Rows m >= M read row M-1 (unpredicated loads); their outputs are dropped.
  const f16* xrow = x + (int64_t)(r < M ? r : M - 1) * ldx + quad * 32;

  f32x4 acc[NT];
#pragma unroll
  for (int j = 0; j < NT; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};

  int s = wave;
  u32x4 wv[NT];
  u32x4 xv[4];
  f16 sv[NT];
  uint8_t zv[NT];
  if (s < nsteps) {
    const int g = (s * 128 + quad * 32) / gs;
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      wv[j] = load16(wrow[j] + (int64_t)s * 64);
      sv[j] = srow[j][g];
      zv[j] = zrow[j][g];
    }
#pragma unroll
    for (int t = 0; t < 4; ++t) xv[t] = load16(xrow + (int64_t)s * 128 + t * 8);
  }
  while (s < nsteps) {
    f16x2 zoff[NT], scale[NT];
    u32x4 wc[NT], xc[4];
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      zoff[j] = splat2((f16)(float)(1024 + zv[j]));
      scale[j] = splat2(sv[j]);
      wc[j] = wv[j];
    }
#pragma unroll
    for (int t = 0; t < 4; ++t) xc[t] = xv[t];
    const int sn = s + KW;
    if (sn < nsteps) {  // prefetch the next step (weights, scales, zeros) before the math of this one
      const int gn = (sn * 128 + quad * 32) / gs;
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        wv[j] = load16(wrow[j] + (int64_t)sn * 64);
        sv[j] = srow[j][gn];
        zv[j] = zrow[j][gn];
      }
#pragma unroll
      for (int t = 0; t < 4; ++t) xv[t] = load16(xrow + (int64_t)sn * 128 + t * 8);
    }
#pragma unroll
    for (int j = 0; j < NT; ++j) {
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        f16x8 b = dequant8(wc[j][t], zoff[j], scale[j]);
        f16x8 a = bit_cast<f16x8>(xc[t]);
        acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, acc[j], 0, 0, 0);
      }
    }
    s = sn;
  }

#pragma unroll
  for (int j = 0; j < NT; ++j) red[wave][j][lane] = acc[j];
  __syncthreads();
  // 16x16 MFMA result layout: lane l holds column l%16, rows (l/16)*4 + i.
  for (int o = threadIdx.x; o < 256 * NT; o += 64 * KW) {
    const int j = o >> 8;
    const int m = (o >> 4) & 15;
    const int nc = o & 15;
    const int src = (m >> 2) * 16 + nc;
    float sum = 0.f;
#pragma unroll
    for (int w = 0; w < KW; ++w) sum += red[w][j][src][m & 3];
    const int n = n_base + j * 16 + nc;
    if (m < M && n < N) y[(int64_t)m * ldy + n] = (f16)sum;
  }
}


// Cache policy of the packed-weight loads of the decode kernels: every weight
// byte is read once per launch, so the loads are non-temporal (the NT bit of
// the buffer instruction's cache-policy operand). Measured on the same box:
// M = 1 3.30 -> 3.22 us, M = 16 6.99 -> 6.63 us. (Q4_K records, whose header
// line is read by four lanes, measured 3% slower with it.)
constexpr int kWeightPolicy = 2;

// ---- 4 <= M <= 16: MFMA GEMV with every load issued up front ------------------
// Same split and MFMA operand roles as w4a16_gemv_kernel: 16 weight rows per
// workgroup, KW waves taking 128-wide K steps in turn, lane (r, quad) holding
// k = step*128 + quad*32 + t*8 + [0, 8) of weight row n0 + r (bytes quad*16 ..
// of the step, one 16-byte load) and of activation row r. A wave owns at most
// SPW steps and issues all of its loads before the first MFMA.
//
// Loads are laid out for the L1, whose request slots bound this kernel:
//  * scales and zeros of the workgroup's 16 rows are fetched once, first, as
//    contiguous row segments (wave w: row w), packed into LDS records and read
//    back after one barrier (per-lane scattered u16/u8 loads cost 1.6 us at
//    M = 16, K = N = 4096);
//  * activations are loaded as whole cache lines, four rows x 256 bytes per
//    instruction, and moved into operand order through a wave-private LDS
//    stage (one write and one read of 16 bytes per lane and piece).
// Activation rows r >= M lie past the end of the x buffer resource (its size
// is exactly the bytes of rows 0..M-1), so their loads return zeros without a
// memory access. The product of a step is exact in fp32; the KW partial tiles
// are summed through LDS in wave order and rounded to f16 once.
constexpr int kFrontMaxGroups = 256;
constexpr int kFrontXRow = 272;  // bytes per activation row in a wave's LDS stage (256 + 16)
constexpr int kFrontWRow = 144;  // bytes per weight row in a wave's LDS stage (128 + 16)

template <int KW, int SPW, bool kPairRec>
__global__ __launch_bounds__(64 * KW) void w4a16_gemv_front_kernel(
    const f16* __restrict__ x, int ldx, int x_bytes, const uint8_t* __restrict__ wq, int ldw,
    const f16* __restrict__ sc, const uint8_t* __restrict__ zp, int ldq, int nsteps, int G, float inv_cpg, int N,
    f16* __restrict__ y, int ldy, int M) {
  static_assert(KW == 16, "the record fetch gives wave w row w");
  __shared__ f32x4 red[KW][64];
  __shared__ uint32_t rec[16][kFrontMaxGroups];
  __shared__ __attribute__((aligned(16))) uint8_t xstage[KW][16 * kFrontXRow];
  // SPW == 2: a wave's two steps are adjacent, so its 16 weight rows are 128
  // contiguous bytes each, loaded as whole lines and sorted through LDS.
  constexpr bool kLineW = SPW == 2;
  __shared__ __attribute__((aligned(16))) uint8_t wstage[kLineW ? KW : 1][kLineW ? 16 * kFrontWRow : 16];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane & 15;
  const int quad = lane >> 4;
  const int n0 = blockIdx.x * 16;
  const int nr = n0 + r < N ? r : N - 1 - n0;  // tail rows compute on a valid row; their outputs are dropped
  // Step i of a wave: adjacent steps with whole-line weight loads, else
  // interleaved (wave w takes w, w + KW, ...).
  auto step_of = [](int w, int i) { return kLineW ? SPW * w + i : w + KW * i; };

  // Records of row n0 + wave (clamped): groups lane, lane + 64, ...
  // kPairRec (G even, 4-byte scale rows, 2-byte zero rows): item t of the
  // workgroup = (row t / G2, group pair t % G2), a scale dword and a zero
  // u16 per item, 16 * G2 items over the 1024 threads (8 instructions at
  // G = 32 instead of 32).
  constexpr int RPL = kPairRec ? (16 * kFrontMaxGroups / 2 + 64 * KW - 1) / (64 * KW) : kFrontMaxGroups / 64;
  uint32_t sq[RPL], zq[RPL];
  const int G2 = G >> 1;
  if constexpr (kPairRec) {
#pragma unroll
    for (int u = 0; u < RPL; ++u) {
      const int t = threadIdx.x + 64 * KW * u;
      if (64 * KW * u < 16 * G2) {  // uniform
        const int row = min(t / G2, 15);
        const int rn = n0 + row < N ? row : N - 1 - n0;
        const int p = t < 16 * G2 ? t - row * G2 : 0;
        sq[u] = __builtin_amdgcn_raw_buffer_load_b32(make_rsrc(sc + (int64_t)n0 * ldq), (rn * ldq + 2 * p) * 2, 0, 0);
        zq[u] = __builtin_amdgcn_raw_buffer_load_b16(make_rsrc(zp + (int64_t)n0 * ldq), rn * ldq + 2 * p, 0, 0);
      }
    }
  } else {
    const int rn = n0 + wave < N ? wave : N - 1 - n0;
    const auto srs = make_rsrc(sc + (int64_t)(n0 + rn) * ldq);
    const auto zrs = make_rsrc(zp + (int64_t)(n0 + rn) * ldq);
#pragma unroll
    for (int u = 0; u < RPL; ++u) {
      if (u * 64 < G) {  // uniform
        const int g = min(lane + u * 64, G - 1);
        sq[u] = __builtin_amdgcn_raw_buffer_load_b16(srs, g * 2, 0, 0);
        zq[u] = __builtin_amdgcn_raw_buffer_load_b8(zrs, g, 0, 0);
      }
    }
  }
  __builtin_amdgcn_sched_barrier(0);

  const auto wrs = make_rsrc(wq + (int64_t)n0 * ldw);
  const auto xrs = __builtin_amdgcn_make_buffer_rsrc(const_cast<f16*>(x), (short)0, x_bytes, 0x00020000);
  const int wvo = nr * ldw + quad * 16;
  // Activations of a step: load j covers rows 4j .. 4j + 3 x 256 contiguous
  // bytes (lane l: row 4j + l / 16, bytes (l % 16) * 16), eight whole cache
  // lines per instruction. (Loading each lane's own 64-byte row segment
  // directly, 16 rows x 64 bytes per instruction, took 2.3 us longer at
  // M = 16, K = N = 4096: the same bytes, twice the lines per instruction.)
  const int xvo = (lane >> 4) * ldx * 2 + (lane & 15) * 16;
  // All activation loads (L2 hits after the first workgroups) go out before
  // the weight loads (HBM): behind the weight misses they waited for slots.
  u32x4 wv[SPW], xl[SPW][4];
#pragma unroll
  for (int i = 0; i < SPW; ++i) {
    const int s = min(step_of(wave, i), nsteps - 1);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      xl[i][j] = __builtin_amdgcn_raw_buffer_load_b128(xrs, xvo, 4 * j * ldx * 2 + s * 256, 0);
  }
  u32x4 wl[2];
  if constexpr (kLineW) {
    // load h: rows 8h .. 8h + 7 x 128 bytes (lane l: row 8h + l / 8, step
    // 2 * wave + (l % 8) / 4, bytes (l % 4) * 16 of it)
    const int ls = min(2 * wave + ((lane & 7) >> 2), nsteps - 1);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int row = 8 * h + (lane >> 3);
      const int rr = n0 + row < N ? row : N - 1 - n0;
      wl[h] = __builtin_amdgcn_raw_buffer_load_b128(wrs, rr * ldw + ls * 64 + (lane & 3) * 16, 0, kWeightPolicy);
    }
  } else {
#pragma unroll
    for (int i = 0; i < SPW; ++i) {
      const int s = min(step_of(wave, i), nsteps - 1);
      wv[i] = __builtin_amdgcn_raw_buffer_load_b128(wrs, wvo, s * 64, kWeightPolicy);
    }
  }
  __builtin_amdgcn_sched_barrier(0);

  if constexpr (kPairRec) {
#pragma unroll
    for (int u = 0; u < RPL; ++u) {
      const int t = threadIdx.x + 64 * KW * u;
      if (t < 16 * G2) {
        const int row = t / G2, p = t - row * G2;
        rec[row][2 * p] = (sq[u] & 0xffffu) | ((zq[u] & 0xffu) << 16);
        rec[row][2 * p + 1] = (sq[u] >> 16) | ((zq[u] & 0xff00u) << 8);
      }
    }
  } else {
#pragma unroll
    for (int u = 0; u < RPL; ++u)
      if (u * 64 < G && lane + u * 64 < G) rec[wave][lane + u * 64] = (sq[u] & 0xffffu) | ((zq[u] & 0xffu) << 16);
  }
  __syncthreads();

  // Into operand order through the wave's own LDS rows (no barrier: a wave's
  // LDS operations complete in order): lane (r, quad) then reads piece t =
  // k step*128 + quad*32 + t*8 .. + 8 of row r. Rows are 272 bytes apart, so
  // the 16 rows of a read fall into different banks.
  uint8_t* xw = xstage[wave];
  u32x4 xv[SPW][4];
#pragma unroll
  for (int i = 0; i < SPW; ++i) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      *reinterpret_cast<u32x4*>(xw + (4 * j + (lane >> 4)) * kFrontXRow + (lane & 15) * 16) = xl[i][j];
#pragma unroll
    for (int t = 0; t < 4; ++t) xv[i][t] = *reinterpret_cast<const u32x4*>(xw + r * kFrontXRow + quad * 64 + t * 16);
  }
  if constexpr (kLineW) {
    uint8_t* ww = wstage[wave];
#pragma unroll
    for (int h = 0; h < 2; ++h)
      *reinterpret_cast<u32x4*>(ww + (8 * h + (lane >> 3)) * kFrontWRow + (lane & 7) * 16) = wl[h];
#pragma unroll
    for (int i = 0; i < 2; ++i) wv[i] = *reinterpret_cast<const u32x4*>(ww + r * kFrontWRow + i * 64 + quad * 16);
  }

  // No branch on a step's validity (a branch lets the compiler sink that
  // step's loads behind the first wait): a step past K, a repeat of the last
  // one, gets scale 0, so its weights dequantize to exact zeros.
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < SPW; ++i) {
    const int sraw = step_of(wave, i);
    const int s = min(sraw, nsteps - 1);
    const int g = (int)(((float)(s * 4 + quad) + 0.5f) * inv_cpg);  // chunk -> group (exact for these magnitudes)
    const uint32_t rq = rec[r][g];
    const f16x2 zoff = splat2((f16)(float)(1024 + (rq >> 16)));
    const f16x2 scale = splat2(sraw < nsteps ? bit_cast<f16>((uint16_t)rq) : (f16)0.0f);
#pragma unroll
    for (int t = 0; t < 4; ++t)
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(bit_cast<f16x8>(xv[i][t]), dequant8(wv[i][t], zoff, scale), acc, 0,
                                                   0, 0);
  }
  red[wave][lane] = acc;
  __syncthreads();
  // 16x16 MFMA result layout: lane l holds column l%16, rows (l/16)*4 + i.
  if (threadIdx.x < 256) {
    const int o = threadIdx.x;
    const int m = o >> 4;
    const int nc = o & 15;
    const int src = (m >> 2) * 16 + nc;
    float sum = 0.f;
#pragma unroll
    for (int w = 0; w < KW; ++w) sum += red[w][src][m & 3];
    const int n = n0 + nc;
    if (m < M && n < N) y[(int64_t)m * ldy + n] = (f16)sum;
  }
}


// ---- M <= 5: K-resident dot-product GEMV --------------------------------------
// (Measured at K = N = 4096, launch included: M = 1..5 take 3.53, 3.94, 4.58,
// 5.14, 6.09 us here against 5.78, 5.89, 5.99, 6.10, 6.13 us on the MFMA
// front kernel; from M = 6 on the per-row dot work makes it the slower one.)
//
// A lane owns CH fixed 32-element K chunks (chunk c = lane + 64*i: bytes
// [16c, 16c+16) of every weight row, so a wave reads 1 KB contiguous per row
// and load). Its activations for those chunks are loaded once and kept in
// registers, pre-paired to match the nibble decode below; each wave then
// streams RW weight rows, issuing every load of the kernel up front.
//
// Decode without per-element dequantization: for a weight dword d (8 nibbles,
// byte b = k 2b low / 2b+1 high), 0x64006400 | (d & 0x000F000F) is the f16
// pair (1024+q0, 1024+q4) and 0x64006400 | (d & 0x00F000F0) is
// (1024+16*q1, 1024+16*q5); the same on d >> 8 gives (q2, q6) and (q3, q7).
// v_dot2_f32_f16 multiplies each pair with the matching activation pair
// (products are exact in fp32), into acc1 (x1 pairs) and acc16 (x16 pairs).
// Per chunk (one quant group): sum_k x_k (q_k - z) =
//   acc1 + acc16/16 - (1024*xs1 + 64*xs16) - z*(xs1 + xs16),
// where xs1 / xs16 are the activation sums over the x1 / x16 positions; the
// result is scaled by s once per chunk. Lane partials are reduced across the
// wave with cross-lane shuffles in a fixed order.
template <int M, int CH, int RW, int WPB = 4>
__global__ __launch_bounds__(64 * WPB) void w4a16_gemv_dot_kernel(const f16* __restrict__ x, int64_t ldx, int K,
                                                             const uint8_t* __restrict__ wq, int64_t ldw,
                                                             const f16* __restrict__ sc,
                                                             const uint8_t* __restrict__ zp, int64_t ldq, int gs,
                                                             f16* __restrict__ y, int64_t ldy, int N) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int row0 = (blockIdx.x * WPB + __builtin_amdgcn_readfirstlane(wave)) * RW;
  if (row0 >= N) return;  // wave-uniform
  const int nchunks = K >> 5;

  // Every load is unconditional (chunks past K are clamped to a valid address
  // and zeroed later through their scale) and raw values are converted only
  // where they are consumed, so all loads of the wave are in flight together.
  // Issue order: activations (mostly L2 hits, needed first), then per weight
  // row its chunks, scales and zeros; vmcnt retires in order, so row r can be
  // consumed while later rows are still arriving.
  int cc[CH];
  bool cvalid[CH];
  uint32_t grp[CH];
#pragma unroll
  for (int i = 0; i < CH; ++i) {
    const int c = lane + 64 * i;
    cvalid[i] = c < nchunks;
    cc[i] = cvalid[i] ? c : nchunks - 1;
    grp[i] = (uint32_t)((cc[i] << 5) / gs);
  }
  // Buffer loads: the row bases are wave-uniform and live in scalar
  // registers; lanes add only their 32-bit chunk offsets.
  u32x4 xraw[M][CH][4];
#pragma unroll
  for (int m = 0; m < M; ++m) {
    const auto xr = make_rsrc(x + (int64_t)m * ldx);
#pragma unroll
    for (int i = 0; i < CH; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        xraw[m][i][j] = __builtin_amdgcn_raw_buffer_load_b128(xr, cc[i] * 64, j * 16, 0);
  }
  u32x4 wv[RW][CH];
  uint32_t sraw[RW][CH];
  uint32_t zraw[RW][CH];
#pragma unroll
  for (int r = 0; r < RW; ++r) {
    const int n = row0 + r < N ? row0 + r : N - 1;
    const auto wr = make_rsrc(wq + (int64_t)n * ldw);
    const auto sr = make_rsrc(sc + (int64_t)n * ldq);
    const auto zr = make_rsrc(zp + (int64_t)n * ldq);
#pragma unroll
    for (int i = 0; i < CH; ++i) wv[r][i] = __builtin_amdgcn_raw_buffer_load_b128(wr, cc[i] * 16, 0, 0);
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      sraw[r][i] = __builtin_amdgcn_raw_buffer_load_b16(sr, grp[i] * 2, 0, 0);
      zraw[r][i] = __builtin_amdgcn_raw_buffer_load_b8(zr, grp[i], 0, 0);
    }
  }
  // Keep every load above this point: the scheduler would otherwise sink some
  // of them below the first wait to save registers, adding a round trip.
  __builtin_amdgcn_sched_barrier(0);

  // Activation pairs: for weight dword j of chunk i, a1 = (x0,x4), b1 = (x2,x6)
  // meet the x1 nibble pairs, a16 = (x1,x5), b16 = (x3,x7) the x16 pairs.
  // Their sums come from v_dot2 against (1, 1).
  const f16x2 ones = splat2((f16)1.0f);
  f16x2 xa1[M][CH][4], xb1[M][CH][4], xa16[M][CH][4], xb16[M][CH][4];
  float c0[M][CH], c1[M][CH];
#pragma unroll
  for (int m = 0; m < M; ++m) {
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      float s1 = 0.f, s16 = 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const u32x4 v = xraw[m][i][j];
        xa1[m][i][j] = bit_cast<f16x2>(__builtin_amdgcn_perm(v[2], v[0], 0x05040100u));
        xa16[m][i][j] = bit_cast<f16x2>(__builtin_amdgcn_perm(v[2], v[0], 0x07060302u));
        xb1[m][i][j] = bit_cast<f16x2>(__builtin_amdgcn_perm(v[3], v[1], 0x05040100u));
        xb16[m][i][j] = bit_cast<f16x2>(__builtin_amdgcn_perm(v[3], v[1], 0x07060302u));
        s1 = __builtin_amdgcn_fdot2(xa1[m][i][j], ones, s1, false);
        s1 = __builtin_amdgcn_fdot2(xb1[m][i][j], ones, s1, false);
        s16 = __builtin_amdgcn_fdot2(xa16[m][i][j], ones, s16, false);
        s16 = __builtin_amdgcn_fdot2(xb16[m][i][j], ones, s16, false);
      }
      c0[m][i] = 1024.f * s1 + 64.f * s16;
      c1[m][i] = s1 + s16;
    }
  }

  uint32_t magic = 0x64006400u;
  asm("" : "+v"(magic));  // keep the constant in a register for v_bfi_b32
  float part[M][RW];
#pragma unroll
  for (int r = 0; r < RW; ++r) {
#pragma unroll
    for (int m = 0; m < M; ++m) part[m][r] = 0.f;
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      float acc1[M], acc16[M];
#pragma unroll
      for (int m = 0; m < M; ++m) acc1[m] = acc16[m] = 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t d = wv[r][i][j];
        const uint32_t d8 = d >> 8;
        const f16x2 lo = bit_cast<f16x2>(bfi(0x000F000Fu, d, magic));
        const f16x2 hi = bit_cast<f16x2>(bfi(0x00F000F0u, d, magic));
        const f16x2 lo8 = bit_cast<f16x2>(bfi(0x000F000Fu, d8, magic));
        const f16x2 hi8 = bit_cast<f16x2>(bfi(0x00F000F0u, d8, magic));
#pragma unroll
        for (int m = 0; m < M; ++m) {
          acc1[m] = __builtin_amdgcn_fdot2(lo, xa1[m][i][j], acc1[m], false);
          acc1[m] = __builtin_amdgcn_fdot2(lo8, xb1[m][i][j], acc1[m], false);
          acc16[m] = __builtin_amdgcn_fdot2(hi, xa16[m][i][j], acc16[m], false);
          acc16[m] = __builtin_amdgcn_fdot2(hi8, xb16[m][i][j], acc16[m], false);
        }
      }
      const float sv = (float)bit_cast<f16>((uint16_t)sraw[r][i]) * (cvalid[i] ? 1.f : 0.f);
      const float zv = (float)zraw[r][i];
#pragma unroll
      for (int m = 0; m < M; ++m) {
        const float t = (acc1[m] + acc16[m] * 0.0625f) - (c0[m][i] + zv * c1[m][i]);
        part[m][r] = __builtin_fmaf(sv, t, part[m][r]);
      }
    }
  }

  // Wave totals without LDS; lane 16R of row R writes the values it holds.
  using Red = WaveReduce<M * RW>;
  float flat[M * RW];
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int r = 0; r < RW; ++r) flat[m * RW + r] = part[m][r];
  float tot[Red::OUT];
  Red::run(flat, tot);
  const int R = lane >> 4;
  const bool writer = (lane & 15) == 0 && (Red::S16 || (R & 1) == 0) && (Red::S32 || R < 2);
  if (writer) {
#pragma unroll
    for (int j = 0; j < Red::OUT; ++j) {
      const int idx = Red::index(R, j);
      const int m = idx / RW, r = idx % RW;
      if (row0 + r < N) y[(int64_t)m * ldy + row0 + r] = (f16)tot[j];
    }
  }
}

// ---- M <= 3: dot-product GEMV with workgroup-shared operands -----------------
// The per-lane arithmetic of w4a16_gemv_dot_kernel (lane l owns chunks
// c = l + 64i of every weight row of its wave; nibble pairs decoded by v_bfi_b32
// straight into v_dot2_f32_f16 operands), with everything the waves of a
// workgroup have in common loaded once per workgroup instead of once per wave:
// * activations: thread t loads the 16-byte pieces (m, c, j) = t, t + NTH, ...
//   (j = dword-quad of chunk c), permutes each into the four v_dot2 operand
//   pairs and stores them to LDS as xp[m][j][c]; the chunk sums
//   c0 = 1024*xs1 + 64*xs16 and c1 = xs1 + xs16 are reduced over the four
//   pieces of a chunk (four adjacent lanes) with DPP into xs[m][c];
// * scales and zeros of the workgroup's R weight rows (G = K/gs groups each):
//   thread t loads one dword of scales and one u16 of zeros (a pair of groups)
//   per item and stores (scale bits | zero << 16) records rec[r][g] to LDS.
// Issue order: activation pieces, scale/zero pairs, then all weight loads of
// the wave. vmcnt retires in order, so the producer step waits only for the
// first two kinds while the weights keep streaming from HBM. Measured at
// K = N = 4096 this cuts the load instructions per wave from 32 to 12.
// Arguments are ordered so that everything the loads need sits in the first
// 16 kernarg dwords, which the library preloads into SGPRs.
template <int M, int CH, int RW, int WPB, int QI>
__global__ __launch_bounds__(64 * WPB) void w4a16_gemv_dot_shared_kernel(
    const f16* __restrict__ x, const uint8_t* __restrict__ wq, const f16* __restrict__ sc,
    const uint8_t* __restrict__ zp, int ldw, int ldq, int K, int G2, int N, float inv_g2, int ldx, float inv_cpg,
    f16* __restrict__ y, int ldy) {
  constexpr int NTH = 64 * WPB;
  constexpr int R = RW * WPB;    // weight rows per workgroup
  constexpr int CMAX = 64 * CH;  // chunk capacity: K <= 32 * CMAX
  constexpr int XI = (M * CMAX * 4 + NTH - 1) / NTH;
  __shared__ u32x4 xp[M][4][CMAX];
  __shared__ f32x2 xs[M][CMAX];
  __shared__ uint32_t rec[R][CMAX];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int rbase = blockIdx.x * R;
  const int nchunks = K >> 5;

  // Producer loads: activation pieces, then scale/zero pairs.
  u32x4 xr[XI];
  bool xok[XI];
#pragma unroll
  for (int i = 0; i < XI; ++i) {
    const int item = tid + i * NTH;
    const int m = item / (4 * CMAX);
    const int rem = item % (4 * CMAX);
    const bool ok = m < M && (rem >> 2) < nchunks;
    xok[i] = ok;
    // one buffer over x, per-lane byte offsets (a per-lane resource would
    // need a waterfall loop)
    xr[i] = __builtin_amdgcn_raw_buffer_load_b128(make_rsrc(x), ok ? m * ldx * 2 + rem * 16 : 0, 0, 0);
  }
  uint32_t sq[QI], zq[QI];
  int qr[QI], qp[QI];
  const auto srs = make_rsrc(sc + (int64_t)rbase * ldq);
  const auto zrs = make_rsrc(zp + (int64_t)rbase * ldq);
#pragma unroll
  for (int i = 0; i < QI; ++i) {
    const int item = tid + i * NTH;
    int r = (int)(((float)item + 0.5f) * inv_g2);  // item / G2 (exact for these magnitudes)
    r = r < R ? r : R - 1;
    const int p = item - r * G2;
    qr[i] = r;
    qp[i] = p;
    const int n = (rbase + r < N ? r : N - 1 - rbase);
    // items past the records read offset 0; a mask rather than a select keeps
    // the address math branch-free, so the weight loads issue sooner
    const int keep = -(int)(p < G2);
    sq[i] = __builtin_amdgcn_raw_buffer_load_b32(srs, (n * ldq * 2 + p * 4) & keep, 0, 0);
    zq[i] = __builtin_amdgcn_raw_buffer_load_b16(zrs, (n * ldq + p * 2) & keep, 0, 0);
  }

  // Weight loads of this wave.
  const int row0 = rbase + wave * RW;
  int cc[CH];
#pragma unroll
  for (int i = 0; i < CH; ++i) {
    const int c = lane + 64 * i;
    cc[i] = c < nchunks ? c : nchunks - 1;  // past K: a valid row address, zero activations
  }
  u32x4 wv[RW][CH];
#pragma unroll
  for (int r = 0; r < RW; ++r) {
    const int n = row0 + r < N ? row0 + r : N - 1;
    const auto wr = make_rsrc(wq + (int64_t)n * ldw);
#pragma unroll
    for (int i = 0; i < CH; ++i)
      wv[r][i] = __builtin_amdgcn_raw_buffer_load_b128(wr, cc[i] * 16, 0, kWeightPolicy);
  }
  __builtin_amdgcn_sched_barrier(0);

  // Producer step: activation pairs and chunk sums, scale/zero records.
  const f16x2 ones = splat2((f16)1.0f);
#pragma unroll
  for (int i = 0; i < XI; ++i) {
    const int item = tid + i * NTH;
    const int m = item / (4 * CMAX);
    const int c = (item >> 2) % CMAX;
    const int j = item & 3;
    // chunks past K get zero activations: their products and sums vanish
    const u32x4 v = xok[i] ? xr[i] : u32x4{0u, 0u, 0u, 0u};
    const uint32_t a1 = __builtin_amdgcn_perm(v[2], v[0], 0x05040100u);
    const uint32_t a16 = __builtin_amdgcn_perm(v[2], v[0], 0x07060302u);
    const uint32_t b1 = __builtin_amdgcn_perm(v[3], v[1], 0x05040100u);
    const uint32_t b16 = __builtin_amdgcn_perm(v[3], v[1], 0x07060302u);
    float s1 = __builtin_amdgcn_fdot2(bit_cast<f16x2>(a1), ones, 0.f, false);
    s1 = __builtin_amdgcn_fdot2(bit_cast<f16x2>(b1), ones, s1, false);
    float s16 = __builtin_amdgcn_fdot2(bit_cast<f16x2>(a16), ones, 0.f, false);
    s16 = __builtin_amdgcn_fdot2(bit_cast<f16x2>(b16), ones, s16, false);
    s1 += dpp_f32<0xB1>(s1);  // quad_perm [1,0,3,2]
    s16 += dpp_f32<0xB1>(s16);
    s1 += dpp_f32<0x4E>(s1);  // quad_perm [2,3,0,1]
    s16 += dpp_f32<0x4E>(s16);
    if (m < M) {
      xp[m][j][c] = u32x4{a1, b1, a16, b16};
      if (j == 0) xs[m][c] = f32x2{1024.f * s1 + 64.f * s16, s1 + s16};
    }
  }
#pragma unroll
  for (int i = 0; i < QI; ++i) {
    if (qp[i] < G2 && tid + i * NTH < R * G2) {
      const uint32_t lo = (sq[i] & 0xffffu) | ((zq[i] & 0xffu) << 16);
      const uint32_t hi = (sq[i] >> 16) | ((zq[i] & 0xff00u) << 8);
      *reinterpret_cast<u32x2*>(&rec[qr[i]][2 * qp[i]]) = u32x2{lo, hi};
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  __syncthreads();
  __builtin_amdgcn_sched_barrier(0);

  f16x2 xa1[M][CH][4], xb1[M][CH][4], xa16[M][CH][4], xb16[M][CH][4];
  float c0[M][CH], c1[M][CH];
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int i = 0; i < CH; ++i) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const u32x4 v = xp[m][j][lane + 64 * i];  // zero past K
        xa1[m][i][j] = bit_cast<f16x2>(v[0]);
        xb1[m][i][j] = bit_cast<f16x2>(v[1]);
        xa16[m][i][j] = bit_cast<f16x2>(v[2]);
        xb16[m][i][j] = bit_cast<f16x2>(v[3]);
      }
      const f32x2 t = xs[m][lane + 64 * i];
      c0[m][i] = t[0];
      c1[m][i] = t[1];
    }
  uint32_t qrec[RW][CH];
#pragma unroll
  for (int i = 0; i < CH; ++i) {
    const int g = (int)(((float)cc[i] + 0.5f) * inv_cpg);  // chunk -> group (exact for these magnitudes)
#pragma unroll
    for (int r = 0; r < RW; ++r) qrec[r][i] = rec[wave * RW + r][g];
  }
  // Every LDS operand is in registers before the first weight is needed:
  // left to itself the scheduler interleaves these reads with the dot
  // products, each behind its own lgkmcnt wait, and their latency then
  // lands after the weights arrive, on the kernel's critical path.
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
  __builtin_amdgcn_sched_barrier(0);

  uint32_t magic = 0x64006400u, mhi = 0x54005400u;
  asm("" : "+v"(magic));  // keep the constants in registers for v_bfi_b32
  asm("" : "+v"(mhi));
  float part[M][RW];
#pragma unroll
  for (int r = 0; r < RW; ++r) {
#pragma unroll
    for (int m = 0; m < M; ++m) part[m][r] = 0.f;
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      float acc1[M], acc16[M];
#pragma unroll
      for (int m = 0; m < M; ++m) acc1[m] = acc16[m] = 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t d = wv[r][i][j];
        const uint32_t d8 = d >> 8;
        const f16x2 lo = bit_cast<f16x2>(bfi(0x000F000Fu, d, magic));
        const f16x2 hi = bit_cast<f16x2>(bfi(0x00F000F0u, d, mhi));   // 64 + q
        const f16x2 lo8 = bit_cast<f16x2>(bfi(0x000F000Fu, d8, magic));
        const f16x2 hi8 = bit_cast<f16x2>(bfi(0x00F000F0u, d8, mhi));
#pragma unroll
        for (int m = 0; m < M; ++m) {
          acc1[m] = __builtin_amdgcn_fdot2(lo, xa1[m][i][j], acc1[m], false);
          acc1[m] = __builtin_amdgcn_fdot2(lo8, xb1[m][i][j], acc1[m], false);
          acc16[m] = __builtin_amdgcn_fdot2(hi, xa16[m][i][j], acc16[m], false);
          acc16[m] = __builtin_amdgcn_fdot2(hi8, xb16[m][i][j], acc16[m], false);
        }
      }
      const float sv = (float)bit_cast<f16>((uint16_t)qrec[r][i]);
      const float zv = (float)(qrec[r][i] >> 16);
#pragma unroll
      for (int m = 0; m < M; ++m) {
        const float t = (acc1[m] + acc16[m]) - __builtin_fmaf(zv, c1[m][i], c0[m][i]);
        part[m][r] = __builtin_fmaf(sv, t, part[m][r]);
      }
    }
  }

  using Red = WaveReduce<M * RW>;
  float flat[M * RW];
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int r = 0; r < RW; ++r) flat[m * RW + r] = part[m][r];
  float tot[Red::OUT];
  Red::run(flat, tot);
  const int Rr = lane >> 4;
  const bool writer = (lane & 15) == 0 && (Red::S16 || (Rr & 1) == 0) && (Red::S32 || Rr < 2);
  if (writer) {
#pragma unroll
    for (int j = 0; j < Red::OUT; ++j) {
      const int idx = Red::index(Rr, j);
      const int m = idx / RW, r = idx % RW;
      if (row0 + r < N) y[(int64_t)m * ldy + row0 + r] = (f16)tot[j];
    }
  }
}

template <int M, int CH, int RW, int WPB, int QI>
void launch_dot_shared(const f16* x, int64_t ldx, int K, const uint8_t* wq, int64_t ldw, const f16* sc,
                       const uint8_t* zp, int64_t ldq, int gs, f16* y, int64_t ldy, int N, hipStream_t st) {
  constexpr int R = RW * WPB;
  const int blocks = (N + R - 1) / R;
  const int G2 = K / gs / 2;
  hipLaunchKernelGGL((w4a16_gemv_dot_shared_kernel<M, CH, RW, WPB, QI>), dim3(blocks), dim3(64 * WPB), 0, st, x, wq,
                     sc, zp, (int)ldw, (int)ldq, K, G2, N, 1.0f / (float)G2, (int)ldx, 32.0f / (float)gs, y, (int)ldy);
}

template <int M, int CH>
void launch_dot(const f16* x, int64_t ldx, int K, const uint8_t* wq, int64_t ldw, const f16* sc, const uint8_t* zp,
                int64_t ldq, int gs, f16* y, int64_t ldy, int N, hipStream_t st) {
  constexpr int RW = CH >= 8 ? 1 : 8 / CH;  // eight 16-byte weight loads per lane
  const int waves = (N + RW - 1) / RW;
  const int blocks = (waves + 3) / 4;
  hipLaunchKernelGGL((w4a16_gemv_dot_kernel<M, CH, RW>), dim3(blocks), dim3(256), 0, st, x, ldx, K, wq, ldw, sc, zp,
                     ldq, gs, y, ldy, N);
}



// Picks the chunk count CH (K <= 2048*CH) for the dot kernel; returns false if
// M*CH exceeds the register budget.
template <int M>
bool dispatch_dot(const f16* x, int64_t ldx, int K, const uint8_t* wq, int64_t ldw, const f16* sc, const uint8_t* zp,
                  int64_t ldq, int gs, f16* y, int64_t ldy, int N, hipStream_t st) {
  const int ch = (K + 2047) / 2048;
  if (ch <= 1) {
    launch_dot<M, 1>(x, ldx, K, wq, ldw, sc, zp, ldq, gs, y, ldy, N, st);
    return true;
  }
  if (ch <= 2) {
    launch_dot<M, 2>(x, ldx, K, wq, ldw, sc, zp, ldq, gs, y, ldy, N, st);
    return true;
  }
  if constexpr (M <= 2) {
    if (ch <= 4) {
      launch_dot<M, 4>(x, ldx, K, wq, ldw, sc, zp, ldq, gs, y, ldy, N, st);
      return true;
    }
  }
  if constexpr (M == 1) {
    if (ch <= 8) {
      launch_dot<M, 8>(x, ldx, K, wq, ldw, sc, zp, ldq, gs, y, ldy, N, st);
      return true;
    }
  }
  return false;
}


// The workgroup-shared dot kernel with four weight rows per wave and four
// waves (one per SIMD). Measured at K = N = 4096 against two rows x eight
// waves: M = 1..5 take 3.24, 3.69, 4.49, 5.00, 6.00 us against 3.37, 3.74,
// 4.49, 5.14, 6.06 us (every weight load is still issued up front; a lone
// wave per SIMD works through its rows as they arrive without sharing the
// SIMD with a second wave's dot products). CH chunks per lane as dispatch_dot, QI scale/zero pairs per thread. Scales
// and zeros are read as group pairs (a dword of scales, a u16 of zeros), so
// the group count must be even and the rows aligned; returns false otherwise.
template <int M, int CH>
bool launch_shared_qi(const f16* x, int64_t ldx, int K, const uint8_t* wq, int64_t ldw, const f16* sc,
                      const uint8_t* zp, int64_t ldq, int gs, f16* y, int64_t ldy, int N, hipStream_t st) {
  const int G = K / gs;
  if (G <= 32) {
    launch_dot_shared<M, CH, 4, 4, 1>(x, ldx, K, wq, ldw, sc, zp, ldq, gs, y, ldy, N, st);
  } else if (G <= 64) {
    launch_dot_shared<M, CH, 4, 4, 2>(x, ldx, K, wq, ldw, sc, zp, ldq, gs, y, ldy, N, st);
  } else if (G <= 128) {
    launch_dot_shared<M, CH, 4, 4, 4>(x, ldx, K, wq, ldw, sc, zp, ldq, gs, y, ldy, N, st);
  } else if (G <= 256) {
    launch_dot_shared<M, CH, 4, 4, 8>(x, ldx, K, wq, ldw, sc, zp, ldq, gs, y, ldy, N, st);
  } else {
    return false;
  }
  return true;
}

template <int M>
bool dispatch_dot_shared(const f16* x, int64_t ldx, int K, const uint8_t* wq, int64_t ldw, const f16* sc,
                         const uint8_t* zp, int64_t ldq, int gs, f16* y, int64_t ldy, int N, hipStream_t st) {
  if ((K / gs) % 2 != 0 || ldq % 2 != 0 || (reinterpret_cast<uintptr_t>(sc) & 3) != 0 ||
      (reinterpret_cast<uintptr_t>(zp) & 1) != 0)
    return false;
  const int ch = (K + 2047) / 2048;
  if (ch <= 1) return launch_shared_qi<M, 1>(x, ldx, K, wq, ldw, sc, zp, ldq, gs, y, ldy, N, st);
  if (ch <= 2) return launch_shared_qi<M, 2>(x, ldx, K, wq, ldw, sc, zp, ldq, gs, y, ldy, N, st);
  if constexpr (M <= 2) {
    if (ch <= 4) return launch_shared_qi<M, 4>(x, ldx, K, wq, ldw, sc, zp, ldq, gs, y, ldy, N, st);
  }
  if constexpr (M == 1) {
    if (ch <= 8) return launch_shared_qi<M, 8>(x, ldx, K, wq, ldw, sc, zp, ldq, gs, y, ldy, N, st);
  }
  return false;
}


// ---- W8A16 GEMV (M <= 16) ----------------------------------------------------
// Same split as the W4 MFMA GEMV: a workgroup owns 16 weight rows, its KW
// waves take 64-wide K steps in turn. Lane (r = lane%16, quad = lane/16) loads
// 16 int8 weights of row n0+r (k = step*64 + quad*16 ..) and the matching 16
// activations of row r; two v_mfma_f32_16x16x32_f16 cover the step. The int8 ->
// f16 conversion is exact; the channel scale multiplies the fp32 sum once.
template <int KW>
__global__ __launch_bounds__(64 * KW) void w8a16_gemv_kernel(const f16* __restrict__ x, int64_t ldx, int M, int K,
                                                             const int8_t* __restrict__ w, int64_t ldw,
                                                             const f16* __restrict__ sc, f16* __restrict__ y,
                                                             int64_t ldy, int N) {
  __shared__ f32x4 red[KW][64];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int r = lane & 15;
  const int quad = lane >> 4;
  const int n_base = blockIdx.x * 16;
  const int n = n_base + r < N ? n_base + r : N - 1;
  const int8_t* wrow = w + (int64_t)n * ldw + quad * 16;
  const f16* xrow = x + (int64_t)(r < M ? r : M - 1) * ldx + quad * 16;
  const int nsteps = K >> 6;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int s = wave; s < nsteps; s += KW) {
    const u32x4 wv = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wrow + (int64_t)s * 64));  // read once
    const u32x4 x0 = load16(xrow + (int64_t)s * 64);
    const u32x4 x1 = load16(xrow + (int64_t)s * 64 + 8);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(bit_cast<f16x8>(x0), int8x8_to_f16(wv[0], wv[1]), acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(bit_cast<f16x8>(x1), int8x8_to_f16(wv[2], wv[3]), acc, 0, 0, 0);
  }
  red[wave][lane] = acc;
  __syncthreads();
  // 16x16 MFMA result layout: lane l holds column l%16, rows (l/16)*4 + i.
  for (int o = threadIdx.x; o < 256; o += 64 * KW) {
    const int m = o >> 4;
    const int nc = o & 15;
    const int src = (m >> 2) * 16 + nc;
    float sum = 0.f;
#pragma unroll
    for (int ww = 0; ww < KW; ++ww) sum += red[ww][src][m & 3];
    const int nn = n_base + nc;
    if (m < M && nn < N) y[(int64_t)m * ldy + nn] = (f16)(sum * (float)sc[nn]);
  }
}

template <int SPW>
void launch_front(const f16* x, int64_t ldx, int M, int K, const uint8_t* wq, int64_t ldw, const f16* sc,
                  const uint8_t* zp, int64_t ldq, int gs, f16* y, int64_t ldy, int N, hipStream_t st) {
  const int x_bytes = (int)(((int64_t)(M - 1) * ldx + K) * 2);
  const bool pair = (K / gs) % 2 == 0 && ldq % 2 == 0 && (reinterpret_cast<uintptr_t>(sc) & 3) == 0 &&
                    (reinterpret_cast<uintptr_t>(zp) & 1) == 0;
  if (pair)
    hipLaunchKernelGGL((w4a16_gemv_front_kernel<16, SPW, true>), dim3((N + 15) / 16), dim3(1024), 0, st, x, (int)ldx,
                       x_bytes, wq, (int)ldw, sc, zp, (int)ldq, K / 128, K / gs, 32.0f / (float)gs, N, y, (int)ldy, M);
  else
    hipLaunchKernelGGL((w4a16_gemv_front_kernel<16, SPW, false>), dim3((N + 15) / 16), dim3(1024), 0, st, x,
                       (int)ldx, x_bytes, wq, (int)ldw, sc, zp, (int)ldq, K / 128, K / gs, 32.0f / (float)gs, N, y,
                       (int)ldy, M);
}

template <int NT, int KW>
void launch_gemv(const f16* x, int64_t ldx, int M, int K, const uint8_t* wq, int64_t ldw, const f16* sc,
                 const uint8_t* zp, int64_t ldq, int gs, f16* y, int64_t ldy, int N, hipStream_t st) {
  const int tiles = (N + 16 * NT - 1) / (16 * NT);
  hipLaunchKernelGGL((w4a16_gemv_kernel<NT, KW>), dim3(tiles), dim3(64 * KW), 0, st, x, ldx, M, K, wq, ldw, sc, zp,
                     ldq, gs, y, ldy, N);
}

// ---- the reference's own W4 layout, read in place (M <= 5) -------------------
// weight_only_int4_matmul (examples/kernels/contraction/weight_only_int4.py:18-51):
// packed int32 [K/8, N], word (r, n) holding k = 8r .. 8r+7 of column n at
// nibble k % 8 (signed, two's complement), scales f16 [K/64, N];
//   y[m, n] = f16(sum_k x[m, k] * (signed(k, n) * s[k/64, n])).
// A word has the nibble order of a dword of the [N, K/2] layout, so the
// decode above applies unchanged: d ^ 0x88888888 turns the signed nibbles
// into q' = q + 8 (the zero point is 8) and the bfi pairs feed v_dot2 with the
// activation pairs of the workgroup-shared x stage. Each workgroup owns 4 CS
// columns; lane t takes the four columns 4 (t % CS) .. of them and the 64-k
// groups t / CS + 64 i (the eight words of a group are its eight loads), so
// one load instruction covers 64 / CS k-rows x 16 CS contiguous bytes.
// Workgroups are numbered XCD-major (xcd_swizzle), so the two workgroups that
// share a 128-byte line of a k-row meet in one L2. Partial sums are reduced
// over the lanes of a column set with shuffles in a fixed order, then over the
// waves in wave order. The layout puts consecutive k-rows of a column strip
// N * 4 bytes apart, which a strip's reads cannot turn into whole DRAM pages:
// 5.9 us at M = 1, K = N = 4096, against 3.4 us for the [N, K/2] layout (and
// 17.9 us with the per-call repack the kernel replaces).
template <int M, int GPL, int CS>
__global__ __launch_bounds__(64 * CS) void w4a16_sym_gemv_kernel(const f16* __restrict__ x, int ldx, int K,
                                                                const int32_t* __restrict__ wq, int ldw,
                                                                const f16* __restrict__ sc, int lds, int N,
                                                                f16* __restrict__ y, int ldy) {
  constexpr int NTH = 64 * CS;     // CS column sets of four columns x 64 group slots
  constexpr int NW = NTH / 64;
  constexpr int NC = 4 * CS;       // columns per workgroup
  constexpr int CMAX = 128 * GPL;  // 32-k chunks: K <= 64 * 64 * GPL
  constexpr int XI = (M * CMAX * 4 + NTH - 1) / NTH;
  __shared__ u32x4 xp[M][4][CMAX];
  __shared__ f32x2 xs[M][CMAX];
  __shared__ float red[NW][M][NC];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int nchunks = K >> 5;
  const int G = K >> 6;
  const int n0 = xcd_swizzle(blockIdx.x, gridDim.x) * NC;
  const int cg = tid % CS;
  const int nc = n0 + 4 * cg;
  const int ncl = nc + 3 < N ? nc : N - 4;  // column set past N: a valid address, never stored

  // Activation pieces first (needed for the x stage), then every weight load.
  u32x4 xr[XI];
  bool xok[XI];
#pragma unroll
  for (int i = 0; i < XI; ++i) {
    const int item = tid + i * NTH;
    const int m = item / (4 * CMAX);
    const int rem = item % (4 * CMAX);
    const bool ok = m < M && (rem >> 2) < nchunks;
    xok[i] = ok;
    xr[i] = __builtin_amdgcn_raw_buffer_load_b128(make_rsrc(x), ok ? m * ldx * 2 + rem * 16 : 0, 0, 0);
  }
  u32x4 wv[GPL][8];
  uint32_t sraw[GPL][2];
  bool gok[GPL];
  const auto wr = make_rsrc(wq + ncl);
  const auto sr = make_rsrc(sc + ncl);
#pragma unroll
  for (int u = 0; u < GPL; ++u) {
    const int g = tid / CS + 64 * u;
    gok[u] = g < G;
    const int gg = gok[u] ? g : 0;
#pragma unroll
    for (int r = 0; r < 8; ++r) wv[u][r] = __builtin_amdgcn_raw_buffer_load_b128(wr, (gg * 8 + r) * ldw * 4, 0, 0);
    const u32x2 s2 = __builtin_amdgcn_raw_buffer_load_b64(sr, gg * lds * 2, 0, 0);
    sraw[u][0] = s2[0];
    sraw[u][1] = s2[1];
  }
  __builtin_amdgcn_sched_barrier(0);

  // x stage: activation pairs for v_dot2 and the chunk sums, as in the
  // [N, K/2] decode kernel above.
  const f16x2 ones = splat2((f16)1.0f);
#pragma unroll
  for (int i = 0; i < XI; ++i) {
    const int item = tid + i * NTH;
    const int m = item / (4 * CMAX);
    const int c = (item >> 2) % CMAX;
    const int j = item & 3;
    const u32x4 v = xok[i] ? xr[i] : u32x4{0u, 0u, 0u, 0u};
    const uint32_t a1 = __builtin_amdgcn_perm(v[2], v[0], 0x05040100u);
    const uint32_t a16 = __builtin_amdgcn_perm(v[2], v[0], 0x07060302u);
    const uint32_t b1 = __builtin_amdgcn_perm(v[3], v[1], 0x05040100u);
    const uint32_t b16 = __builtin_amdgcn_perm(v[3], v[1], 0x07060302u);
    float s1 = __builtin_amdgcn_fdot2(bit_cast<f16x2>(a1), ones, 0.f, false);
    s1 = __builtin_amdgcn_fdot2(bit_cast<f16x2>(b1), ones, s1, false);
    float s16 = __builtin_amdgcn_fdot2(bit_cast<f16x2>(a16), ones, 0.f, false);
    s16 = __builtin_amdgcn_fdot2(bit_cast<f16x2>(b16), ones, s16, false);
    s1 += dpp_f32<0xB1>(s1);
    s16 += dpp_f32<0xB1>(s16);
    s1 += dpp_f32<0x4E>(s1);
    s16 += dpp_f32<0x4E>(s16);
    if (m < M) {
      xp[m][j][c] = u32x4{a1, b1, a16, b16};
      if (j == 0) xs[m][c] = f32x2{1024.f * s1 + 64.f * s16, s1 + s16};
    }
  }
  __syncthreads();

  uint32_t magic = 0x64006400u, mhi = 0x54005400u;
  asm("" : "+v"(magic));
  asm("" : "+v"(mhi));
  float part[M][4];
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) part[m][jj] = 0.f;
#pragma unroll
  for (int u = 0; u < GPL; ++u) {
    if (!gok[u]) continue;
    const int g = tid / CS + 64 * u;
    float sv[4];
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) sv[jj] = (float)bit_cast<f16>((uint16_t)(sraw[u][jj >> 1] >> (16 * (jj & 1))));
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int c = 2 * g + h;
      float acc1[M][4], acc16[M][4];
#pragma unroll
      for (int m = 0; m < M; ++m)
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) acc1[m][jj] = acc16[m][jj] = 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        u32x4 xv[M];
#pragma unroll
        for (int m = 0; m < M; ++m) xv[m] = xp[m][j][c];
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const uint32_t d = wv[u][4 * h + j][jj] ^ 0x88888888u;
          const uint32_t d8 = d >> 8;
          const f16x2 lo = bit_cast<f16x2>(bfi(0x000F000Fu, d, magic));
          const f16x2 hi = bit_cast<f16x2>(bfi(0x00F000F0u, d, mhi));
          const f16x2 lo8 = bit_cast<f16x2>(bfi(0x000F000Fu, d8, magic));
          const f16x2 hi8 = bit_cast<f16x2>(bfi(0x00F000F0u, d8, mhi));
#pragma unroll
          for (int m = 0; m < M; ++m) {
            acc1[m][jj] = __builtin_amdgcn_fdot2(lo, bit_cast<f16x2>(xv[m][0]), acc1[m][jj], false);
            acc1[m][jj] = __builtin_amdgcn_fdot2(lo8, bit_cast<f16x2>(xv[m][1]), acc1[m][jj], false);
            acc16[m][jj] = __builtin_amdgcn_fdot2(hi, bit_cast<f16x2>(xv[m][2]), acc16[m][jj], false);
            acc16[m][jj] = __builtin_amdgcn_fdot2(hi8, bit_cast<f16x2>(xv[m][3]), acc16[m][jj], false);
          }
        }
      }
#pragma unroll
      for (int m = 0; m < M; ++m) {
        const f32x2 cs = xs[m][c];
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const float t = (acc1[m][jj] + acc16[m][jj]) - __builtin_fmaf(8.f, cs[1], cs[0]);
          part[m][jj] = __builtin_fmaf(sv[jj], t, part[m][jj]);
        }
      }
    }
  }
  // Over the 64 / CS lanes of a column set within the wave, then over the waves.
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      float v = part[m][jj];
#pragma unroll
      for (int d = CS; d < 64; d <<= 1) v += __shfl_xor(v, d);
      part[m][jj] = v;
    }
  if (lane < CS) {
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) red[wave][m][4 * lane + jj] = part[m][jj];
  }
  __syncthreads();
  if (tid < NC * M) {
    const int m = tid / NC, col = tid % NC;
    float v = red[0][m][col];
#pragma unroll
    for (int w = 1; w < NW; ++w) v += red[w][m][col];
    if (n0 + col < N) y[(int64_t)m * ldy + n0 + col] = (f16)v;
  }
}

// Four column sets (16 columns, 256 lanes) per workgroup: 32 columns (whole
// 128-byte lines per k-row, 512 lanes, half the workgroups) measured 9.68 vs
// 5.92 us at M = 1, K = N = 4096.
constexpr int kSymCS = 4;

template <int M>
void launch_sym(const f16* x, int64_t ldx, int K, const int32_t* wq, int64_t ldw, const f16* sc, int64_t lds, int N,
                f16* y, int64_t ldy, hipStream_t st) {
  const dim3 grid((unsigned)((N + 4 * kSymCS - 1) / (4 * kSymCS)));
  if (K <= 4096)
    hipLaunchKernelGGL((w4a16_sym_gemv_kernel<M, 1, kSymCS>), grid, dim3(64 * kSymCS), 0, st, x, (int)ldx, K, wq,
                       (int)ldw, sc, (int)lds, N, y, (int)ldy);
  else
    hipLaunchKernelGGL((w4a16_sym_gemv_kernel<M, 2, kSymCS>), grid, dim3(64 * kSymCS), 0, st, x, (int)ldx, K, wq,
                       (int)ldw, sc, (int)lds, N, y, (int)ldy);
}

}  // namespace

namespace intent {

// Validity of a W4A16 call (any shape the operator defines: K even and a
// multiple of the group size). The tiled kernels also need w4a16_fast.
int w4a16_check(const void* x, int64_t M, int64_t K, int64_t x_ld, const uint8_t* packed, int64_t N,
                int64_t packed_ld, const void* scales, const uint8_t* zeros, int64_t qparam_ld, int64_t gs,
                const void* y, int64_t y_ld) {
  INTENT_REQUIRE(M >= 0 && N >= 0 && K >= 0, INTENT_ERR_INVALID_ARGUMENT, "negative extent (M=%lld N=%lld K=%lld)",
                 (long long)M, (long long)N, (long long)K);
  INTENT_REQUIRE(M <= INT32_MAX && N <= INT32_MAX && K <= INT32_MAX, INTENT_ERR_UNSUPPORTED, "extent exceeds int32");
  INTENT_REQUIRE(gs > 0, INTENT_ERR_INVALID_ARGUMENT, "group_size must be positive, got %lld", (long long)gs);
  INTENT_REQUIRE(K % 2 == 0 && K % gs == 0, INTENT_ERR_INVALID_ARGUMENT,
                 "K must be even and a multiple of group_size (K=%lld group=%lld)", (long long)K, (long long)gs);
  if (M == 0 || N == 0) return INTENT_OK;
  // an empty K reads no operand (y = 0, on the generic kernel): they may be null
  INTENT_REQUIRE(y && (K == 0 || (x && packed && scales && zeros)), INTENT_ERR_INVALID_ARGUMENT,
                 "null pointer argument");
  INTENT_REQUIRE(x_ld >= K && packed_ld >= K / 2 && qparam_ld >= K / gs && y_ld >= N, INTENT_ERR_INVALID_ARGUMENT,
                 "leading stride smaller than the row (x_ld=%lld packed_ld=%lld qparam_ld=%lld y_ld=%lld)",
                 (long long)x_ld, (long long)packed_ld, (long long)qparam_ld, (long long)y_ld);
  return INTENT_OK;
}

// Shapes the GEMV and tiled GEMM kernels take: whole 128-k steps, groups of
// 32 k or more, 16-byte aligned activation and weight rows.
bool w4a16_fast(const void* x, int64_t K, int64_t x_ld, const uint8_t* packed, int64_t packed_ld, int64_t gs) {
  return gs % 32 == 0 && K % 128 == 0 && K > 0 && aligned16(x) && aligned16(packed) && x_ld % 8 == 0 &&
         packed_ld % 16 == 0;
}

int w4a16_gemv_launch(const void* x, int64_t M, int64_t K, int64_t x_ld, const uint8_t* packed, int64_t N,
                      int64_t packed_ld, const void* scales, const uint8_t* zeros, int64_t qparam_ld, int64_t gs,
                      void* y, int64_t y_ld, void* stream) {
  INTENT_REQUIRE(M <= 16, INTENT_ERR_UNSUPPORTED, "the GEMV kernel covers M <= 16, got M=%lld", (long long)M);
  if (M == 0 || N == 0) return INTENT_OK;
  hipStream_t st = (hipStream_t)stream;
  const f16* xx = (const f16*)x;
  const f16* ss = (const f16*)scales;
  f16* yy = (f16*)y;
  bool done = false;
  switch (M) {
    case 1: done = dispatch_dot_shared<1>(xx, x_ld, (int)K, packed, packed_ld, ss, zeros, qparam_ld, (int)gs, yy, y_ld, (int)N, st); break;
    case 2: done = dispatch_dot_shared<2>(xx, x_ld, (int)K, packed, packed_ld, ss, zeros, qparam_ld, (int)gs, yy, y_ld, (int)N, st); break;
    case 3: done = dispatch_dot_shared<3>(xx, x_ld, (int)K, packed, packed_ld, ss, zeros, qparam_ld, (int)gs, yy, y_ld, (int)N, st); break;
    case 4: done = dispatch_dot_shared<4>(xx, x_ld, (int)K, packed, packed_ld, ss, zeros, qparam_ld, (int)gs, yy, y_ld, (int)N, st); break;
    case 5: done = dispatch_dot_shared<5>(xx, x_ld, (int)K, packed, packed_ld, ss, zeros, qparam_ld, (int)gs, yy, y_ld, (int)N, st); break;
    default: break;
  }
  if (done) {
    const int ch = (int)((K + 2047) / 2048);
    const int chv = ch <= 1 ? 1 : ch <= 2 ? 2 : ch <= 4 ? 4 : 8;
    const int64_t G = K / gs;
    return launch_status_fmt("w4a16_gemv_dot_shared_kernel<%d, %d, 4, 4, %d>", (int)M, chv,
                             G <= 32 ? 1 : G <= 64 ? 2 : G <= 128 ? 4 : 8);
  }
  if (!done) switch (M) {
    case 1: done = dispatch_dot<1>(xx, x_ld, (int)K, packed, packed_ld, ss, zeros, qparam_ld, (int)gs, yy, y_ld, (int)N, st); break;
    case 2: done = dispatch_dot<2>(xx, x_ld, (int)K, packed, packed_ld, ss, zeros, qparam_ld, (int)gs, yy, y_ld, (int)N, st); break;
    case 3: done = dispatch_dot<3>(xx, x_ld, (int)K, packed, packed_ld, ss, zeros, qparam_ld, (int)gs, yy, y_ld, (int)N, st); break;
    default: break;
  }
  if (done) {
    const int ch = (int)((K + 2047) / 2048);
    const int chv = ch <= 1 ? 1 : ch <= 2 ? 2 : ch <= 4 ? 4 : 8;
    return launch_status_fmt("w4a16_gemv_dot_kernel<%d, %d, %d, 4>", (int)M, chv, chv >= 8 ? 1 : 8 / chv);
  }
  const int steps = (int)(K / 128);
  if (fits_offset(M, x_ld * 2) && fits_offset(N, packed_ld) && fits_offset(N, qparam_ld * 2) && steps <= 64 &&
      K / gs <= kFrontMaxGroups) {
    if (steps <= 16)
      launch_front<1>(xx, x_ld, (int)M, (int)K, packed, packed_ld, ss, zeros, qparam_ld, (int)gs, yy, y_ld, (int)N, st);
    else if (steps <= 32)
      launch_front<2>(xx, x_ld, (int)M, (int)K, packed, packed_ld, ss, zeros, qparam_ld, (int)gs, yy, y_ld, (int)N, st);
    else
      launch_front<4>(xx, x_ld, (int)M, (int)K, packed, packed_ld, ss, zeros, qparam_ld, (int)gs, yy, y_ld, (int)N, st);
    const bool pair = (K / gs) % 2 == 0 && qparam_ld % 2 == 0 && (reinterpret_cast<uintptr_t>(ss) & 3) == 0 &&
                      (reinterpret_cast<uintptr_t>(zeros) & 1) == 0;
    return launch_status_fmt("w4a16_gemv_front_kernel<16, %d, %s>", steps <= 16 ? 1 : steps <= 32 ? 2 : 4,
                             pair ? "true" : "false");
  }
  if (steps >= 16)
    launch_gemv<1, 16>(xx, x_ld, (int)M, (int)K, packed, packed_ld, ss, zeros, qparam_ld, (int)gs, yy, y_ld, (int)N, st);
  else if (steps >= 8)
    launch_gemv<1, 8>(xx, x_ld, (int)M, (int)K, packed, packed_ld, ss, zeros, qparam_ld, (int)gs, yy, y_ld, (int)N, st);
  else
    launch_gemv<1, 4>(xx, x_ld, (int)M, (int)K, packed, packed_ld, ss, zeros, qparam_ld, (int)gs, yy, y_ld, (int)N, st);
  return launch_status_fmt("w4a16_gemv_kernel<1, %d>", steps >= 16 ? 16 : steps >= 8 ? 8 : 4);
}

int w8a16_gemv_launch(const void* x, int64_t M, int64_t K, int64_t x_ld, const int8_t* w, int64_t N, int64_t w_ld,
                      const void* scales, void* y, int64_t y_ld, void* stream) {
  const int steps = (int)(K / 64);
  const unsigned tiles = (unsigned)((N + 15) / 16);
  hipStream_t st = (hipStream_t)stream;
  if (steps >= 16)
    hipLaunchKernelGGL(w8a16_gemv_kernel<16>, dim3(tiles), dim3(1024), 0, st, (const f16*)x, x_ld, (int)M, (int)K, w,
                       w_ld, (const f16*)scales, (f16*)y, y_ld, (int)N);
  else if (steps >= 4)
    hipLaunchKernelGGL(w8a16_gemv_kernel<4>, dim3(tiles), dim3(256), 0, st, (const f16*)x, x_ld, (int)M, (int)K, w,
                       w_ld, (const f16*)scales, (f16*)y, y_ld, (int)N);
  else
    hipLaunchKernelGGL(w8a16_gemv_kernel<1>, dim3(tiles), dim3(64), 0, st, (const f16*)x, x_ld, (int)M, (int)K, w,
                       w_ld, (const f16*)scales, (f16*)y, y_ld, (int)N);
  return launch_status("w8a16_gemv");
}

}  // namespace intent

extern "C" int intent_w4a16_sym_gemv(const void* x, int64_t M, int64_t K, int64_t x_ld, const int32_t* packed,
                                     int64_t N, int64_t packed_ld, const void* scales, int64_t scales_ld, void* y,
                                     int64_t y_ld, void* stream) {
  intent::clear_error();
  INTENT_REQUIRE(M >= 0 && N >= 0 && K >= 0 && M <= INT32_MAX && N <= INT32_MAX && K <= INT32_MAX,
                 INTENT_ERR_INVALID_ARGUMENT, "bad extents");
  INTENT_REQUIRE(M <= 5, INTENT_ERR_UNSUPPORTED, "w4a16_sym_gemv covers M <= 5, got %lld", (long long)M);
  INTENT_REQUIRE(K % 64 == 0 && K <= 8192, INTENT_ERR_UNSUPPORTED,
                 "w4a16_sym_gemv: K must be a multiple of 64 up to 8192, got %lld", (long long)K);
  INTENT_REQUIRE(N % 4 == 0, INTENT_ERR_UNSUPPORTED, "w4a16_sym_gemv: N must be a multiple of 4, got %lld",
                 (long long)N);
  if (M == 0 || N == 0) return INTENT_OK;
  INTENT_REQUIRE(K > 0, INTENT_ERR_UNSUPPORTED, "w4a16_sym_gemv: K must be positive");
  INTENT_REQUIRE(x && packed && scales && y, INTENT_ERR_INVALID_ARGUMENT, "null pointer argument");
  INTENT_REQUIRE(x_ld >= K && packed_ld >= N && scales_ld >= N && y_ld >= N, INTENT_ERR_INVALID_ARGUMENT,
                 "leading stride smaller than the row");
  INTENT_REQUIRE(intent::aligned16(x) && x_ld % 8 == 0 && intent::aligned16(packed) && packed_ld % 4 == 0 &&
                     (reinterpret_cast<uintptr_t>(scales) & 7) == 0 && scales_ld % 4 == 0,
                 INTENT_ERR_ALIGNMENT, "w4a16_sym_gemv: 16-byte aligned x and packed rows, 8-byte aligned scale rows");
  INTENT_REQUIRE(intent::fits_offset(K / 8, packed_ld * 4) && intent::fits_offset(M, x_ld * 2),
                 INTENT_ERR_UNSUPPORTED, "w4a16_sym_gemv: operand too large for 31-bit buffer offsets");
  const f16* xx = (const f16*)x;
  const f16* ss = (const f16*)scales;
  f16* yy = (f16*)y;
  hipStream_t st = (hipStream_t)stream;
  switch (M) {
    case 1: launch_sym<1>(xx, x_ld, (int)K, packed, packed_ld, ss, scales_ld, (int)N, yy, y_ld, st); break;
    case 2: launch_sym<2>(xx, x_ld, (int)K, packed, packed_ld, ss, scales_ld, (int)N, yy, y_ld, st); break;
    case 3: launch_sym<3>(xx, x_ld, (int)K, packed, packed_ld, ss, scales_ld, (int)N, yy, y_ld, st); break;
    case 4: launch_sym<4>(xx, x_ld, (int)K, packed, packed_ld, ss, scales_ld, (int)N, yy, y_ld, st); break;
    default: launch_sym<5>(xx, x_ld, (int)K, packed, packed_ld, ss, scales_ld, (int)N, yy, y_ld, st); break;
  }
  return intent::launch_status("w4a16_sym_gemv_kernel");
}
