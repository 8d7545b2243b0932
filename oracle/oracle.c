/*
 * CPU oracle for the quantized-contraction hot path — TEST INFRASTRUCTURE ONLY.
 *
 * This file restates, in plain C, the numerics of the reference's CPU path for
 * each function of the hot path. It is the checker: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it, and
 * never as the thing measured or shipped.
 *
 * Numerics follow the reference's CPU contraction semantics:
 *   - float contraction: acc = fma(f32(a), f32(b), acc), zero-initialised,
 *     sequential in k (lib/Conversion/KIRToCPU/Contractions.cpp:12-41,53-112);
 *   - integer contraction: i8 x i8 sign-extended, int32 accumulate modulo 2^32
 *     (Contractions.cpp:30-35,79-83; doc/dsl/types-numerics-and-effects.en.md:40);
 *   - casts to f16/bf16 round to nearest even
 *     (doc/dsl/types-numerics-and-effects.en.md:80).
 * Build with -ffp-contract=off so that only the explicit fmaf() fuses.
 * OpenMP splits whole output elements across threads; every element is
 * computed by one thread in a fixed order, so results do not depend on the
 * thread count.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

/* ---- scalar conversions --------------------------------------------------- */

float orc_f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t exp = (h >> 10) & 0x1fu;
  uint32_t mant = h & 0x3ffu;
  uint32_t bits;
  if (exp == 0) {
    if (mant == 0) {
      bits = sign;
    } else { /* subnormal: normalise */
      int e = -1;
      do {
        mant <<= 1;
        ++e;
      } while ((mant & 0x400u) == 0);
      mant &= 0x3ffu;
      bits = sign | ((uint32_t)(127 - 15 - e) << 23) | (mant << 13);
    }
  } else if (exp == 0x1f) {
    bits = sign | 0x7f800000u | (mant << 13);
  } else {
    bits = sign | ((exp + 127 - 15) << 23) | (mant << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

uint16_t orc_f32_to_f16(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
  const uint32_t absx = x & 0x7fffffffu;
  if (absx > 0x7f800000u) return sign | 0x7e00u; /* NaN */
  if (absx >= 0x47800000u) return sign | 0x7c00u; /* >= 65536 (and inf) */
  const int e = (int)(absx >> 23) - 127 + 15;
  const uint32_t mant = absx & 0x7fffffu;
  if (e >= 1) {
    uint32_t h = ((uint32_t)e << 10) | (mant >> 13);
    const uint32_t rem = mant & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h; /* carry may reach inf: correct */
    return sign | (uint16_t)h;
  }
  /* f16 subnormal or zero: value / 2^-24 rounded to nearest even */
  const int shift = 14 - e;
  if (shift > 24) return sign;
  const uint32_t m = mant | 0x800000u;
  uint32_t h = m >> shift;
  const uint32_t rem = m & ((1u << shift) - 1u);
  const uint32_t half = 1u << (shift - 1);
  if (rem > half || (rem == half && (h & 1u))) ++h;
  return sign | (uint16_t)h;
}

uint16_t orc_f32_to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

/* ---- W8A16 ------------------------------------------------------------------
 * y[m,n] = f16( f32(s[n]) * sum_k fma(f32(x[m,k]), f32(w[n,k])) ).
 * Weight-only int8 written as I.cast(W, f16) -> I.matmul(acc f32) -> scale
 * (doc/dsl/core.en.md:246); the int8 -> f32 decode is exact.
 */
void orc_w8a16(const uint16_t* x, int64_t M, int64_t K, const int8_t* w, int64_t N, const uint16_t* s, uint16_t* y,
               int threads) {
  int64_t i;
#pragma omp parallel for num_threads(threads) schedule(static)
  for (i = 0; i < M * N; ++i) {
    const int64_t m = i / N, n = i % N;
    float acc = 0.f;
    for (int64_t k = 0; k < K; ++k) acc = fmaf(orc_f16_to_f32(x[m * K + k]), (float)w[n * K + k], acc);
    y[m * N + n] = orc_f32_to_f16(acc * orc_f16_to_f32(s[n]));
  }
}

/* ---- W4A16 asymmetric group dequant ---------------------------------------------
 * deq[n,k] = f32(q[n,k] - z[n,k/g]) * f32(s[n,k/g]) (dequantization in f32, as
 * experiments/cpu/baselines/pytorch/cpu_runtime.py:97-102 does for the signed
 * variant of examples/kernels/contraction/weight_only_int4.py:18-51);
 * q from packed[n, k/2]: low nibble for even k, high nibble for odd k
 * (weight_only_int4.py:66-70 packing; doc/dsl/quantized-operations.en.md:17).
 * y[m,n] = f16( sum_k fma(f32(x[m,k]), deq[n,k]) ).
 */
void orc_w4a16(const uint16_t* x, int64_t M, int64_t K, const uint8_t* packed, int64_t N, const uint16_t* scales,
               const uint8_t* zeros, int64_t gs, uint16_t* y, int threads) {
  const int64_t G = K / gs;
  int64_t i;
#pragma omp parallel for num_threads(threads) schedule(static)
  for (i = 0; i < M * N; ++i) {
    const int64_t m = i / N, n = i % N;
    float acc = 0.f;
    for (int64_t k = 0; k < K; ++k) {
      const uint8_t byte = packed[n * (K / 2) + k / 2];
      const int q = (k & 1) ? (byte >> 4) : (byte & 15);
      const int64_t g = k / gs;
      const float deq = (float)(q - (int)zeros[n * G + g]) * orc_f16_to_f32(scales[n * G + g]);
      acc = fmaf(orc_f16_to_f32(x[m * K + k]), deq, acc);
    }
    y[m * N + n] = orc_f32_to_f16(acc);
  }
}

/* ---- int8 contractions ------------------------------------------------------------
 * acc[m,n] = sum_k i32(a[m,k]) * i32(w[n,k]) modulo 2^32 (gemm_i8,
 * examples/kernels/contraction/gemm.py:29-39, weight K-contiguous [N,K]).
 */
static int32_t i8_dot(const int8_t* a, const int8_t* w, int64_t K) {
  uint32_t acc = 0;
  for (int64_t k = 0; k < K; ++k) acc += (uint32_t)((int32_t)a[k] * (int32_t)w[k]);
  return (int32_t)acc;
}

void orc_i8_gemm_i32(const int8_t* a, int64_t M, int64_t K, const int8_t* w, int64_t N, const int32_t* bias,
                     int32_t* c, int threads) {
  int64_t i;
#pragma omp parallel for num_threads(threads) schedule(static)
  for (i = 0; i < M * N; ++i) {
    const int64_t m = i / N, n = i % N;
    uint32_t v = (uint32_t)i8_dot(a + m * K, w + n * K, K);
    if (bias) v += (uint32_t)bias[n];
    c[m * N + n] = (int32_t)v;
  }
}

/* out[m,n] = bf16( (f32(acc) * sa[m]) * sw[n] ), two fp32 multiplies left to
 * right, then round to nearest even. */
void orc_w8a8(const int8_t* a, int64_t M, int64_t K, const float* sa, const int8_t* w, int64_t N, const float* sw,
              uint16_t* out, int threads) {
  int64_t i;
#pragma omp parallel for num_threads(threads) schedule(static)
  for (i = 0; i < M * N; ++i) {
    const int64_t m = i / N, n = i % N;
    float f = (float)i8_dot(a + m * K, w + n * K, K);
    f = f * sa[m];
    f = f * sw[n];
    out[m * N + n] = orc_f32_to_bf16(f);
  }
}

/* ---- MoE router ---------------------------------------------------------------------
 * Top-k by raw logit (softmax is monotonic); a later expert replaces the best
 * only if strictly greater, so ties keep the lower index (argmax convention,
 * doc/dsl/types-numerics-and-effects.en.md:129). Probabilities:
 * p_e = expf(l_e - max) / sum_e' expf(l_e' - max), sums sequential in e;
 * renormalised as p_j / sum_{selected} p when renorm != 0.
 */
void orc_moe_route(const float* logits, int64_t T, int64_t E, int64_t top_k, int renorm, int32_t* ids,
                   float* weights) {
  for (int64_t t = 0; t < T; ++t) {
    const float* l = logits + t * E;
    float mx = l[0];
    for (int64_t e = 1; e < E; ++e) mx = l[e] > mx ? l[e] : mx;
    float sum = 0.f;
    for (int64_t e = 0; e < E; ++e) sum += expf(l[e] - mx);
    unsigned char taken[1024];
    memset(taken, 0, sizeof(taken));
    float p[64];
    float psum = 0.f;
    for (int64_t j = 0; j < top_k; ++j) {
      int64_t best = -1;
      float bv = 0.f;
      for (int64_t e = 0; e < E; ++e) {
        if (taken[e]) continue;
        if (best < 0 || l[e] > bv) {
          best = e;
          bv = l[e];
        }
      }
      taken[best] = 1;
      ids[t * top_k + j] = (int32_t)best;
      p[j] = expf(bv - mx) / sum;
      psum += p[j];
    }
    for (int64_t j = 0; j < top_k; ++j) weights[t * top_k + j] = renorm ? p[j] / psum : p[j];
  }
}

/* ---- MoE alignment ---------------------------------------------------------------------
 * moe_align_block_size (experiments/cpu/baselines/pytorch/cpu_runtime.py:
 * 1081-1098): histogram, block-padded cumulative offsets, route ids in stable
 * order (the order of a stable argsort of the expert ids) inside each expert
 * segment, sentinel R = T*top_k in unused slots, expert id per block
 * (-1 past the padded total). Ids outside [0,E) are dropped.
 */
void orc_moe_align(const int32_t* ids, int64_t T, int64_t top_k, int64_t E, int64_t B, int32_t* sorted,
                   int64_t capacity, int32_t* blocks, int64_t nblocks, int32_t* offsets, int32_t* total) {
  const int64_t R = T * top_k;
  int64_t* counts = (int64_t*)calloc((size_t)E, sizeof(int64_t));
  int64_t* cursor = (int64_t*)calloc((size_t)E, sizeof(int64_t));
  for (int64_t r = 0; r < R; ++r)
    if (ids[r] >= 0 && ids[r] < E) counts[ids[r]]++;
  offsets[0] = 0;
  for (int64_t e = 0; e < E; ++e) offsets[e + 1] = offsets[e] + (int32_t)((counts[e] + B - 1) / B * B);
  total[0] = offsets[E];
  for (int64_t i = 0; i < capacity; ++i) sorted[i] = (int32_t)R;
  for (int64_t r = 0; r < R; ++r) {
    const int32_t e = ids[r];
    if (e < 0 || e >= E) continue;
    sorted[offsets[e] + cursor[e]++] = (int32_t)r;
  }
  for (int64_t b = 0; b < nblocks; ++b) blocks[b] = -1;
  for (int64_t e = 0; e < E; ++e)
    for (int64_t b = offsets[e] / B; b < offsets[e + 1] / B; ++b) blocks[b] = (int32_t)e;
  free(counts);
  free(cursor);
}

/* ---- MoE expert FFN (W4, SiLU-gated) -------------------------------------------------------
 * For route r = t*top_k + j with expert e = ids[r] (moe_expert_ffn,
 * examples/kernels/ragged/moe.py:12-53, with a SiLU-gated first layer):
 *   g[f] = sum_h fma(x[t,h], deq(Wgu[e])[f,h]);  u[f] = same with row F+f
 *   a[f] = f16( (g / (1 + expf(-g))) * u )       (hidden cast to f16, moe.py:43)
 *   o[d] = sum_f fma(f32(a[f]), deq(Wd[e])[d,f])
 * and y[t,:] (f32, accumulated) gets y = y + w[r]*o slot by slot in order.
 */
static float w4_deq(const uint8_t* packed, const uint16_t* scales, const uint8_t* zeros, int64_t Kdim, int64_t gs,
                    int64_t row, int64_t k) {
  const uint8_t byte = packed[row * (Kdim / 2) + k / 2];
  const int q = (k & 1) ? (byte >> 4) : (byte & 15);
  const int64_t G = Kdim / gs;
  return (float)(q - (int)zeros[row * G + k / gs]) * orc_f16_to_f32(scales[row * G + k / gs]);
}

void orc_moe_ffn_w4(const uint16_t* x, int64_t T, int64_t H, const int32_t* ids, const float* weights, int64_t top_k,
                    int64_t E, const uint8_t* wgu, const uint16_t* sgu, const uint8_t* zgu, const uint8_t* wd,
                    const uint16_t* sd, const uint8_t* zd, int64_t F, int64_t gs, float* y, int threads) {
  const int64_t R = T * top_k;
  float* out = (float*)malloc(sizeof(float) * (size_t)(R * H));
  uint16_t* act = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)(R * F));
  const int64_t gu_rows = 2 * F;
  int64_t i;
#pragma omp parallel for num_threads(threads) schedule(static)
  for (i = 0; i < R * F; ++i) {
    const int64_t r = i / F, f = i % F;
    const int64_t t = r / top_k;
    const int32_t e = ids[r];
    if (e < 0 || e >= E) {
      act[i] = 0;
      continue;
    }
    const uint8_t* q = wgu + (int64_t)e * gu_rows * (H / 2);
    const uint16_t* s = sgu + (int64_t)e * gu_rows * (H / gs);
    const uint8_t* z = zgu + (int64_t)e * gu_rows * (H / gs);
    float g = 0.f, u = 0.f;
    for (int64_t h = 0; h < H; ++h) {
      const float xv = orc_f16_to_f32(x[t * H + h]);
      g = fmaf(xv, w4_deq(q, s, z, H, gs, f, h), g);
      u = fmaf(xv, w4_deq(q, s, z, H, gs, F + f, h), u);
    }
    const float silu = g / (1.0f + expf(-g));
    act[i] = orc_f32_to_f16(silu * u);
  }
#pragma omp parallel for num_threads(threads) schedule(static)
  for (i = 0; i < R * H; ++i) {
    const int64_t r = i / H, d = i % H;
    const int32_t e = ids[r];
    if (e < 0 || e >= E) {
      out[i] = 0.f;
      continue;
    }
    const uint8_t* q = wd + (int64_t)e * H * (F / 2);
    const uint16_t* s = sd + (int64_t)e * H * (F / gs);
    const uint8_t* z = zd + (int64_t)e * H * (F / gs);
    float acc = 0.f;
    for (int64_t f = 0; f < F; ++f) acc = fmaf(orc_f16_to_f32(act[r * F + f]), w4_deq(q, s, z, F, gs, d, f), acc);
    out[i] = acc;
  }
  for (int64_t t = 0; t < T; ++t)
    for (int64_t d = 0; d < H; ++d) {
      float acc = y[t * H + d];
      for (int64_t j = 0; j < top_k; ++j) {
        const int64_t r = t * top_k + j;
        if (ids[r] < 0 || ids[r] >= E) continue;
        const float prod = weights[r] * out[r * H + d];
        acc = acc + prod;
      }
      y[t * H + d] = acc;
    }
  free(out);
  free(act);
}

/* ---- K-quant records: Q8_K quantize and Q4_K x Q8_K dot --------------------
 * Record formats and numerics: doc/dsl/quantized-operations.en.md:11-70
 * (Q4_K 144 bytes: f16 d, f16 dmin, 12 bytes of 6-bit sc/m, 128 bytes of
 * nibbles; Q8_K 292 bytes: f32 ds, 256 i8, 16 i16 bsum). The same algorithm
 * appears as the reference's RVV baseline,
 * experiments/cpu/baselines/weft/tianchenrv/contraction/q4_k_projection/
 * q4_k_projection.py:29-72 (quantize_row, compute), whose result starts from
 * +0.0 and adds the records in increasing order. */

static float orc_ld_f32(const uint8_t* p) {
  float f;
  memcpy(&f, p, 4);
  return f;
}

/* quantized-operations.en.md:62-70. */
void orc_q8k_quantize(const float* x, int64_t G, uint8_t* out) {
  for (int64_t g = 0; g < G; ++g) {
    const float* v = x + g * 256;
    uint8_t* r = out + g * 292;
    float mx = v[0], mn = v[0];
    for (int i = 1; i < 256; ++i) {
      if (v[i] > mx) mx = v[i];
      if (v[i] < mn) mn = v[i];
    }
    const float extreme = fabsf(mx) > fabsf(mn) ? mx : mn; /* ties pick the minimum */
    float inverse = 0.0f, ds = 0.0f;
    int8_t q[256];
    if (extreme != 0.0f) {
      inverse = -127.0f / extreme;
      ds = 1.0f / inverse;
      for (int i = 0; i < 256; ++i) {
        const float t = rintf(v[i] * inverse); /* round half to even (default mode) */
        q[i] = (int8_t)(t > 127.0f ? 127 : t < -128.0f ? -128 : (int)t);
      }
    } else {
      memset(q, 0, sizeof q);
    }
    memcpy(r, &ds, 4);
    memcpy(r + 4, q, 256);
    for (int j = 0; j < 16; ++j) {
      int s = 0;
      for (int i = 0; i < 16; ++i) s += q[16 * j + i];
      const int16_t b = (int16_t)s;
      memcpy(r + 260 + 2 * j, &b, 2);
    }
  }
}

/* Field r (0 = sc, 1 = m) of a Q4_K record: quantized-operations.en.md:28-36. */
static int orc_q4k_field(const uint8_t* a, int r, int i) {
  if (i < 4) return a[4 + 4 * r + i] & 63;
  const int t = i - 4;
  return ((a[12 + t] >> (4 * r)) & 15) | ((a[4 + 4 * r + t] >> 6) << 4);
}

/* v_b of one record pair: quantized-operations.en.md:44-54. */
static float orc_q4k_q8k_record(const uint8_t* w, const uint8_t* x) {
  int32_t S = 0, T = 0;
  for (int s = 0; s < 8; ++s) {
    int32_t dot = 0;
    for (int i = 0; i < 32; ++i) {
      const int e = 32 * s + i;
      const int packed = w[16 + 32 * (e / 64) + (e % 32)];
      const int q = (packed >> ((e % 64) < 32 ? 0 : 4)) & 15;
      dot += q * (int32_t)(int8_t)x[4 + e];
    }
    S += orc_q4k_field(w, 0, s) * dot;
    int16_t b0, b1;
    memcpy(&b0, x + 260 + 2 * (2 * s), 2);
    memcpy(&b1, x + 260 + 2 * (2 * s + 1), 2);
    T += orc_q4k_field(w, 1, s) * ((int32_t)b0 + (int32_t)b1);
  }
  uint16_t dh, mh;
  memcpy(&dh, w, 2);
  memcpy(&mh, w + 2, 2);
  const float p = orc_f16_to_f32(dh) * (float)S;
  const float n = orc_f16_to_f32(mh) * (float)T;
  const float diff = p - n;
  return orc_ld_f32(x) * diff;
}

float orc_q4k_q8k_dot(const uint8_t* w, const uint8_t* x, int64_t G) {
  float result = 0.0f;
  for (int64_t g = 0; g < G; ++g) result = result + orc_q4k_q8k_record(w + 144 * g, x + 292 * g);
  return result;
}

/* quantized_projection (examples/kernels/quantization/quantized_projection.py:5-19):
 * y[n] = quantized_dot(w[n], quantize(x)). */
void orc_q4k_gemv(const uint8_t* w, int64_t N, int64_t G, int64_t w_ld, const uint8_t* xq, float* y, int threads) {
  (void)threads;
#pragma omp parallel for num_threads(threads > 0 ? threads : 1) schedule(static)
  for (int64_t n = 0; n < N; ++n) y[n] = orc_q4k_q8k_dot(w + n * w_ld, xq, G);
}

/* ---- groupwise FP8 (E4M3FN) activation quantizers ---------------------------
 * examples/kernels/quantization/fp8.py:11-69 (bf16_groupwise_fp8_quantize,
 * f32_groupwise_fp8_quantize), the same as the reference's CPU comparison
 * side experiments/cpu/baselines/pytorch/cpu_runtime.py:142-147:
 *   scale = max(absmax(group of 128), eps) / 448      (eps 1e-12 bf16, 1e-4 f32)
 *   q     = e4m3fn(min(max(x / scale, -448), 448))    (round to nearest even)
 * Columns past N belong to no group element (masked out of the max). */

/* f32 -> OCP E4M3FN bits (bias 7, no infinities, NaN = S.1111.111), round to
 * nearest even. Inputs of magnitude above 448 saturate to 448 (callers clamp
 * first, so this never triggers for the quantizers). */
uint8_t orc_f32_to_e4m3fn(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  const uint8_t sign = (uint8_t)((u >> 24) & 0x80u);
  const uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return (uint8_t)(sign | 0x7f); /* NaN */
  float mag;
  memcpy(&mag, &a, 4);
  if (mag >= 448.0f) return (uint8_t)(sign | 0x7e);
  if (mag < 0.015625f) { /* below 2^-6: subnormal step 2^-9 */
    const float m = rintf(mag * 512.0f); /* exact scaling, then round half even */
    return (uint8_t)(sign | (uint8_t)m);  /* m == 8 is the smallest normal, 0x08 */
  }
  /* normal: keep 3 mantissa bits, round half to even on the 20 dropped bits */
  const uint32_t r = a + 0x7ffffu + ((a >> 20) & 1u);
  const uint32_t e = (r >> 23) - 127 + 7;
  const uint32_t m = (r >> 20) & 7u;
  return (uint8_t)(sign | (e << 3) | m);
}

void orc_fp8_groupwise_quantize(const float* x, int64_t M, int64_t N, int64_t ldx, int64_t G, float eps,
                                uint8_t* q, int64_t ldq, float* scales, int64_t lds_) {
  for (int64_t r = 0; r < M; ++r) {
    for (int64_t g = 0; g < G; ++g) {
      float amax = -INFINITY;
      for (int64_t c = g * 128; c < g * 128 + 128 && c < N; ++c) {
        const float v = x[r * ldx + c];
        const float av = fmaxf(v, -v);
        if (av > amax) amax = av;
      }
      const float scale = fmaxf(amax, eps) / 448.0f;
      scales[r * lds_ + g] = scale;
      for (int64_t c = g * 128; c < g * 128 + 128 && c < N; ++c) {
        const float t = x[r * ldx + c] / scale;
        q[r * ldq + c] = orc_f32_to_e4m3fn(fminf(fmaxf(t, -448.0f), 448.0f));
      }
    }
  }
}

/* ---- low-bit weight x int8 activation, exact int32 ---------------------------
 * w4a8_packed_matmul (examples/kernels/contraction/weight_only_int4.py:54-91):
 *   nibble k of row n = (packed[n, k/2] >> 4*(k%2)) & 15, signed = n - ((n & 8) << 1),
 *   out[n, m] = sum_k signed[n, k] * a[m, k]          (output [N, M]).
 * bitnet_int2_matmul (weight_only_int4.py:94-124):
 *   value k of row n = (packed[n, (k/16)*4 + k%4] >> 2*((k/4)%4)) & 3,
 *   out[m, n] = sum_k a[m, k] * value[n, k]            (output [M, N]).
 * int32 accumulation, modulo 2^32 (types-numerics-and-effects.en.md:40). */
void orc_w4a8(const int8_t* a, int64_t M, int64_t K, const uint8_t* packed, int64_t N, int32_t* out, int threads) {
#pragma omp parallel for num_threads(threads > 0 ? threads : 1) schedule(static)
  for (int64_t n = 0; n < N; ++n) {
    for (int64_t m = 0; m < M; ++m) {
      uint32_t acc = 0;
      for (int64_t k = 0; k < K; ++k) {
        const int nib = (packed[n * (K / 2) + k / 2] >> (4 * (k % 2))) & 15;
        const int w = nib - ((nib & 8) << 1);
        acc += (uint32_t)(w * (int32_t)a[m * K + k]);
      }
      out[n * M + m] = (int32_t)acc;
    }
  }
}

void orc_bitnet_int2(const int8_t* a, int64_t M, int64_t K, const uint8_t* packed, int64_t N, int32_t* out,
                     int threads) {
#pragma omp parallel for num_threads(threads > 0 ? threads : 1) schedule(static)
  for (int64_t m = 0; m < M; ++m) {
    for (int64_t n = 0; n < N; ++n) {
      uint32_t acc = 0;
      for (int64_t k = 0; k < K; ++k) {
        const int v = (packed[n * (K / 4) + (k / 16) * 4 + k % 4] >> (2 * ((k / 4) % 4))) & 3;
        acc += (uint32_t)((int32_t)a[m * K + k] * v);
      }
      out[m * N + n] = (int32_t)acc;
    }
  }
}

/* ---- MX block-scaled FP8 contraction ------------------------------------------
 * block_scaled_matmul (examples/kernels/contraction/block_scaled.py:11-39) with
 * the CPU semantics of lib/Conversion/KIRToCPU/Contractions.cpp:177-259: each
 * E4M3FN element widens exactly to f32 and is multiplied by its E8M0 scale
 * (bits e << 23; e == 0 gives 2^-127 = 0x00400000, e == 255 NaN), then
 * out = f32 contraction with fma accumulation in k order (Contractions.cpp:12-41). */
float orc_e4m3fn_to_f32(uint8_t v) {
  const int sign = v >> 7, e = (v >> 3) & 15, m = v & 7;
  float mag;
  if (e == 15 && m == 7) mag = NAN;
  else if (e == 0) mag = ldexpf((float)m, -9);
  else mag = ldexpf(1.0f + (float)m / 8.0f, e - 7);
  return sign ? -mag : mag;
}

float orc_e8m0_to_f32(uint8_t e) {
  const uint32_t bits = e == 0 ? 0x00400000u : e == 255 ? 0x7fc00000u : (uint32_t)e << 23;
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

void orc_mxfp8_gemm(const uint8_t* a, const uint8_t* sa, int64_t M, int64_t K, const uint8_t* b, const uint8_t* sb,
                    int64_t N, float* out, int threads) {
#pragma omp parallel for num_threads(threads > 0 ? threads : 1) schedule(static)
  for (int64_t m = 0; m < M; ++m) {
    for (int64_t n = 0; n < N; ++n) {
      float acc = 0.0f;
      for (int64_t k = 0; k < K; ++k) {
        const float x = orc_e4m3fn_to_f32(a[m * K + k]) * orc_e8m0_to_f32(sa[m * (K / 32) + k / 32]);
        const float y = orc_e4m3fn_to_f32(b[n * K + k]) * orc_e8m0_to_f32(sb[n * (K / 32) + k / 32]);
        acc = fmaf(x, y, acc);
      }
      out[m * N + n] = acc;
    }
  }
}

/* ---- per-tensor scaled FP8 GEMM and its split-K form ---------------------------
 * scaled_fp8_matmul (examples/kernels/contraction/block_scaled.py:42-63):
 *   out = f16((acc * lhs_scale) * rhs_scale), acc the f32 contraction (fma in
 *   k order, Contractions.cpp:12-41) of E4M3FN values widened exactly to f32.
 * scaled_fp8_splitk_matmul (block_scaled.py:66-98; CPU baseline
 * experiments/cpu/baselines/pytorch/cpu_runtime.py:133-139): lhs [M, IT, SP, 256]
 * and rhs [IT, SP, 256, N] share k = (it*SP + s)*256 + r; for s = 0 .. SP-1 in
 * order, p = f16((acc_s * lhs_scale) * rhs_scale) and out = f16(out + p).
 * Here a is [M, K] (K contiguous) and b is [K, N] (N contiguous), as the
 * reference passes them; splits == 1 without accumulate is the plain form. */
void orc_scaled_fp8_gemm(const uint8_t* a, int64_t M, int64_t K, const uint8_t* b, int64_t N, float ls, float rs,
                         int64_t splits, int accumulate, uint16_t* out, int threads) {
  const int64_t chunks = K / 256;
#pragma omp parallel for num_threads(threads > 0 ? threads : 1) schedule(static)
  for (int64_t m = 0; m < M; ++m) {
    for (int64_t n = 0; n < N; ++n) {
      float o = accumulate ? orc_f16_to_f32(out[m * N + n]) : 0.0f;
      for (int64_t s = 0; s < splits; ++s) {
        float acc = 0.0f;
        if (splits == 1) {
          for (int64_t k = 0; k < K; ++k)
            acc = fmaf(orc_e4m3fn_to_f32(a[m * K + k]), orc_e4m3fn_to_f32(b[k * N + n]), acc);
        } else {
          for (int64_t c = s; c < chunks; c += splits)
            for (int64_t r = 0; r < 256; ++r) {
              const int64_t k = c * 256 + r;
              acc = fmaf(orc_e4m3fn_to_f32(a[m * K + k]), orc_e4m3fn_to_f32(b[k * N + n]), acc);
            }
        }
        const float scaled = (acc * ls) * rs;
        const float p = orc_f16_to_f32(orc_f32_to_f16(scaled));
        o = accumulate ? orc_f16_to_f32(orc_f32_to_f16(o + p)) : p;
      }
      out[m * N + n] = orc_f32_to_f16(o);
    }
  }
}

/* ---- DeepGEMM-style FP8 GEMM with f32 block scales -----------------------------
 * deepgemm_fp8_2xacc (block_scaled.py:101-122; CPU baseline cpu_runtime.py:127-131):
 * lhs [M, KB, 128] and rhs [N, KB, 128] E4M3FN, lhs_scale f32 [M, KB], rhs_scale
 * f32 [N/128, KB] (one scale per 128 x 128 block of rhs):
 *   left = f32(lhs) * lhs_scale[m, kb], right = f32(rhs) * rhs_scale[n/128, kb]
 *   out = bf16(sum_k left * right), fma in k order. */
void orc_deepgemm_fp8(const uint8_t* a, const float* sa, int64_t M, int64_t KB, const uint8_t* b, const float* sb,
                      int64_t N, uint16_t* out, int threads) {
  const int64_t K = KB * 128;
#pragma omp parallel for num_threads(threads > 0 ? threads : 1) schedule(static)
  for (int64_t m = 0; m < M; ++m) {
    for (int64_t n = 0; n < N; ++n) {
      float acc = 0.0f;
      for (int64_t k = 0; k < K; ++k) {
        const float x = orc_e4m3fn_to_f32(a[m * K + k]) * sa[m * KB + k / 128];
        const float y = orc_e4m3fn_to_f32(b[n * K + k]) * sb[(n / 128) * KB + k / 128];
        acc = fmaf(x, y, acc);
      }
      out[m * N + n] = orc_f32_to_bf16(acc);
    }
  }
}

/* ---- FP8 x FP8 -> FP8 contractions ---------------------------------------------
 * fp8_e4m3_matmul / fp8_e5m2_matmul (examples/kernels/contraction/weight_only_int4.py:
 * 178-215): out = cast(f32 contraction, format), fma in k order. Casts follow
 * doc/dsl/types-numerics-and-effects.en.md:86-89: nearest-even; E5M2 (sign1,
 * exponent5 bias 15, fraction2, subnormals) overflows to infinity; E4M3FN
 * results beyond 448 are outside the cast's contract (saturated here). */
float orc_e5m2_to_f32(uint8_t v) {
  const int sign = v >> 7, e = (v >> 2) & 31, m = v & 3;
  float mag;
  if (e == 31) mag = m ? NAN : INFINITY;
  else if (e == 0) mag = ldexpf((float)m, -16);
  else mag = ldexpf(1.0f + (float)m / 4.0f, e - 15);
  return sign ? -mag : mag;
}

uint8_t orc_f32_to_e5m2(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  const uint8_t sign = (uint8_t)((u >> 24) & 0x80u);
  const uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return (uint8_t)(sign | 0x7f); /* NaN */
  if (a == 0x7f800000u) return (uint8_t)(sign | 0x7c);
  float mag;
  memcpy(&mag, &a, 4);
  if (mag < ldexpf(1.0f, -14)) /* subnormal step 2^-16; 4 is the smallest normal */
    return (uint8_t)(sign | (uint8_t)rintf(mag * 65536.0f));
  /* normal: keep 2 mantissa bits, round half to even on the 21 dropped bits */
  const uint32_t r = a + 0xfffffu + ((a >> 21) & 1u);
  const uint32_t e = (r >> 23) - 127 + 15;
  if (e >= 31) return (uint8_t)(sign | 0x7c); /* finite overflow -> infinity */
  return (uint8_t)(sign | (e << 2) | ((r >> 21) & 3u));
}

void orc_fp8_gemm(int format, const uint8_t* a, int64_t M, int64_t K, const uint8_t* bt, int64_t N, uint8_t* out,
                  int threads) {
#pragma omp parallel for num_threads(threads > 0 ? threads : 1) schedule(static)
  for (int64_t m = 0; m < M; ++m) {
    for (int64_t n = 0; n < N; ++n) {
      float acc = 0.0f;
      for (int64_t k = 0; k < K; ++k) {
        const float x = format ? orc_e5m2_to_f32(a[m * K + k]) : orc_e4m3fn_to_f32(a[m * K + k]);
        const float y = format ? orc_e5m2_to_f32(bt[n * K + k]) : orc_e4m3fn_to_f32(bt[n * K + k]);
        acc = fmaf(x, y, acc);
      }
      out[m * N + n] = format ? orc_f32_to_e5m2(acc) : orc_f32_to_e4m3fn(acc);
    }
  }
}

/* ---- FP4 (E2M1) weights x bf16 activations ----------------------------------------
 * dequant_bf16_fp4_matmul (examples/kernels/contraction/weight_only_int4.py:127-175;
 * CPU baseline experiments/cpu/baselines/pytorch/cpu_runtime.py:117-124): row n holds
 * big-endian 16-bit words w = (p[2i] << 8) | p[2i+1], each carrying k = 4i .. 4i+3 at
 * the bf16 bit patterns below; decoded = bf16(f32(bf16 pattern) * 2^126);
 * out = bf16(sum_k f32(x) * decoded), fma in k order. */
static float bf16_bits_to_f32(uint16_t b) {
  const uint32_t u = (uint32_t)b << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

float orc_fp4_decode(const uint8_t* row, int64_t k) {
  const int64_t pair = (k / 4) * 2;
  const uint32_t w = ((uint32_t)row[pair] << 8) | row[pair + 1];
  uint32_t bits;
  switch (k % 4) {
    case 0: bits = w & 0x81C0u; break;
    case 1: bits = (w << 3) & 0x81C0u; break;
    case 2: bits = (w << 6) & 0x81C0u; break;
    default: bits = ((w << 1) & 0x8000u) | ((w >> 3) & 0x0180u) | ((w >> 7) & 0x0040u); break;
  }
  const float v = bf16_bits_to_f32((uint16_t)bits) * ldexpf(1.0f, 126);
  return bf16_bits_to_f32(orc_f32_to_bf16(v));
}

void orc_fp4_bf16_matmul(const uint16_t* x, int64_t M, int64_t K, const uint8_t* packed, int64_t N, uint16_t* out,
                         int threads) {
#pragma omp parallel for num_threads(threads > 0 ? threads : 1) schedule(static)
  for (int64_t m = 0; m < M; ++m) {
    for (int64_t n = 0; n < N; ++n) {
      float acc = 0.0f;
      for (int64_t k = 0; k < K; ++k) acc = fmaf(bf16_bits_to_f32(x[m * K + k]), orc_fp4_decode(packed + n * (K / 2), k), acc);
      out[m * N + n] = orc_f32_to_bf16(acc);
    }
  }
}

/* ---- the reference's own W4 layout -------------------------------------------------
 * weight_only_int4_matmul (examples/kernels/contraction/weight_only_int4.py:18-51;
 * CPU baseline experiments/cpu/baselines/pytorch/cpu_runtime.py:97-102): packed int32
 * [K/8, N], nibble k % 8 of word [k/8, n] at bits 4(k % 8), two's complement; scales
 * f16 [K/64, N]; dequantized = f32(signed) * f32(scale) (exact); y = f16(sum_k
 * f32(x) * dequantized), fma in k order. */
void orc_w4_sym(const uint16_t* x, int64_t M, int64_t K, const int32_t* packed, const uint16_t* scales, int64_t N,
                uint16_t* y, int threads) {
#pragma omp parallel for num_threads(threads > 0 ? threads : 1) schedule(static)
  for (int64_t m = 0; m < M; ++m) {
    for (int64_t n = 0; n < N; ++n) {
      float acc = 0.0f;
      for (int64_t k = 0; k < K; ++k) {
        const uint32_t word = (uint32_t)packed[(k / 8) * N + n];
        const int nib = (int)((word >> (4 * (k % 8))) & 15u);
        const int sgn = nib - ((nib & 8) << 1);
        const float w = (float)sgn * orc_f16_to_f32(scales[(k / 64) * N + n]);
        acc = fmaf(orc_f16_to_f32(x[m * K + k]), w, acc);
      }
      y[m * N + n] = orc_f32_to_f16(acc);
    }
  }
}

/* ---- quantized_gemm -------------------------------------------------------------
 * examples/kernels/contraction/gemm.py:83-106; CPU baseline
 * experiments/cpu/baselines/pytorch/cpu_runtime.py:91-94: acc = f32 contraction of
 * f16 a [M, K] and b [K, N] (fma in k order); v = relu(acc + bias[n]) + f32(residual);
 * out = i8(trunc(clamp(v / output_scale[n], -128, 127))). */
void orc_quantized_gemm(const uint16_t* a, int64_t M, int64_t K, const uint16_t* b, int64_t N, const float* bias,
                        const uint16_t* residual, const float* oscale, int8_t* out, int threads) {
#pragma omp parallel for num_threads(threads > 0 ? threads : 1) schedule(static)
  for (int64_t m = 0; m < M; ++m) {
    for (int64_t n = 0; n < N; ++n) {
      float acc = 0.0f;
      for (int64_t k = 0; k < K; ++k) acc = fmaf(orc_f16_to_f32(a[m * K + k]), orc_f16_to_f32(b[k * N + n]), acc);
      float v = acc + bias[n];
      v = v < 0.0f ? 0.0f : v;
      v = v + orc_f16_to_f32(residual[m * N + n]);
      v = v / oscale[n];
      v = fminf(fmaxf(v, -128.0f), 127.0f);
      out[m * N + n] = (int8_t)(int32_t)v;
    }
  }
}

/* ---- f16 / bf16 grouped GEMMs ------------------------------------------------------
 * ragged_grouped_gemm(_bf16) (examples/kernels/ragged/grouped_gemm.py:11-70; CPU
 * baseline cpu_runtime.py:859-864): y[rows of g] = x[rows of g] @ W[g], W [G, K, N].
 * routed_expert_projection_bf16 (grouped_gemm.py:101-138; cpu_runtime.py:874-881):
 * route r = routes[i] for i in the expert's range reads token r / top_k, writes
 * output row r of [T * top_k, N]; W [E, N, K]. f32 accumulation (fma in k order),
 * one rounding to the element type. */
static float u16_to_f32(uint16_t v, int bf16) { return bf16 ? bf16_bits_to_f32(v) : orc_f16_to_f32(v); }

void orc_grouped_gemm(const uint16_t* x, int bf16, int64_t K, const int32_t* offsets, int64_t G, const int32_t* routes,
                      int64_t top_k, const uint16_t* w, int64_t N, uint16_t* out, int threads) {
  for (int64_t g = 0; g < G; ++g) {
    const int64_t b = offsets[g], e = offsets[g + 1];
#pragma omp parallel for num_threads(threads > 0 ? threads : 1) schedule(static)
    for (int64_t i = b; i < e; ++i) {
      const int64_t orow = routes ? routes[i] : i;
      const int64_t xrow = routes ? routes[i] / top_k : i;
      for (int64_t n = 0; n < N; ++n) {
        float acc = 0.0f;
        for (int64_t k = 0; k < K; ++k) {
          const uint16_t wv = routes ? w[(g * N + n) * K + k] : w[(g * K + k) * N + n];
          acc = fmaf(u16_to_f32(x[xrow * K + k], bf16), u16_to_f32(wv, bf16), acc);
        }
        out[orow * N + n] = bf16 ? orc_f32_to_bf16(acc) : orc_f32_to_f16(acc);
      }
    }
  }
}

/* ---- f16 MoE expert FFN ---------------------------------------------------------------
 * moe_expert_ffn (examples/kernels/ragged/moe.py:12-53; host reference
 * experiments/_common/support.py:133-151): for expert e in order and each member i of
 * [route_offsets[e], route_offsets[e+1]): route r = member_routes[i], token t =
 * route_token[r]; hidden = f16(max(x[t] @ w1[e], 0)) (f32 fma in k order, ReLU in f32,
 * one rounding); out = hidden @ w2[e] (f32 fma in f order); y[t] += route_weights[r] * out
 * (f32 product, then f32 add: scatter_reduce add). w1 [E, D, F], w2 [E, F, D] f16.
 * token_sel (T entries, or NULL = all): members of unselected tokens are skipped. */
void orc_moe_expert_ffn(const uint16_t* x, int64_t T, int64_t D, const int32_t* route_offsets, int64_t E,
                        const int32_t* member_routes, const int32_t* route_token, const float* route_weights,
                        const uint16_t* w1, const uint16_t* w2, int64_t F, float* y, const uint8_t* token_sel,
                        int threads) {
  float* hid = (float*)malloc(sizeof(float) * (size_t)(F > 0 ? F : 1));
  float* out = (float*)malloc(sizeof(float) * (size_t)(D > 0 ? D : 1));
  for (int64_t e = 0; e < E; ++e) {
    for (int64_t i = route_offsets[e]; i < route_offsets[e + 1]; ++i) {
      const int64_t r = member_routes[i];
      const int64_t t = route_token[r];
      if (token_sel && !token_sel[t]) continue;
      const uint16_t* xr = x + t * D;
      const uint16_t* a = w1 + e * D * F;
#pragma omp parallel for num_threads(threads > 0 ? threads : 1) schedule(static)
      for (int64_t f = 0; f < F; ++f) {
        float acc = 0.0f;
        for (int64_t k = 0; k < D; ++k) acc = fmaf(orc_f16_to_f32(xr[k]), orc_f16_to_f32(a[k * F + f]), acc);
        acc = acc < 0.0f ? 0.0f : acc;
        hid[f] = orc_f16_to_f32(orc_f32_to_f16(acc));
      }
      const uint16_t* b = w2 + e * F * D;
#pragma omp parallel for num_threads(threads > 0 ? threads : 1) schedule(static)
      for (int64_t d = 0; d < D; ++d) {
        float acc = 0.0f;
        for (int64_t f = 0; f < F; ++f) acc = fmaf(hid[f], orc_f16_to_f32(b[f * D + d]), acc);
        out[d] = acc;
      }
      const float wt = route_weights[r];
      for (int64_t d = 0; d < D; ++d) y[t * D + d] = y[t * D + d] + wt * out[d];
    }
  }
  free(hid);
  free(out);
}

/* ---- float GEMMs ----------------------------------------------------------------------
 * gemm (examples/kernels/contraction/gemm.py:42-61, ACTIVATION RELU: max(acc, 0)) and
 * bf16_gemm (gemm.py:64-80): c = cast(f32 contraction (fma in k order)); b is [K, N]. */
void orc_float_gemm(const uint16_t* a, int64_t M, int64_t K, const uint16_t* b, int64_t N, int bf16, int relu,
                    uint16_t* c, int threads) {
#pragma omp parallel for num_threads(threads > 0 ? threads : 1) schedule(static)
  for (int64_t m = 0; m < M; ++m) {
    for (int64_t n = 0; n < N; ++n) {
      float acc = 0.0f;
      for (int64_t k = 0; k < K; ++k) acc = fmaf(u16_to_f32(a[m * K + k], bf16), u16_to_f32(b[k * N + n], bf16), acc);
      if (relu) acc = acc < 0.0f ? 0.0f : acc;
      c[m * N + n] = bf16 ? orc_f32_to_bf16(acc) : orc_f32_to_f16(acc);
    }
  }
}

/* ---- NVFP4 quantization -----------------------------------------------------------------
 * nvfp4_quantize (examples/kernels/quantization/nvfp4.py; CPU baseline
 * experiments/cpu/baselines/pytorch/cpu_runtime.py:1325-1340), per row and group of 16:
 * scale = e4m3fn(max((amax / 6) * gs, 1.5258789e-5)); multiplier = gs / f32(scale);
 * v = x * multiplier; E2M1 code by thresholds on |v| (> 0.25, >= 0.75, > 1.25, >= 1.75,
 * > 2.5, >= 3.5, > 5.0) with the sign bit of v; packed byte = code(2i) | code(2i+1) << 4;
 * the scale byte at scales[row/128][group/4][row%32][(row%128)/32][group%4] (NT = the
 * number of 4-group blocks). */
void orc_nvfp4_quantize(const uint16_t* x, int64_t M, int64_t N, float gs, uint8_t* packed, uint8_t* scales) {
  const int64_t G = N / 16, NT = (G + 3) / 4;
  static const float thr[7] = {0.25f, 0.75f, 1.25f, 1.75f, 2.5f, 3.5f, 5.0f};
  for (int64_t r = 0; r < M; ++r) {
    for (int64_t g = 0; g < G; ++g) {
      float v[16], amax = 0.0f;
      for (int i = 0; i < 16; ++i) {
        v[i] = bf16_bits_to_f32(x[r * N + g * 16 + i]);
        amax = fmaxf(amax, fabsf(v[i]));
      }
      float s = (amax / 6.0f) * gs;
      if (s < 1.5258789e-5f) s = 1.5258789e-5f;
      /* torch's E4M3FN cast (the CPU formula's) rounds (448, 464] to 448 and gives NaN
       * above; a NaN scale makes every value NaN and every code of the group 0 */
      const int nan_scale = !(s <= 464.0f);
      const uint8_t sb = nan_scale ? (uint8_t)0x7f : orc_f32_to_e4m3fn(s);
      const float mult = nan_scale ? 0.0f : gs / orc_e4m3fn_to_f32(sb);
      uint8_t code[16];
      for (int i = 0; i < 16; ++i) {
        const float t = v[i] * mult, a = fabsf(t);
        uint8_t c = 0;
        if (nan_scale) {
          code[i] = 0;
          continue;
        }
        for (int q = 0; q < 7; ++q) {
          const int sel = (q % 2 == 0) ? a > thr[q] : a >= thr[q]; /* codes 1,3,5,7 strict; 2,4,6 inclusive */
          if (sel) c = (uint8_t)(q + 1);
        }
        uint32_t bits;
        memcpy(&bits, &t, 4);
        code[i] = (uint8_t)(c | ((bits >> 31) << 3));
      }
      for (int i = 0; i < 8; ++i) packed[r * (N / 2) + g * 8 + i] = (uint8_t)(code[2 * i] | (code[2 * i + 1] << 4));
      scales[((((r / 128) * NT + g / 4) * 32 + r % 32) * 4 + (r % 128) / 32) * 4 + g % 4] = sb;
    }
  }
}

/* ---- per-token symmetric int8 activation quantizer -------------------------
 * absmax = max |x[m,:]|, scale = absmax / 127, inv = 127 / absmax (f32
 * divisions), q = rne(clamp(x * inv, -128, 127)); a zero row gives scale 0 and
 * q 0. The clamp-then-round-half-even rule is the reference's integer
 * quantization (lib/Conversion/KIRToGPU/Quantization.cpp:191-203), written
 * here with floor and the parity of the floor as it does. */
void orc_i8_per_token_quantize(const float* x, int64_t M, int64_t K, int64_t ldx, int8_t* q, int64_t ldq,
                               float* scales) {
  for (int64_t m = 0; m < M; ++m) {
    float amax = 0.0f;
    for (int64_t k = 0; k < K; ++k) {
      const float a = fabsf(x[m * ldx + k]);
      if (a > amax) amax = a;
    }
    const float scale = amax == 0.0f ? 0.0f : amax / 127.0f;
    const float inv = amax == 0.0f ? 0.0f : 127.0f / amax;
    scales[m] = scale;
    for (int64_t k = 0; k < K; ++k) {
      float t = x[m * ldx + k] * inv;
      t = t < -128.0f ? -128.0f : (t > 127.0f ? 127.0f : t);
      const float fl = floorf(t);
      const float frac = t - fl;
      const int32_t base = (int32_t)fl;
      const int up = frac > 0.5f || (frac == 0.5f && (base & 1) != 0);
      q[m * ldq + k] = (int8_t)(base + up);
    }
  }
}
