// The reference's f16 MoE expert FFN (examples/kernels/ragged/moe.py:12-53)
// on the grouped [K, N] kernel (grouped_kn.h): two grouped projections over
// the ragged routing, then a deterministic per-token combine.
#include "grouped_kn.h"

using namespace gkn;

namespace {

// ---- the expert FFN's combine: y[token] += contributions of its members, in
// member order (the reference adds expert by expert: experts.py index_add_
// loop), through a per-token member list built on the device.
//
// One workgroup builds the list: counts per token (order-free atomics), an
// exclusive scan, a placement with per-token cursors (order-free), then each
// token's entries sorted ascending (a token has at most a few members), so
// the list is the same on every run.
constexpr int kListThreads = 1024;

// Token counts and placement cursors live in LDS up to this many tokens
// (64 KB), in the count array of the workspace beyond.
constexpr int kListLdsTokens = 16384;

// Inclusive sum of v over the workgroup's kListThreads threads, in thread
// order (wave prefix by shuffles, then the wave totals); `wsum` holds one
// slot per wave.
INTENT_DEVICE int block_inclusive_scan(int v, int* wsum) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int o = __shfl_up(v, d);
    if (lane >= d) v += o;
  }
  if (lane == 63) wsum[wave] = v;
  __syncthreads();
  if (wave == 0) {
    int w = lane < kListThreads / 64 ? wsum[lane] : 0;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int o = __shfl_up(w, d);
      if (lane >= d) w += o;
    }
    if (lane < kListThreads / 64) wsum[lane] = w;
  }
  __syncthreads();
  return v + (wave > 0 ? wsum[wave - 1] : 0);
}

// End of the member range: m1 = clampi(route_offsets[g + 1], m1, R) over the
// groups g in order from m1 = m0 (as find_tile clamps it) equals
// min(max(m0, max_g route_offsets[g + 1]), R): one block-wide max instead of
// E dependent loads. Every thread of the workgroup calls it.
INTENT_DEVICE int member_end(const int32_t* __restrict__ route_offsets, int E, int m0, int R, int* slot) {
  if (threadIdx.x == 0) *slot = m0;
  __syncthreads();
  int mx = m0;
  for (int g = threadIdx.x; g < E; g += blockDim.x) mx = max(mx, route_offsets[g + 1]);
  atomicMax(slot, mx);
  __syncthreads();
  return min(*slot, R);
}

template <bool kLds>
__global__ __launch_bounds__(kListThreads) void token_member_list_kernel(
    const int32_t* __restrict__ route_offsets, int E, const int32_t* __restrict__ members,
    const int32_t* __restrict__ route_token, int T, int R, int NR, int32_t* __restrict__ count,
    int32_t* __restrict__ start, int32_t* __restrict__ list) {
  __shared__ int32_t lds_cnt[kLds ? kListLdsTokens : 1];
  __shared__ int32_t wsum[kListThreads / 64];
  int32_t* cnt = kLds ? lds_cnt : count;
  const int tid = threadIdx.x;
  __shared__ int m1_slot;
  const int m0 = clampi(route_offsets[0], 0, R);
  const int m1 = member_end(route_offsets, E, m0, R, &m1_slot);
  auto token_of = [&](int i) { return clampi(route_token[clampi(members[i], 0, NR - 1)], 0, T - 1); };
  for (int t = tid; t < T; t += kListThreads) cnt[t] = 0;
  __syncthreads();
  for (int i = m0 + tid; i < m1; i += kListThreads) atomicAdd(&cnt[token_of(i)], 1);
  __syncthreads();
  // exclusive scan of the counts: each thread takes a contiguous slice of tokens
  const int per = (T + kListThreads - 1) / kListThreads;
  const int t0 = tid * per;
  int sum = 0;
  for (int t = t0; t < t0 + per && t < T; ++t) sum += cnt[t];
  const int incl = block_inclusive_scan(sum, wsum);
  int run = incl - sum;
  if (tid == kListThreads - 1) start[T] = incl;
  for (int t = t0; t < t0 + per && t < T; ++t) {
    start[t] = run;
    run += cnt[t];
    cnt[t] = 0;  // reused as the placement cursor
  }
  __syncthreads();
  for (int i = m0 + tid; i < m1; i += kListThreads) {
    const int t = token_of(i);
    const int pos = atomicAdd(&cnt[t], 1);
    list[start[t] + pos] = i;
  }
  __syncthreads();
  for (int t = tid; t < T; t += kListThreads) {
    const int b = start[t], e = start[t + 1];
    for (int a = b + 1; a < e; ++a) {  // insertion sort: ascending member index
      const int v = list[a];
      int c = a - 1;
      while (c >= b && list[c] > v) {
        list[c + 1] = list[c];
        --c;
      }
      list[c + 1] = v;
    }
  }
}

// The same list with every array in LDS (T, R <= kListLdsAll): the token of
// each member is gathered once, all loads of a thread issued together (the
// global-memory kernel above pays two dependent load latencies per member in
// each of its passes, and its sort reads the list back from global memory);
// counts, scan, placement and the per-token sort then run on LDS, and start /
// list are written out at the end. The list is the same as the kernel above
// produces: per token, its members in ascending index order.
constexpr int kListLdsAll = 8192;
constexpr int kListPer = kListLdsAll / kListThreads;  // members per thread

__global__ __launch_bounds__(kListThreads) void token_member_list_lds_kernel(
    const int32_t* __restrict__ route_offsets, int E, const int32_t* __restrict__ members,
    const int32_t* __restrict__ route_token, int T, int R, int NR, int32_t* __restrict__ start_out,
    int32_t* __restrict__ list_out) {
  extern __shared__ int32_t list_lds[];
  int32_t* cnt = list_lds;                 // T: counts, then placement cursors
  int32_t* start = cnt + T;                // T + 1
  int32_t* tok = start + T + 1;            // kListLdsAll: token of member m0 + j
  int32_t* list = tok + kListLdsAll;       // kListLdsAll
  __shared__ int32_t wsum[kListThreads / 64];
  const int tid = threadIdx.x;
  __shared__ int m1_slot;
  const int m0 = clampi(route_offsets[0], 0, R);
  const int m1 = member_end(route_offsets, E, m0, R, &m1_slot);
  const int n = m1 - m0;  // <= R <= kListLdsAll
  int mem[kListPer];
#pragma unroll
  for (int j = 0; j < kListPer; ++j) {
    const int i = tid + j * kListThreads;
    mem[j] = i < n ? members[m0 + i] : 0;
  }
#pragma unroll
  for (int j = 0; j < kListPer; ++j)
    if (tid + j * kListThreads < n) mem[j] = route_token[clampi(mem[j], 0, NR - 1)];
  for (int t = tid; t < T; t += kListThreads) cnt[t] = 0;
  __syncthreads();
#pragma unroll
  for (int j = 0; j < kListPer; ++j) {
    const int i = tid + j * kListThreads;
    if (i < n) {
      const int t = clampi(mem[j], 0, T - 1);
      tok[i] = t;
      atomicAdd(&cnt[t], 1);
    }
  }
  __syncthreads();
  const int per = (T + kListThreads - 1) / kListThreads;
  const int t0 = tid * per;
  int sum = 0;
  for (int t = t0; t < t0 + per && t < T; ++t) sum += cnt[t];
  const int incl = block_inclusive_scan(sum, wsum);
  int run = incl - sum;
  if (tid == kListThreads - 1) start[T] = incl;
  for (int t = t0; t < t0 + per && t < T; ++t) {
    start[t] = run;
    run += cnt[t];
    cnt[t] = 0;
  }
  __syncthreads();
  for (int i = tid; i < n; i += kListThreads) {
    const int t = tok[i];
    list[start[t] + atomicAdd(&cnt[t], 1)] = m0 + i;
  }
  __syncthreads();
  for (int t = tid; t < T; t += kListThreads) {
    const int b = start[t], e = start[t + 1];
    for (int a = b + 1; a < e; ++a) {  // insertion sort: ascending member index
      const int v = list[a];
      int c = a - 1;
      while (c >= b && list[c] > v) {
        list[c + 1] = list[c];
        --c;
      }
      list[c + 1] = v;
    }
  }
  __syncthreads();
  for (int t = tid; t <= T; t += kListThreads) start_out[t] = start[t];
  for (int i = tid; i < n; i += kListThreads) list_out[i] = list[i];
}

// y[t, d] += contrib[i, d] for the members i of token t in ascending order
// (one add per member, no fma): f32 throughout.
__global__ __launch_bounds__(256) void token_combine_kernel(const float* __restrict__ contrib, int64_t ldc,
                                                            const int32_t* __restrict__ start,
                                                            const int32_t* __restrict__ list, int T, int D,
                                                            float* __restrict__ y, int64_t ldy) {
  const int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int d4 = (D + 3) / 4;
  if (id >= (int64_t)T * d4) return;
  const int t = (int)(id / d4);
  const int d = (int)(id % d4) * 4;
  const int b = start[t], e = start[t + 1];
  float* yo = y + (int64_t)t * ldy + d;
  if (d + 3 < D && (ldy & 3) == 0 && (ldc & 3) == 0) {
    f32x4 acc = *reinterpret_cast<const f32x4*>(yo);
    for (int k = b; k < e; ++k) {
      const f32x4 c = *reinterpret_cast<const f32x4*>(contrib + (int64_t)list[k] * ldc + d);
      acc = f32x4{__fadd_rn(acc[0], c[0]), __fadd_rn(acc[1], c[1]), __fadd_rn(acc[2], c[2]), __fadd_rn(acc[3], c[3])};
    }
    *reinterpret_cast<f32x4*>(yo) = acc;
  } else {
    for (int c = 0; c < 4 && d + c < D; ++c) {
      float acc = yo[c];
      for (int k = b; k < e; ++k) acc = __fadd_rn(acc, contrib[(int64_t)list[k] * ldc + d + c]);
      yo[c] = acc;
    }
  }
}

size_t round256(size_t v) { return (v + 255) & ~(size_t)255; }

struct FfnLayout {
  size_t hidden, contrib, count, start, list, bytes;
};

FfnLayout ffn_layout(int64_t T, int64_t R, int64_t D, int64_t F) {
  FfnLayout L{};
  size_t o = 0;
  L.hidden = o;  o = round256(o + sizeof(uint16_t) * (size_t)R * F);
  L.contrib = o; o = round256(o + sizeof(float) * (size_t)R * D);
  L.count = o;   o = round256(o + sizeof(int32_t) * (size_t)T);
  L.start = o;   o = round256(o + sizeof(int32_t) * (size_t)(T + 1));
  L.list = o;    o = round256(o + sizeof(int32_t) * (size_t)R);
  L.bytes = o;
  return L;
}

}  // namespace

extern "C" size_t intent_moe_expert_ffn_workspace_size(int64_t T, int64_t R, int64_t D, int64_t F) {
  if (T < 0 || R < 0 || D < 0 || F < 0) return 0;
  return ffn_layout(T, R, D, F).bytes;
}

extern "C" int intent_moe_expert_ffn(const void* x, int64_t T, int64_t D, int64_t x_ld, const int32_t* route_offsets,
                                     int64_t E, const int32_t* member_routes, int64_t R, const int32_t* route_token,
                                     const float* route_weights, int64_t NR, const void* w1, const void* w2,
                                     int64_t F, float* y, int64_t y_ld, void* workspace, size_t workspace_bytes,
                                     void* stream) {
  intent::clear_error();
  INTENT_REQUIRE(T >= 0 && D >= 0 && E >= 1 && R >= 0 && NR >= 0 && F >= 0 && T <= INT32_MAX && R <= INT32_MAX &&
                     D <= INT32_MAX && F <= INT32_MAX && E <= (1 << 20),
                 INTENT_ERR_INVALID_ARGUMENT, "bad extents");
  if (T == 0 || D == 0 || R == 0) return INTENT_OK;
  int st = kn_shape_check(D, F, F, w1, "moe_expert_ffn (w1)");
  if (st != INTENT_OK) return st;
  st = kn_shape_check(F, D, D, w2, "moe_expert_ffn (w2)");
  if (st != INTENT_OK) return st;
  INTENT_REQUIRE(x && route_offsets && member_routes && route_token && route_weights && y,
                 INTENT_ERR_INVALID_ARGUMENT, "null pointer argument");
  INTENT_REQUIRE(x_ld >= D && y_ld >= D, INTENT_ERR_INVALID_ARGUMENT, "leading stride smaller than the row");
  INTENT_REQUIRE(intent::aligned16(x) && x_ld % 8 == 0, INTENT_ERR_ALIGNMENT,
                 "x must be 16-byte aligned with 16-byte row strides");
  INTENT_REQUIRE(intent::fits_offset(T, x_ld * 2) && intent::fits_offset(R, F * 2) && intent::fits_offset(R, D * 4),
                 INTENT_ERR_UNSUPPORTED, "moe_expert_ffn: operands exceed 31-bit buffer offsets");
  const FfnLayout L = ffn_layout(T, R, D, F);
  INTENT_REQUIRE(workspace && workspace_bytes >= L.bytes, INTENT_ERR_WORKSPACE, "workspace needs %zu bytes, got %zu",
                 L.bytes, workspace_bytes);
  INTENT_REQUIRE(intent::aligned16(workspace), INTENT_ERR_ALIGNMENT, "workspace must be 16-byte aligned");
  char* ws = (char*)workspace;
  uint16_t* hidden = (uint16_t*)(ws + L.hidden);
  float* contrib = (float*)(ws + L.contrib);
  int32_t* count = (int32_t*)(ws + L.count);
  int32_t* start = (int32_t*)(ws + L.start);
  int32_t* list = (int32_t*)(ws + L.list);
  hipStream_t s = (hipStream_t)stream;
  const int64_t ntiles = (R + GTile::BM - 1) / GTile::BM + E;
  INTENT_REQUIRE(ntiles * ((F + GTile::BN - 1) / GTile::BN) < (1ll << 31), INTENT_ERR_UNSUPPORTED, "grid too large");
  // hidden[i] = f16(relu(x[token(i)] @ w1[e])) for the members i of expert e
  launch_grouped<mp::F16Math, true, GEpi::kReluF16>(x, x_ld, route_offsets, E, R, member_routes, route_token, NR, T,
                                                    nullptr, w1, F, D * F, F, D, (int)ntiles, hidden, F, s);
  st = intent::launch_status("grouped_kn_kernel<moe w1 relu>");
  if (st != INTENT_OK) return st;
  // contrib[i] = route_weight * (hidden[i] @ w2[e])
  launch_grouped<mp::F16Math, false, GEpi::kRouteWeight>(hidden, F, route_offsets, E, R, member_routes, nullptr, NR,
                                                         T, route_weights, w2, D, F * D, D, F, (int)ntiles, contrib,
                                                         D, s);
  st = intent::launch_status("grouped_kn_kernel<moe w2 weighted>");
  if (st != INTENT_OK) return st;
  if (T <= kListLdsAll && R <= kListLdsAll) {
    const size_t lds = sizeof(int32_t) * (size_t)(2 * T + 1 + 2 * kListLdsAll);
    if (lds > 65536) {
      const hipError_t e = hipFuncSetAttribute((const void*)token_member_list_lds_kernel,
                                               hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
      INTENT_REQUIRE(e == hipSuccess, INTENT_ERR_LAUNCH, "token_member_list: %zu bytes of LDS refused (%s)", lds,
                     hipGetErrorString(e));
    }
    hipLaunchKernelGGL(token_member_list_lds_kernel, dim3(1), dim3(kListThreads), lds, s, route_offsets, (int)E,
                       member_routes, route_token, (int)T, (int)R, (int)NR, start, list);
  } else {
    hipLaunchKernelGGL(T <= kListLdsTokens ? token_member_list_kernel<true> : token_member_list_kernel<false>, dim3(1),
                       dim3(kListThreads), 0, s, route_offsets, (int)E, member_routes, route_token, (int)T, (int)R,
                       (int)NR, count, start, list);
  }
  st = intent::launch_status("token_member_list");
  if (st != INTENT_OK) return st;
  const int64_t items = T * ((D + 3) / 4);
  hipLaunchKernelGGL(token_combine_kernel, dim3((unsigned)((items + 255) / 256)), dim3(256), 0, s, contrib, D, start,
                     list, (int)T, (int)D, y, y_ld);
  return intent::launch_status("token_combine");
}
