/*
 * intent_amd.h — C ABI of the MI355X (gfx950) quantized-contraction library.
 *
 * One flat C entry per kernel family. Every view is passed as a device pointer
 * plus int64 extents and an int64 leading (row) stride in ELEMENTS; the inner
 * axis must be unit-stride. This is the slot model the reference host uses for
 * natively compiled entries (python/intent/runtime/native.py:14-120: pointer,
 * extent and stride slots per view, one C symbol per entry), with three
 * additions:
 *   - a `stream` argument (a hipStream_t passed as void*): launches are
 *     asynchronous on that stream, as GPU artifact calls run on the provider's
 *     current stream (python/intent/runtime/artifact.py:149-162);
 *   - an int status return (INTENT_OK or a negative INTENT_ERR_* code) instead
 *     of void (python/intent/runtime/mojo/program.py:255);
 *   - intent_amd_last_error(), a thread-local message for the last failure.
 *
 * The library never allocates user-visible memory: outputs and workspaces
 * belong to the caller. No entry synchronises the stream.
 *
 * Empty extents: M = 0 or N = 0 is a no-op. An empty K (K = 0, no groups or
 * blocks) is a contraction that sums nothing (doc/dsl/core.en.md:213): the
 * entry writes its epilogue of a zero accumulator to the whole output (zeros,
 * the bias, quantized_gemm's epilogue, the in-place output plus zero) and
 * reads no operand along K, whose pointers may then be null.
 *
 * Quantized formats (row-major, K contiguous):
 *   W4 asymmetric group quant: packed uint8 [N, K/2]; byte j of row n holds
 *       k = 2j in its low nibble and k = 2j+1 in its high nibble; scales f16
 *       [N, K/group]; zeros uint8 [N, K/group] (values 0..15);
 *       w[n,k] = (q[n,k] - zero[n,k/g]) * scale[n,k/g].
 *   W8 per-channel symmetric: int8 [N, K]; scales f16 [N]; w = q * scale[n].
 *   W8A8: int8 activations [M, K] with f32 per-token scales [M]; int8 weights
 *       [N, K] with f32 per-channel scales [N].
 */
#ifndef INTENT_AMD_H
#define INTENT_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define INTENT_AMD_ABI_VERSION 1

#define INTENT_OK 0
#define INTENT_ERR_INVALID_ARGUMENT (-1) /* bad extent, stride, null pointer */
#define INTENT_ERR_ALIGNMENT (-2)        /* pointer/stride not 16-byte aligned */
#define INTENT_ERR_UNSUPPORTED (-3)      /* shape outside what the kernels cover */
#define INTENT_ERR_LAUNCH (-4)           /* HIP launch or device query failed */
#define INTENT_ERR_WORKSPACE (-5)        /* workspace too small */

/* Library facts. */
int intent_amd_abi_version(void);
const char* intent_amd_last_error(void);
/* Name of the last kernel the calling thread launched through this library
 * (the kernel variant an entry dispatched to, e.g. for profiling reports);
 * "" before the first launch. */
const char* intent_amd_last_kernel(void);
/* Writes the gcnArchName of `device` into buf; returns INTENT_OK or an error. */
int intent_amd_device_arch(int device, char* buf, int64_t buf_len);

/*
 * W8A16: y[m,n] = f16( scale[n] * sum_k f32(x[m,k]) * f32(w[n,k]) ), fp32
 * accumulation.
 * Replaces: weight-only int8 contraction written as I.cast(W_i8, f16) ->
 * I.matmul(acc_dtype=f32) -> scale (doc/dsl/core.en.md:246,
 * lib/Conversion/KIRToCPU/Contractions.cpp:12-41).
 * x f16 [M,K] (stride x_ld); w int8 [N,K] (w_ld); scales f16 [N]; y f16 [M,N].
 * Any K and strides: K % 64 == 0 with 16-byte aligned rows runs the tiled
 * kernels, other shapes a generic kernel (same arithmetic, lower throughput).
 */
int intent_w8a16_matmul(const void* x, int64_t M, int64_t K, int64_t x_ld,
                        const int8_t* w, int64_t N, int64_t w_ld,
                        const void* scales,
                        void* y, int64_t y_ld, void* stream);

/*
 * W4A16 asymmetric group-dequant contraction:
 * y[m,n] = f16( sum_k f32(x[m,k]) * (q[n,k] - z[n,k/g]) * s[n,k/g] ).
 * Replaces weight_only_int4_matmul (examples/kernels/contraction/
 * weight_only_int4.py:18-51; CPU oracle experiments/cpu/baselines/pytorch/
 * cpu_runtime.py:97-102) for the asymmetric uint4, [N, K/2]-packed format.
 * Requires K even and K % group == 0 (else INTENT_ERR_INVALID_ARGUMENT).
 * K % 128 == 0, group % 32 == 0 and 16-byte aligned rows (x_ld % 8 == 0,
 * packed_ld % 16 == 0) take the fast kernels, other shapes a generic kernel
 * (same per-element dequantisation, f32 sums).
 * `intent_w4a16_matmul` picks the decode GEMV kernel for M <= 16 and the
 * MFMA tile kernel otherwise; the _gemv / _gemm entries force one kernel
 * (the _gemv entry covers M <= 16).
 */
int intent_w4a16_matmul(const void* x, int64_t M, int64_t K, int64_t x_ld,
                        const uint8_t* packed, int64_t N, int64_t packed_ld,
                        const void* scales, const uint8_t* zeros, int64_t qparam_ld,
                        int64_t group_size,
                        void* y, int64_t y_ld, void* stream);
int intent_w4a16_gemv(const void* x, int64_t M, int64_t K, int64_t x_ld,
                      const uint8_t* packed, int64_t N, int64_t packed_ld,
                      const void* scales, const uint8_t* zeros, int64_t qparam_ld,
                      int64_t group_size,
                      void* y, int64_t y_ld, void* stream);
int intent_w4a16_gemm(const void* x, int64_t M, int64_t K, int64_t x_ld,
                      const uint8_t* packed, int64_t N, int64_t packed_ld,
                      const void* scales, const uint8_t* zeros, int64_t qparam_ld,
                      int64_t group_size,
                      void* y, int64_t y_ld, void* stream);

/*
 * W8A8: out[m,n] = bf16( f32(acc[m,n]) * a_scale[m] * w_scale[n] ), with
 * acc[m,n] = sum_k i32(a[m,k]) * i32(w[n,k]) computed exactly in int32
 * (modulo 2^32). The two multiplies are evaluated left to right in fp32 and
 * rounded to bf16 to nearest-even.
 * Replaces the integer contraction branch (lib/Conversion/KIRToCPU/
 * Contractions.cpp:30-35,79-80) plus per-token/per-channel scale epilogue
 * (examples/kernels/contraction/gemm.py:83-106 pattern).
 * Any K and strides (K % 64 == 0 with 16-byte aligned rows: the tiled
 * kernels; else a generic kernel with the same exact sums and epilogue).
 */
int intent_w8a8_gemm(const int8_t* a, int64_t M, int64_t K, int64_t a_ld,
                     const float* a_scales,
                     const int8_t* w, int64_t N, int64_t w_ld,
                     const float* w_scales,
                     void* out, int64_t out_ld, void* stream);

/*
 * int8 x int8 -> int32 contraction with optional int32 bias (nullable):
 * c[m,n] = sum_k i32(a[m,k]) * i32(w[n,k]) + bias[n], modulo 2^32.
 * Replaces gemm_i8 (examples/kernels/contraction/gemm.py:29-39), with the
 * weight given K-contiguous as [N, K]. Any K and strides, as intent_w8a8_gemm.
 */
int intent_i8_gemm_i32(const int8_t* a, int64_t M, int64_t K, int64_t a_ld,
                       const int8_t* w, int64_t N, int64_t w_ld,
                       const int32_t* bias,
                       int32_t* c, int64_t c_ld, void* stream);

/*
 * The same contraction with the weight as the reference's gemm_i8 passes it
 * (examples/kernels/contraction/gemm.py:29-39, b [K, N], N contiguous, b_ld
 * bytes), read in place (no transposed copy):
 * c[m,n] = sum_k i32(a[m,k]) * i32(b[k,n]) + bias[n], modulo 2^32.
 * K a positive multiple of 128, N % 16 == 0, 16-byte aligned rows.
 */
int intent_i8_gemm_i32_kn(const int8_t* a, int64_t M, int64_t K, int64_t a_ld,
                          const int8_t* b, int64_t N, int64_t b_ld,
                          const int32_t* bias,
                          int32_t* c, int64_t c_ld, void* stream);

/*
 * MoE router: per token, top_k experts by logit (ties -> lower expert index)
 * and their softmax probabilities (fp32, over all E experts; renormalised
 * over the selected top_k when `renormalize` != 0).
 * No reference counterpart exists (the reference takes topk_ids as an input,
 * experiments/_common/support.py:113-130); this is the producer of that input.
 * logits f32 [T,E]; topk_ids i32 [T,top_k]; topk_weights f32 [T,top_k].
 * Requires 1 <= top_k <= min(E, 8). E <= 256 runs one wave per token, larger E
 * one thread per token (same selections and ties).
 */
int intent_moe_route(const float* logits, int64_t T, int64_t E, int64_t top_k,
                     int renormalize, int32_t* topk_ids, float* topk_weights,
                     void* stream);

/*
 * MoE alignment: expert histogram, block-padded exclusive prefix, STABLE
 * scatter of route ids (route = token*top_k + choice) into expert segments,
 * and the expert id of every block.
 * Replaces moe_count_routes / moe_prefix_routes / moe_scatter_routes /
 * moe_mark_expert_blocks (examples/kernels/routing/moe_align.py:14-86) as
 * composed by MoEAlignment (examples/programs/composition.py:134-174), with
 * the deterministic order of moe_align_block_size
 * (experiments/cpu/baselines/pytorch/cpu_runtime.py:1081-1098).
 *   sorted_route_ids i32 [capacity], capacity >= R + E*(block_size-1),
 *     R = T*top_k; unused slots hold the sentinel R;
 *   expert_blocks i32 [num_blocks], num_blocks >= ceil(capacity/block_size);
 *     blocks past the padded total hold -1;
 *   expert_offsets i32 [E+1]; total_padded i32 [1].
 * Route ids whose expert is outside [0,E) are dropped.
 * Requires E <= 2048 (its LDS holds 19 counters per expert).
 */
int intent_moe_align(const int32_t* topk_ids, int64_t T, int64_t top_k, int64_t E,
                     int64_t block_size,
                     int32_t* sorted_route_ids, int64_t capacity,
                     int32_t* expert_blocks, int64_t num_blocks,
                     int32_t* expert_offsets, int32_t* total_padded, void* stream);

/*
 * Grouped W4 gate/up projection with SiLU gating over the aligned routes:
 * for every padded row p with route r = sorted_route_ids[p] < R, token
 * t = r / top_k and expert e = expert_blocks[p / block_size]:
 *   g[f] = sum_h x[t,h] * Wgu[e][f, h],  u[f] = sum_h x[t,h] * Wgu[e][F+f, h]
 *   act[p,f] = f16( silu(g) * u ),  silu(g) = g / (1 + exp(-g))  (fp32)
 * Rows with r == R are written as zeros.
 * Wgu: packed [E][2F, H/2], scales f16 / zeros u8 [E][2F, H/g].
 * act f16 [num_blocks*block_size, F].
 * Replaces the first contraction + activation of moe_expert_ffn
 * (examples/kernels/ragged/moe.py:28-45) for SiLU-gated W4 experts.
 * Requires H even and a multiple of group_size. Block size 64 or 128 with
 * H % 128 == 0, F % 64 == 0, group 32 or a multiple of 64 and aligned rows
 * runs the tiled kernels, block size 160 too when the group is a multiple of
 * 64, H / group a multiple of 4 and scales/zeros 4-byte aligned; any other
 * block size or shape a generic kernel.
 */
int intent_moe_gate_up_w4(const void* x, int64_t T, int64_t H, int64_t x_ld,
                          const int32_t* sorted_route_ids, const int32_t* expert_blocks,
                          int64_t num_blocks, int64_t block_size, int64_t top_k,
                          const uint8_t* w_packed, const void* w_scales,
                          const uint8_t* w_zeros, int64_t E, int64_t F, int64_t group_size,
                          void* act, int64_t act_ld, void* stream);

/*
 * Grouped W4 down projection: for every padded row p with route r < R,
 *   out[r, d] = sum_f f32(act[p,f]) * Wd[e][d, f]   (fp32 result)
 * Wd: packed [E][H, F/2], scales/zeros [E][H, F/g]; out f32 [R, H].
 * Replaces the second contraction of moe_expert_ffn
 * (examples/kernels/ragged/moe.py:46-53).
 * Requires F even and a multiple of group_size. Block size 64 or 128 with
 * F % 128 == 0, group 32 or a multiple of 64 and aligned rows runs the
 * tiled kernels, block size 160 too when the group is a multiple of 64,
 * F / group a multiple of 4 and scales/zeros 4-byte aligned; any other
 * block size or shape a generic kernel.
 */
int intent_moe_down_w4(const void* act, int64_t act_ld,
                       const int32_t* sorted_route_ids, const int32_t* expert_blocks,
                       int64_t num_blocks, int64_t block_size, int64_t R,
                       const uint8_t* w_packed, const void* w_scales,
                       const uint8_t* w_zeros, int64_t E, int64_t H, int64_t F,
                       int64_t group_size,
                       float* out, int64_t out_ld, void* stream);

/*
 * Weighted combine: y[t,:] += w[t,0]*out[t*k+0,:]; y[t,:] += w[t,1]*out[...]
 * ... slot by slot in order (each step one fp32 multiply then one fp32 add).
 * Replaces the scatter_reduce(add) of moe_expert_ffn
 * (examples/kernels/ragged/moe.py:48-53), in a fixed order.
 * y f32 [T,H] is read and written.
 */
int intent_moe_combine(const float* route_out, int64_t out_ld,
                       const float* topk_weights, int64_t T, int64_t top_k,
                       float* y, int64_t H, int64_t y_ld, void* stream);

/*
 * Whole quantized MoE expert FFN from router logits: route -> align ->
 * gate/up(SiLU) -> down -> combine into y (f32 [T,H], accumulated).
 * Replaces moe_expert_ffn (examples/kernels/ragged/moe.py:12-53) together
 * with its host alignment (examples/programs/composition.py:134-174).
 * `workspace` must hold intent_moe_workspace_size(T, top_k, E, H, F, 0) bytes
 * (16-byte aligned); the composite aligns routes to 160-row blocks when
 * experts average at least 96 routes (T*top_k >= 96*E) and both projections
 * take the 160-row tile, else to 128-row blocks.
 * intent_moe_workspace_size with block_size > 0 gives the staged pipeline's
 * buffers for that block size; block_size <= 0 gives the composite's, which
 * covers either block size it may pick.
 * If topk_ids_out / topk_weights_out are non-null the routing results are
 * also copied there ([T,top_k] each).
 */
size_t intent_moe_workspace_size(int64_t T, int64_t top_k, int64_t E, int64_t H,
                                 int64_t F, int64_t block_size);
int intent_moe_expert_ffn_w4(const float* router_logits, const void* x, int64_t T,
                             int64_t H, int64_t E, int64_t top_k, int renormalize,
                             const uint8_t* wgu_packed, const void* wgu_scales,
                             const uint8_t* wgu_zeros,
                             const uint8_t* wd_packed, const void* wd_scales,
                             const uint8_t* wd_zeros,
                             int64_t F, int64_t group_size,
                             float* y, void* workspace, size_t workspace_bytes,
                             int32_t* topk_ids_out, float* topk_weights_out,
                             void* stream);

/*
 * GGUF K-quant records (doc/dsl/quantized-operations.en.md:11-70).
 * Q4_K record: 144 bytes (f16 d, f16 dmin, 6-bit sc[8]/m[8] in bytes 4..15,
 * 256 nibbles in bytes 16..143). Q8_K record: 292 bytes (f32 ds, 256 x i8,
 * 16 x i16 bsum). Little-endian, no padding.
 *
 * intent_q8k_quantize: f32 x [G, 256] (row stride x_ld elements, 16-byte
 * aligned, x_ld % 4 == 0) -> G Q8_K records (row stride records_ld bytes,
 * 4-byte aligned). Replaces I.quantize(values, format=I.quant.q8_k)
 * (quantized-operations.en.md:5-10,62-70; RVV baseline quantize_row,
 * experiments/cpu/baselines/weft/tianchenrv/contraction/q4_k_projection/
 * q4_k_projection.py:29-48). Bit-exact: IEEE division for the inverse and
 * ds, one f32 multiply per value, round half to even, saturation to i8.
 */
int intent_q8k_quantize(const float* x, int64_t G, int64_t x_ld,
                        uint8_t* records, int64_t records_ld, void* stream);

/*
 * y[n] = quantized_dot(W[n, 0..G), Xq[0..G)) for N rows of G Q4_K records
 * (row stride w_ld bytes, 16-byte aligned) and one vector of G Q8_K records
 * (contiguous, 4-byte aligned); y f32 [N]. Replaces I.quantized_dot(...,
 * lhs_format=q4_k, rhs_format=q8_k, acc_dtype=f32)
 * (quantized-operations.en.md:38-58; baseline compute, q4_k_projection.py:
 * 56-72) applied per row as in quantized_projection
 * (examples/kernels/quantization/quantized_projection.py:15-19).
 * Bit-exact: integer sub-sums, one rounding per f32 operation, records
 * added in increasing order starting from +0. G == 0 gives +0 per row.
 */
int intent_q4k_q8k_gemv(const uint8_t* w, int64_t N, int64_t G, int64_t w_ld,
                        const uint8_t* xq, float* y, void* stream);

/*
 * Whole quantized_projection (examples/kernels/quantization/
 * quantized_projection.py:5-19): quantize x (f32 [G, 256]) into xq_records
 * (caller-provided, G * 292 bytes, 4-byte aligned; left holding the Q8_K
 * records) and run intent_q4k_q8k_gemv into y f32 [N].
 */
int intent_q4k_projection(const uint8_t* w, int64_t N, int64_t G, int64_t w_ld,
                          const float* x, int64_t x_ld, uint8_t* xq_records,
                          float* y, void* stream);

/*
 * intent_q4k_projection without the caller's record buffer: no counterpart in
 * the reference; for callers that cannot allocate (code under HIP graph
 * capture, serving loops, harnesses that forbid hipMalloc). Same arguments and
 * result as intent_q4k_projection minus xq_records; the Q8_K records live in a
 * fixed device array of the library (one per GPU, 299,008 bytes, kept until
 * the process ends), so G <= 1024 (K <= 262144), else INTENT_ERR_UNSUPPORTED.
 * Allocates nothing (the array's device address is looked up on the first
 * call on each device, with that device current: make that first call
 * outside graph capture). Calls that overlap on one GPU share the array and
 * race; serialise them (one stream, or events).
 */
int intent_q4k_projection_noalloc(const uint8_t* w, int64_t N, int64_t G, int64_t w_ld,
                                  const float* x, int64_t x_ld, float* y, void* stream);

/*
 * Groupwise FP8 activation quantizer, bit-exact: for each row and group of
 * 128 columns, scale = max(absmax, eps) / 448 (eps = 1e-12 for bf16 input,
 * 1e-4 for f32), q = E4M3FN(min(max(x / scale, -448), 448)) rounded to
 * nearest even. x is f32 or bf16 (x_is_bf16) [M, N] with row stride x_ld
 * elements; q E4M3FN bytes [M, N] (row stride q_ld); scales f32 [M, G]
 * (G >= ceil(N/128); groups past N get eps / 448). Replaces
 * bf16_groupwise_fp8_quantize / f32_groupwise_fp8_quantize
 * (examples/kernels/quantization/fp8.py:11-69; CPU side
 * experiments/cpu/baselines/pytorch/cpu_runtime.py:142-147). N % 4 == 0.
 */
int intent_fp8_groupwise_quantize(const void* x, int x_is_bf16, int64_t M, int64_t N,
                                  int64_t x_ld, uint8_t* q, int64_t q_ld, float* scales,
                                  int64_t G, int64_t scales_ld, void* stream);

/*
 * Low-bit weight x int8 activation GEMMs, exact int32 (modulo 2^32).
 * a: int8 [M, K] (row stride a_ld, 16-byte aligned rows); K % 128 == 0.
 *
 * intent_w4a8_gemm: w_packed u8 [N, K/2] (row stride w_ld bytes, 8-byte
 * aligned), two's-complement nibbles, low nibble = even k;
 * out[n, m] = sum_k w[n, k] * a[m, k], out int32 [N, M] (row stride out_ld).
 * Replaces w4a8_packed_matmul (examples/kernels/contraction/
 * weight_only_int4.py:54-91).
 *
 * intent_bitnet_int2_gemm: w_packed u8 [N, K/4] (row stride w_ld bytes,
 * 4-byte aligned), values 0..3 interleaved: k in byte (k/16)*4 + k%4 at bit
 * 2*((k/4)%4); out[m, n] = sum_k a[m, k] * w[n, k], out int32 [M, N].
 * Replaces bitnet_int2_matmul (weight_only_int4.py:94-124).
 */
int intent_w4a8_gemm(const int8_t* a, int64_t M, int64_t K, int64_t a_ld,
                     const uint8_t* w_packed, int64_t N, int64_t w_ld,
                     int32_t* out, int64_t out_ld, void* stream);
int intent_bitnet_int2_gemm(const int8_t* a, int64_t M, int64_t K, int64_t a_ld,
                            const uint8_t* w_packed, int64_t N, int64_t w_ld,
                            int32_t* out, int64_t out_ld, void* stream);

/*
 * MX block-scaled FP8 GEMM: out[m, n] = sum_k (a[m,k] * 2^(sa[m,k/32]-127)) *
 * (b[n,k] * 2^(sb[n,k/32]-127)), a and b OCP E4M3FN bytes with K contiguous
 * (row strides a_ld, b_ld bytes, 16-byte aligned), E8M0 scales u8 [M, K/32]
 * and [N, K/32] (row strides a_scales_ld, b_scales_ld, multiples of 4), out
 * f32 [M, N]; K % 128 == 0. f32 accumulation on v_mfma_scale_f32_32x32x64_f8f6f4.
 * Replaces block_scaled_matmul (examples/kernels/contraction/block_scaled.py:
 * 11-39; CPU semantics lib/Conversion/KIRToCPU/Contractions.cpp:177-259),
 * whose rhs [KB, 32, N] is here passed as rows n with K contiguous (the
 * layout of the reference's own benchmark view, experiments/cpu/providers/
 * mojo/contraction.py:285-305).
 */
int intent_mxfp8_gemm(const uint8_t* a, int64_t M, int64_t K, int64_t a_ld,
                      const uint8_t* a_scales, int64_t a_scales_ld,
                      const uint8_t* b, int64_t N, int64_t b_ld,
                      const uint8_t* b_scales, int64_t b_scales_ld,
                      float* out, int64_t out_ld, void* stream);

/* Byte-matrix transpose: dst[c * dst_ld + r] = src[r * src_ld + c] for an
 * R x C matrix of one-byte elements (FP8). Plumbing for the contractions whose
 * right operand the reference passes as [K, N] (N contiguous): the FP8 MFMA
 * reads both operands K-contiguous. Replaces no reference function.
 */
int intent_fp8_transpose(const uint8_t* src, int64_t rows, int64_t cols, int64_t src_ld,
                         uint8_t* dst, int64_t dst_ld, void* stream);

/* Per-tensor scaled FP8 (E4M3FN) GEMM with an f16 result. Replaces
 * scaled_fp8_matmul (examples/kernels/contraction/block_scaled.py:42-63) with
 * splits == 1, accumulate == 0: out = f16((acc * a_scale) * b_scale), acc the
 * f32 sum over k; and scaled_fp8_splitk_matmul (block_scaled.py:66-98) with
 * splits == SP, accumulate == 1, where k = (it*SP + s)*256 + r (the operands'
 * [.., IT, SP, 256] layout): for s = 0 .. SP-1 in order,
 * out = f16(out + f16((acc_s * a_scale) * b_scale)) (the reference's CPU
 * baseline order, experiments/cpu/baselines/pytorch/cpu_runtime.py:133-139;
 * its GPU form adds the splits with relaxed atomics, in no fixed order).
 * a: [M, K] (K contiguous, a_ld bytes); bt: the right operand as [N, K] rows
 * (bt_ld bytes; use intent_fp8_transpose for a [K, N] operand); out: f16
 * [M, N] (out_ld elements, read and written when accumulate).
 * K % 128 == 0 (K % (256 * splits) == 0 when splits > 1).
 */
int intent_scaled_fp8_gemm(const uint8_t* a, int64_t M, int64_t K, int64_t a_ld,
                           const uint8_t* bt, int64_t N, int64_t bt_ld,
                           float a_scale, float b_scale, int64_t splits, int accumulate,
                           void* out, int64_t out_ld, void* stream);

/* intent_scaled_fp8_gemm with the right operand as the reference passes it:
 * b [K, N] E4M3FN (N contiguous, b_ld bytes), read in place (no transposed
 * copy). Same semantics, splits and K rules; additionally N % 16 == 0.
 * Replaces the same functions (block_scaled.py:42-63 and :66-98, whose rhs is
 * [K, N] and [IT, SP, 256, N]).
 */
int intent_scaled_fp8_gemm_kn(const uint8_t* a, int64_t M, int64_t K, int64_t a_ld,
                              const uint8_t* b, int64_t N, int64_t b_ld,
                              float a_scale, float b_scale, int64_t splits, int accumulate,
                              void* out, int64_t out_ld, void* stream);

/* DeepGEMM-style FP8 GEMM with f32 block scales. Replaces deepgemm_fp8_2xacc
 * (examples/kernels/contraction/block_scaled.py:101-122; CPU baseline
 * experiments/cpu/baselines/pytorch/cpu_runtime.py:127-131).
 * a: [M, K] E4M3FN (K = KB * 128 contiguous, a_ld bytes); a_scales: f32 [M, KB]
 * (a_scales_ld elements); b: [N, K] E4M3FN rows (b_ld bytes); b_scales: f32
 * [ceil(N / 128), KB], one per 128-row block of b and 128-k block;
 * out: bf16 bits [M, N] (out_ld elements):
 *   out[m, n] = bf16(sum_kb (sum_k a*b) * a_scales[m, kb] * b_scales[n/128, kb])
 * The reference scales the operands before the product; the sums agree to
 * rounding.
 */
int intent_deepgemm_fp8(const uint8_t* a, int64_t M, int64_t K, int64_t a_ld,
                        const float* a_scales, int64_t a_scales_ld,
                        const uint8_t* b, int64_t N, int64_t b_ld,
                        const float* b_scales, int64_t b_scales_ld,
                        void* out, int64_t out_ld, void* stream);

/* FP8 x FP8 -> FP8 GEMM. Replaces fp8_e4m3_matmul (format 0) and
 * fp8_e5m2_matmul (format 1) (examples/kernels/contraction/weight_only_int4.py:
 * 178-215): out[m, n] = cast(sum_k a[m, k] * bt[n, k] in f32, format), nearest
 * even (doc/dsl/types-numerics-and-effects.en.md:86-89: E5M2 overflows to
 * infinity; E4M3FN results must lie within +-448, larger ones saturate here).
 * a: [M, K], bt: [N, K] rows (K contiguous, K % 128 == 0), out: [M, N] bytes.
 */
int intent_fp8_gemm(const uint8_t* a, int64_t M, int64_t K, int64_t a_ld,
                    const uint8_t* bt, int64_t N, int64_t bt_ld, int format,
                    uint8_t* out, int64_t out_ld, void* stream);

/* FP4 (E2M1) weight x bf16 activation GEMM. Replaces dequant_bf16_fp4_matmul
 * (examples/kernels/contraction/weight_only_int4.py:127-175; CPU baseline
 * experiments/cpu/baselines/pytorch/cpu_runtime.py:117-124).
 * x: bf16 bits [M, K] (x_ld elements); packed: [N, K/2] bytes, each big-endian
 * 16-bit word (p[2i] << 8 | p[2i+1]) holding k = 4i .. 4i+3 in the reference's
 * bit layout; y: bf16 bits [M, N]: y = bf16(sum_k x * e2m1(W)), f32 accumulation.
 * K % 64 == 0.
 */
int intent_fp4_bf16_matmul(const void* x, int64_t M, int64_t K, int64_t x_ld,
                           const uint8_t* packed, int64_t N, int64_t packed_ld,
                           void* y, int64_t y_ld, void* stream);

/* Repacks the reference's own W4 layout for the W4A16 entries. Used by
 * weight_only_int4_matmul (examples/kernels/contraction/weight_only_int4.py:18-51):
 * packed int32 [P = K/8, N] (eight signed nibbles of consecutive k per word,
 * nibble k % 8 at bits 4(k % 8); packed_ld elements) and f16 scales [G, N]
 * (scales_ld elements) become q_out [N, K/2] bytes (low nibble = even k, each
 * nibble with its top bit flipped), s_out f16 [N, G] and z_out [N, G] = 8, so
 * that (q - z) * s equals the reference's signed nibble times its scale.
 */
int intent_w4_sym_repack(const int32_t* packed, int64_t P, int64_t N, int64_t packed_ld,
                         const void* scales, int64_t G, int64_t scales_ld,
                         uint8_t* q_out, int64_t q_ld, void* s_out, uint8_t* z_out, int64_t sz_ld,
                         void* stream);

/* weight_only_int4_matmul (examples/kernels/contraction/weight_only_int4.py:18-51)
 * for M <= 5, reading the reference's layout in place (no repack):
 *   y[m, n] = f16(sum_k x[m, k] * (signed nibble (k, n) * scales[k / 64, n]))
 * x: f16 [M, K] (x_ld elements); packed: int32 [K/8, N] (packed_ld elements),
 * word (r, n) holding k = 8r .. 8r+7 at nibble k % 8; scales: f16 [K/64, N]
 * (scales_ld elements); y: f16 [M, N] (y_ld elements).
 * K % 64 == 0 and K <= 8192, N % 4 == 0, x and packed rows 16-byte aligned,
 * scale rows 8-byte aligned.
 */
int intent_w4a16_sym_gemv(const void* x, int64_t M, int64_t K, int64_t x_ld,
                          const int32_t* packed, int64_t N, int64_t packed_ld,
                          const void* scales, int64_t scales_ld,
                          void* y, int64_t y_ld, void* stream);

/* The same function for any M on the tiled W4 GEMM (producer waves decode the
 * reference's words in place into the f16 LDS tile; no repack). K % 64 == 0,
 * x rows 16-byte aligned.
 */
int intent_w4a16_sym_gemm(const void* x, int64_t M, int64_t K, int64_t x_ld,
                          const int32_t* packed, int64_t N, int64_t packed_ld,
                          const void* scales, int64_t scales_ld,
                          void* y, int64_t y_ld, void* stream);

/* f16 matrix transpose: dst[c * dst_ld + r] = src[r * src_ld + c] (elements).
 * Plumbing for quantized_gemm, whose right operand the reference passes as
 * [K, N]. Replaces no reference function.
 */
int intent_f16_transpose(const void* src, int64_t rows, int64_t cols, int64_t src_ld,
                         void* dst, int64_t dst_ld, void* stream);

/* f16 GEMM with the fused int8 epilogue of quantized_gemm
 * (examples/kernels/contraction/gemm.py:83-106; CPU baseline
 * experiments/cpu/baselines/pytorch/cpu_runtime.py:91-94):
 *   out = i8(trunc(clamp((relu(acc + bias[n]) + residual[m, n]) / output_scale[n],
 *                        -128, 127)))
 * a: f16 [M, K]; bt: the right operand as f16 [N, K] rows (use
 * intent_f16_transpose for a [K, N] operand); bias, output_scale: f32 [N];
 * residual: f16 [M, N]; out: int8 [M, N]. K % 64 == 0.
 */
int intent_quantized_gemm(const void* a, int64_t M, int64_t K, int64_t a_ld,
                          const void* bt, int64_t N, int64_t bt_ld,
                          const float* bias, const void* residual, int64_t residual_ld,
                          const float* output_scale, int8_t* out, int64_t out_ld, void* stream);

/* Batched f16/bf16 transpose: matrix b (b < batch) of src (rows x cols,
 * src_ld elements, src_batch elements apart) to dst (cols x rows). Plumbing
 * for ragged_grouped_gemm, whose weights the reference passes as [G, K, N].
 * Replaces no reference function.
 */
int intent_f16_transpose_batched(const void* src, int64_t batch, int64_t rows, int64_t cols,
                                 int64_t src_ld, int64_t src_batch, void* dst, int64_t dst_ld,
                                 int64_t dst_batch, void* stream);

/* f16 / bf16 grouped GEMM over row groups. Replaces ragged_grouped_gemm and
 * ragged_grouped_gemm_bf16 (examples/kernels/ragged/grouped_gemm.py:11-70;
 * routes == NULL: group g owns rows offsets[g] .. offsets[g+1] of x and out)
 * and routed_expert_projection_bf16 (grouped_gemm.py:101-138; routes != NULL:
 * group g owns routes[offsets[g] .. offsets[g+1]], route r reads x row r / top_k
 * and writes out row r of [T * top_k, N]).
 * x: [rows, K] (x_ld elements); w: group g's weights as [N, K] rows at
 * w + g * w_group_stride (w_ld elements; use intent_f16_transpose_batched for
 * [G, K, N]); bf16 selects bf16 (else f16) elements; f32 accumulation.
 * `rows` bounds the rows (routes) a group can hold. K % 64 == 0.
 */
int intent_grouped_gemm(const void* x, int64_t rows, int64_t K, int64_t x_ld, const int32_t* offsets,
                        int64_t G, const int32_t* routes, int64_t top_k, const void* w, int64_t N,
                        int64_t w_ld, int64_t w_group_stride, int bf16, void* out, int64_t out_ld,
                        void* stream);

/* Float GEMM on the same tiles as intent_quantized_gemm. Replaces gemm
 * (examples/kernels/contraction/gemm.py:42-61; epilogue 0: c = f16(acc),
 * 1: ACTIVATION RELU, c = f16(max(acc, 0))) and bf16_gemm (gemm.py:64-80;
 * epilogue 2: bf16 operands, c = bf16(acc)). a: [M, K]; bt: the right operand
 * as [N, K] rows (use intent_f16_transpose for [K, N]); f32 accumulation;
 * c: [M, N] of the operands' type. K % 64 == 0.
 */
int intent_f16_gemm(const void* a, int64_t M, int64_t K, int64_t a_ld, const void* bt, int64_t N,
                    int64_t bt_ld, int epilogue, void* c, int64_t c_ld, void* stream);

/* The float GEMMs with the right operand as the reference passes it: b
 * [K, N] with N contiguous (b_ld elements per k-row), read in place (no
 * transposed copy): gemm / bf16_gemm (examples/kernels/contraction/gemm.py:42-80,
 * epilogue as intent_f16_gemm) and quantized_gemm (gemm.py:83-106, epilogue as
 * intent_quantized_gemm). N % 8 == 0, b_ld % 8 == 0, 16-byte aligned operands,
 * K % 64 == 0; otherwise INTENT_ERR_UNSUPPORTED / INTENT_ERR_ALIGNMENT.
 */
int intent_f16_gemm_kn(const void* a, int64_t M, int64_t K, int64_t a_ld, const void* b, int64_t N,
                       int64_t b_ld, int epilogue, void* c, int64_t c_ld, void* stream);
int intent_quantized_gemm_kn(const void* a, int64_t M, int64_t K, int64_t a_ld, const void* b, int64_t N,
                             int64_t b_ld, const float* bias, const void* residual, int64_t residual_ld,
                             const float* output_scale, int8_t* out, int64_t out_ld, void* stream);

/* ragged_grouped_gemm / ragged_grouped_gemm_bf16 (examples/kernels/ragged/
 * grouped_gemm.py:11-70) with the weights as the reference lays them out,
 * [G][K][N] (w_ld elements per k-row, w_group_stride per group), read in
 * place. Rows offsets[g] .. offsets[g+1] of x [rows, K] and out [rows, N]
 * belong to group g (offsets clamped to [0, rows]). N and w_ld multiples of 8,
 * K % 64 == 0, 16-byte aligned operands.
 */
int intent_grouped_gemm_kn(const void* x, int64_t rows, int64_t K, int64_t x_ld, const int32_t* offsets,
                           int64_t G, const void* w, int64_t N, int64_t w_ld, int64_t w_group_stride, int bf16,
                           void* out, int64_t out_ld, void* stream);

/* The reference's f16 MoE expert FFN, moe_expert_ffn
 * (examples/kernels/ragged/moe.py:12-53; host reference
 * experiments/_common/support.py:133-151): x f16 [T, D] (x_ld), route_offsets
 * i32 [E + 1], member_routes i32 [R], route_token i32 [NR], route_weights f32
 * [NR], w1 f16 [E, D, F], w2 f16 [E, F, D] (both contiguous), y f32 [T, D]
 * (y_ld) updated in place:
 *   for each expert e, member i in route_offsets[e] .. route_offsets[e+1]:
 *     r = member_routes[i], t = route_token[r]
 *     y[t] += route_weights[r] * (f16(max(x[t] @ w1[e], 0)) @ w2[e])
 * with f32 accumulation; a token's contributions are added in member order
 * (deterministic). Out-of-range routing entries are clamped, never
 * dereferenced. D and F multiples of 64. workspace: at least
 * intent_moe_expert_ffn_workspace_size(T, R, D, F) bytes, 16-byte aligned.
 */
size_t intent_moe_expert_ffn_workspace_size(int64_t T, int64_t R, int64_t D, int64_t F);
int intent_moe_expert_ffn(const void* x, int64_t T, int64_t D, int64_t x_ld, const int32_t* route_offsets,
                          int64_t E, const int32_t* member_routes, int64_t R, const int32_t* route_token,
                          const float* route_weights, int64_t NR, const void* w1, const void* w2, int64_t F,
                          float* y, int64_t y_ld, void* workspace, size_t workspace_bytes, void* stream);

/* NVFP4 activation quantizer. Replaces nvfp4_quantize
 * (examples/kernels/quantization/nvfp4.py; CPU baseline
 * experiments/cpu/baselines/pytorch/cpu_runtime.py:1325-1340): x bf16 [M, N]
 * (x_ld elements, N % 16 == 0), global_scale f32 [1] (device); per row and group
 * of 16: scale = e4m3fn(max((amax / 6) * gs, 1.5258789e-5)), values
 * x * (gs / scale) encoded as E2M1 (thresholds of the reference), two per byte
 * into packed [M, N/2]; scale bytes into the reference's swizzled blocks
 * scales[ceil(M/128)][ceil(G/4)][32][4][4] exactly (row r, group g at
 * [r/128][g/4][r%32][(r%128)/32][g%4]; the block stride follows from N).
 * Only valid groups are written. As torch's E4M3FN cast in the CPU formula,
 * a scale in (448, 464] rounds to 448 and one above 464 is NaN (0x7f), whose
 * group then encodes every value as code 0.
 */
int intent_nvfp4_quantize(const void* x, int64_t M, int64_t N, int64_t x_ld, const float* global_scale,
                          uint8_t* packed, int64_t packed_ld, uint8_t* scales, void* stream);

/* Per-token symmetric int8 activation quantizer, the producer of
 * intent_w8a8_gemm's int8 activations and f32 per-token scales. Applies the
 * reference's integer quantization rule (clamp to [-128, 127], then round half
 * to even: lib/Conversion/KIRToGPU/Quantization.cpp:191-203) per row:
 * scale[m] = absmax / 127, q = rne(clamp(x * (127 / absmax))), both divisions
 * IEEE f32; a zero row gives scale 0 and q 0. x f16 (x_is_bf16 = 0) or bf16
 * [M, K] (x_ld elements, 16-byte aligned rows, K % 8 == 0); q int8 [M, K]
 * (q_ld, 8-byte aligned rows); scales f32 [M]. Inputs are finite.
 */
int intent_i8_per_token_quantize(const void* x, int x_is_bf16, int64_t M, int64_t K, int64_t x_ld,
                                 int8_t* q, int64_t q_ld, float* scales, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* INTENT_AMD_H */
