/* CPU oracle of the quantized-contraction hot path — test infrastructure only.
 * f16 / bf16 values are passed as their uint16 bit patterns. `threads` is the
 * OpenMP thread count (results do not depend on it). */
#ifndef INTENT_ORACLE_H
#define INTENT_ORACLE_H

#include <stdint.h>

float orc_f16_to_f32(uint16_t h);
uint16_t orc_f32_to_f16(float f);
uint16_t orc_f32_to_bf16(float f);

void orc_w8a16(const uint16_t* x, int64_t M, int64_t K, const int8_t* w, int64_t N, const uint16_t* s, uint16_t* y,
               int threads);
void orc_w4a16(const uint16_t* x, int64_t M, int64_t K, const uint8_t* packed, int64_t N, const uint16_t* scales,
               const uint8_t* zeros, int64_t gs, uint16_t* y, int threads);
void orc_i8_gemm_i32(const int8_t* a, int64_t M, int64_t K, const int8_t* w, int64_t N, const int32_t* bias,
                     int32_t* c, int threads);
void orc_w8a8(const int8_t* a, int64_t M, int64_t K, const float* sa, const int8_t* w, int64_t N, const float* sw,
              uint16_t* out, int threads);
void orc_moe_route(const float* logits, int64_t T, int64_t E, int64_t top_k, int renorm, int32_t* ids,
                   float* weights);
void orc_moe_align(const int32_t* ids, int64_t T, int64_t top_k, int64_t E, int64_t B, int32_t* sorted,
                   int64_t capacity, int32_t* blocks, int64_t nblocks, int32_t* offsets, int32_t* total);
void orc_moe_ffn_w4(const uint16_t* x, int64_t T, int64_t H, const int32_t* ids, const float* weights, int64_t top_k,
                    int64_t E, const uint8_t* wgu, const uint16_t* sgu, const uint8_t* zgu, const uint8_t* wd,
                    const uint16_t* sd, const uint8_t* zd, int64_t F, int64_t gs, float* y, int threads);

void orc_q8k_quantize(const float* x, int64_t G, uint8_t* out);
float orc_q4k_q8k_dot(const uint8_t* w, const uint8_t* x, int64_t G);
void orc_q4k_gemv(const uint8_t* w, int64_t N, int64_t G, int64_t w_ld, const uint8_t* xq, float* y, int threads);
uint8_t orc_f32_to_e4m3fn(float f);
void orc_fp8_groupwise_quantize(const float* x, int64_t M, int64_t N, int64_t ldx, int64_t G, float eps,
                                uint8_t* q, int64_t ldq, float* scales, int64_t lds_);
void orc_i8_per_token_quantize(const float* x, int64_t M, int64_t K, int64_t ldx, int8_t* q, int64_t ldq,
                               float* scales);
void orc_w4a8(const int8_t* a, int64_t M, int64_t K, const uint8_t* packed, int64_t N, int32_t* out, int threads);
void orc_bitnet_int2(const int8_t* a, int64_t M, int64_t K, const uint8_t* packed, int64_t N, int32_t* out,
                     int threads);
float orc_e4m3fn_to_f32(uint8_t v);
float orc_e8m0_to_f32(uint8_t e);
void orc_mxfp8_gemm(const uint8_t* a, const uint8_t* sa, int64_t M, int64_t K, const uint8_t* b, const uint8_t* sb,
                    int64_t N, float* out, int threads);
void orc_scaled_fp8_gemm(const uint8_t* a, int64_t M, int64_t K, const uint8_t* b, int64_t N, float ls, float rs,
                         int64_t splits, int accumulate, uint16_t* out, int threads);
void orc_deepgemm_fp8(const uint8_t* a, const float* sa, int64_t M, int64_t KB, const uint8_t* b, const float* sb,
                      int64_t N, uint16_t* out, int threads);
float orc_e5m2_to_f32(uint8_t v);
uint8_t orc_f32_to_e5m2(float f);
void orc_fp8_gemm(int format, const uint8_t* a, int64_t M, int64_t K, const uint8_t* bt, int64_t N, uint8_t* out,
                  int threads);
float orc_fp4_decode(const uint8_t* row, int64_t k);
void orc_fp4_bf16_matmul(const uint16_t* x, int64_t M, int64_t K, const uint8_t* packed, int64_t N, uint16_t* out,
                         int threads);
void orc_w4_sym(const uint16_t* x, int64_t M, int64_t K, const int32_t* packed, const uint16_t* scales, int64_t N,
                uint16_t* y, int threads);
void orc_quantized_gemm(const uint16_t* a, int64_t M, int64_t K, const uint16_t* b, int64_t N, const float* bias,
                        const uint16_t* residual, const float* oscale, int8_t* out, int threads);
void orc_grouped_gemm(const uint16_t* x, int bf16, int64_t K, const int32_t* offsets, int64_t G, const int32_t* routes,
                      int64_t top_k, const uint16_t* w, int64_t N, uint16_t* out, int threads);
void orc_moe_expert_ffn(const uint16_t* x, int64_t T, int64_t D, const int32_t* route_offsets, int64_t E,
                        const int32_t* member_routes, const int32_t* route_token, const float* route_weights,
                        const uint16_t* w1, const uint16_t* w2, int64_t F, float* y, const uint8_t* token_sel,
                        int threads);
void orc_float_gemm(const uint16_t* a, int64_t M, int64_t K, const uint16_t* b, int64_t N, int bf16, int relu,
                    uint16_t* c, int threads);
void orc_nvfp4_quantize(const uint16_t* x, int64_t M, int64_t N, float gs, uint8_t* packed, uint8_t* scales);

#endif
