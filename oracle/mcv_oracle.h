/*
 * mcv_oracle.h -- CPU restatement of the reference's quantized-matmul arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the checker
 * (or, in bench.py, as the timed CPU baseline).  The product library never links
 * or calls it; its entry points fail loudly when the HIP build is missing.
 *
 * Every function names the reference file:line it restates.  Paths are relative
 * to the reference repository root (lvyufeng/minicpm-v-4.6-orangepi).
 *
 * Pinning status (what checks each function, see tests/test_oracle_*.py):
 *   or_h2f / or_h2f_ftz / or_f2h_trunc / or_f2h_rne  -- exhaustive over all 65536
 *       fp16 bit patterns against numpy's IEEE conversions, and a brute-force
 *       "largest fp16 not above |f|" characterisation of truncation.
 *   or_bf16_to_f16_trunc -- exhaustive over all 65536 bf16 patterns: exact (numpy
 *       float32 -> float16) wherever the value is an fp16 normal, signed zero
 *       below, signed infinity above and for NaN.
 *   or_unpack_awq / or_unpack_gptq  -- hand-built known-answer words, a vectorised
 *       numpy restatement written from the format description, and round trips.
 *   or_quantize_int4_awq  -- build-defined (the reference has no int4 quantizer);
 *       pinned by invariants only: range, error bound, exact min/max recovery.
 *       Parity with any upstream quantizer is unpinned by construction.
 *   or_w4a16_matmul  -- float64 numpy matmul of the dequantised matrix, linearity,
 *       integer special case (unit scales) computed exactly.
 *   or_w4a16_dequant_f16 -- numpy float64 product rounded by numpy's fp16 RNE.
 *   or_quantize_i8 / or_w8a8_quantize_weight / or_w8a8_quantize_act -- tie and
 *       clamp known answers, the error bound |q - v/s| <= 1/2, max|q| == 127.
 *   or_gemm_i32 -- numpy int64 matmul (exact).
 *   or_w8a8_dequant -- the reference test's deterministic vectors
 *       (tests/test_w8a8_dequant.cpp:42-46) and its bound (:58-63).
 *   or_silu_mul -- float64 silu rounded to fp16, within 1 fp16 ulp.
 *   or_argmax_f16 -- numpy argmax (first maximum) over the flushed values and the
 *       reference's modular-pattern lm_head test (tests/test_lm_head_pipeline.cpp).
 *   or_rms_norm -- float64 numpy RMSNorm rounded to fp16, within 1 fp16 ulp.
 *       The reference computes it with a CANN builtin (aclnnRmsNorm, not vendored):
 *       its rounding is parity unpinned; the formula is the definition.
 */
#ifndef MCV_ORACLE_H
#define MCV_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* fp16 <-> fp32 bit conversions */
float or_h2f(uint16_t h);
float or_h2f_ftz(uint16_t h);
uint16_t or_f2h_trunc(float f);
uint16_t or_f2h_rne(float f);
uint16_t or_bf16_to_f16_trunc(uint16_t bf);
void or_bf16_to_f16_trunc_array(const uint16_t* bf, int64_t n, uint16_t* out);
void or_h2f_array(const uint16_t* h, int64_t n, float* out);
void or_f2h_rne_array(const float* f, int64_t n, uint16_t* out);
void or_f2h_trunc_array(const float* f, int64_t n, uint16_t* out);

/* int4 checkpoint unpackers: produce (q - z) as int8 [K, N] */
int or_unpack_awq(const int32_t* qweight, const int32_t* qzeros, int64_t K, int64_t N, int8_t* w8);
int or_unpack_gptq(const int32_t* qweight, const int32_t* qzeros, const int32_t* g_idx,
                   int64_t K, int64_t N, int64_t groups, int8_t* w8);

/* build-defined synthetic int4 quantizer (AWQ packing) */
int or_quantize_int4_awq(const uint16_t* w_kn, int64_t K, int64_t N,
                         int32_t* qweight, int32_t* qzeros, uint16_t* scales);

/* W4A16 CPU formula, fp32 accumulation, out fp32 [M, N] */
void or_w4a16_matmul(const uint16_t* x, const int8_t* w8, const uint16_t* scales,
                     int64_t M, int64_t K, int64_t N, float* out, int nthreads);
/* dequantised weight values fp16 RNE((q - z) * s), [K, N] */
void or_w4a16_dequant_f16(const int8_t* w8, const uint16_t* scales, int64_t K, int64_t N, uint16_t* out);

/* W8A8 */
int8_t or_quantize_i8(float value, float inv_scale);
void or_w8a8_quantize_weight(const uint16_t* w_kn, int64_t K, int64_t N,
                             int8_t* q_kn, float* scale_f32, uint16_t* scale_f16);
void or_w8a8_quantize_act(const uint16_t* x, int64_t M, int64_t K,
                          int8_t* xq, float* scale_f32, uint16_t* scale_f16);
void or_gemm_i32(const int8_t* x, const int8_t* w_kn, int64_t M, int64_t K, int64_t N,
                 int32_t* out, int nthreads);
void or_w8a8_dequant(const int32_t* acc, const float* x_scale, const float* w_scale,
                     int64_t M, int64_t N, uint16_t* out);

/* elementwise and argmax */
void or_silu_mul(const uint16_t* gate, const uint16_t* up, int64_t n, uint16_t* out);
int64_t or_argmax_f16(const uint16_t* logits, int64_t n);
void or_rms_norm(const uint16_t* x, const uint16_t* gamma, int64_t M, int64_t H, float eps, uint16_t* out);

#ifdef __cplusplus
}
#endif

#endif
