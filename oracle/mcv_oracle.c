/*
 * mcv_oracle.c -- CPU restatement of the reference's quantized-matmul arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY (the checker, and the CPU baseline timed by bench.py).
 * Nothing in the product library links or calls this file.
 *
 * Build: oracle/Makefile (gcc -O3 -fno-fast-math -ffp-contract=off -fopenmp).
 * Floating point contraction is off so every multiply and add rounds on its own,
 * which is the arithmetic the reference's CPU formulas spell out.
 *
 * Reference paths are relative to the root of lvyufeng/minicpm-v-4.6-orangepi.
 */
#include "mcv_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define GROUP 128

static inline uint32_t f32_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float bits_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* ------------------------------------------------------------------------- */
/* fp16 <-> fp32                                                              */
/* ------------------------------------------------------------------------- */

/* Decode with subnormals kept: src/csrc/lib/quantized_weight.cpp:162-184
 * (same function in tests/test_matmul_w4a16.cpp:33-54). */
float or_h2f(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    if (e == 0) {
        if (m == 0) return bits_f32(sign);
        /* value = m * 2^-24 exactly; scale in fp32 (exact, m < 2^10) */
        float v = (float)m * 5.9604644775390625e-08f;
        return sign ? -v : v;
    }
    if (e == 31) return bits_f32(sign | 0x7f800000u | (m << 13));
    return bits_f32(sign | ((e + 112u) << 23) | (m << 13));
}

/* Decode with subnormals flushed to signed zero: the lambda inside
 * lm_head_greedy, src/csrc/lib/language_model.cpp:444-459 (also
 * tests/test_w8a8_dequant.cpp h2f). */
float or_h2f_ftz(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    if (e == 0) return bits_f32(sign);
    if (e == 31) return bits_f32(sign | 0x7f800000u | (m << 13));
    return bits_f32(sign | ((e + 112u) << 23) | (m << 13));
}

/* Truncating encode, underflow to signed zero, exponent overflow (incl. NaN
 * input) to signed infinity: src/csrc/lib/quantized_weight.cpp:186-195. */
uint16_t or_f2h_trunc(float f) {
    uint32_t x = f32_bits(f);
    uint32_t sign = (x >> 16) & 0x8000u;
    int32_t e = (int32_t)((x >> 23) & 0xffu) - 127 + 15;
    uint32_t m = x & 0x7fffffu;
    if (e <= 0) return (uint16_t)sign;
    if (e >= 31) return (uint16_t)(sign | 0x7c00u);
    return (uint16_t)(sign | ((uint32_t)e << 10) | (m >> 13));
}

/* bf16 -> fp16 as the reference loads bf16 checkpoint tensors
 * (src/csrc/lib/weights.cpp:25-33): rebias the exponent, keep the top 10
 * mantissa bits (bf16 has 7, so nothing is lost for fp16 normals), flush
 * what falls below the fp16 normal range to signed zero and send what falls
 * above it -- NaN included -- to signed infinity. */
uint16_t or_bf16_to_f16_trunc(uint16_t bf) {
    uint32_t x = (uint32_t)bf << 16;
    uint32_t sign = (x >> 16) & 0x8000u;
    int32_t e = (int32_t)((x >> 23) & 0xffu) - 127 + 15;
    if (e <= 0) return (uint16_t)sign;
    if (e >= 31) return (uint16_t)(sign | 0x7c00u);
    return (uint16_t)(sign | ((uint32_t)e << 10) | ((x & 0x7fffffu) >> 13));
}

void or_bf16_to_f16_trunc_array(const uint16_t* bf, int64_t n, uint16_t* out) {
    for (int64_t i = 0; i < n; ++i) out[i] = or_bf16_to_f16_trunc(bf[i]);
}

/* IEEE-754 round-to-nearest-even encode with subnormals.  Build-defined: the
 * synthetic generators and the fp16 outputs of every kernel use this rounding
 * (the reference's AscendC casts use CAST_RINT, e.g.
 * src/csrc/custom_ops/op_kernel/w8a8_dequant_custom.cpp:62). */
uint16_t or_f2h_rne(float f) {
    uint32_t x = f32_bits(f);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) {                 /* inf or NaN */
        if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);
        return (uint16_t)(sign | 0x7c00u);
    }
    int32_t e = (int32_t)(ax >> 23) - 127;    /* unbiased exponent */
    if (e > 15) return (uint16_t)(sign | 0x7c00u);
    uint32_t mant = (ax & 0x7fffffu) | 0x800000u;  /* 24-bit significand, value mant*2^(e-23) */
    int32_t shift;                            /* bits to drop from the 24-bit significand */
    uint32_t base;
    if (e >= -14) {                           /* normal fp16 range */
        shift = 13;
        base = (uint32_t)(e + 15) << 10;
        mant &= 0x7fffffu;                    /* implicit bit carried by base */
        uint32_t q = mant >> shift;
        uint32_t rem = mant & ((1u << shift) - 1);
        uint32_t half = 1u << (shift - 1);
        uint32_t r = base + q;
        if (rem > half || (rem == half && (q & 1u))) r += 1;   /* carry may bump exponent: correct */
        return (uint16_t)(sign | r);
    }
    if (ax == 0) return (uint16_t)sign;
    /* subnormal: value = mant * 2^(e-23); fp16 subnormal unit is 2^-24 */
    shift = -e - 1;                           /* mant * 2^(e-23) / 2^-24 = mant >> (-e-1) */
    if (shift > 25) return (uint16_t)sign;
    {
        uint32_t q = mant >> shift;
        uint32_t rem = mant & ((1u << shift) - 1);
        uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1u))) q += 1;
        return (uint16_t)(sign | q);         /* q == 0x400 becomes the smallest normal: correct */
    }
}

void or_h2f_array(const uint16_t* h, int64_t n, float* out) {
    for (int64_t i = 0; i < n; ++i) out[i] = or_h2f(h[i]);
}
void or_f2h_rne_array(const float* f, int64_t n, uint16_t* out) {
    for (int64_t i = 0; i < n; ++i) out[i] = or_f2h_rne(f[i]);
}
void or_f2h_trunc_array(const float* f, int64_t n, uint16_t* out) {
    for (int64_t i = 0; i < n; ++i) out[i] = or_f2h_trunc(f[i]);
}

/* ------------------------------------------------------------------------- */
/* int4 checkpoint unpackers                                                  */
/* ------------------------------------------------------------------------- */

/* AutoAWQ "gemm" packing: src/csrc/lib/quantized_weight.cpp:122-160 with the
 * nibble order of :17.  qweight int32 [K, N/8], qzeros int32 [K/128, N/8];
 * nibble slot s of word j holds column 8j + order[s]; out = q - z. */
int or_unpack_awq(const int32_t* qweight, const int32_t* qzeros, int64_t K, int64_t N, int8_t* w8) {
    static const int order[8] = {0, 2, 4, 6, 1, 3, 5, 7};
    if (K <= 0 || N <= 0 || K % GROUP != 0 || N % 8 != 0) return 1;
    const int64_t np = N / 8;
    for (int64_t k = 0; k < K; ++k) {
        const int64_t g = k / GROUP;
        for (int64_t j = 0; j < np; ++j) {
            uint32_t qw = (uint32_t)qweight[k * np + j];
            uint32_t zw = (uint32_t)qzeros[g * np + j];
            for (int s = 0; s < 8; ++s) {
                int q = (int)((qw >> (4 * s)) & 15u);
                int z = (int)((zw >> (4 * s)) & 15u);
                w8[k * N + j * 8 + order[s]] = (int8_t)(q - z);
            }
        }
    }
    return 0;
}

/* GPTQ v1 packing: src/csrc/lib/quantized_weight.cpp:75-120.  qweight int32
 * [K/8, N] packs 8 consecutive k per word (nibble i -> k = 8*k0 + i); qzeros
 * int32 [G, N/8] packs 8 consecutive n; the stored zero is off by one
 * (zero = nibble + 1, :112); the group of row k is g_idx[k] (act-order). */
int or_unpack_gptq(const int32_t* qweight, const int32_t* qzeros, const int32_t* g_idx,
                   int64_t K, int64_t N, int64_t groups, int8_t* w8) {
    if (K <= 0 || N <= 0 || K % 8 != 0 || N % 8 != 0 || groups * GROUP != K) return 1;
    const int64_t kp = K / 8;
    for (int64_t k0 = 0; k0 < kp; ++k0) {
        for (int64_t n = 0; n < N; ++n) {
            uint32_t qw = (uint32_t)qweight[k0 * N + n];
            for (int i = 0; i < 8; ++i) {
                int64_t k = k0 * 8 + i;
                int64_t g = g_idx[k];
                if (g < 0 || g >= groups) return 2;
                uint32_t zw = (uint32_t)qzeros[g * (N / 8) + n / 8];
                int z = (int)((zw >> (4 * (n % 8))) & 15u) + 1;
                int q = (int)((qw >> (4 * i)) & 15u);
                w8[k * N + n] = (int8_t)(q - z);
            }
        }
    }
    return 0;
}

/* ------------------------------------------------------------------------- */
/* Build-defined synthetic int4 quantizer.  The reference has none (it only     */
/* unpacks AutoAWQ/GPTQ checkpoints).  Per (group g, column n) over 128 fp16    */
/* values: s = fp16_rne(max(hi - lo, 1e-5) / 15); z = clamp(rne(-lo / s), 0,   */
/* 15); q = clamp(rne(w / s) + z, 0, 15); packed AWQ-style so the reference's   */
/* unpacker (quantized_weight.cpp:122-160) reads it unchanged.                   */
/* ------------------------------------------------------------------------- */
int or_quantize_int4_awq(const uint16_t* w_kn, int64_t K, int64_t N,
                         int32_t* qweight, int32_t* qzeros, uint16_t* scales) {
    static const int order[8] = {0, 2, 4, 6, 1, 3, 5, 7};
    if (K <= 0 || N <= 0 || K % GROUP != 0 || N % 8 != 0) return 1;
    const int64_t G = K / GROUP, np = N / 8;
    uint8_t* q = (uint8_t*)malloc((size_t)K * (size_t)N);
    uint8_t* z = (uint8_t*)malloc((size_t)G * (size_t)N);
    if (!q || !z) { free(q); free(z); return 3; }
    for (int64_t g = 0; g < G; ++g) {
        for (int64_t n = 0; n < N; ++n) {
            float lo = INFINITY, hi = -INFINITY;
            for (int64_t kk = 0; kk < GROUP; ++kk) {
                float v = or_h2f(w_kn[(g * GROUP + kk) * N + n]);
                if (v < lo) lo = v;
                if (v > hi) hi = v;
            }
            float range = hi - lo;
            if (range < 1e-5f) range = 1e-5f;
            uint16_t s16 = or_f2h_rne(range / 15.0f);
            float s = or_h2f(s16);
            float zf = rintf(-lo / s);
            if (!(zf > 0.0f)) zf = 0.0f;   /* NaN (inf / inf) -> 0 */
            if (zf > 15.0f) zf = 15.0f;
            int zi = (int)zf;
            scales[g * N + n] = s16;
            z[g * N + n] = (uint8_t)zi;
            for (int64_t kk = 0; kk < GROUP; ++kk) {
                int64_t k = g * GROUP + kk;
                float v = or_h2f(w_kn[k * N + n]);
                float qf = rintf(v / s) + (float)zi;
                if (!(qf > 0.0f)) qf = 0.0f;
                if (qf > 15.0f) qf = 15.0f;
                q[k * N + n] = (uint8_t)qf;
            }
        }
    }
    for (int64_t k = 0; k < K; ++k) {
        for (int64_t j = 0; j < np; ++j) {
            uint32_t word = 0;
            for (int s = 0; s < 8; ++s) word |= (uint32_t)q[k * N + j * 8 + order[s]] << (4 * s);
            qweight[k * np + j] = (int32_t)word;
        }
    }
    for (int64_t g = 0; g < G; ++g) {
        for (int64_t j = 0; j < np; ++j) {
            uint32_t word = 0;
            for (int s = 0; s < 8; ++s) word |= (uint32_t)z[g * N + j * 8 + order[s]] << (4 * s);
            qzeros[g * np + j] = (int32_t)word;
        }
    }
    free(q);
    free(z);
    return 0;
}

/* ------------------------------------------------------------------------- */
/* W4A16 CPU formula: tests/test_matmul_w4a16.cpp:217-227 (and                 */
/* tests/test_matmul_awq.cpp:205-215), per output row for M > 1:                */
/*   partial = sum_{kk<128} h2f(x[k]) * (float)w8[k,n]   (kk ascending, fp32)   */
/*   out[n] += partial * h2f(scales[g, n])                (g ascending, fp32)   */
/* The loops run n innermost so each element sees exactly that sequence of      */
/* roundings; OpenMP splits n, which leaves every element's sequence unchanged. */
/* ------------------------------------------------------------------------- */
void or_w4a16_matmul(const uint16_t* x, const int8_t* w8, const uint16_t* scales,
                     int64_t M, int64_t K, int64_t N, float* out, int nthreads) {
    const int64_t G = K / GROUP;
#ifdef _OPENMP
    if (nthreads <= 0) nthreads = omp_get_max_threads();
#else
    (void)nthreads;
#endif
    for (int64_t m = 0; m < M; ++m) {
        const uint16_t* xr = x + m * K;
        float* o = out + m * N;
#pragma omp parallel num_threads(nthreads)
        {
            int64_t n0 = 0, n1 = N;
#ifdef _OPENMP
            int nt = omp_get_num_threads(), t = omp_get_thread_num();
            int64_t per = ((N + nt - 1) / nt + 15) / 16 * 16;
            n0 = per * t; n1 = n0 + per;
            if (n0 > N) n0 = N;
            if (n1 > N) n1 = N;
#endif
            const int64_t len = n1 - n0;
            float* partial = (float*)malloc(sizeof(float) * (size_t)(len > 0 ? len : 1));
            for (int64_t n = n0; n < n1; ++n) o[n] = 0.0f;
            for (int64_t g = 0; g < G && len > 0; ++g) {
                for (int64_t i = 0; i < len; ++i) partial[i] = 0.0f;
                for (int64_t kk = 0; kk < GROUP; ++kk) {
                    const int64_t k = g * GROUP + kk;
                    const float xk = or_h2f(xr[k]);
                    const int8_t* wr = w8 + k * N + n0;
                    for (int64_t i = 0; i < len; ++i) partial[i] += xk * (float)wr[i];
                }
                const uint16_t* sr = scales + g * N + n0;
                for (int64_t i = 0; i < len; ++i) o[n0 + i] += partial[i] * or_h2f(sr[i]);
            }
            free(partial);
        }
    }
}

/* Dequantised weight values: fp16 RNE of (q - z) * s.  (q - z) has <= 5
 * significant bits and s <= 11, so the fp32 product is exact and one RNE
 * gives the correctly rounded fp16 value.  Follows the dequant the reference's
 * CPU formula implies (tests/test_matmul_w4a16.cpp:5,223-225). */
void or_w4a16_dequant_f16(const int8_t* w8, const uint16_t* scales, int64_t K, int64_t N, uint16_t* out) {
    for (int64_t k = 0; k < K; ++k) {
        const int64_t g = k / GROUP;
        for (int64_t n = 0; n < N; ++n)
            out[k * N + n] = or_f2h_rne((float)w8[k * N + n] * or_h2f(scales[g * N + n]));
    }
}

/* ------------------------------------------------------------------------- */
/* W8A8                                                                        */
/* ------------------------------------------------------------------------- */

/* src/csrc/lib/quantized_weight.cpp:197-202: clamp first, then round half
 * away from zero by +-0.5 and truncation (each step one fp32 rounding).  A
 * NaN product is 0, what the reference's (undefined) float-to-int8 cast gives
 * on aarch64 (fcvtzs) and x86-64 (cvttss2si, low byte of 0x80000000). */
int8_t or_quantize_i8(float value, float inv_scale) {
    float q = value * inv_scale;
    if (q != q) return 0;
    if (q > 127.0f) q = 127.0f;
    if (q < -128.0f) q = -128.0f;
    return (int8_t)(q >= 0.0f ? q + 0.5f : q - 0.5f);
}

/* Per-output-channel symmetric weight quantizer:
 * src/csrc/lib/quantized_weight.cpp:231-268.  scale = max_k|w| / 127 (fp32),
 * floored at 1e-8; inv = 1 / scale; the stored fp16 scale is the truncating
 * encode (:253).  Both the fp32 and the fp16 scale are returned. */
void or_w8a8_quantize_weight(const uint16_t* w_kn, int64_t K, int64_t N,
                             int8_t* q_kn, float* scale_f32, uint16_t* scale_f16) {
    for (int64_t n = 0; n < N; ++n) {
        float max_abs = 0.0f;
        for (int64_t k = 0; k < K; ++k) {
            float a = fabsf(or_h2f(w_kn[k * N + n]));
            if (a > max_abs) max_abs = a;
        }
        float scale = max_abs / 127.0f;
        if (scale < 0.00000001f) scale = 0.00000001f;
        const float inv = 1.0f / scale;
        scale_f32[n] = scale;
        scale_f16[n] = or_f2h_trunc(scale);
        for (int64_t k = 0; k < K; ++k) q_kn[k * N + n] = or_quantize_i8(or_h2f(w_kn[k * N + n]), inv);
    }
}

/* Per-token symmetric activation quantizer, one row at a time:
 * src/csrc/custom_ops/op_kernel/w8a8_quantize_custom.cpp:25-41 (the kernel is
 * per-tensor over [1, K]; per row it is the same closed form).  The fp16 scale
 * uses RNE (static_cast<half> at :41; its NPU rounding is unpinned). */
void or_w8a8_quantize_act(const uint16_t* x, int64_t M, int64_t K,
                          int8_t* xq, float* scale_f32, uint16_t* scale_f16) {
    for (int64_t m = 0; m < M; ++m) {
        const uint16_t* xr = x + m * K;
        float max_abs = 0.0f;
        for (int64_t k = 0; k < K; ++k) {
            float v = or_h2f(xr[k]);
            if (v < 0.0f) v = -v;
            if (v > max_abs) max_abs = v;
        }
        float scale = max_abs / 127.0f;
        if (scale < 0.00000001f) scale = 0.00000001f;
        const float inv = 1.0f / scale;
        for (int64_t k = 0; k < K; ++k) {
            float v = or_h2f(xr[k]) * inv;
            if (v > 127.0f) v = 127.0f;
            if (v < -128.0f) v = -128.0f;
            int32_t qi = (int32_t)(v >= 0.0f ? v + 0.5f : v - 0.5f);
            xq[m * K + k] = (int8_t)qi;
        }
        scale_f32[m] = scale;
        if (scale_f16) scale_f16[m] = or_f2h_rne(scale);
    }
}

/* Exact int32 product: tests/test_matmul_w8a8_i32.cpp:40-49, per row. */
void or_gemm_i32(const int8_t* x, const int8_t* w_kn, int64_t M, int64_t K, int64_t N,
                 int32_t* out, int nthreads) {
#ifdef _OPENMP
    if (nthreads <= 0) nthreads = omp_get_max_threads();
#else
    (void)nthreads;
#endif
    for (int64_t m = 0; m < M; ++m) {
#pragma omp parallel for num_threads(nthreads) schedule(static)
        for (int64_t nb = 0; nb < (N + 63) / 64; ++nb) {
            int32_t acc[64];
            const int64_t n0 = nb * 64, n1 = n0 + 64 < N ? n0 + 64 : N;
            for (int64_t n = n0; n < n1; ++n) acc[n - n0] = 0;
            for (int64_t k = 0; k < K; ++k) {
                const int32_t xv = x[m * K + k];
                const int8_t* wr = w_kn + k * N;
                for (int64_t n = n0; n < n1; ++n) acc[n - n0] += xv * (int32_t)wr[n];
            }
            for (int64_t n = n0; n < n1; ++n) out[m * N + n] = acc[n - n0];
        }
    }
}

/* Dequant epilogue: src/csrc/custom_ops/op_kernel/w8a8_dequant_custom.cpp:55-62
 * out = RINT_fp16( ((float)acc * w_scale[n]) * x_scale[m] ), fp32 throughout. */
void or_w8a8_dequant(const int32_t* acc, const float* x_scale, const float* w_scale,
                     int64_t M, int64_t N, uint16_t* out) {
    for (int64_t m = 0; m < M; ++m)
        for (int64_t n = 0; n < N; ++n) {
            float v = (float)acc[m * N + n] * w_scale[n];
            v = v * x_scale[m];
            out[m * N + n] = or_f2h_rne(v);
        }
}

/* ------------------------------------------------------------------------- */
/* silu * mul: src/csrc/custom_ops/op_kernel/silu_mul_custom.cpp:59-75        */
/* t = -g; t = exp(t); t = t + 1; t = g / t; t = t * u; RINT to fp16.           */
/* ------------------------------------------------------------------------- */
void or_silu_mul(const uint16_t* gate, const uint16_t* up, int64_t n, uint16_t* out) {
    for (int64_t i = 0; i < n; ++i) {
        float g = or_h2f(gate[i]);
        float u = or_h2f(up[i]);
        float t = expf(-g);
        t = t + 1.0f;
        t = g / t;
        t = t * u;
        out[i] = or_f2h_rne(t);
    }
}

/* Greedy argmax over fp16 logits: src/csrc/lib/language_model.cpp:462-479.
 * Values are decoded with subnormals flushed (:444-459), the scan is in
 * ascending index with a strict '>', starting from -inf and token 0: the first
 * maximum wins, NaNs never win, an all -inf/NaN row returns 0. */
int64_t or_argmax_f16(const uint16_t* logits, int64_t n) {
    int64_t best = 0;
    float best_v = -INFINITY;
    for (int64_t i = 0; i < n; ++i) {
        float v = or_h2f_ftz(logits[i]);
        if (v > best_v) { best_v = v; best = i; }
    }
    return best;
}

/* RMSNorm before the vocabulary projection: lm_head_greedy calls rms_norm
 * (src/csrc/lib/language_model.cpp:424 -> ops.cpp rms_norm -> aclnnRmsNorm, a
 * CANN builtin whose internal rounding is not vendored).  Restated from the
 * definition: y = x / sqrt(mean(x^2) + eps) * gamma, fp32 with a sequential sum. */
void or_rms_norm(const uint16_t* x, const uint16_t* gamma, int64_t M, int64_t H, float eps, uint16_t* out) {
    for (int64_t m = 0; m < M; ++m) {
        float ss = 0.0f;
        for (int64_t i = 0; i < H; ++i) {
            float v = or_h2f(x[m * H + i]);
            ss += v * v;
        }
        float rstd = 1.0f / sqrtf(ss / (float)H + eps);
        for (int64_t i = 0; i < H; ++i) out[m * H + i] = or_f2h_rne((or_h2f(x[m * H + i]) * rstd) * or_h2f(gamma[i]));
    }
}
