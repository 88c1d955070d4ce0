// common.h -- shared helpers for the gfx950 quantized-matmul library.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <string>

#include "mcv_quant.h"

namespace mcv {

constexpr int kGroup = 128;       // quantisation group along K
constexpr int kSlab = 64;         // output columns per slab (one per lane)
constexpr int kChunkK = 32;       // k per 16-byte lane chunk

// Last error message of this thread, returned by mcv_last_error().
std::string& last_error();

// Records a formatted message and returns `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

inline int ok() { return MCV_OK; }

// Checks the launch that was just issued; HIP launch errors become MCV_ERR_HIP.
int check_launch(const char* what);

// Returns MCV_ERR_NO_DEVICE unless the current device is a gfx950 (the only
// target the code objects are built for); cached per device id.
int require_device();

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// ------------------------------------------------------------ device helpers --
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef float float16_t __attribute__((ext_vector_type(16)));
typedef int int4_t __attribute__((ext_vector_type(4)));
typedef int int16_t_v __attribute__((ext_vector_type(16)));

__device__ __forceinline__ half2_t as_h2(uint32_t u) { return __builtin_bit_cast(half2_t, u); }
__device__ __forceinline__ uint32_t as_u32(half2_t h) { return __builtin_bit_cast(uint32_t, h); }

// (a & smask) | vmagic in one v_and_or_b32, the mask in an SGPR.
__device__ __forceinline__ uint32_t and_or_b32(uint32_t a, uint32_t smask, uint32_t vmagic) {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "s"(smask), "v"(vmagic));
    return r;
}

// The W4A16 GEMMs' weight operands: two packed words (k-octets: k 2p at bits
// 4p..4p+3, k 2p+1 at bits 16+4p..19+4p) widened into the fp16 MFMA operands
// k0..k7 = RNE((q - z) * s), the values mcv_w4a16_dequant materialises.  A
// nibble pair becomes half2(1024 + q) through the fp16 exponent (mlo =
// 0x000F000F, vmagic = 0x64006400), minus zz = half2(1024 + z) (exact), times
// ss = half2(s) (one rounding).  The eight pairs of the two words go through
// each step together, so each step's eight instructions are independent: a
// VALU result read by the next instruction costs a wait state on gfx950, and
// one word at a time as a single chain left a nop between most of them.
__device__ __forceinline__ void dequant_pair(uint32_t qa, uint32_t qb, uint32_t zza, uint32_t ssa, uint32_t zzb,
                                             uint32_t ssb, uint32_t mlo, uint32_t vmagic, half8_t& ra, half8_t& rb) {
    uint32_t t[8];
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        t[2 * p] = and_or_b32(p ? qa >> (4 * p) : qa, mlo, vmagic);
        t[2 * p + 1] = and_or_b32(p ? qb >> (4 * p) : qb, mlo, vmagic);
    }
    half2_t d[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) d[i] = as_h2(t[i]) - as_h2((i & 1) ? zzb : zza);
#pragma unroll
    for (int i = 0; i < 8; ++i) d[i] = d[i] * as_h2((i & 1) ? ssb : ssa);
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        ra[2 * p] = d[2 * p][0];
        ra[2 * p + 1] = d[2 * p][1];
        rb[2 * p] = d[2 * p + 1][0];
        rb[2 * p + 1] = d[2 * p + 1][1];
    }
}

__device__ __forceinline__ float h2f(uint16_t h) {
    return static_cast<float>(__builtin_bit_cast(_Float16, h));
}
// fp32 -> fp16 with IEEE round-to-nearest-even (v_cvt_f16_f32 in the default
// mode) of exactly this fp32 value.  The empty asm hides where `f` came from:
// otherwise the backend folds a preceding fp32 multiply or add into one
// v_fma_mixlo_f16, which rounds the exact result to fp16 once instead of
// rounding to fp32 first -- a different answer in about 1 of 8192 cases, and
// not the reference's Mul/Muls-then-Cast(RINT) sequence.
__device__ __forceinline__ uint16_t f2h(float f) {
    asm volatile("" : "+v"(f));
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

// Order-preserving 16-bit key of an fp16 value for the greedy argmax: fp16
// subnormals and -0 map to +0 (the reference decodes logits with subnormals
// flushed, language_model.cpp:444-459, and compares with '>'); NaN and -inf
// return 0, a key no candidate has, because they can never win the scan.
__device__ __forceinline__ uint32_t argmax_key16(uint16_t h) {
    const uint32_t e = (h >> 10) & 0x1fu;
    if (e == 0x1f) {                       // inf or NaN
        if ((h & 0x3ffu) != 0 || (h & 0x8000u)) return 0u;
        return 0xfc00u | 0x8000u;          // +inf
    }
    if (e == 0) h = 0;                     // subnormal or zero -> +0
    return (h & 0x8000u) ? (~static_cast<uint32_t>(h) & 0xffffu) : (static_cast<uint32_t>(h) | 0x8000u);
}

// 64-bit argmax key: larger value first, then smaller index.  0 = no candidate.
__device__ __forceinline__ unsigned long long argmax_key64(uint32_t key16, uint32_t idx) {
    if (key16 == 0) return 0ull;
    return (static_cast<unsigned long long>(key16) << 32) | static_cast<unsigned long long>(0xffffffffu - idx);
}
__device__ __host__ __forceinline__ int64_t argmax_index(unsigned long long key) {
    if (key == 0ull) return 0;
    return static_cast<int64_t>(0xffffffffu - static_cast<uint32_t>(key & 0xffffffffull));
}

// fp16 RNE((g / (1 + exp(-g))) * u) with every step in fp32: the operation
// sequence of src/csrc/custom_ops/op_kernel/silu_mul_custom.cpp:59-75.  Shared
// by silu_mul_kernel and the fused gate/up GEMV so both round identically.
__device__ __forceinline__ uint16_t silu_mul_f16(uint16_t g, uint16_t u) {
    const float gv = h2f(g);
    float t = expf(-gv);
    t = __fadd_rn(t, 1.0f);
    t = __fdiv_rn(gv, t);
    t = __fmul_rn(t, h2f(u));
    return f2h(t);
}

// A bounded wait for another workgroup's words gave up: sets the u32 give-up
// word of the workspace (device scope) and, when the caller passed one, the
// status word -- a plain system-scope store of 1, so a word in host-mapped
// pinned memory turns non-zero where the host can read it without
// synchronising, and no PCIe atomic is needed.  Vector memory operations
// only; reached only on the give-up path.
__device__ __forceinline__ void flag_gave_up(unsigned* ws_word, unsigned* status) {
    __hip_atomic_fetch_or(ws_word, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (status != nullptr) __hip_atomic_store(status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

__device__ __forceinline__ unsigned long long wave_max_u64(unsigned long long v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        unsigned long long o = __shfl_xor(v, off, 64);
        v = o > v ? o : v;
    }
    return v;
}

// ---- row kernels shared by RMSNorm, activation quantisation and their fusion
// (one 256-thread workgroup per row; the same code in every kernel, so the
// fused kernel is bit-identical to the two separate launches).

// rstd = 1 / sqrt(mean(x^2) + eps): per-thread fp32 sums of squares over the
// strided elements i = tid, tid + 256, ... in that order (`ss`), folded by a
// wave shuffle tree and then across the four waves in order.
__device__ __forceinline__ float block_rstd(float ss, int H, float eps) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) ss += __shfl_xor(ss, off, 64);
    __shared__ float part[4];
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
    __syncthreads();
    float tot = 0.f;
    for (int w = 0; w < static_cast<int>(blockDim.x >> 6); ++w) tot += part[w];
    return __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(__fdiv_rn(tot, static_cast<float>(H)), eps)));
}

__device__ __forceinline__ float row_rstd(const uint16_t* __restrict__ xr, int H, float eps) {
    float ss = 0.f;
    for (int i = threadIdx.x; i < H; i += blockDim.x) {
        const float v = h2f(xr[i]);
        ss = fmaf(v, v, ss);
    }
    return block_rstd(ss, H, eps);
}

// fp16 RNE((x * rstd) * gamma), each product an IEEE fp32 multiply.
__device__ __forceinline__ uint16_t rms_apply(uint16_t x, float rstd, uint16_t g) {
    return f2h(__fmul_rn(__fmul_rn(h2f(x), rstd), h2f(g)));
}

// Workgroup maximum of per-thread |x| maxima (NaN never becomes the maximum).
__device__ __forceinline__ float row_absmax(float m) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const float o = __shfl_xor(m, off, 64);
        m = o > m ? o : m;
    }
    __shared__ float wmax[4];
    if ((threadIdx.x & 63) == 0) wmax[threadIdx.x >> 6] = m;
    __syncthreads();
    m = wmax[0];
    for (int w = 1; w < static_cast<int>(blockDim.x >> 6); ++w) m = wmax[w] > m ? wmax[w] : m;
    return m;
}

// scale = max / 127 floored at 1e-8 (op_kernel/w8a8_quantize_custom.cpp:25-41).
__device__ __forceinline__ float act_scale(float absmax) {
    const float scale = __fdiv_rn(absmax, 127.0f);
    return scale < 0.00000001f ? 0.00000001f : scale;
}

// quantize_i8 (src/csrc/lib/quantized_weight.cpp:197-202): clamp, then
// round half away from zero by truncating v +- 0.5.
__device__ __forceinline__ int8_t act_quant(uint16_t x, float inv) {
    float v = __fmul_rn(h2f(x), inv);
    v = v > 127.0f ? 127.0f : v;
    v = v < -128.0f ? -128.0f : v;
    const float r = v >= 0.0f ? __fadd_rn(v, 0.5f) : __fsub_rn(v, 0.5f);
    return static_cast<int8_t>(static_cast<int>(r));
}

}  // namespace mcv
