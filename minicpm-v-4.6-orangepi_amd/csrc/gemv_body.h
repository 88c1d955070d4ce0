// gemv_body.h -- the W4A16 GEMV inner loop shared by the decode kernels
// (w4a16_gemv.hip, decode_mlp.hip): kernels built from these pieces add the
// same fp32 terms in the same order, so their outputs agree bit for bit when
// their k-splits do.
#pragma once

#include "common.h"

namespace mcv {

// (a & mask) | magic in one v_and_or_b32.  gfx9 VOP3 encodings take no
// literal and at most one SGPR, so the mask rides in an SGPR and the magic
// exponent pattern in a VGPR; left to itself the compiler emits v_and + v_or.
__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t smask, uint32_t vmagic) {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "s"(smask), "v"(vmagic));
    return r;
}

// One 16-byte chunk of packed weights.  Every weight byte is read once per
// call, so the loads are non-temporal.  Measured on MI355X (same-box A/B):
// with the weights streamed from HBM, as in a decode step whose layers and
// lm_head together exceed the 256 MB MALL, the lm_head step went from 26.7 to
// 24.8 us and the K=N=1024 GEMV from 3.20 to 2.99 us; with a working set that
// fits the MALL the GEMVs are 0.2-0.4 us slower than with ordinary loads.
__device__ __forceinline__ uint4 load_weights(const uint4* p) {
    typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
    const u32x4 t = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    return make_uint4(t.x, t.y, t.z, t.w);
}

// The group's 128 activation values as 64 half2 words.  The index is
// wave-uniform, so these become scalar loads into SGPRs.
__device__ __forceinline__ void load_x_group(const uint32_t* __restrict__ xw, int g, uint32_t (&xs)[64]) {
#pragma unroll
    for (int i = 0; i < 64; ++i) xs[i] = xw[g * 64 + i];
}

// Every load of one trip (weights, scale, zero word, activations) is issued
// before the first wait: left alone, the scheduler sinks the scale and the
// activation loads below the waits for the weight words, which costs each
// trip a second full memory latency.
__device__ __forceinline__ void issue_fence() { __builtin_amdgcn_sched_barrier(0); }

// One quantisation group (four 16-byte chunks of this lane's column,
// activations `xs`): group_sum is its sum of (q - z) * x before the scale,
// group_dot adds sum * scale to `acc` in one fma -- so a kernel may form the
// two steps in different waves and still add exactly what group_dot adds.
__device__ __forceinline__ float group_sum(const uint4 (&wv)[4], const uint32_t (&xs)[64], uint32_t z,
                                           uint32_t vmagic) {
    const uint32_t zlo = (0x6400u + z) * 0x10001u;          // half2(1024 + z)
    const uint32_t zhi = (0x6400u + (z << 4)) * 0x10001u;   // half2(1024 + 16 z)
    const uint32_t mlo = __builtin_amdgcn_readfirstlane(0x000F000Fu);
    const uint32_t mhi = __builtin_amdgcn_readfirstlane(0x00F000F0u);
    float alo = 0.f, ahi = 0.f;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const uint32_t words[4] = {wv[c].x, wv[c].y, wv[c].z, wv[c].w};
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const int kw = (c * kChunkK + w * 8) >> 1;                // half2 index into xs
            const uint32_t q = words[w];
            const uint32_t q8 = q >> 8;
            const half2_t p0 = as_h2(and_or(q, mlo, vmagic)) - as_h2(zlo);    // k+0, k+1
            const half2_t p1 = as_h2(and_or(q, mhi, vmagic)) - as_h2(zhi);    // k+2, k+3 (x16)
            const half2_t p2 = as_h2(and_or(q8, mlo, vmagic)) - as_h2(zlo);   // k+4, k+5
            const half2_t p3 = as_h2(and_or(q8, mhi, vmagic)) - as_h2(zhi);   // k+6, k+7 (x16)
            alo = __builtin_amdgcn_fdot2(p0, as_h2(xs[kw + 0]), alo, false);
            ahi = __builtin_amdgcn_fdot2(p1, as_h2(xs[kw + 1]), ahi, false);
            alo = __builtin_amdgcn_fdot2(p2, as_h2(xs[kw + 2]), alo, false);
            ahi = __builtin_amdgcn_fdot2(p3, as_h2(xs[kw + 3]), ahi, false);
        }
    }
    return alo + ahi * 0.0625f;
}

__device__ __forceinline__ float group_dot(const uint4 (&wv)[4], const uint32_t (&xs)[64], uint32_t z, float scale,
                                           float acc, uint32_t vmagic) {
    return fmaf(group_sum(wv, xs, z, vmagic), scale, acc);
}

// group_sum in two steps, for a kernel that has the weights long before the
// activations: the widened operands first (p[j] pairs with xs[j]), then the
// same fdot2 chains in the same order, so the sum is group_sum's bit for bit.
__device__ __forceinline__ void group_operands(const uint4 (&wv)[4], uint32_t z, uint32_t vmagic, half2_t (&p)[64]) {
    const uint32_t zlo = (0x6400u + z) * 0x10001u;
    const uint32_t zhi = (0x6400u + (z << 4)) * 0x10001u;
    const uint32_t mlo = __builtin_amdgcn_readfirstlane(0x000F000Fu);
    const uint32_t mhi = __builtin_amdgcn_readfirstlane(0x00F000F0u);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const uint32_t words[4] = {wv[c].x, wv[c].y, wv[c].z, wv[c].w};
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const int j = 16 * c + 4 * w;
            const uint32_t q = words[w];
            const uint32_t q8 = q >> 8;
            p[j + 0] = as_h2(and_or(q, mlo, vmagic)) - as_h2(zlo);
            p[j + 1] = as_h2(and_or(q, mhi, vmagic)) - as_h2(zhi);
            p[j + 2] = as_h2(and_or(q8, mlo, vmagic)) - as_h2(zlo);
            p[j + 3] = as_h2(and_or(q8, mhi, vmagic)) - as_h2(zhi);
        }
    }
}

__device__ __forceinline__ float group_sum_operands(const half2_t (&p)[64], const uint32_t (&xs)[64]) {
    float alo = 0.f, ahi = 0.f;
#pragma unroll
    for (int j = 0; j < 64; j += 4) {
        alo = __builtin_amdgcn_fdot2(p[j + 0], as_h2(xs[j + 0]), alo, false);
        ahi = __builtin_amdgcn_fdot2(p[j + 1], as_h2(xs[j + 1]), ahi, false);
        alo = __builtin_amdgcn_fdot2(p[j + 2], as_h2(xs[j + 2]), alo, false);
        ahi = __builtin_amdgcn_fdot2(p[j + 3], as_h2(xs[j + 3]), ahi, false);
    }
    return alo + ahi * 0.0625f;
}

// One lane's column of a W4A16 weight in the slab-64 layout: its packed
// words (slab base + lane), its scale and zero-word columns, and the zero
// bias.  `zshift` selects the lane's nibble in the shared zero word.
struct W4Column {
    const uint4* __restrict__ q;         // + g * 4 * kSlab per group, + c * kSlab per chunk
    const uint16_t* __restrict__ s;      // + g * Npad per group
    const uint32_t* __restrict__ z;      // + g * (Npad / 8) per group
    uint32_t zshift;
    uint32_t zero_bias;
    int npad;
};

__device__ __forceinline__ W4Column w4_column(const uint4* qw, const uint16_t* scales, const uint32_t* zeros,
                                              uint32_t zero_bias, int K, int Npad, int slab, int lane) {
    const int n = slab * kSlab + lane;
    return W4Column{qw + static_cast<size_t>(slab) * (K / kChunkK) * kSlab + lane, scales + n, zeros + (n >> 3),
                    static_cast<uint32_t>(n & 7) * 4u, zero_bias, Npad};
}

// One weight's sum for one lane's column over the groups g0, g0 + step, ...
// below G, in that order (a GEMV wave's chain; the fused gate+up kernels run
// the gate and the up chain of a column on two lanes).
__device__ __forceinline__ float w4_partials(const uint32_t* __restrict__ xw, const W4Column& c, int g0, int step,
                                             int G, uint32_t vmagic) {
    float a = 0.f;
    for (int g = g0; g < G; g += step) {
        uint4 wv[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) wv[i] = load_weights(c.q + static_cast<size_t>(g * 4 + i) * kSlab);
        const uint16_t sv = c.s[static_cast<size_t>(g) * c.npad];
        const uint32_t zv = c.z[static_cast<size_t>(g) * (c.npad >> 3)];
        uint32_t xs[64];
        load_x_group(xw, g, xs);
        issue_fence();
        a = group_dot(wv, xs, ((zv >> c.zshift) & 15u) + c.zero_bias, h2f(sv), a, vmagic);
    }
    return a;
}

}  // namespace mcv
