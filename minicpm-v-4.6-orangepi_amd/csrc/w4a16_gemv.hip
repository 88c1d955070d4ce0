// w4a16_gemv.hip -- W4A16 decode kernels for gfx950.
//
// Streaming GEMV over the slab-64 layout (see include/mcv_quant.h): each lane
// owns one output column and walks K in 16-byte chunks, so every wave-wide
// 128-bit load is one contiguous 1 KiB line.  Nibbles are widened in registers
// with the fp16 exponent-bias identity: bits 0x6400 | q form the fp16 value
// 1024 + q, and 0x6400 | (q << 4) the value 1024 + 16 q; subtracting
// 1024 + z (or 1024 + 16 z) leaves the exact q - z (or 16 (q - z)).  Pairs of
// consecutive k then go through v_dot2_f32_f16 against the activation pairs,
// accumulating in fp32.  The activation row is wave-uniform and is read with
// scalar loads.  Waves of a workgroup split K; partial sums meet in LDS.
//
// Replaces the NPU kernel src/csrc/custom_ops/op_kernel/matmul_w4a16_custom.cpp
// (8 AICore blocks, int8 tiles, fp16 Axpy accumulation) and its host wrapper
// src/csrc/lib/ops.cpp:1030-1095.
#include <algorithm>
#include <cstdint>
#include <cstdlib>
#include <atomic>
#include <mutex>

#include "argmax_exchange.h"
#include "common.h"
#include "gemv_body.h"

namespace mcv {
namespace {

constexpr int kSlotWords = 64;                                // slots of the host-finished route

// ARGMAX modes of the GEMV epilogue (M == 1 only).
constexpr int kArgNone = 0;
constexpr int kArgPartials = 1;   // plain store of the slab's key to keys[slab]

// grid = (Nslab, M), block = 64 * KSPLIT.  Wave w handles groups
// {w*GPW + r*KSPLIT*GPW + i : i < GPW}.
template <int KSPLIT, int GPW, int ARGMAX>
__global__ __launch_bounds__(64 * KSPLIT) void w4a16_gemv_kernel(
    const uint16_t* __restrict__ x, const uint4* __restrict__ qw, const uint16_t* __restrict__ scales,
    const uint32_t* __restrict__ zeros, uint32_t zero_bias, uint16_t* __restrict__ out, int K, int N,
    int Npad, unsigned long long* __restrict__ keys, int64_t* __restrict__ token) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // wave-uniform: keeps x loads scalar
    const int slab = blockIdx.x;
    const int m = blockIdx.y;
    const int n = slab * kSlab + lane;
    const int G = K / kGroup;
    uint32_t vmagic;                                                     // 0x64006400 = half2(1024, 1024)
    asm("v_mov_b32 %0, 0x64006400" : "=v"(vmagic));
    const int C = K / kChunkK;
    const uint4* __restrict__ wp = qw + static_cast<size_t>(slab) * C * kSlab + lane;
    const uint32_t* __restrict__ xw = reinterpret_cast<const uint32_t*>(x + static_cast<size_t>(m) * K);
    const uint16_t* __restrict__ sp = scales + n;
    const uint32_t* __restrict__ zp = zeros + (n >> 3);
    const uint32_t zshift = (n & 7) * 4;
    const int zstride = Npad >> 3;

    float acc = 0.f;
    for (int gb = wave * GPW; gb < G; gb += KSPLIT * GPW) {
        uint4 wv[GPW][4];
        uint16_t sv[GPW];
        uint32_t zv[GPW];
#pragma unroll
        for (int i = 0; i < GPW; ++i) {
            const int g = gb + i;
            if (g < G) {
#pragma unroll
                for (int c = 0; c < 4; ++c) wv[i][c] = load_weights(wp + static_cast<size_t>(g * 4 + c) * kSlab);
                sv[i] = sp[static_cast<size_t>(g) * Npad];
                zv[i] = zp[static_cast<size_t>(g) * zstride];
            }
        }
#pragma unroll
        for (int i = 0; i < GPW; ++i) {
            const int g = gb + i;
            if (g < G) {
                uint32_t xs[64];
                load_x_group(xw, g, xs);
                if (i == 0) issue_fence();
                acc = group_dot(wv[i], xs, ((zv[i] >> zshift) & 15u) + zero_bias, h2f(sv[i]), acc, vmagic);
            }
        }
    }

    if constexpr (KSPLIT > 1) {
        __shared__ float red[KSPLIT][kSlab];
        red[wave][lane] = acc;
        __syncthreads();
        if (wave != 0) return;
        acc = red[0][lane];
#pragma unroll
        for (int w = 1; w < KSPLIT; ++w) acc += red[w][lane];
    }

    const uint16_t h = f2h(acc);
    if (out != nullptr && n < N) out[static_cast<size_t>(m) * N + n] = h;
    if constexpr (ARGMAX != kArgNone) {
        unsigned long long key = n < N ? argmax_key64(argmax_key16(h), static_cast<uint32_t>(n)) : 0ull;
        key = wave_max_u64(key);
        if (lane == 0) keys[slab] = key;
    }
}

// Greedy lm_head: the GEMV with the argmax folded in.  Eight waves per
// workgroup, wave w owning quantisation groups w, w + 8, ...; a workgroup
// walks SPW consecutive slabs.  When K <= 1024 (one group per wave) the
// activation group stays in SGPRs for the whole workgroup and the next slab's
// weight, scale and zero loads are issued before the current slab is
// decoded.  Per-slab partial sums go to LDS and meet after one barrier (idle
// waves contribute -0.0, the exact additive identity, so the sums equal the
// GEMV's whenever that also gives each wave one group).  The best key then
// leaves through one of two routes:
//   kLmTree  -- the call-tagged key words above; the grid's last workgroup
//               polls them and writes the token on the device;
//   kLmSlots -- one fire-and-forget atomicMax of a call-tagged key into one
//               of 64 slots; whoever reads the token takes the maximum of the
//               slots that carry this call's tag (the host, after the copy it
//               makes anyway).  Slot key bits: 63..40 tag, 39..24 the fp16
//               key, 23..0 the complement of the column index.
// Measured on the lm_head shape (MI355X, 8 rotated weight copies, graph-
// replayed): SPW 16 (243 workgroups) with the tree 26.9-27.2 us, with slots
// 25.7-26.0 us; SPW 8 27.1-27.3 / 26.4-27.0 us; SPW 1-4 28-30 us; the former
// one-slab, four-wave kernel ~27.9 us.  Direct launches run ~1 us faster.
// 256 workgroups with 15 or 16 slabs each (one per CU, the slabs even over
// the XCDs) measured 0.5-1.1 us slower than 243 with 16 on the full
// vocabulary, and 0.6 us slower at V = 124047.
constexpr int kLmWaves = 8;
constexpr int kLmTree = 0;
constexpr int kLmSlots = 1;
constexpr int kSlotStride = 16;                              // u64 words per slot: 128 B

template <int SPW, int MODE>
__global__ __launch_bounds__(64 * kLmWaves) void w4a16_lm_head_kernel(
    const uint16_t* __restrict__ x, const uint4* __restrict__ qw, const uint16_t* __restrict__ scales,
    const uint32_t* __restrict__ zeros, uint32_t zero_bias, uint16_t* __restrict__ logits, int K, int V, int Npad,
    int nslab, unsigned long long* __restrict__ ws, int64_t* __restrict__ token, uint32_t tag, unsigned* status) {
    __shared__ float part[SPW][kLmWaves][kSlab];
    __shared__ unsigned long long wbest[kLmWaves];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int G = K / kGroup;
    const int C = K / kChunkK;
    const int zstride = Npad >> 3;
    const uint32_t* __restrict__ xw = reinterpret_cast<const uint32_t*>(x);
    uint32_t vmagic;                                                     // 0x64006400 = half2(1024, 1024)
    asm("v_mov_b32 %0, 0x64006400" : "=v"(vmagic));
    const int s0 = static_cast<int>(blockIdx.x) * SPW;
    // the call's generation word (device-token route), issued before the
    // weight loads and needed only at the end
    unsigned gen = 0;
    if constexpr (MODE == kLmTree)
        if (wave == 0)
            gen = __hip_atomic_load(reinterpret_cast<unsigned*>(ws) + kLmGen, __ATOMIC_RELAXED,
                                    __HIP_MEMORY_SCOPE_AGENT);
    const int ns = nslab - s0 < SPW ? nslab - s0 : SPW;                  // workgroup-uniform
    const uint32_t zshift = (lane & 7) * 4;                              // slab bases are multiples of 8 columns
    const uint4* __restrict__ wbase = qw + lane;
    const uint16_t* __restrict__ sbase = scales + lane;
    const uint32_t* __restrict__ zbase = zeros + (lane >> 3);
    auto issue = [&](uint4 (&wv)[4], uint16_t& sv, uint32_t& zv, int slab, int g) {
        const uint4* __restrict__ p = wbase + (static_cast<size_t>(slab) * C + g * 4) * kSlab;
#pragma unroll
        for (int c = 0; c < 4; ++c) wv[c] = load_weights(p + c * kSlab);
        sv = sbase[static_cast<size_t>(g) * Npad + slab * kSlab];
        zv = zbase[static_cast<size_t>(g) * zstride + slab * (kSlab / 8)];
    };

    if (G <= kLmWaves && ns == SPW) {
        if (wave < G) {
            uint32_t xs[64];
            load_x_group(xw, wave, xs);
            uint4 wv[2][4];
            uint16_t sv[2];
            uint32_t zv[2];
            issue(wv[0], sv[0], zv[0], s0, wave);
#pragma unroll
            for (int i = 0; i < SPW; ++i) {
                if (i + 1 < SPW) issue(wv[(i + 1) & 1], sv[(i + 1) & 1], zv[(i + 1) & 1], s0 + i + 1, wave);
                issue_fence();
                part[i][wave][lane] = group_dot(wv[i & 1], xs, ((zv[i & 1] >> zshift) & 15u) + zero_bias,
                                                h2f(sv[i & 1]), 0.f, vmagic);
            }
        } else {
#pragma unroll
            for (int i = 0; i < SPW; ++i) part[i][wave][lane] = -0.0f;
        }
    } else {
        for (int i = 0; i < ns; ++i) {
            float acc = -0.0f;
            for (int g = wave; g < G; g += kLmWaves) {
                uint4 wv[4];
                uint16_t sv;
                uint32_t zv;
                issue(wv, sv, zv, s0 + i, g);
                uint32_t xs[64];
                load_x_group(xw, g, xs);
                issue_fence();
                acc = group_dot(wv, xs, ((zv >> zshift) & 15u) + zero_bias, h2f(sv), g == wave ? 0.f : acc, vmagic);
            }
            part[i][wave][lane] = acc;
        }
    }
    __syncthreads();

    unsigned long long best = 0ull;
    for (int i = wave; i < ns; i += kLmWaves) {
        float acc = part[i][0][lane];
#pragma unroll
        for (int w = 1; w < kLmWaves; ++w) acc += part[i][w][lane];
        const int n = (s0 + i) * kSlab + lane;
        const uint16_t h = f2h(acc);
        if (logits != nullptr && n < V) logits[n] = h;
        const unsigned long long key = n < V ? argmax_key64(argmax_key16(h), static_cast<uint32_t>(n)) : 0ull;
        best = key > best ? key : best;
    }
    best = wave_max_u64(best);
    if (lane == 0) wbest[wave] = best;
    __syncthreads();
    if (wave != 0) return;
    best = wave_max_u64(lane < kLmWaves ? wbest[lane] : 0ull);
    if constexpr (MODE == kLmTree) {
        argmax_publish(ws, best, gen, tag, static_cast<int>(blockIdx.x), static_cast<int>(gridDim.x), lane, token,
                       status);
    } else {
        if (lane == 0) {
            // argmax_key64 -> slot key: the fp16 key moves to bits 39..24, the
            // index complement keeps its low 24 bits (V < 2^24)
            const unsigned long long k16 = best >> 32;
            const unsigned long long idx = best & 0xffffffull;
            atomicMax(ws + (blockIdx.x & (kSlotWords - 1)) * kSlotStride,
                      (static_cast<unsigned long long>(tag) << 40) | (k16 << 24) | (k16 ? idx : 0ull));
        }
    }
}

// Several projections of one activation row in one launch (q/k/v,
// decoder_layer.cpp:970-972; qkv and z, :1108-1110): the grid runs over the
// concatenated slabs of up to kMaxParts weights, each workgroup picks its
// weight from the running slab ends and then does exactly what the GEMV above
// does with GPW = 1, so with the same k-split the outputs are bit-identical to
// separate launches.
constexpr int kMaxParts = 4;
struct GemvPart {
    const uint4* qw;
    const uint16_t* scales;
    const uint32_t* zeros;
    uint16_t* out;
    int N;
    int Npad;
    int slab_end;          // running total of slabs up to and including this part
    uint32_t zero_bias;
};
struct GemvParts {
    GemvPart p[kMaxParts];
    int count;
};

template <int KSPLIT>
__global__ __launch_bounds__(64 * KSPLIT) void w4a16_gemv_multi_kernel(const uint16_t* __restrict__ x, GemvParts parts,
                                                                        int K) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int gslab = blockIdx.x;
    const int m = blockIdx.y;
    // the part this slab belongs to (constant indices only: the kernel
    // arguments stay in SGPRs)
    GemvPart P = parts.p[0];
    int slab0 = 0;
#pragma unroll
    for (int j = 1; j < kMaxParts; ++j) {
        if (j < parts.count && gslab >= parts.p[j - 1].slab_end) {
            P = parts.p[j];
            slab0 = parts.p[j - 1].slab_end;
        }
    }
    const int slab = gslab - slab0;
    const int n = slab * kSlab + lane;
    const int G = K / kGroup;
    const int C = K / kChunkK;
    uint32_t vmagic;                                                     // 0x64006400 = half2(1024, 1024)
    asm("v_mov_b32 %0, 0x64006400" : "=v"(vmagic));
    const uint4* __restrict__ wp = P.qw + static_cast<size_t>(slab) * C * kSlab + lane;
    const uint32_t* __restrict__ xw = reinterpret_cast<const uint32_t*>(x + static_cast<size_t>(m) * K);
    const uint32_t zshift = (n & 7) * 4;
    const int zstride = P.Npad >> 3;
    float acc = 0.f;
    for (int g = wave; g < G; g += KSPLIT) {
        uint4 wv[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) wv[c] = load_weights(wp + static_cast<size_t>(g * 4 + c) * kSlab);
        const uint16_t sv = P.scales[static_cast<size_t>(g) * P.Npad + n];
        const uint32_t zv = P.zeros[static_cast<size_t>(g) * zstride + (n >> 3)];
        uint32_t xs[64];
        load_x_group(xw, g, xs);
        issue_fence();
        acc = group_dot(wv, xs, ((zv >> zshift) & 15u) + P.zero_bias, h2f(sv), acc, vmagic);
    }
    if constexpr (KSPLIT > 1) {
        __shared__ float red[KSPLIT][kSlab];
        red[wave][lane] = acc;
        __syncthreads();
        if (wave != 0) return;
        acc = red[0][lane];
#pragma unroll
        for (int w = 1; w < KSPLIT; ++w) acc += red[w][lane];
    }
    if (n < P.N) P.out[static_cast<size_t>(m) * P.N + n] = f2h(acc);
}

// Decode MLP front half in one launch: act = silu(x . Wgate) * (x . Wup).
// Each workgroup owns one 32-column half of a slab of both weights: lanes
// 0-31 run the gate chains of its columns and lanes 32-63 the up chains of
// the same columns (one chain per lane, half a slab's bytes per workgroup);
// its waves split K exactly like the GEMV (the same group_dot per weight), the
// partial sums meet in LDS, and wave 0 rounds gate and up to fp16 -- as the
// separate GEMV launches store them -- before silu_mul_f16, so the result is
// bit-identical to gate GEMV + up GEMV + silu_mul.  Measured on MI355X inside
// the one-launch MLP block (H=1024, I=3584), half slabs against whole slabs
// with both chains per lane: 6.98 against 7.62 us per block.
// grid = (2 Nslab, M).
template <int KSPLIT>
__global__ __launch_bounds__(64 * KSPLIT) void w4a16_gate_up_silu_kernel(
    const uint16_t* __restrict__ x, const uint4* __restrict__ qg, const uint16_t* __restrict__ sg,
    const uint32_t* __restrict__ zg, uint32_t zbg, const uint4* __restrict__ qu, const uint16_t* __restrict__ su,
    const uint32_t* __restrict__ zu, uint32_t zbu, uint16_t* __restrict__ act, int K, int N, int Npad) {
    __shared__ float red[2][KSPLIT][32];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int slab = blockIdx.x >> 1;
    const int col = 32 * (blockIdx.x & 1) + (lane & 31), pj = lane >> 5;
    const int m = blockIdx.y;
    const int G = K / kGroup;
    const uint32_t* __restrict__ xw = reinterpret_cast<const uint32_t*>(x + static_cast<size_t>(m) * K);
    uint32_t vmagic;                                                     // 0x64006400 = half2(1024, 1024)
    asm("v_mov_b32 %0, 0x64006400" : "=v"(vmagic));
    red[pj][wave][lane & 31] = w4_partials(xw, pj ? w4_column(qu, su, zu, zbu, K, Npad, slab, col)
                                                  : w4_column(qg, sg, zg, zbg, K, Npad, slab, col),
                                           wave, KSPLIT, G, vmagic);
    __syncthreads();
    if (wave != 0 || lane >= 32) return;
    float ag = red[0][0][lane], au = red[1][0][lane];
#pragma unroll
    for (int w = 1; w < KSPLIT; ++w) {
        ag += red[0][w][lane];
        au += red[1][w][lane];
    }
    const int n = slab * kSlab + col;
    if (n < N) act[static_cast<size_t>(m) * N + n] = silu_mul_f16(f2h(ag), f2h(au));
}

// One workgroup folds the per-slab keys into the token (first maximum wins:
// the key orders by value, then by smallest index).
__global__ __launch_bounds__(1024) void argmax_reduce_kernel(const unsigned long long* __restrict__ keys, int n,
                                                             int64_t* __restrict__ token) {
    unsigned long long best = 0ull;
    for (int i = threadIdx.x; i < n; i += blockDim.x) best = keys[i] > best ? keys[i] : best;
    best = wave_max_u64(best);
    __shared__ unsigned long long wbest[16];
    if ((threadIdx.x & 63) == 0) wbest[threadIdx.x >> 6] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < static_cast<int>(blockDim.x >> 6); ++w) best = wbest[w] > best ? wbest[w] : best;
        *token = argmax_index(best);
    }
}

template <int ARGMAX>
using GemvFn = void (*)(const uint16_t*, const uint4*, const uint16_t*, const uint32_t*, uint32_t, uint16_t*, int,
                        int, int, unsigned long long*, int64_t*);

template <int ARGMAX>
GemvFn<ARGMAX> pick_kernel(int ks, int gpw) {
    if (gpw != 1) return nullptr;                 // one group per wave per trip (choose_gemv)
    switch (ks) {
        case 1: return w4a16_gemv_kernel<1, 1, ARGMAX>;
        case 2: return w4a16_gemv_kernel<2, 1, ARGMAX>;
        case 4: return w4a16_gemv_kernel<4, 1, ARGMAX>;
        case 8: return w4a16_gemv_kernel<8, 1, ARGMAX>;
        default: return w4a16_gemv_kernel<16, 1, ARGMAX>;
    }
}

struct GemvCfg {
    int ksplit;
    int gpw;
};

// One quantisation group (four 16-byte loads per lane) per wave per trip,
// and enough waves per workgroup (up to 16, at most one per group) that the
// grid holds >= 8K waves, 32 per CU.  Measured on the lm_head shape (K=1024,
// 3877 slabs) with graph-replayed launches: 4 waves x 1 group (two trips)
// 25.4 us, 8 x 1 25.8 us, 4 x 2 27.1 us, 2 x 4 31.0 us; the decode is VALU
// heavy, so more loads in flight per wave do not pay.  On the decoder's
// narrow projections the grid is tiny and the serial trips per wave set the
// time: K=3584 N=1024 8 x 1 6.45 us, 16 x 1 5.39 us; K=2048 N=1024 4.56 us
// vs 4.07 us.
GemvCfg choose_gemv(int64_t G, int64_t blocks) {
    int ks = 1;
    while (ks < 16 && blocks * ks < 8192 && ks * 2 <= G) ks *= 2;
    return GemvCfg{ks, 1};
}

bool w4_args_ok(const void* qw, const void* scales, const void* zeros, int zero_bias, int64_t K, int64_t N,
                const char* who, int* rc) {
    if (!qw || !scales || !zeros) { *rc = fail(MCV_ERR_INVALID_ARG, "%s: null weight pointer", who); return false; }
    if (zero_bias != 0 && zero_bias != 1) { *rc = fail(MCV_ERR_INVALID_ARG, "%s: zero_bias must be 0 or 1", who); return false; }
    if (K <= 0 || K % kGroup != 0 || K > (int64_t(1) << 24)) {
        *rc = fail(MCV_ERR_SHAPE, "%s: K must be a positive multiple of 128 (K=%lld)", who, (long long)K);
        return false;
    }
    if (N <= 0 || N > (int64_t(1) << 30)) {
        *rc = fail(MCV_ERR_SHAPE, "%s: N out of range (N=%lld)", who, (long long)N);
        return false;
    }
    return true;
}

// ------------------------------------------------------------- dequant --
// grid = (Nslab, K/32), block = 64: lane -> column, blockIdx.y -> chunk.
__global__ __launch_bounds__(64) void w4a16_dequant_kernel(const uint4* __restrict__ qw,
                                                           const uint16_t* __restrict__ scales,
                                                           const uint32_t* __restrict__ zeros, uint32_t zero_bias,
                                                           int K, int N, int Npad, uint16_t* __restrict__ wf,
                                                           int8_t* __restrict__ w8) {
    const int lane = threadIdx.x;
    const int slab = blockIdx.x;
    const int c = blockIdx.y;
    const int n = slab * kSlab + lane;
    if (n >= N) return;
    const int C = K / kChunkK;
    const int g = c / 4;
    const uint4 v = qw[(static_cast<size_t>(slab) * C + c) * kSlab + lane];
    const float s = h2f(scales[static_cast<size_t>(g) * Npad + n]);
    const int z = static_cast<int>(((zeros[static_cast<size_t>(g) * (Npad >> 3) + (n >> 3)] >> ((n & 7) * 4)) & 15u) + zero_bias);
    const uint32_t words[4] = {v.x, v.y, v.z, v.w};
    constexpr int kSlotOfK[8] = {0, 4, 1, 5, 2, 6, 3, 7};
#pragma unroll
    for (int w = 0; w < 4; ++w) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int k = c * kChunkK + w * 8 + j;
            const int d = static_cast<int>((words[w] >> (4 * kSlotOfK[j])) & 15u) - z;
            const size_t o = static_cast<size_t>(k) * N + n;
            if (w8) w8[o] = static_cast<int8_t>(d);
            if (wf) wf[o] = f2h(static_cast<float>(d) * s);   // exact product, one RNE
        }
    }
}

// ------------------------------------------- reference int8 tile format --
// The reference's own device format (quantized_weight.cpp:41-73): int8 (q - z)
// in [128][tileLen] tiles ordered (group, block b of 8, tile t, k, i), column
// b * blockLen + t * tileLen + i.  A tile's tileLen / 16 chunks of 16 columns
// are split into slices of CS chunks, one workgroup of kTiWaves waves per
// (tile, slice): all of a tile when there are >= 64 tiles, down to one chunk
// per workgroup for the narrow projections (8 tiles).  Lane l of a wave takes
// chunk l % CS of the slice in row r = l / CS of each R-row band (R = the
// largest power of two with R * CS <= 64; lanes past R * CS idle), one
// 16-byte load per band; the waves take the bands of a group in turn, so a
// lane holds JPG = 128 / (kTiWaves * R) rows of each group (or, when a step
// of all waves spans several groups, one row of every gstep-th group).  Per
// group a lane sums x * (q - z) over its rows in fp32, multiplies the sum by
// its columns' scales and adds it to its accumulators; the next group's loads
// are in flight meanwhile.  The lanes of one chunk then add up across the
// rows by shuffles, the waves through LDS.  The same terms as the
// reference's per-group partial sums, added in another order.  Measured on
// MI355X (graph-replayed, rotated weights): the former one-thread-per-column
// kernel took 74 us at K=N=1024, 390 us at K=3584 N=1024 and 140 us at
// K=1024 N=248064.
constexpr int kTiWaves = 8;
constexpr int kTiMaxJ = 8;                               // rows per lane per group: 128 / (8 * 2)

struct Ti8Group {
    uint4 q[kTiMaxJ];
    float xv[kTiMaxJ];
    uint4 s[2];
};

__global__ __launch_bounds__(64 * kTiWaves) void w4a16_tiled_i8_kernel(const uint16_t* __restrict__ x,
                                                                      const int8_t* __restrict__ w,
                                                                      const uint16_t* __restrict__ scales,
                                                                      uint16_t* __restrict__ out, int K, int N,
                                                                      int blockLen, int tileLen, int tilesPerBlock,
                                                                      int CS, int slices) {
    __shared__ float red[kTiWaves][448];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int CN = tileLen >> 4;
    int R = 1;
    while (R * 2 * CS <= 64) R *= 2;
    const int tile = static_cast<int>(blockIdx.x) / slices, sl = static_cast<int>(blockIdx.x) % slices;
    const int b = tile / tilesPerBlock, t = tile % tilesPerBlock;
    const int CSa = CN - sl * CS < CS ? CN - sl * CS : CS;          // chunks of this slice
    const int cl = lane % CS, r = lane / CS;
    const int c = sl * CS + cl;
    // blockLen and tile offsets are multiples of 16, so a chunk lies wholly
    // inside the block or wholly in the last tile's padding (no scales there)
    const bool live = r < R && cl < CSa && t * tileLen + 16 * c < blockLen;
    const int col0 = b * blockLen + t * tileLen + 16 * c;
    const int G = K / kGroup;
    const int band = kTiWaves * R;                       // rows per step of all waves
    const int row0 = wave * R + r;
    // rows of group g this lane holds: g * 128 + rowin + j * band, j < jpg
    const int jpg = band <= kGroup ? kGroup / band : 1;
    const int gstep = band <= kGroup ? 1 : band / kGroup;
    const int gsub = band <= kGroup ? 0 : row0 / kGroup;
    const int rowin = band <= kGroup ? row0 : row0 % kGroup;
    const size_t tile_bytes = static_cast<size_t>(kGroup) * tileLen;
    const int8_t* __restrict__ wl = w + (static_cast<size_t>(b) * tilesPerBlock + t) * tile_bytes + 16 * c +
                                    static_cast<size_t>(rowin) * tileLen;
    const size_t gstride = static_cast<size_t>(8) * tilesPerBlock * tile_bytes;    // bytes per group
    float acc[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[e] = 0.f;
    auto load = [&](int g, Ti8Group& d) {
        const int8_t* p = wl + static_cast<size_t>(g) * gstride;
#pragma unroll
        for (int jj = 0; jj < kTiMaxJ; ++jj)
            if (jj < jpg) {
                d.q[jj] = *reinterpret_cast<const uint4*>(p + static_cast<size_t>(jj) * band * tileLen);
                d.xv[jj] = h2f(x[g * kGroup + rowin + jj * band]);
            }
        const uint4* sp = reinterpret_cast<const uint4*>(scales + static_cast<size_t>(g) * N + col0);
        d.s[0] = sp[0];
        d.s[1] = sp[1];
    };
    auto sum = [&](const Ti8Group& d) {
        float part[16];
#pragma unroll
        for (int e = 0; e < 16; ++e) part[e] = 0.f;
#pragma unroll
        for (int jj = 0; jj < kTiMaxJ; ++jj)
            if (jj < jpg) {
                const uint32_t words[4] = {d.q[jj].x, d.q[jj].y, d.q[jj].z, d.q[jj].w};
#pragma unroll
                for (int wd = 0; wd < 4; ++wd)
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        part[4 * wd + e] = fmaf(d.xv[jj],
                                                static_cast<float>(static_cast<int8_t>((words[wd] >> (8 * e)) & 0xffu)),
                                                part[4 * wd + e]);
            }
        const uint32_t sw[8] = {d.s[0].x, d.s[0].y, d.s[0].z, d.s[0].w, d.s[1].x, d.s[1].y, d.s[1].z, d.s[1].w};
#pragma unroll
        for (int e = 0; e < 16; ++e)
            acc[e] = fmaf(part[e], h2f(static_cast<uint16_t>(sw[e >> 1] >> (16 * (e & 1)))), acc[e]);
    };
    if (live && gsub < G) {
        Ti8Group A, B;
        load(gsub, A);
        for (int g = gsub; g < G; g += 2 * gstep) {
            const int g1 = g + gstep, g2 = g + 2 * gstep;
            if (g1 < G) load(g1, B);
            sum(A);
            if (g1 >= G) break;
            if (g2 < G) load(g2, A);
            sum(B);
        }
    }
    // rows r of one chunk meet in lane cl (r = 0): a tree over offsets
    // CS, 2 CS, ... (idle lanes hold zeros; a lane that adds reads r + 2^i < R)
    for (int m = 1; m < R; m <<= 1)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[e] += __shfl_down(acc[e], m * CS, 64);
    if (r == 0 && cl < CSa) {
#pragma unroll
        for (int e = 0; e < 16; ++e) red[wave][16 * cl + e] = acc[e];
    }
    __syncthreads();
    for (int col = threadIdx.x; col < 16 * CSa; col += blockDim.x) {
        float total = 0.f;
#pragma unroll
        for (int v = 0; v < kTiWaves; ++v) total += red[v][col];
        const int i = t * tileLen + 16 * sl * CS + col;
        const int n = b * blockLen + i;
        if (i < blockLen && n < N) out[n] = f2h(total);
    }
}

// ---- the lm_head's workspace in library memory, for callers that cannot
// allocate (mcv_w4a16_lm_head_argmax_noalloc).  Every GPU the library runs on
// holds its own copy of this array until the process ends; host code never
// passes the array's name to a kernel (on the host it is only a stand-in):
// it uses the device address hipGetSymbolAddress returns for the current GPU.
constexpr int64_t kNoallocMaxV = int64_t(1) << 20;
constexpr int64_t kNoallocWords = kLmKeysByte / 8 + (kNoallocMaxV + kSlab - 1) / kSlab;   // u64 words for V = kNoallocMaxV
static __device__ __align__(256) unsigned long long scratch[kNoallocWords];

}  // namespace

// The GEMV launchers' k-split, for kernels that must add in the same order
// (decode_mlp.hip).
int gemv_ksplit(int64_t G, int64_t blocks) { return choose_gemv(G, blocks).ksplit; }

// Internal entry used by the dispatcher in w4a16_gemm.hip.
int launch_w4a16_gemv(const void* x, int64_t M, int64_t K, int64_t N, const void* qw, const void* scales,
                      const void* zeros, int zero_bias, void* out, hipStream_t stream) {
    int rc = MCV_OK;
    if (!w4_args_ok(qw, scales, zeros, zero_bias, K, N, "mcv_w4a16_gemv", &rc)) return rc;
    if (!x || !out) return fail(MCV_ERR_INVALID_ARG, "mcv_w4a16_gemv: null x/out");
    if (M <= 0 || M > 65535) return fail(MCV_ERR_SHAPE, "mcv_w4a16_gemv: M must be in [1, 65535] (M=%lld)", (long long)M);
    if ((rc = require_device()) != MCV_OK) return rc;
    const int64_t nslab = ceil_div(N, kSlab);
    const GemvCfg cfg = choose_gemv(K / kGroup, nslab * M);
    auto fn = pick_kernel<kArgNone>(cfg.ksplit, cfg.gpw);
    hipLaunchKernelGGL(fn, dim3(static_cast<unsigned>(nslab), static_cast<unsigned>(M)), dim3(64 * cfg.ksplit), 0,
                       stream, static_cast<const uint16_t*>(x), static_cast<const uint4*>(qw),
                       static_cast<const uint16_t*>(scales), static_cast<const uint32_t*>(zeros),
                       static_cast<uint32_t>(zero_bias), static_cast<uint16_t*>(out), static_cast<int>(K),
                       static_cast<int>(N), static_cast<int>(nslab * kSlab), nullptr, nullptr);
    return check_launch("w4a16_gemv_kernel");
}

// Slabs per workgroup: the most (up to 16) that still leave >= 240
// workgroups, except that a grid of one slab per workgroup is used whenever
// it fits two workgroups per CU.  Measured on MI355X (K=1024, rotated weight
// copies past the MALL, 5000 direct launches, us per call, SPW 1/2/4/8/16):
// the full vocabulary V=248094 (3877 slabs) -/-/-/24.7/24.1; a half,
// V=124047: 18.6/16.0/15.4/14.8/19.1; a quarter, V=62024: 10.9/9.9/9.9/
// 11.8/18.6; an eighth, V=31012 (485 slabs): 6.9/7.6/8.4/11.6/18.5 -- long
// double-buffered runs of slabs pay while the grid still covers the CUs,
// and at a few slabs per workgroup more workgroups hide more latency.  A
// function of V alone, so a workspace (sized for one workgroup per slab)
// always meets the same grid.
int lm_head_spw(int64_t nslab) {
    int spw = 16;
    while (spw > 1 && ceil_div(nslab, spw) < 240) spw /= 2;
    if (spw == 2 && nslab <= 512) spw = 1;
    return spw;
}

// Test hook (mcv_testing_lm_head_skew_poll): the device-token route's poller
// expects a tag no key carries.
std::atomic<unsigned> g_lm_poll_skew{0};

// ... also for the W8A8 lm_head (w8a8_tiled.hip).
unsigned lm_poll_skew() { return g_lm_poll_skew.load(std::memory_order_relaxed); }

// Shared launcher of both argmax routes (`tag`: the slots route's call tag;
// the device-token route passes the poll skew in its place).
int launch_lm_head(const void* x, int64_t K, int64_t N, int64_t V, const void* qw, const void* scales,
                   const void* zeros, int zero_bias, void* logits, int64_t* token, void* ws, uint32_t tag, int mode,
                   unsigned* status, hipStream_t stream) {
    const int64_t nslab = ceil_div(V, kSlab);
    const int64_t npad = ceil_div(N, kSlab) * kSlab;
    const int spw = lm_head_spw(nslab);
    using LmFn = void (*)(const uint16_t*, const uint4*, const uint16_t*, const uint32_t*, uint32_t, uint16_t*, int, int,
                          int, int, unsigned long long*, int64_t*, uint32_t, unsigned*);
    LmFn fn = nullptr;
#define MCV_LM(SPW_)                                                                                  \
    if (spw == SPW_)                                                                                  \
        fn = mode == kLmTree ? w4a16_lm_head_kernel<SPW_, kLmTree> : w4a16_lm_head_kernel<SPW_, kLmSlots>;
    MCV_LM(1) MCV_LM(2) MCV_LM(4) MCV_LM(8) MCV_LM(16)
#undef MCV_LM
    const int64_t nblk = ceil_div(nslab, spw);
    hipLaunchKernelGGL(fn, dim3(static_cast<unsigned>(nblk)), dim3(64 * kLmWaves), 0, stream,
                       static_cast<const uint16_t*>(x), static_cast<const uint4*>(qw),
                       static_cast<const uint16_t*>(scales), static_cast<const uint32_t*>(zeros),
                       static_cast<uint32_t>(zero_bias), static_cast<uint16_t*>(logits), static_cast<int>(K),
                       static_cast<int>(V), static_cast<int>(npad), static_cast<int>(nslab),
                       static_cast<unsigned long long*>(ws), token,
                       mode == kLmTree ? g_lm_poll_skew.load(std::memory_order_relaxed) : tag, status);
    return check_launch("w4a16_lm_head_kernel");
}


namespace {

// Per-GPU state of the no-allocation route: the scratch array's device
// address on that GPU (fixed-size, so looking a device up allocates nothing).
// The array needs no host-side bookkeeping beyond that: it starts zero-filled
// with the code object, and its generation word and fixed-offset key words
// stay consistent from call to call, for any V, in eager calls and graph
// replays alike.
constexpr int kNoallocMaxDevices = 64;
unsigned long long* g_noalloc[kNoallocMaxDevices];
std::mutex g_noalloc_mu;

}  // namespace

}  // namespace mcv

using namespace mcv;

extern "C" {

int mcv_w4a16_gemv(const void* x, int64_t M, int64_t K, int64_t N, const void* qw, const void* scales,
                   const void* zeros, int zero_bias, void* out, mcv_stream_t stream) {
    return launch_w4a16_gemv(x, M, K, N, qw, scales, zeros, zero_bias, out, static_cast<hipStream_t>(stream));
}

int64_t mcv_lm_head_workspace_bytes(int64_t V) {
    if (V <= 0 || V >= (int64_t(1) << 24)) return 0;
    // one key word per slab: room for the grid of this V and of every smaller one
    return kLmKeysByte + ceil_div(V, kSlab) * 8;
}

int64_t mcv_lm_head_slabs_per_workgroup(int64_t V) {
    if (V <= 0 || V >= (int64_t(1) << 24)) return 0;
    return lm_head_spw(ceil_div(V, kSlab));
}

int mcv_w4a16_gemv_argmax_partials(const void* x, int64_t K, int64_t N, int64_t V, const void* qw,
                                   const void* scales, const void* zeros, int zero_bias, void* logits,
                                   void* keys, mcv_stream_t stream) {
    int rc = MCV_OK;
    if (!w4_args_ok(qw, scales, zeros, zero_bias, K, N, "mcv_w4a16_gemv_argmax_partials", &rc)) return rc;
    if (!x || !keys) return fail(MCV_ERR_INVALID_ARG, "mcv_w4a16_gemv_argmax_partials: null x/keys");
    if (V <= 0 || V > N) return fail(MCV_ERR_SHAPE, "lm_head: need 0 < V <= N (V=%lld N=%lld)", (long long)V, (long long)N);
    if (reinterpret_cast<uintptr_t>(keys) % 8 != 0)
        return fail(MCV_ERR_INVALID_ARG, "lm_head: workspace must be 8-byte aligned");
    if ((rc = require_device()) != MCV_OK) return rc;
    // Only the slabs holding columns < V run; the scale/zero row stride is the
    // packed width of the weight (N), not of V.
    const int64_t nslab = ceil_div(V, kSlab);
    const int64_t npad = ceil_div(N, kSlab) * kSlab;
    const GemvCfg cfg = choose_gemv(K / kGroup, nslab);
    auto fn = pick_kernel<kArgPartials>(cfg.ksplit, cfg.gpw);
    hipLaunchKernelGGL(fn, dim3(static_cast<unsigned>(nslab), 1u), dim3(64 * cfg.ksplit), 0,
                       static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(x),
                       static_cast<const uint4*>(qw), static_cast<const uint16_t*>(scales),
                       static_cast<const uint32_t*>(zeros), static_cast<uint32_t>(zero_bias),
                       static_cast<uint16_t*>(logits), static_cast<int>(K), static_cast<int>(V),
                       static_cast<int>(npad), static_cast<unsigned long long*>(keys), nullptr);
    return check_launch("w4a16_gemv_kernel<partials>");
}

int mcv_argmax_reduce_keys(const void* keys, int64_t n_keys, int64_t* token, mcv_stream_t stream) {
    if (!keys || !token) return fail(MCV_ERR_INVALID_ARG, "mcv_argmax_reduce_keys: null pointer");
    if (n_keys <= 0 || n_keys > 0x7fffffff) return fail(MCV_ERR_SHAPE, "mcv_argmax_reduce_keys: bad n_keys");
    int rc = require_device();
    if (rc != MCV_OK) return rc;
    hipLaunchKernelGGL(argmax_reduce_kernel, dim3(1), dim3(1024), 0, static_cast<hipStream_t>(stream),
                       static_cast<const unsigned long long*>(keys), static_cast<int>(n_keys), token);
    return check_launch("argmax_reduce_kernel");
}

int mcv_w4a16_lm_head_argmax(const void* x, int64_t K, int64_t N, int64_t V, const void* qw, const void* scales,
                             const void* zeros, int zero_bias, void* logits, int64_t* token, void* workspace,
                             uint32_t* status, mcv_stream_t stream) {
    int rc = MCV_OK;
    if (!w4_args_ok(qw, scales, zeros, zero_bias, K, N, "mcv_w4a16_lm_head_argmax", &rc)) return rc;
    if (!x || !token || !workspace) return fail(MCV_ERR_INVALID_ARG, "mcv_w4a16_lm_head_argmax: null x/token/workspace");
    if (V <= 0 || V > N) return fail(MCV_ERR_SHAPE, "mcv_w4a16_lm_head_argmax: need 0 < V <= N (V=%lld N=%lld)",
                                     (long long)V, (long long)N);
    if (V >= (int64_t(1) << 24))
        return fail(MCV_ERR_SHAPE, "mcv_w4a16_lm_head_argmax: V must be below 2^24 (V=%lld)", (long long)V);
    if (reinterpret_cast<uintptr_t>(workspace) % 128 != 0)
        return fail(MCV_ERR_INVALID_ARG, "mcv_w4a16_lm_head_argmax: workspace must be 128-byte aligned");
    if ((rc = require_device()) != MCV_OK) return rc;
    return launch_lm_head(x, K, N, V, qw, scales, zeros, zero_bias, logits, token, workspace, 0u, kLmTree,
                          static_cast<unsigned*>(status), static_cast<hipStream_t>(stream));
}

int64_t mcv_lm_head_noalloc_max_vocab(void) { return kNoallocMaxV; }

void mcv_testing_lm_head_skew_poll(int on) { g_lm_poll_skew.store(on ? 1u : 0u, std::memory_order_relaxed); }

int mcv_w4a16_lm_head_argmax_noalloc(const void* x, int64_t K, int64_t N, int64_t V, const void* qw,
                                     const void* scales, const void* zeros, int zero_bias, void* logits,
                                     int64_t* token, uint32_t* status, mcv_stream_t stream) {
    const char* who = "mcv_w4a16_lm_head_argmax_noalloc";
    int rc = MCV_OK;
    if (!w4_args_ok(qw, scales, zeros, zero_bias, K, N, who, &rc)) return rc;
    if (!x || !token) return fail(MCV_ERR_INVALID_ARG, "%s: null x/token", who);
    if (V <= 0 || V > N) return fail(MCV_ERR_SHAPE, "%s: need 0 < V <= N (V=%lld N=%lld)", who, (long long)V, (long long)N);
    if (V > kNoallocMaxV)
        return fail(MCV_ERR_SHAPE, "%s: V=%lld exceeds the library scratch, which holds V <= %lld", who, (long long)V,
                    (long long)kNoallocMaxV);
    if ((rc = require_device()) != MCV_OK) return rc;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kNoallocMaxDevices)
        return fail(MCV_ERR_HIP, "%s: no usable current device (%d)", who, dev);
    const hipStream_t st = static_cast<hipStream_t>(stream);
    unsigned long long* ptr = nullptr;
    {
        std::lock_guard<std::mutex> lock(g_noalloc_mu);
        if (g_noalloc[dev] == nullptr) {
            // once per GPU, with that GPU current: the array's address on it
            void* p = nullptr;
            const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
            if (e != hipSuccess || p == nullptr)
                return fail(MCV_ERR_HIP, "%s: hipGetSymbolAddress failed (%s)", who, hipGetErrorString(e));
            g_noalloc[dev] = static_cast<unsigned long long*>(p);
        }
        ptr = g_noalloc[dev];
    }
    return launch_lm_head(x, K, N, V, qw, scales, zeros, zero_bias, logits, token, ptr, 0u, kLmTree,
                          static_cast<unsigned*>(status), st);
}

int64_t mcv_lm_head_slots_bytes(void) { return int64_t(kSlotWords) * kSlotStride * 8; }

int mcv_w4a16_lm_head_argmax_slots(const void* x, int64_t K, int64_t N, int64_t V, const void* qw,
                                   const void* scales, const void* zeros, int zero_bias, void* logits, void* slots,
                                   uint32_t tag, mcv_stream_t stream) {
    int rc = MCV_OK;
    if (!w4_args_ok(qw, scales, zeros, zero_bias, K, N, "mcv_w4a16_lm_head_argmax_slots", &rc)) return rc;
    if (!x || !slots) return fail(MCV_ERR_INVALID_ARG, "mcv_w4a16_lm_head_argmax_slots: null x/slots");
    if (V <= 0 || V > N) return fail(MCV_ERR_SHAPE, "mcv_w4a16_lm_head_argmax_slots: need 0 < V <= N (V=%lld N=%lld)",
                                     (long long)V, (long long)N);
    if (V >= (int64_t(1) << 24))
        return fail(MCV_ERR_SHAPE, "mcv_w4a16_lm_head_argmax_slots: V must be below 2^24 (V=%lld)", (long long)V);
    if (tag == 0 || tag > MCV_LM_SLOT_TAG_MAX)
        return fail(MCV_ERR_INVALID_ARG, "mcv_w4a16_lm_head_argmax_slots: tag must be in [1, 2^24 - 1] (tag=%u)", tag);
    if (reinterpret_cast<uintptr_t>(slots) % 128 != 0)
        return fail(MCV_ERR_INVALID_ARG, "mcv_w4a16_lm_head_argmax_slots: slots must be 128-byte aligned");
    if ((rc = require_device()) != MCV_OK) return rc;
    return launch_lm_head(x, K, N, V, qw, scales, zeros, zero_bias, logits, nullptr, slots, tag, kLmSlots, nullptr,
                          static_cast<hipStream_t>(stream));
}

int64_t mcv_lm_head_slots_token(const uint64_t* slots_host, uint32_t tag) {
    if (!slots_host) return fail(MCV_ERR_INVALID_ARG, "mcv_lm_head_slots_token: null slots");
    uint64_t best = 0;
    for (int j = 0; j < kSlotWords; ++j) {
        const uint64_t k = slots_host[static_cast<size_t>(j) * kSlotStride];
        if ((k >> 40) != tag) continue;                                  // no workgroup of this call used slot j
        const uint64_t v = k & 0xffffffffffull;
        best = v > best ? v : best;
    }
    if ((best >> 24) == 0) return 0;                                    // no candidate (every logit NaN or -inf)
    return static_cast<int64_t>(0xffffffu - static_cast<uint32_t>(best & 0xffffffu));
}

int mcv_w4a16_gemv_multi(const void* x, int64_t M, int64_t K, const mcv_w4a16_part* parts, int n_parts,
                         mcv_stream_t stream) {
    if (!x || !parts) return fail(MCV_ERR_INVALID_ARG, "mcv_w4a16_gemv_multi: null x/parts");
    if (n_parts < 1 || n_parts > kMaxParts)
        return fail(MCV_ERR_INVALID_ARG, "mcv_w4a16_gemv_multi: 1..%d parts (got %d)", kMaxParts, n_parts);
    if (M <= 0 || M > 65535) return fail(MCV_ERR_SHAPE, "mcv_w4a16_gemv_multi: M must be in [1, 65535] (M=%lld)", (long long)M);
    GemvParts gp{};
    int64_t total = 0;
    int64_t min_slabs = INT64_MAX;
    for (int i = 0; i < n_parts; ++i) {
        const mcv_w4a16_part& q = parts[i];
        int rc = MCV_OK;
        if (!w4_args_ok(q.qw_dev, q.scales_dev, q.zeros_dev, q.zero_bias, K, q.N, "mcv_w4a16_gemv_multi", &rc)) return rc;
        if (!q.out_dev) return fail(MCV_ERR_INVALID_ARG, "mcv_w4a16_gemv_multi: null out for part %d", i);
        const int64_t ns = ceil_div(q.N, kSlab);
        total += ns;
        min_slabs = ns < min_slabs ? ns : min_slabs;
        if (total > 0x7fffffff) return fail(MCV_ERR_SHAPE, "mcv_w4a16_gemv_multi: too many columns");
        gp.p[i] = GemvPart{static_cast<const uint4*>(q.qw_dev), static_cast<const uint16_t*>(q.scales_dev),
                           static_cast<const uint32_t*>(q.zeros_dev), static_cast<uint16_t*>(q.out_dev),
                           static_cast<int>(q.N), static_cast<int>(ns * kSlab), static_cast<int>(total),
                           static_cast<uint32_t>(q.zero_bias)};
    }
    gp.count = n_parts;
    int rc = require_device();
    if (rc != MCV_OK) return rc;
    // The k-split the smallest part would get on its own (the decode shapes
    // with K = 1024 all get 8, so the outputs equal separate launches').
    const GemvCfg cfg = choose_gemv(K / kGroup, min_slabs * M);
    const int ks = cfg.ksplit;
    using Fn = void (*)(const uint16_t*, GemvParts, int);
    Fn fn = ks >= 16 ? w4a16_gemv_multi_kernel<16>
          : ks == 8 ? w4a16_gemv_multi_kernel<8>
          : ks == 4 ? w4a16_gemv_multi_kernel<4>
          : ks == 2 ? w4a16_gemv_multi_kernel<2> : w4a16_gemv_multi_kernel<1>;
    hipLaunchKernelGGL(fn, dim3(static_cast<unsigned>(total), static_cast<unsigned>(M)), dim3(64 * ks), 0,
                       static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(x), gp, static_cast<int>(K));
    return check_launch("w4a16_gemv_multi_kernel");
}

int mcv_w4a16_gate_up_silu(const void* x, int64_t M, int64_t K, int64_t N, const void* qw_gate,
                           const void* scales_gate, const void* zeros_gate, int zero_bias_gate, const void* qw_up,
                           const void* scales_up, const void* zeros_up, int zero_bias_up, void* act,
                           mcv_stream_t stream) {
    int rc = MCV_OK;
    if (!w4_args_ok(qw_gate, scales_gate, zeros_gate, zero_bias_gate, K, N, "mcv_w4a16_gate_up_silu", &rc) ||
        !w4_args_ok(qw_up, scales_up, zeros_up, zero_bias_up, K, N, "mcv_w4a16_gate_up_silu", &rc))
        return rc;
    if (!x || !act) return fail(MCV_ERR_INVALID_ARG, "mcv_w4a16_gate_up_silu: null x/act");
    if (M <= 0 || M > 65535) return fail(MCV_ERR_SHAPE, "mcv_w4a16_gate_up_silu: M must be in [1, 65535] (M=%lld)", (long long)M);
    if ((rc = require_device()) != MCV_OK) return rc;
    const int64_t nslab = ceil_div(N, kSlab);
    const GemvCfg cfg = choose_gemv(K / kGroup, nslab * M);
    using Fn = void (*)(const uint16_t*, const uint4*, const uint16_t*, const uint32_t*, uint32_t, const uint4*,
                        const uint16_t*, const uint32_t*, uint32_t, uint16_t*, int, int, int);
    // Same k-split as the GEMV so the fp32 partial sums add in the same order.
    const int ks = cfg.ksplit;
    Fn fn = ks >= 16 ? w4a16_gate_up_silu_kernel<16>
          : ks == 8 ? w4a16_gate_up_silu_kernel<8>
          : ks == 4 ? w4a16_gate_up_silu_kernel<4>
          : ks == 2 ? w4a16_gate_up_silu_kernel<2> : w4a16_gate_up_silu_kernel<1>;
    hipLaunchKernelGGL(fn, dim3(static_cast<unsigned>(2 * nslab), static_cast<unsigned>(M)), dim3(64 * ks), 0,
                       static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(x),
                       static_cast<const uint4*>(qw_gate), static_cast<const uint16_t*>(scales_gate),
                       static_cast<const uint32_t*>(zeros_gate), static_cast<uint32_t>(zero_bias_gate),
                       static_cast<const uint4*>(qw_up), static_cast<const uint16_t*>(scales_up),
                       static_cast<const uint32_t*>(zeros_up), static_cast<uint32_t>(zero_bias_up),
                       static_cast<uint16_t*>(act), static_cast<int>(K), static_cast<int>(N),
                       static_cast<int>(nslab * kSlab));
    return check_launch("w4a16_gate_up_silu_kernel");
}

int mcv_w4a16_dequant(const void* qw, const void* scales, const void* zeros, int zero_bias, int64_t K, int64_t N,
                      void* w_f16, int8_t* w8, mcv_stream_t stream) {
    int rc = MCV_OK;
    if (!w4_args_ok(qw, scales, zeros, zero_bias, K, N, "mcv_w4a16_dequant", &rc)) return rc;
    if (!w_f16 && !w8) return fail(MCV_ERR_INVALID_ARG, "mcv_w4a16_dequant: no output");
    if ((rc = require_device()) != MCV_OK) return rc;
    const int64_t nslab = ceil_div(N, kSlab);
    hipLaunchKernelGGL(w4a16_dequant_kernel, dim3(static_cast<unsigned>(nslab), static_cast<unsigned>(K / kChunkK)),
                       dim3(64), 0, static_cast<hipStream_t>(stream), static_cast<const uint4*>(qw),
                       static_cast<const uint16_t*>(scales), static_cast<const uint32_t*>(zeros),
                       static_cast<uint32_t>(zero_bias), static_cast<int>(K), static_cast<int>(N),
                       static_cast<int>(nslab * kSlab), static_cast<uint16_t*>(w_f16), w8);
    return check_launch("w4a16_dequant_kernel");
}

int mcv_w4a16_gemv_tiled_i8(const void* x, int64_t K, int64_t N, int64_t tile_len, int64_t packed_rows,
                            const int8_t* w, const void* scales, void* out, mcv_stream_t stream) {
    if (!x || !w || !scales || !out) return fail(MCV_ERR_INVALID_ARG, "matmul_w4a16: null pointer");
    // Same constraints as src/csrc/lib/ops.cpp:1058-1079.
    if (tile_len <= 0 || tile_len > 448 || tile_len % 16 != 0)
        return fail(MCV_ERR_SHAPE, "matmul_w4a16 tile_len must be a multiple of 16 and <= 448");
    if (K <= 0 || N <= 0 || K % kGroup != 0 || N % 128 != 0)
        return fail(MCV_ERR_SHAPE, "matmul_w4a16 K and N must be multiples of 128");
    const int64_t blockLen = (N + 7) / 8;
    const int64_t tilesPerBlock = (blockLen + tile_len - 1) / tile_len;
    if (packed_rows != (K / kGroup) * 8 * tilesPerBlock * kGroup)
        return fail(MCV_ERR_SHAPE, "matmul_w4a16 w packed_rows mismatch");
    int rc = require_device();
    if (rc != MCV_OK) return rc;
    if (8 * tilesPerBlock > 0x7fffffff || (K / kGroup) * 8 * tilesPerBlock * kGroup * tile_len >= (int64_t(1) << 40))
        return fail(MCV_ERR_SHAPE, "matmul_w4a16: weight too large");
    // chunks of 16 columns per workgroup: a whole tile from 64 tiles on, else
    // fewer, so the grid reaches ~256 workgroups where it can (MI355X, us per
    // call: K=N=1024, 8 tiles, 9.9 whole / 6.3 sliced; K=3584 N=1024 29.2 /
    // 12.5; K=1024 N=31104, 72 tiles, 17.9 whole / 21.6 in 4 slices)
    const int64_t tiles = 8 * tilesPerBlock, cn = tile_len / 16;
    const int64_t want = tiles >= 64 ? 1 : std::min<int64_t>(cn, ceil_div(256, tiles));
    const int64_t cs = ceil_div(cn, want), slices = ceil_div(cn, cs);
    hipLaunchKernelGGL(w4a16_tiled_i8_kernel, dim3(static_cast<unsigned>(tiles * slices)), dim3(64 * kTiWaves), 0,
                       static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(x), w,
                       static_cast<const uint16_t*>(scales), static_cast<uint16_t*>(out), static_cast<int>(K),
                       static_cast<int>(N), static_cast<int>(blockLen), static_cast<int>(tile_len),
                       static_cast<int>(tilesPerBlock), static_cast<int>(cs), static_cast<int>(slices));
    return check_launch("w4a16_tiled_i8_kernel");
}

}  // extern "C"
