// decode_mlp.hip -- the whole W4A16 decode MLP block in one launch, gfx950.
//
//   act = silu(x . gate) * (x . up)      [I]   (phase 1, one workgroup per act slab)
//   out = act . down                     [H]   (phase 2)
//
// The phases meet inside the kernel instead of at a kernel boundary, so the
// block costs one launch, and every phase-2 wave issues the loads of its
// down-projection weights at the start: by the time the act row is complete
// those bytes are in registers.
//
// Phase 1 is w4a16_gate_up_silu_kernel's loop, phase 2 the down GEMV's
// arithmetic with its k-split ks2: "wave slot" w of an output slab adds the
// groups w, w + ks2 in that order (one fma chain), and the slab's output is
// slot 0 + slot 1 + ... in slot order.  Here each group's sum is formed by its
// own wave, spread over ceil(ks2/2) workgroups per slab (four waves each, one
// per SIMD), and the chains and the slot sum are then done in exactly that
// order -- so the result is bit for bit that of the two-launch sequence
// (tested).  Spreading matters: the moment the act row lands every phase-2
// wave starts its arithmetic, and with one workgroup per slab (16 waves on one
// CU) the SIMDs ran four waves' decode back to back, ~3.4 us.
//
// Cross-workgroup exchange without barriers or fences (the L2s of the eight
// XCDs are not coherent with each other): every value travels in a word that
// also carries a call tag -- act elements as (tag << 16 | fp16), slot
// partials as (tag << 32 | fp32) -- written with device-scope stores, which go
// through to the coherent point, and polled with device-scope loads until the
// tag is this call's.  The tag comes from a per-workgroup call counter in the
// workspace: every workgroup reads its own counter once and bumps it, so all
// workgroups of a call agree without talking to each other, and a graph
// replay (which reads the counters afresh) gets a new tag.  A grid barrier on
// an arrival counter was measured first: its arrival, reset and release
// round trips (~0.7 us each at device scope) cost more than the second launch
// they replace.  Every poll is bounded (a fraction of a second), after which
// the wave sets the workspace's error word and carries on, so a broken launch
// cannot hang the device; the launcher admits only grids that are resident
// all at once, so every tag a wave waits for does get written.
//
// Replaces the reference's MLP sequence (src/csrc/lib/decoder_layer.cpp:1029-1046:
// gate matmul_w4a16, up matmul_w4a16, silu_mul, down matmul_w4a16).
#include <cstdint>
#include <cstdlib>
#include <mutex>
#include <unordered_map>

#include "common.h"
#include "gemv_body.h"

namespace mcv {

// Same choice as the GEMV launchers (w4a16_gemv.hip).
int gemv_ksplit(int64_t G, int64_t blocks);

namespace {

constexpr int kMaxWaves = 16;                 // largest k-split of the GEMV launchers
constexpr int kP2Waves = 4;                   // phase-2 waves per workgroup: two slots x two groups
constexpr int kWsError = 0;                   // u32 word offsets in the workspace
constexpr int kWsEpoch = 64;                  // one call counter per workgroup
constexpr int kMaxBlocks = 1024;
constexpr int64_t kWsHeader = 4 * (kWsEpoch + kMaxBlocks);   // bytes before the tagged act row
constexpr int kSpinLimit = 1 << 18;

struct W4Ptrs {
    const uint4* q;
    const uint16_t* s;
    const uint32_t* z;
    uint32_t zero_bias;
};

__host__ __device__ inline int64_t act_bytes(int64_t I) { return (I + kSlab - 1) / kSlab * kSlab * 4; }

// Bounded poll: load_all(v) re-reads N tagged words per lane until every
// tag_of(v[i]) equals `tag` (v then holds them), or gives up and flags the
// workspace.  All loads of one read are issued before any is compared.
template <int N, typename Load, typename TagOf>
__device__ __forceinline__ void poll_words(uint64_t (&v)[N], Load load_all, TagOf tag_of, uint32_t tag,
                                           unsigned* __restrict__ ws, unsigned* status, int lane) {
    for (int spins = 0;; ++spins) {
        load_all(v);
        uint32_t bad = 0;
#pragma unroll
        for (int i = 0; i < N; ++i) bad |= tag_of(v[i]) ^ tag;
        if (__all(bad == 0)) return;
        if (spins > kSpinLimit) {
            if (lane == 0) flag_gave_up(ws + kWsError, status);
            return;
        }
        __builtin_amdgcn_s_sleep(1);
    }
}

// grid = nslab2 * npair + 2 * nslab1 with npair = ceil(ks2 / 2), block =
// 64 * max(ks1, 4).  Workgroups below nslab2 * npair are phase 2 (dispatched
// first, so their weight loads start earliest): workgroup (slab, pair p) owns
// wave slots 2p and 2p + 1 of that output slab.  The rest are phase 1, one
// half of an act slab each: lanes 0-31 on the half's 32 gate columns, lanes
// 32-63 on the same up columns, so each lane runs one of the gate+up
// kernel's chains (MI355X, H=1024, I=3584: 6.98 us per block against 7.62
// with whole slabs and both chains per lane).  Requires ceil(G2 / ks2) <= 2
// (two groups per slot).
__global__ __launch_bounds__(64 * kMaxWaves) void w4a16_mlp_kernel(const uint16_t* __restrict__ x, W4Ptrs gate,
                                                                   W4Ptrs up, W4Ptrs down, uint16_t* __restrict__ out,
                                                                   int H, int I, int ks1, int ks2,
                                                                   unsigned* __restrict__ ws, unsigned* status) {
    __shared__ float red[2][kMaxWaves][kSlab];
    __shared__ uint32_t xg[kP2Waves][kSlab];                             // one act group per wave, half2 words
    __shared__ unsigned s_epoch;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int b = blockIdx.x;
    const int nslab1 = (I + kSlab - 1) / kSlab, nslab2 = (H + kSlab - 1) / kSlab;
    const int npair = (ks2 + 1) / 2;
    const int G1 = H / kGroup, G2 = I / kGroup;
    uint32_t* __restrict__ act = reinterpret_cast<uint32_t*>(reinterpret_cast<uint8_t*>(ws) + kWsHeader);
    uint64_t* __restrict__ part = reinterpret_cast<uint64_t*>(reinterpret_cast<uint8_t*>(act) + act_bytes(I));
    uint32_t vmagic;                                                     // 0x64006400 = half2(1024, 1024)
    asm("v_mov_b32 %0, 0x64006400" : "=v"(vmagic));

    // This call's tag: the workgroup's own call counter, read once by wave 0
    // (issued first, needed only after the weight loads) and bumped by it; in
    // phase 2 it reaches the other waves through LDS -- a read of the counter
    // by another wave could already see the bump.
    const unsigned epoch =
        wave == 0 ? __hip_atomic_load(ws + kWsEpoch + b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0u;
    auto bump_epoch = [&]() {
        if (wave == 0 && lane == 0)
            __hip_atomic_store(ws + kWsEpoch + b, epoch + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    };

    if (b >= nslab2 * npair) {
        // ---- phase 1, half h of an act slab, published as tagged words:
        // lane l runs the gate (l < 32) or up (l >= 32) chain of column
        // 32 h + l % 32
        const int j = b - nslab2 * npair;
        const int slab = j >> 1, col = 32 * (j & 1) + (lane & 31), pj = lane >> 5;
        if (wave < ks1) {
            const W4Ptrs w = pj ? up : gate;
            const int npad1 = nslab1 * kSlab;
            red[pj][wave][lane & 31] = w4_partials(reinterpret_cast<const uint32_t*>(x),
                                                   w4_column(w.q, w.s, w.z, w.zero_bias, H, npad1, slab, col), wave,
                                                   ks1, G1, vmagic);
        }
        __syncthreads();
        if (wave != 0) return;
        bump_epoch();
        const uint32_t tag = (epoch + 1u) & 0xffffu;
        if (lane >= 32) return;
        float ag = red[0][0][lane], au = red[1][0][lane];
        for (int w = 1; w < ks1; ++w) {
            ag += red[0][w][lane];
            au += red[1][w][lane];
        }
        const int n = slab * kSlab + col;
        if (n < I)
            __hip_atomic_store(act + n, (tag << 16) | silu_mul_f16(f2h(ag), f2h(au)), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        return;
    }
    // ---- phase 2: wave j of workgroup (slab, pair) forms the sum of group
    // g = slot + i * ks2, slot = 2 pair + j / 2, i = j % 2
    const int slab = b / npair, pair = b - slab * npair;
    const int slot = 2 * pair + (wave >> 1);
    const int g = slot + (wave & 1) * ks2;
    const bool present = wave < kP2Waves && slot < ks2 && g < G2;       // wave-uniform
    const W4Column dc = w4_column(down.q, down.s, down.z, down.zero_bias, I, nslab2 * kSlab, slab, lane);
    uint4 wv[4];
    uint16_t sv = 0;
    uint32_t zv = 0;
    if (present) {
#pragma unroll
        for (int c = 0; c < 4; ++c) wv[c] = load_weights(dc.q + static_cast<size_t>(g * 4 + c) * kSlab);
        sv = dc.s[static_cast<size_t>(g) * dc.npad];
        zv = dc.z[static_cast<size_t>(g) * (dc.npad >> 3)];
    }
    if (wave == 0 && lane == 0) s_epoch = epoch;
    bump_epoch();
    __syncthreads();
    const uint32_t tag = (s_epoch + 1u) & 0xffffu;
    float y = 0.f;
    if (present) {
        // the weights arrive long before the act row: widen them now, so
        // that only the dot products remain once it lands
        half2_t pw[64];
        group_operands(wv, ((zv >> dc.zshift) & 15u) + dc.zero_bias, vmagic, pw);
        // (left alone, the compiler sinks the widening below the poll loop,
        // next to its only use)
#pragma unroll
        for (int j = 0; j < 64; ++j) asm volatile("" ::"v"(pw[j]) : "memory");
        // lane l holds act elements 2l and 2l + 1 of the group; the word's
        // tag is `tag` only if both element tags are
        const uint64_t* src = reinterpret_cast<const uint64_t*>(act + g * kGroup) + lane;
        uint64_t av[1];
        poll_words<1>(
            av, [&](uint64_t (&v)[1]) { v[0] = __hip_atomic_load(src, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); },
            [](uint64_t v) {
                const uint32_t t0 = static_cast<uint32_t>(v) >> 16, t1 = static_cast<uint32_t>(v >> 48);
                return t0 == t1 ? t0 : ~t0;
            },
            tag, ws, status, lane);
        xg[wave][lane] = (static_cast<uint32_t>(av[0]) & 0xffffu) | (static_cast<uint32_t>(av[0] >> 32) << 16);
        uint32_t xs[64];
#pragma unroll
        for (int k = 0; k < 64; ++k) xs[k] = __builtin_amdgcn_readfirstlane(xg[wave][k]);
        y = group_sum_operands(pw, xs);
    }
    if (wave < kP2Waves) {
        red[0][wave][lane] = y;
        red[1][wave][lane] = h2f(sv);
    }
    __syncthreads();
    if (wave != 0) return;

    // wave 0: the fma chains of the workgroup's two slots ...
    float p[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        const int s = 2 * pair + t;
        p[t] = 0.f;
        if (s < ks2) p[t] = fmaf(red[0][2 * t][lane], red[1][2 * t][lane], 0.f);
        if (s < ks2 && s + ks2 < G2) p[t] = fmaf(red[0][2 * t + 1][lane], red[1][2 * t + 1][lane], p[t]);
    }
    uint64_t* __restrict__ slab_part = part + static_cast<size_t>(slab) * kMaxWaves * kSlab + lane;
    if (pair != 0) {
        // ... published for the slab's first workgroup
#pragma unroll
        for (int t = 0; t < 2; ++t)
            if (2 * pair + t < ks2)
                __hip_atomic_store(slab_part + (2 * pair + t) * kSlab,
                                   (static_cast<uint64_t>(tag) << 32) | __float_as_uint(p[t]), __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
        return;
    }
    // ... and, in the slab's first workgroup, the slot sum in slot order; the
    // other slots' partials are read together (slots past ks2 re-read slot 2)
    float acc = p[0];
    if (ks2 > 1) acc += p[1];
    if (ks2 > 2) {
        uint64_t pv[kMaxWaves - 2];
        poll_words<kMaxWaves - 2>(
            pv,
            [&](uint64_t (&v)[kMaxWaves - 2]) {
#pragma unroll
                for (int i = 0; i < kMaxWaves - 2; ++i)
                    v[i] = __hip_atomic_load(slab_part + (2 + i < ks2 ? 2 + i : 2) * kSlab, __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT);
            },
            [](uint64_t v) { return static_cast<uint32_t>(v >> 32); }, tag, ws, status, lane);
#pragma unroll
        for (int i = 0; i < kMaxWaves - 2; ++i)
            if (2 + i < ks2) acc += __uint_as_float(static_cast<uint32_t>(pv[i]));
    }
    const int col = slab * kSlab + lane;
    if (col < H) out[col] = f2h(acc);
}

// ---------------------------------------------------------------- W8A8 --
// The W8A8 decode MLP block from the normed fp16 row, in one launch:
//   xq, xs = quantize(x); act = silu(deq(xq . gate)) * deq(xq . up);
//   aq, as = quantize(act); out = deq(aq . down)
// with every step as the separate kernels do it (mcv_w8a8_quantize_act,
// mcv_w8a8_gate_up_silu, mcv_w8a8_gemm_f16 with fp32 scales) -- bit-identical,
// since the int32 sums are exact in any order and a row maximum is a maximum.
// Phase 1: one workgroup per 32-column half of an act slab quantises x itself
// (H values, into LDS), runs the dual int8 GEMV over the tiled weights and
// publishes its act values (tag << 16 | fp16) and the maximum of their
// magnitudes (tag << 32 | fp32).  Phase 2: workgroup (half of an output slab,
// k-part) loads its down-projection operand lines at the start, polls the
// half maxima and its k-range of act words, quantises that range with the row
// scale into LDS, forms its int32 partial sums and publishes them; the
// k-part-0 workgroup adds the parts and applies the epilogue.
constexpr int kW8Line = 1024;                 // bytes of one 32-column x 32-k operand line
constexpr int kW8Waves = 8;
constexpr int kW8U = 4;                       // k-blocks per wave per trip (phase 1) / per part (phase 2)
constexpr int kW8PartBlocks = kW8Waves * kW8U;  // k-blocks of one phase-2 part
constexpr int kW8MaxH = 8192;                 // the quantised x row staged in LDS
constexpr int kW8XWords = kW8MaxH / 2 / (64 * kW8Waves);   // fp16 pairs of x per thread
constexpr int kW8MaxParts = 16;               // phase-2 k-parts per output half: I <= 16384

__device__ __forceinline__ __amdgpu_buffer_rsrc_t w8_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, static_cast<int>(bytes), 0x00020000);
}

// Maximum over the workgroup's eight waves (values are magnitudes, >= 0).
__device__ __forceinline__ float block_max8(float m, float* __restrict__ scratch8) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const float o = __shfl_xor(m, off, 64);
        m = o > m ? o : m;
    }
    if ((threadIdx.x & 63) == 0) scratch8[threadIdx.x >> 6] = m;
    __syncthreads();
    m = scratch8[0];
#pragma unroll
    for (int w = 1; w < kW8Waves; ++w) m = scratch8[w] > m ? scratch8[w] : m;
    return m;
}

struct W8Layout {                             // word offsets into the workspace
    int act;                                  // u32 [I]
    int amax;                                 // u64 [2 nslab1]
    int part;                                 // u64 [2 nslab2][nparts][32]
};

__host__ __device__ inline W8Layout w8_layout(int H, int I, int nparts) {
    const int nslab1 = (I + 63) / 64;
    W8Layout l;
    l.act = static_cast<int>(kWsHeader / 4);
    l.amax = (l.act + nslab1 * 64 + 1) / 2;                             // u64 index
    l.part = l.amax + 2 * nslab1;
    (void)H;
    (void)nparts;
    return l;
}

// Per-channel weight scale n as fp32: fp32 storage, or (REF16) the
// reference's truncated fp16 copy widened exactly.
template <bool REF16>
__device__ __forceinline__ float w8_scale(const void* __restrict__ s, int n) {
    if constexpr (REF16) return h2f(static_cast<const uint16_t*>(s)[n]);
    else return static_cast<const float*>(s)[n];
}

// The scale a row's epilogue multiplies by: the quantiser's fp32 scale, or
// (REF16) its fp16 RNE encoding widened back, the value the reference stores
// in w8a8_quantize's fp16 x_scale and its dequant reads
// (op_kernel/w8a8_quantize_custom.cpp:41, w8a8_dequant_custom.cpp:43-44).
template <bool REF16>
__device__ __forceinline__ float epilogue_scale(float xs) {
    if constexpr (REF16) return h2f(f2h(xs));
    else return xs;
}

// grid = 2 nslab2 nparts (phase 2, first) + 2 nslab1 (phase 1), block = 512.
// REF16: fp16 weight scales and fp16-rounded activation scales in every
// epilogue, the reference's precision; otherwise fp32 throughout.
template <bool REF16>
__global__ __launch_bounds__(64 * kW8Waves) void w8a8_mlp_kernel(
    const uint16_t* __restrict__ x, const int8_t* __restrict__ wg, const void* __restrict__ sg,
    const int8_t* __restrict__ wu, const void* __restrict__ su, const int8_t* __restrict__ wd,
    const void* __restrict__ sd, uint16_t* __restrict__ out, int H, int I, int nparts, unsigned* __restrict__ ws,
    unsigned* status) {
    __shared__ __attribute__((aligned(16))) int8_t xq_lds[kW8MaxH];
    __shared__ int red[kW8Waves][2][64];
    __shared__ float scratch8[kW8Waves];
    __shared__ unsigned s_epoch;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int h = lane >> 5;
    const int b = blockIdx.x;
    const int nslab1 = (I + 63) / 64, nslab2 = (H + 63) / 64;
    const int KB1 = (H + 127) / 128 * 4, KB2 = (I + 127) / 128 * 4;
    const W8Layout L = w8_layout(H, I, nparts);
    uint32_t* __restrict__ act = reinterpret_cast<uint32_t*>(ws) + L.act;
    uint64_t* __restrict__ amax = reinterpret_cast<uint64_t*>(ws) + L.amax;
    uint64_t* __restrict__ part = reinterpret_cast<uint64_t*>(ws) + L.part;
    constexpr uint32_t kNowhere = 0xFFFFFF00u;
    const unsigned epoch =
        wave == 0 ? __hip_atomic_load(ws + kWsEpoch + b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0u;
    const int n2 = 2 * nslab2 * nparts;

    if (b >= n2) {
        // ---- phase 1: half j of act slab `slab`
        const int u1 = b - n2, slab = u1 >> 1, j = u1 & 1;
        const uint32_t wbytes = static_cast<uint32_t>(nslab1) * KB1 * 2 * kW8Line;
        const __amdgpu_buffer_rsrc_t rg = w8_rsrc(wg, wbytes), ru = w8_rsrc(wu, wbytes);
        // the weight lines of the first trip are in flight while x is quantised
        int4_t wgv[kW8U], wuv[kW8U];
        auto load_w = [&](int kb0) {
#pragma unroll
            for (int u = 0; u < kW8U; ++u) {
                const int kb = kb0 + u * kW8Waves;
                const uint32_t off =
                    kb < KB1 ? ((static_cast<uint32_t>(slab) * KB1 + kb) * 2 + j) * kW8Line + lane * 16u : kNowhere;
                wgv[u] = __builtin_bit_cast(int4_t, __builtin_amdgcn_raw_buffer_load_b128(rg, off, 0, 2));
                wuv[u] = __builtin_bit_cast(int4_t, __builtin_amdgcn_raw_buffer_load_b128(ru, off, 0, 2));
            }
        };
        // x as fp16 pairs, all loads issued at once and ahead of the weights
        const uint32_t* __restrict__ x32 = reinterpret_cast<const uint32_t*>(x);
        uint32_t xw[kW8XWords];
#pragma unroll
        for (int i = 0; i < kW8XWords; ++i) {
            const int k2 = static_cast<int>(threadIdx.x) + i * 64 * kW8Waves;
            xw[i] = k2 < H / 2 ? x32[k2] : 0u;
        }
        load_w(wave);
        const int n = slab * 64 + 32 * j + (lane & 31);
        const float sgv = n < I ? w8_scale<REF16>(sg, n) : 0.f, suv = n < I ? w8_scale<REF16>(su, n) : 0.f;
        // x -> xq with the activation quantiser's arithmetic (H is a multiple
        // of 128, so the k-blocks cover x exactly)
        float m = 0.f;
#pragma unroll
        for (int i = 0; i < kW8XWords; ++i) {
            const float v0 = fabsf(h2f(static_cast<uint16_t>(xw[i]))), v1 = fabsf(h2f(static_cast<uint16_t>(xw[i] >> 16)));
            m = v0 > m ? v0 : m;
            m = v1 > m ? v1 : m;
        }
        const float xs = act_scale(block_max8(m, scratch8));
        const float inv = __fdiv_rn(1.0f, xs);
        const float xse = epilogue_scale<REF16>(xs);
#pragma unroll
        for (int i = 0; i < kW8XWords; ++i) {
            const int k2 = static_cast<int>(threadIdx.x) + i * 64 * kW8Waves;
            if (k2 < H / 2) {
                const uint32_t lo = static_cast<uint8_t>(act_quant(static_cast<uint16_t>(xw[i]), inv));
                const uint32_t hi = static_cast<uint8_t>(act_quant(static_cast<uint16_t>(xw[i] >> 16), inv));
                reinterpret_cast<uint16_t*>(xq_lds)[k2] = static_cast<uint16_t>(lo | (hi << 8));
            }
        }
        __syncthreads();
        int accg = 0, accu = 0;
        for (int kb0 = wave;;) {
#pragma unroll
            for (int u = 0; u < kW8U; ++u) {
                const int kb = kb0 + u * kW8Waves;
                if (kb < KB1) {
                    const int4_t xv = *reinterpret_cast<const int4_t*>(xq_lds + kb * 32 + h * 16);
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        accg = __builtin_amdgcn_sdot4(wgv[u][q], xv[q], accg, false);
                        accu = __builtin_amdgcn_sdot4(wuv[u][q], xv[q], accu, false);
                    }
                }
            }
            kb0 += kW8Waves * kW8U;
            if (kb0 >= KB1) break;
            load_w(kb0);
        }
        red[wave][0][lane] = accg;
        red[wave][1][lane] = accu;
        __syncthreads();
        if (wave != 0) return;
        const uint32_t tag = (epoch + 1u) & 0xffffu;
        if (lane == 0)
            __hip_atomic_store(ws + kWsEpoch + b, epoch + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        // lanes 0-31: columns of the half; both k-halves of every wave
        const int l = lane & 31;
        int g = 0, uu = 0;
        for (int w = 0; w < kW8Waves; ++w) {
            g += red[w][0][l] + red[w][0][l + 32];
            uu += red[w][1][l] + red[w][1][l + 32];
        }
        float a = 0.f;
        if (lane < 32 && n < I) {
            const uint16_t g16 = f2h(__fmul_rn(__fmul_rn(static_cast<float>(g), sgv), xse));
            const uint16_t u16 = f2h(__fmul_rn(__fmul_rn(static_cast<float>(uu), suv), xse));
            const uint16_t a16 = silu_mul_f16(g16, u16);
            a = fabsf(h2f(a16));
            __hip_atomic_store(act + n, (tag << 16) | a16, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) {
            const float o = __shfl_xor(a, off, 64);
            a = o > a ? o : a;
        }
        if (lane == 0)
            __hip_atomic_store(amax + u1, (static_cast<uint64_t>(tag) << 32) | __float_as_uint(a), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        return;
    }

    // ---- phase 2: half j of output slab `slab`, k-part p
    const int p = b % nparts, u2 = b / nparts, slab = u2 >> 1, j = u2 & 1;
    const int kbp = (KB2 + nparts - 1) / nparts;
    const int kb_beg = p * kbp, kb_end = kb_beg + kbp < KB2 ? kb_beg + kbp : KB2;
    const uint32_t wbytes = static_cast<uint32_t>(nslab2) * KB2 * 2 * kW8Line;
    const __amdgpu_buffer_rsrc_t rd = w8_rsrc(wd, wbytes);
    int4_t wdv[kW8U];
#pragma unroll
    for (int u = 0; u < kW8U; ++u) {
        const int kb = kb_beg + wave + u * kW8Waves;
        const uint32_t off =
            kb < kb_end ? ((static_cast<uint32_t>(slab) * KB2 + kb) * 2 + j) * kW8Line + lane * 16u : kNowhere;
        wdv[u] = __builtin_bit_cast(int4_t, __builtin_amdgcn_raw_buffer_load_b128(rd, off, 0, 2));
    }
    const int ncol = slab * 64 + 32 * j + (lane & 31);
    const float sdv = p == 0 && wave == 0 && ncol < H ? w8_scale<REF16>(sd, ncol) : 0.f;
    if (wave == 0 && lane == 0) {
        s_epoch = epoch;
        __hip_atomic_store(ws + kWsEpoch + b, epoch + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    const uint32_t tag = (s_epoch + 1u) & 0xffffu;
    // poll: thread t reads half maximum t (if any) and act words k0 + t, k0 + t + 512 of the k-range
    const int k0 = kb_beg * 32, klen = (kb_end - kb_beg) * 32;
    const int nmax = 2 * nslab1;
    float am = 0.f;
    uint32_t av[2] = {0u, 0u};
    for (int spins = 0;; ++spins) {
        bool ok = true;
        am = 0.f;
        if (static_cast<int>(threadIdx.x) < nmax) {
            const uint64_t v = __hip_atomic_load(amax + threadIdx.x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            ok = static_cast<uint32_t>(v >> 32) == tag;
            am = __uint_as_float(static_cast<uint32_t>(v));
        }
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int k = static_cast<int>(threadIdx.x) + i * 64 * kW8Waves;
            if (k < klen && k0 + k < I) {
                av[i] = __hip_atomic_load(act + k0 + k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                ok = ok && (av[i] >> 16) == tag;
            }
        }
        if (!__syncthreads_or(ok ? 0 : 1)) break;
        if (spins > kSpinLimit) {
            if (threadIdx.x == 0) flag_gave_up(ws + kWsError, status);
            break;
        }
        __builtin_amdgcn_s_sleep(1);
    }
    // the act row's scale (maximum of the half maxima), its k-range quantised into LDS
    const float as = act_scale(block_max8(am, scratch8));
    const float inv = __fdiv_rn(1.0f, as);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int k = static_cast<int>(threadIdx.x) + i * 64 * kW8Waves;
        if (k < klen) xq_lds[k] = k0 + k < I ? act_quant(static_cast<uint16_t>(av[i] & 0xffffu), inv) : int8_t(0);
    }
    __syncthreads();
    int acc = 0;
#pragma unroll
    for (int u = 0; u < kW8U; ++u) {
        const int kb = kb_beg + wave + u * kW8Waves;
        if (kb < kb_end) {
            const int4_t xv = *reinterpret_cast<const int4_t*>(xq_lds + (kb - kb_beg) * 32 + h * 16);
#pragma unroll
            for (int q = 0; q < 4; ++q) acc = __builtin_amdgcn_sdot4(wdv[u][q], xv[q], acc, false);
        }
    }
    red[wave][0][lane] = acc;
    __syncthreads();
    if (wave != 0) return;
    const int l = lane & 31;
    int sum = 0;
    for (int w = 0; w < kW8Waves; ++w) sum += red[w][0][l] + red[w][0][l + 32];
    uint64_t* __restrict__ mypart = part + (static_cast<size_t>(u2) * nparts) * 32 + l;
    if (p != 0) {
        if (lane < 32)
            __hip_atomic_store(mypart + p * 32, (static_cast<uint64_t>(tag) << 32) | static_cast<uint32_t>(sum),
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return;
    }
    // k-part 0: add the other parts (exact int32; read together, parts past
    // nparts re-read part 1) and apply the epilogue
    if (nparts > 1) {
        uint64_t v[kW8MaxParts - 1];
        poll_words<kW8MaxParts - 1>(
            v,
            [&](uint64_t (&w)[kW8MaxParts - 1]) {
#pragma unroll
                for (int q = 0; q < kW8MaxParts - 1; ++q)
                    w[q] = __hip_atomic_load(mypart + (q + 1 < nparts ? q + 1 : 1) * 32, __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT);
            },
            [](uint64_t w) { return static_cast<uint32_t>(w >> 32); }, tag, ws, status, lane);
#pragma unroll
        for (int q = 0; q < kW8MaxParts - 1; ++q)
            if (q + 1 < nparts) sum += static_cast<int>(static_cast<uint32_t>(v[q]));
    }
    if (lane < 32 && ncol < H)
        out[ncol] = f2h(__fmul_rn(__fmul_rn(static_cast<float>(sum), sdv), epilogue_scale<REF16>(as)));
}

// Workgroups of `kernel` that the current device holds at once (occupancy
// per CU x CUs), cached per device, kernel and block size.
template <typename Kernel>
int resident_blocks(Kernel kernel, int which, int threads) {
    static std::mutex mu;
    static std::unordered_map<int64_t, int> cache;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    const int64_t key = (static_cast<int64_t>(dev) << 20) | (static_cast<int64_t>(which) << 16) | threads;
    std::lock_guard<std::mutex> lock(mu);
    auto it = cache.find(key);
    if (it != cache.end()) return it->second;
    int per_cu = 0, cus = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, threads, 0) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        return 0;
    const int n = per_cu * cus;
    cache.emplace(key, n);
    return n;
}

}  // namespace
}  // namespace mcv

using namespace mcv;

extern "C" {

int64_t mcv_w4a16_mlp_workspace_bytes(int64_t H, int64_t I) {
    if (H <= 0 || I <= 0 || H > (int64_t(1) << 20) || I > (int64_t(1) << 20)) return 0;
    return kWsHeader + act_bytes(I) + ceil_div(H, kSlab) * kMaxWaves * kSlab * 8;
}

int mcv_w4a16_mlp(const void* x, int64_t H, int64_t I, const void* qw_gate, const void* scales_gate,
                  const void* zeros_gate, int zero_bias_gate, const void* qw_up, const void* scales_up,
                  const void* zeros_up, int zero_bias_up, const void* qw_down, const void* scales_down,
                  const void* zeros_down, int zero_bias_down, void* out, void* workspace, uint32_t* status,
                  mcv_stream_t stream) {
    const char* who = "mcv_w4a16_mlp";
    if (!x || !out || !workspace) return fail(MCV_ERR_INVALID_ARG, "%s: null x/out/workspace", who);
    if (!qw_gate || !scales_gate || !zeros_gate || !qw_up || !scales_up || !zeros_up || !qw_down || !scales_down ||
        !zeros_down)
        return fail(MCV_ERR_INVALID_ARG, "%s: null weight pointer", who);
    for (int zb : {zero_bias_gate, zero_bias_up, zero_bias_down})
        if (zb != 0 && zb != 1) return fail(MCV_ERR_INVALID_ARG, "%s: zero_bias must be 0 or 1", who);
    if (H <= 0 || H % kGroup != 0 || I <= 0 || I % kGroup != 0 || H > (int64_t(1) << 20) || I > (int64_t(1) << 20))
        return fail(MCV_ERR_SHAPE, "%s: H and I must be positive multiples of 128 (H=%lld I=%lld)", who, (long long)H,
                    (long long)I);
    if (reinterpret_cast<uintptr_t>(workspace) % 256 != 0)
        return fail(MCV_ERR_INVALID_ARG, "%s: workspace must be 256-byte aligned", who);
    if (reinterpret_cast<uintptr_t>(x) % 4 != 0) return fail(MCV_ERR_INVALID_ARG, "%s: x must be 4-byte aligned", who);
    const int64_t nslab1 = ceil_div(I, kSlab), nslab2 = ceil_div(H, kSlab);
    const int ks1 = gemv_ksplit(H / kGroup, nslab1);
    const int ks2 = gemv_ksplit(I / kGroup, nslab2);
    if (ceil_div(I / kGroup, ks2) > 2)
        return fail(MCV_ERR_SHAPE, "%s: I=%lld needs more than two groups per wave slot (I <= 4096 does not)", who,
                    (long long)I);
    const int64_t grid = nslab2 * ((ks2 + 1) / 2) + 2 * nslab1;
    const int threads = 64 * (ks1 > kP2Waves ? ks1 : kP2Waves);
    if (grid > kMaxBlocks)
        return fail(MCV_ERR_SHAPE, "%s: %lld workgroups exceed %d (H=%lld I=%lld)", who, (long long)grid, kMaxBlocks,
                    (long long)H, (long long)I);
    int rc = require_device();
    if (rc != MCV_OK) return rc;
    const int resident = resident_blocks(w4a16_mlp_kernel, 0, threads);
    if (grid > resident)
        return fail(MCV_ERR_SHAPE, "%s: %lld workgroups of %d threads exceed the %d the device holds at once", who,
                    (long long)grid, threads, resident);
    hipLaunchKernelGGL(w4a16_mlp_kernel, dim3(static_cast<unsigned>(grid)), dim3(threads), 0,
                       static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(x),
                       W4Ptrs{static_cast<const uint4*>(qw_gate), static_cast<const uint16_t*>(scales_gate),
                              static_cast<const uint32_t*>(zeros_gate), static_cast<uint32_t>(zero_bias_gate)},
                       W4Ptrs{static_cast<const uint4*>(qw_up), static_cast<const uint16_t*>(scales_up),
                              static_cast<const uint32_t*>(zeros_up), static_cast<uint32_t>(zero_bias_up)},
                       W4Ptrs{static_cast<const uint4*>(qw_down), static_cast<const uint16_t*>(scales_down),
                              static_cast<const uint32_t*>(zeros_down), static_cast<uint32_t>(zero_bias_down)},
                       static_cast<uint16_t*>(out), static_cast<int>(H), static_cast<int>(I), ks1, ks2,
                       static_cast<unsigned*>(workspace), static_cast<unsigned*>(status));
    return check_launch("w4a16_mlp_kernel");
}

static int w8_parts(int64_t I) { return static_cast<int>(ceil_div(ceil_div(I, 128) * 4, kW8PartBlocks)); }

int64_t mcv_w8a8_mlp_workspace_bytes(int64_t H, int64_t I) {
    if (H <= 0 || I <= 0 || H > kW8MaxH || w8_parts(I) > kW8MaxParts) return 0;
    const W8Layout l = w8_layout(static_cast<int>(H), static_cast<int>(I), w8_parts(I));
    return (static_cast<int64_t>(l.part) + 2 * ceil_div(H, kSlab) * w8_parts(I) * 32) * 8;
}

int mcv_w8a8_mlp(const void* x, int64_t H, int64_t I, const int8_t* w_gate, const void* ws_gate, const int8_t* w_up,
                 const void* ws_up, const int8_t* w_down, const void* ws_down, int scale_dtype, void* out,
                 void* workspace, uint32_t* status, mcv_stream_t stream) {
    const char* who = "mcv_w8a8_mlp";
    if (!x || !out || !workspace) return fail(MCV_ERR_INVALID_ARG, "%s: null x/out/workspace", who);
    if (!w_gate || !ws_gate || !w_up || !ws_up || !w_down || !ws_down)
        return fail(MCV_ERR_INVALID_ARG, "%s: null weight or scale pointer", who);
    if (scale_dtype != MCV_F32 && scale_dtype != MCV_F16)
        return fail(MCV_ERR_INVALID_ARG, "%s: scale_dtype must be MCV_F32 or MCV_F16", who);
    if ((reinterpret_cast<uintptr_t>(w_gate) | reinterpret_cast<uintptr_t>(w_up) | reinterpret_cast<uintptr_t>(w_down)) % 16)
        return fail(MCV_ERR_INVALID_ARG, "%s: weights must be 16-byte aligned", who);
    if (H <= 0 || H % kGroup != 0 || I <= 0 || I % kGroup != 0 || H > kW8MaxH || I > 16384)
        return fail(MCV_ERR_SHAPE, "%s: H, I must be positive multiples of 128, H <= %d, I <= 16384 (H=%lld I=%lld)",
                    who, kW8MaxH, (long long)H, (long long)I);
    if (reinterpret_cast<uintptr_t>(x) % 4 != 0) return fail(MCV_ERR_INVALID_ARG, "%s: x must be 4-byte aligned", who);
    if (reinterpret_cast<uintptr_t>(workspace) % 256 != 0)
        return fail(MCV_ERR_INVALID_ARG, "%s: workspace must be 256-byte aligned", who);
    const int nparts = w8_parts(I);
    const int64_t grid = 2 * ceil_div(H, kSlab) * nparts + 2 * ceil_div(I, kSlab);
    if (grid > kMaxBlocks)
        return fail(MCV_ERR_SHAPE, "%s: %lld workgroups exceed %d (H=%lld I=%lld)", who, (long long)grid, kMaxBlocks,
                    (long long)H, (long long)I);
    int rc = require_device();
    if (rc != MCV_OK) return rc;
    auto kernel = scale_dtype == MCV_F16 ? w8a8_mlp_kernel<true> : w8a8_mlp_kernel<false>;
    const int resident = resident_blocks(kernel, scale_dtype == MCV_F16 ? 2 : 1, 64 * kW8Waves);
    if (grid > resident)
        return fail(MCV_ERR_SHAPE, "%s: %lld workgroups exceed the %d the device holds at once", who, (long long)grid,
                    resident);
    hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(grid)), dim3(64 * kW8Waves), 0,
                       static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(x), w_gate, ws_gate, w_up, ws_up,
                       w_down, ws_down, static_cast<uint16_t*>(out), static_cast<int>(H), static_cast<int>(I), nparts,
                       static_cast<unsigned*>(workspace), static_cast<unsigned*>(status));
    return check_launch("w8a8_mlp_kernel");
}

}  // extern "C"
