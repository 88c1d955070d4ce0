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
                                           unsigned* __restrict__ ws, int lane) {
    for (int spins = 0;; ++spins) {
        load_all(v);
        uint32_t bad = 0;
#pragma unroll
        for (int i = 0; i < N; ++i) bad |= tag_of(v[i]) ^ tag;
        if (__all(bad == 0)) return;
        if (spins > kSpinLimit) {
            if (lane == 0) __hip_atomic_fetch_or(ws + kWsError, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            return;
        }
        __builtin_amdgcn_s_sleep(1);
    }
}

// grid = nslab2 * npair + nslab1 with npair = ceil(ks2 / 2), block =
// 64 * max(ks1, 4).  Workgroups below nslab2 * npair are phase 2 (dispatched
// first, so their weight loads start earliest): workgroup (slab, pair p) owns
// wave slots 2p and 2p + 1 of that output slab.  The rest are phase 1, one act
// slab each.  Requires ceil(G2 / ks2) <= 2 (two groups per slot).
__global__ __launch_bounds__(64 * kMaxWaves) void w4a16_mlp_kernel(const uint16_t* __restrict__ x, W4Ptrs gate,
                                                                   W4Ptrs up, W4Ptrs down, uint16_t* __restrict__ out,
                                                                   int H, int I, int ks1, int ks2,
                                                                   unsigned* __restrict__ ws) {
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
        // ---- phase 1: one act slab, published as tagged words
        const int slab = b - nslab2 * npair;
        float ag = 0.f, au = 0.f;
        if (wave < ks1) {
            const int npad1 = nslab1 * kSlab;
            gate_up_partials(reinterpret_cast<const uint32_t*>(x),
                             w4_column(gate.q, gate.s, gate.z, gate.zero_bias, H, npad1, slab, lane),
                             w4_column(up.q, up.s, up.z, up.zero_bias, H, npad1, slab, lane), wave, ks1, G1, ag, au,
                             vmagic);
            red[0][wave][lane] = ag;
            red[1][wave][lane] = au;
        }
        __syncthreads();
        if (wave != 0) return;
        bump_epoch();
        const uint32_t tag = (epoch + 1u) & 0xffffu;
        ag = red[0][0][lane];
        au = red[1][0][lane];
        for (int w = 1; w < ks1; ++w) {
            ag += red[0][w][lane];
            au += red[1][w][lane];
        }
        const int n = slab * kSlab + lane;
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
        for (int c = 0; c < 4; ++c) wv[c] = dc.q[static_cast<size_t>(g * 4 + c) * kSlab];
        sv = dc.s[static_cast<size_t>(g) * dc.npad];
        zv = dc.z[static_cast<size_t>(g) * (dc.npad >> 3)];
    }
    if (wave == 0 && lane == 0) s_epoch = epoch;
    bump_epoch();
    __syncthreads();
    const uint32_t tag = (s_epoch + 1u) & 0xffffu;
    float y = 0.f;
    if (present) {
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
            tag, ws, lane);
        xg[wave][lane] = (static_cast<uint32_t>(av[0]) & 0xffffu) | (static_cast<uint32_t>(av[0] >> 32) << 16);
        uint32_t xs[64];
#pragma unroll
        for (int k = 0; k < 64; ++k) xs[k] = __builtin_amdgcn_readfirstlane(xg[wave][k]);
        y = group_sum(wv, xs, ((zv >> dc.zshift) & 15u) + dc.zero_bias, vmagic);
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
            [](uint64_t v) { return static_cast<uint32_t>(v >> 32); }, tag, ws, lane);
#pragma unroll
        for (int i = 0; i < kMaxWaves - 2; ++i)
            if (2 + i < ks2) acc += __uint_as_float(static_cast<uint32_t>(pv[i]));
    }
    const int col = slab * kSlab + lane;
    if (col < H) out[col] = f2h(acc);
}

// Workgroups of this kernel that the current device holds at once
// (occupancy per CU x CUs), cached per device and block size.
int resident_blocks(int threads) {
    static std::mutex mu;
    static std::unordered_map<int64_t, int> cache;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    const int64_t key = (static_cast<int64_t>(dev) << 16) | threads;
    std::lock_guard<std::mutex> lock(mu);
    auto it = cache.find(key);
    if (it != cache.end()) return it->second;
    int per_cu = 0, cus = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, w4a16_mlp_kernel, threads, 0) != hipSuccess ||
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
                  const void* zeros_down, int zero_bias_down, void* out, void* workspace, mcv_stream_t stream) {
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
    const int64_t grid = nslab2 * ((ks2 + 1) / 2) + nslab1;
    const int threads = 64 * (ks1 > kP2Waves ? ks1 : kP2Waves);
    if (grid > kMaxBlocks)
        return fail(MCV_ERR_SHAPE, "%s: %lld workgroups exceed %d (H=%lld I=%lld)", who, (long long)grid, kMaxBlocks,
                    (long long)H, (long long)I);
    int rc = require_device();
    if (rc != MCV_OK) return rc;
    const int resident = resident_blocks(threads);
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
                       static_cast<unsigned*>(workspace));
    return check_launch("w4a16_mlp_kernel");
}

}  // extern "C"
