// w8a8_tiled.hip -- W8A8 GEMM and GEMV over the MFMA-tiled int8 weight layout
// (MCV_W8_TILED, include/mcv_quant.h), gfx950.
//
// acc[m][n] = sum_k xq[m][k] * w[k][n] in int32 (exact), optionally followed
// by the fused epilogue out = fp16 RNE((float(acc) * ws[n]) * xs[m]).
//
// The tiled layout stores every 32-column x 32-k block of the weight as one
// contiguous 1 KiB line in the operand order of v_mfma_i32_32x32x32_i8 (lane
// l: column l%32, k-half l/32, 16 bytes).  The GEMM over it (M > 4) stages
// both operands in LDS (w8a8_gemm_lds.hip); this file holds the layout's
// GEMV and the dispatch.
//
// GEMV (M <= 4, or M <= 2 when K > 2048): one workgroup per slab, waves splitting K, v_dot4
// int8 dot products on the same operand lines, partial sums meeting in LDS.
//
// Replaces matmul_w8a8_i32_custom + w8a8_dequant_custom and their host
// wrappers (src/csrc/lib/ops.cpp:1097-1133, 1173-1210) for weights packed by
// quantize_dense_weight_w8a8 (src/csrc/lib/quantized_weight.cpp:231-268).
#include <cstdlib>
#include <cstring>
#include <string>

#include "argmax_exchange.h"
#include "common.h"

namespace mcv {
namespace {

constexpr int kW8Block = 1024;        // bytes of one 32-column x 32-k operand line

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, static_cast<int>(bytes), 0x00020000);
}

// ------------------------------------------------------------------ GEMV --
// M <= 4.  A workgroup owns HALVES 32-column halves of one 64-column slab
// (grid (nslab, 2 / HALVES)); its NW waves split the 32-k blocks, wave v
// taking kb = v, v + NW, ...  Each wave issues the loads of U k-blocks (weight
// lines and x vectors) before it multiplies any of them; k-blocks past the end
// read as zero through an out-of-range buffer offset, so no load is
// conditional.  Lane l of a half accumulates column 32 j + l%32 over k-half
// l/32 with v_dot4_i32_i8 (exact int32); the partial sums meet in LDS.  DUAL:
// the same over a second weight (gate and up) with the fp16 epilogues of both
// and silu_mul_f16 -- bit-identical to two GEMVs and silu_mul, since the int32
// sums are exact and the epilogue code is shared.  ARG (M = 1, both halves in
// the workgroup): the fp16 outputs also leave as one first-maximum argmax key
// per slab (keys[slab], argmax_key64 of the fp16 value and the column), and
// `out` may be null.
template <int MR, int NW, int HALVES, int U, bool OUT_F16, bool DUAL, bool ARG = false>
__global__ __launch_bounds__(64 * NW) void w8a8_tiled_gemv_kernel(
    const int8_t* __restrict__ xq, const int8_t* __restrict__ w, const int8_t* __restrict__ w2, int M, int K, int N,
    int KB, void* __restrict__ out, const void* __restrict__ xs, int xs16, const void* __restrict__ ws,
    const void* __restrict__ ws2, int ws16, int nslab, unsigned long long* __restrict__ keys) {
    static_assert(!ARG || (MR == 1 && HALVES == 2 && OUT_F16 && !DUAL), "argmax epilogue: M = 1, whole slabs");
    constexpr int NWT = DUAL ? 2 : 1;
    __shared__ int red[NW][MR][NWT][HALVES][64];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int slab = blockIdx.x;
    const int j0 = HALVES == 2 ? 0 : static_cast<int>(blockIdx.y);
    const int h = lane >> 5;
    constexpr uint32_t kNowhere = 0xFFFFFF00u;
    const uint32_t wbytes = static_cast<uint32_t>(nslab) * KB * 2 * kW8Block;
    const __amdgpu_buffer_rsrc_t wr[2] = {rsrc(w, wbytes), rsrc(DUAL ? w2 : w, wbytes)};
    const __amdgpu_buffer_rsrc_t xr = rsrc(xq, static_cast<uint32_t>(M) * K);
    int acc[MR][NWT][HALVES];
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
        for (int t = 0; t < NWT; ++t)
#pragma unroll
            for (int jj = 0; jj < HALVES; ++jj) acc[m][t][jj] = 0;
    // the epilogue's scales, loaded now so the tail does not wait for them:
    // thread -> (row em, half ejj, column el of the half)
    const int etid = threadIdx.x;
    const int em = etid / (32 * HALVES), ejj = (etid >> 5) % HALVES, el = etid & 31;
    const int en = slab * kSlab + 32 * (j0 + ejj) + el;
    const bool eok = etid < 32 * HALVES * MR && em < M && en < N;
    // raw bits now, converted in the epilogue (a conversion here would wait)
    uint32_t r_xs = 0, r_ws = 0, r_ws2 = 0;
    if constexpr (OUT_F16) {
        if (eok) {
            r_xs = xs16 ? static_cast<const uint16_t*>(xs)[em] : static_cast<const uint32_t*>(xs)[em];
            r_ws = ws16 ? static_cast<const uint16_t*>(ws)[en] : static_cast<const uint32_t*>(ws)[en];
            if constexpr (DUAL)
                r_ws2 = ws16 ? static_cast<const uint16_t*>(ws2)[en] : static_cast<const uint32_t*>(ws2)[en];
        }
    }
    auto bits_to_f = [](uint32_t r, int is16) { return is16 ? h2f(static_cast<uint16_t>(r)) : __uint_as_float(r); };
    for (int kb0 = wave; kb0 < KB; kb0 += NW * U) {
        int4_t wv[U][NWT][HALVES];
        int4_t xv[U][MR];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int kb = kb0 + u * NW;
            const bool live = kb < KB;
#pragma unroll
            for (int t = 0; t < NWT; ++t)
#pragma unroll
                for (int jj = 0; jj < HALVES; ++jj) {
                    const uint32_t off =
                        live ? ((static_cast<uint32_t>(slab) * KB + kb) * 2 + j0 + jj) * kW8Block + lane * 16u : kNowhere;
                    wv[u][t][jj] = __builtin_bit_cast(int4_t, __builtin_amdgcn_raw_buffer_load_b128(wr[t], off, 0, 2));
                }
#pragma unroll
            for (int m = 0; m < MR; ++m) {
                // k past K in a row meets zero weights; rows past M are not used
                const uint32_t off = live ? static_cast<uint32_t>(m * K + kb * 32 + h * 16) : kNowhere;
                xv[u][m] = __builtin_bit_cast(int4_t, __builtin_amdgcn_raw_buffer_load_b128(xr, off, 0, 0));
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int m = 0; m < MR; ++m)
#pragma unroll
                for (int t = 0; t < NWT; ++t)
#pragma unroll
                    for (int jj = 0; jj < HALVES; ++jj)
#pragma unroll
                        for (int q = 0; q < 4; ++q)
                            acc[m][t][jj] = __builtin_amdgcn_sdot4(wv[u][t][jj][q], xv[u][m][q], acc[m][t][jj], false);
    }
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
        for (int t = 0; t < NWT; ++t)
#pragma unroll
            for (int jj = 0; jj < HALVES; ++jj) red[wave][m][t][jj][lane] = acc[m][t][jj];
    __syncthreads();
    // thread -> (row m, half jj, column l of the half)
    const int tid = threadIdx.x;
    if (tid >= 32 * HALVES * MR) return;
    const int m = tid / (32 * HALVES), jj = (tid >> 5) % HALVES, l = tid & 31;
    int sum[NWT];
#pragma unroll
    for (int t = 0; t < NWT; ++t) {
        sum[t] = 0;
#pragma unroll
        for (int v = 0; v < NW; ++v) sum[t] += red[v][m][t][jj][l] + red[v][m][t][jj][l + 32];
    }
    const int n = slab * kSlab + 32 * (j0 + jj) + l;
    const float e_xs = bits_to_f(r_xs, xs16), e_ws = bits_to_f(r_ws, ws16);
    if constexpr (ARG) {
        // the 64 threads left are wave 0, one column each (columns past N: key 0)
        const uint16_t h16 = f2h(__fmul_rn(__fmul_rn(static_cast<float>(sum[0]), e_ws), e_xs));
        if (out != nullptr && n < N) static_cast<uint16_t*>(out)[n] = h16;
        const unsigned long long key = wave_max_u64(n < N ? argmax_key64(argmax_key16(h16), static_cast<uint32_t>(n))
                                                          : 0ull);
        if (lane == 0) keys[slab] = key;
        return;
    }
    if (m >= M || n >= N) return;
    const size_t o = static_cast<size_t>(m) * N + n;
    if constexpr (DUAL) {
        const float e_ws2 = bits_to_f(r_ws2, ws16);
        const uint16_t g16 = f2h(__fmul_rn(__fmul_rn(static_cast<float>(sum[0]), e_ws), e_xs));
        const uint16_t u16 = f2h(__fmul_rn(__fmul_rn(static_cast<float>(sum[1]), e_ws2), e_xs));
        static_cast<uint16_t*>(out)[o] = silu_mul_f16(g16, u16);
    } else if constexpr (OUT_F16) {
        const float v = __fmul_rn(__fmul_rn(static_cast<float>(sum[0]), e_ws), e_xs);
        static_cast<uint16_t*>(out)[o] = f2h(v);
    } else {
        static_cast<int32_t*>(out)[o] = sum[0];
    }
}

// GEMV launch.  Measured with rotated weights (graph-replayed, M=1): narrow
// outputs (fewer than 128 slabs) want a workgroup per 32-column half -- 8
// waves with 4 k-blocks in flight up to K=2048 (K=1024, N=3584: 3.5 us; one
// workgroup per slab, 8 waves, one block at a time: 4.8 us), 16 waves with 2
// for longer K (K=3584, N=1024: 5.4 us against 10.0); wide ones a workgroup
// per slab with 16 waves and 2 blocks (N=248096: 40.7 us against 47).
template <bool OUT_F16, bool DUAL>
int launch_w8a8_gemv(const int8_t* xq, int64_t M, int64_t K, int64_t N, const int8_t* w, const int8_t* w2, void* out,
                     const void* xs, int xs16, const void* ws, const void* ws2, int ws16, hipStream_t stream) {
    const int64_t nslab = ceil_div(N, kSlab);
    const int64_t KB = ceil_div(K, 128) * 4;
    if (nslab * KB * 2 * kW8Block >= (int64_t(1) << 32) || M * K >= (int64_t(1) << 32))
        return fail(MCV_ERR_SHAPE, "w8a8 tiled GEMV: weight or activation exceeds 4 GiB");
    const bool narrow = nslab < 128;
    const int nw = narrow && KB <= 64 ? 8 : 16, halves = narrow ? 1 : 2, u = narrow && KB <= 64 ? 4 : 2;
    const dim3 grid(static_cast<unsigned>(nslab), halves == 1 ? 2u : 1u);
    const dim3 block(64 * nw);
    const int iM = static_cast<int>(M), iK = static_cast<int>(K), iN = static_cast<int>(N), iKB = static_cast<int>(KB);
    const int ns = static_cast<int>(nslab);
    bool launched = false;
#define MCV_GEMV8V(R, NW_, H_, U_)                                                                                \
    if (!launched && nw == NW_ && halves == H_ && u == U_) {                                                      \
        hipLaunchKernelGGL((w8a8_tiled_gemv_kernel<R, NW_, H_, U_, OUT_F16, DUAL>), grid, block, 0, stream, xq, w, w2, \
                           iM, iK, iN, iKB, out, xs, xs16, ws, ws2, ws16, ns, nullptr);                           \
        launched = true;                                                                                           \
    }
#define MCV_GEMV8(R) MCV_GEMV8V(R, 8, 1, 4) MCV_GEMV8V(R, 16, 1, 2) MCV_GEMV8V(R, 16, 2, 2)
    switch (M) {
        case 1: MCV_GEMV8(1) break;
        case 2: MCV_GEMV8(2) break;
        case 3: MCV_GEMV8(3) break;
        default: MCV_GEMV8(4) break;
    }
#undef MCV_GEMV8
#undef MCV_GEMV8V
    if (!launched) return fail(MCV_ERR_INVALID_ARG, "w8a8 tiled GEMV: no variant %d,%d,%d", nw, halves, u);
    return check_launch(DUAL ? "w8a8_tiled_gemv_kernel<gate_up_silu>" : "w8a8_tiled_gemv_kernel");
}

// The whole W8A8 lm_head step in one launch (M = 1): the activation
// quantisation, the GEMV over the slabs holding columns < V with the fused
// epilogue, and the first-maximum argmax through the device-token exchange
// (argmax_exchange.h).  A workgroup takes SPW consecutive slabs
// (w8a8_lm_head_spw), so the quantisation is paid per workgroup, not per slab.
// 16 waves; for each slab wave w takes k-blocks w,
// w + 16, ... (both 32-column halves) with the next slab's weight lines in
// flight; x is quantised once into LDS with the activation quantiser's
// arithmetic (w8a8_quant_act_kernel: the row maximum is a maximum in any
// order, every element the same act_quant) while the first slab's lines load;
// the int32 partial sums (exact in any order) meet in LDS; wave w then
// applies the GEMV's epilogue to slab w of the workgroup and forms its key.
// So the logits and the token are bit-identical to mcv_w8a8_quantize_act +
// mcv_w8a8_gemv_argmax_partials + mcv_argmax_reduce_keys.
constexpr int kW8LmWaves = 16;

template <int SPW, int U>
__global__ __launch_bounds__(64 * kW8LmWaves) void w8a8_lm_head_kernel(
    const uint16_t* __restrict__ x, const int8_t* __restrict__ w, int K, int V, int KB, int nslab,
    const void* __restrict__ wscale, int ws16, int xs16, uint16_t* __restrict__ logits,
    unsigned long long* __restrict__ ws, int64_t* __restrict__ token, unsigned skew, unsigned* status) {
    constexpr int NW = kW8LmWaves;
    constexpr int XB = NW * U * 32;                      // bytes of the quantised row (zero past K)
    constexpr int XPER = (XB + 64 * NW - 1) / (64 * NW);
    static_assert(SPW <= NW, "one slab per wave in the epilogue");
    __shared__ int part[SPW][NW][64];
    __shared__ __attribute__((aligned(16))) int8_t xq[XB];
    __shared__ float smax[NW];
    __shared__ unsigned long long wbest[NW];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int h = lane >> 5;
    const int s0 = static_cast<int>(blockIdx.x) * SPW;
    const int ns = nslab - s0 < SPW ? nslab - s0 : SPW;  // workgroup-uniform
    // the call's generation word (needed only at the end), x and the
    // epilogue's scale go out first: a wave's loads return in issue order
    unsigned gen = 0;
    if (wave == 0)
        gen = __hip_atomic_load(reinterpret_cast<unsigned*>(ws) + kLmGen, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    uint16_t xv[XPER];
#pragma unroll
    for (int i = 0; i < XPER; ++i) {
        const int k = static_cast<int>(threadIdx.x) + i * 64 * NW;
        xv[i] = k < K ? x[k] : uint16_t(0);
    }
    const int n = (s0 + wave) * kSlab + lane;           // wave w's epilogue column
    uint32_t r_ws = 0;
    if (wave < ns && n < V)
        r_ws = ws16 ? static_cast<const uint16_t*>(wscale)[n] : static_cast<const uint32_t*>(wscale)[n];
    // slab i's lines of this wave into ring slot i & 1; slabs past the
    // workgroup's last re-read its last (never stored); k-blocks past the end
    // get bit 31 in the offset and read zero (the weight is under 2 GiB).  No
    // select in the offsets: a uniform select compiles to a branch, and the
    // waitcnt pass then waits for every load in flight at the join.
    const __amdgpu_buffer_rsrc_t wr = rsrc(w, static_cast<uint32_t>(nslab) * KB * 2 * kW8Block);
    int4_t wv[2][U][2];
    auto issue = [&](int slot, int i) {
        const uint32_t sl = static_cast<uint32_t>(s0 + min(i, ns - 1));
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int kb = wave + u * NW;
            const uint32_t dead = static_cast<uint32_t>(kb >= KB) << 31;
#pragma unroll
            for (int jj = 0; jj < 2; ++jj) {
                const uint32_t off = (((sl * KB + kb) * 2 + jj) * kW8Block + lane * 16u) | dead;
                wv[slot][u][jj] = __builtin_bit_cast(int4_t, __builtin_amdgcn_raw_buffer_load_b128(wr, off, 0, 2));
            }
        }
    };
    issue(0, 0);
    // x -> int8 in LDS with the activation quantiser's arithmetic
    float m = 0.f;
#pragma unroll
    for (int i = 0; i < XPER; ++i) {
        const float v = fabsf(h2f(xv[i]));                // padding contributes 0, never above the max
        m = v > m ? v : m;
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const float o = __shfl_xor(m, off, 64);
        m = o > m ? o : m;
    }
    if (lane == 0) smax[wave] = m;
    __syncthreads();
    m = smax[0];
#pragma unroll
    for (int v = 1; v < NW; ++v) m = smax[v] > m ? smax[v] : m;
    const float scale = act_scale(m);
    const float inv = __fdiv_rn(1.0f, scale);
#pragma unroll
    for (int i = 0; i < XPER; ++i) {
        const int k = static_cast<int>(threadIdx.x) + i * 64 * NW;
        if (k < XB) xq[k] = k < K ? act_quant(xv[i], inv) : int8_t(0);
    }
    __syncthreads();
    int4_t xb[U];
#pragma unroll
    for (int u = 0; u < U; ++u) xb[u] = *reinterpret_cast<const int4_t*>(xq + (wave + u * NW) * 32 + h * 16);
#pragma unroll
    for (int i = 0; i < SPW; ++i) {
        if (i + 1 < SPW) issue((i + 1) & 1, i + 1);
        int a0 = 0, a1 = 0;
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                a0 = __builtin_amdgcn_sdot4(wv[i & 1][u][0][q], xb[u][q], a0, false);
                a1 = __builtin_amdgcn_sdot4(wv[i & 1][u][1][q], xb[u][q], a1, false);
            }
        // lanes l and l ^ 32 hold the two k-halves of the same column
        a0 += __shfl_xor(a0, 32, 64);
        a1 += __shfl_xor(a1, 32, 64);
        part[i][wave][lane] = h ? a1 : a0;               // lane l: column l of the slab
    }
    __syncthreads();
    unsigned long long best = 0ull;
    if (wave < ns) {
        int sum = 0;
#pragma unroll
        for (int v = 0; v < NW; ++v) sum += part[wave][v][lane];
        const float e_ws = ws16 ? h2f(static_cast<uint16_t>(r_ws)) : __uint_as_float(r_ws);
        const float e_xs = xs16 ? h2f(f2h(scale)) : scale;
        const uint16_t h16 = f2h(__fmul_rn(__fmul_rn(static_cast<float>(sum), e_ws), e_xs));
        if (logits != nullptr && n < V) logits[n] = h16;
        best = n < V ? argmax_key64(argmax_key16(h16), static_cast<uint32_t>(n)) : 0ull;
    }
    best = wave_max_u64(best);
    if (lane == 0) wbest[wave] = best;
    __syncthreads();
    if (wave != 0) return;
    best = wave_max_u64(lane < NW ? wbest[lane] : 0ull);
    argmax_publish(ws, best, gen, skew, static_cast<int>(blockIdx.x), static_cast<int>(gridDim.x), lane, token,
                   status);
}

}  // namespace

unsigned lm_poll_skew();

// Slabs per workgroup of the W8A8 lm_head: 4 once that still gives >= 512
// workgroups, fewer below.  Measured at V = 248094 (3877 slabs, 200 back-to-
// back steps, MI355X): 4 slabs (970 workgroups) 41.8 us per step; 2 slabs
// 42.1-42.3; 8 slabs 43.2; 16 slabs (one workgroup per CU, 243) 42.7; 1 slab
// (every workgroup quantising x for one slab) 46-47.  The exchange's last
// workgroup polls the others' keys: workgroups start in index order, so every
// one it waits for has started and waits for nothing.
int w8a8_lm_head_spw(int64_t nslab) {
    int spw = 4;
    while (spw > 1 && ceil_div(nslab, spw) < 512) spw /= 2;
    return spw;
}

// The one-launch W8A8 lm_head (M = 1, K <= 2048).  Shapes were validated by the caller.
int launch_w8a8_lm_head(const void* x, int64_t K, int64_t V, const int8_t* w, const void* wscale, int ws16, int xs16,
                        void* logits, int64_t* token, void* ws, unsigned* status, hipStream_t stream) {
    const int64_t nslab = ceil_div(V, kSlab);
    const int64_t KB = ceil_div(K, 128) * 4;
    if (KB > 4 * kW8LmWaves) return fail(MCV_ERR_SHAPE, "w8a8 lm_head: K=%lld above 2048", (long long)K);
    if (nslab * KB * 2 * kW8Block >= (int64_t(1) << 31))
        return fail(MCV_ERR_SHAPE, "w8a8 lm_head: weight exceeds 2 GiB");
    const int spw = w8a8_lm_head_spw(nslab);
    const int u = KB <= kW8LmWaves ? 1 : (KB <= 2 * kW8LmWaves ? 2 : 4);
    using Fn = void (*)(const uint16_t*, const int8_t*, int, int, int, int, const void*, int, int, uint16_t*,
                        unsigned long long*, int64_t*, unsigned, unsigned*);
    Fn fn = nullptr;
#define MCV_LM8(SPW_)                                                                                        \
    if (spw == SPW_)                                                                                         \
        fn = u == 1 ? w8a8_lm_head_kernel<SPW_, 1> : (u == 2 ? w8a8_lm_head_kernel<SPW_, 2> : w8a8_lm_head_kernel<SPW_, 4>);
    MCV_LM8(1) MCV_LM8(2) MCV_LM8(4)
#undef MCV_LM8
    if (fn == nullptr) return fail(MCV_ERR_INVALID_ARG, "w8a8 lm_head: no kernel for %d slabs per workgroup", spw);
    hipLaunchKernelGGL(fn, dim3(static_cast<unsigned>(ceil_div(nslab, spw))), dim3(64 * kW8LmWaves), 0, stream,
                       static_cast<const uint16_t*>(x), w, static_cast<int>(K), static_cast<int>(V),
                       static_cast<int>(KB), static_cast<int>(nslab), wscale, ws16, xs16,
                       static_cast<uint16_t*>(logits), static_cast<unsigned long long*>(ws), token, lm_poll_skew(),
                       status);
    return check_launch("w8a8_lm_head_kernel");
}

// Columns pad to 64 (a slab), k to 128 (a GEMM stage); padding is zero.
int64_t w8a8_tiled_bytes(int64_t K, int64_t N) {
    if (K <= 0 || N <= 0) return 0;
    return ceil_div(N, kSlab) * kSlab * ceil_div(K, 128) * 128;
}

int launch_w8a8_gemm_lds(const int8_t* xq, int64_t M, int64_t K, int64_t N, const int8_t* w, void* out, bool f16,
                         const void* xs, int xs16, const void* ws, int ws16, hipStream_t stream);
std::string w8a8_gemm_lds_name(int64_t M, int64_t N, bool f16);

// The GEMV takes M <= 4, and M <= 2 past K = 2048 (launch_w8a8_tiled).
bool w8a8_uses_gemv(int64_t M, int64_t K) {
    const int64_t KB = ceil_div(K, 128) * 4;
    return M <= 2 || (M <= 4 && KB <= 64);
}

// The kernel launch_w8a8_tiled runs for M x K x N, as text (report labels).
std::string w8a8_tiled_name(int64_t M, int64_t K, int64_t N, bool f16) {
    if (!w8a8_uses_gemv(M, K)) return w8a8_gemm_lds_name(M, N, f16);
    const int64_t nslab = ceil_div(N, kSlab), KB = ceil_div(K, 128) * 4;
    const bool narrow = nslab < 128;
    const int nw = narrow && KB <= 64 ? 8 : 16, halves = narrow ? 1 : 2, u = narrow && KB <= 64 ? 4 : 2;
    char buf[160];
    std::snprintf(buf, sizeof(buf), "w8a8_tiled_gemv_kernel<%lld, %d, %d, %d, %s, false, false> (v_dot4, %s)",
                  (long long)(M < 4 ? M : 4), nw, halves, u, f16 ? "true" : "false",
                  f16 ? "fused fp16 epilogue" : "int32 out");
    return buf;
}

// xq [M][K] int8 (16-byte aligned rows not required), w tiled; out int32 or
// fp16 [M][N].  Shapes were validated by the caller.
int launch_w8a8_tiled(const int8_t* xq, int64_t M, int64_t K, int64_t N, const int8_t* w, void* out, bool f16,
                      const void* xs, int xs16, const void* ws, int ws16, hipStream_t stream) {
    const int64_t nslab = ceil_div(N, kSlab);
    const int64_t KB = ceil_div(K, 128) * 4;            // 32-k blocks per slab (padded to whole stages)
    if (nslab * KB * 2 * kW8Block >= (int64_t(1) << 32) || M * K >= (int64_t(1) << 32))
        return fail(MCV_ERR_SHAPE, "w8a8 tiled: weight or activation exceeds 4 GiB");
    // The GEMV up to M = 4, but only up to M = 2 past K = 2048, where its
    // serial k-blocks per wave cost more than the GEMM's fixed start
    // (MI355X, graph-replayed, us: K=3584 N=1024 GEMV M=1/2/4 4.8/6.3/8.4,
    // GEMM M=5 6.6; K=1024 N=3584 GEMV M=4 3.8, GEMM M=5 4.0).
    if (w8a8_uses_gemv(M, K)) {
        return f16 ? launch_w8a8_gemv<true, false>(xq, M, K, N, w, nullptr, out, xs, xs16, ws, nullptr, ws16, stream)
                   : launch_w8a8_gemv<false, false>(xq, M, K, N, w, nullptr, out, xs, xs16, ws, nullptr, ws16, stream);
    }
    // M > 4: the LDS-staged GEMM (w8a8_gemm_lds.hip)
    return launch_w8a8_gemm_lds(xq, M, K, N, w, out, f16, xs, xs16, ws, ws16, stream);
}

// Shapes were validated by the caller; M in [1, 4], both weights tiled.
int launch_w8a8_tiled_gate_up_silu(const int8_t* xq, int64_t M, int64_t K, int64_t N, const int8_t* wg,
                                   const void* wsg, const int8_t* wu, const void* wsu, int ws16, const void* xs,
                                   int xs16, void* act, hipStream_t stream) {
    return launch_w8a8_gemv<true, true>(xq, M, K, N, wg, wu, act, xs, xs16, wsg, wsu, ws16, stream);
}

// The GEMV with the argmax epilogue over the slabs holding columns < V
// (M = 1): one workgroup per slab, 16 waves, 2 k-blocks in flight -- the wide
// variant above (V = 248094: the lm_head).
int launch_w8a8_gemv_argmax(const int8_t* xq, int64_t K, int64_t V, const int8_t* w, void* logits, const void* xs,
                            int xs16, const void* ws, int ws16, unsigned long long* keys, hipStream_t stream) {
    const int64_t nslab = ceil_div(V, kSlab);
    const int64_t KB = ceil_div(K, 128) * 4;
    if (nslab * KB * 2 * kW8Block >= (int64_t(1) << 32) || nslab > 0x7fffffff)
        return fail(MCV_ERR_SHAPE, "w8a8 lm_head GEMV: weight exceeds 4 GiB");
    hipLaunchKernelGGL((w8a8_tiled_gemv_kernel<1, 16, 2, 2, true, false, true>), dim3(static_cast<unsigned>(nslab)),
                       dim3(64 * 16), 0, stream, xq, w, w, 1, static_cast<int>(K), static_cast<int>(V),
                       static_cast<int>(KB), logits, xs, xs16, ws, ws, ws16, static_cast<int>(nslab), keys);
    return check_launch("w8a8_tiled_gemv_kernel<argmax>");
}

}  // namespace mcv
