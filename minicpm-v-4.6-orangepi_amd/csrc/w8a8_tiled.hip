// w8a8_tiled.hip -- W8A8 GEMM and GEMV over the MFMA-tiled int8 weight layout
// (MCV_W8_TILED, include/mcv_quant.h), gfx950.
//
// acc[m][n] = sum_k xq[m][k] * w[k][n] in int32 (exact), optionally followed
// by the fused epilogue out = fp16 RNE((float(acc) * ws[n]) * xs[m]).
//
// The tiled layout stores every 32-column x 32-k block of the weight as one
// contiguous 1 KiB line in the operand order of v_mfma_i32_32x32x32_i8 (lane
// l: column l%32, k-half l/32, 16 bytes).  A wave therefore loads its weight
// operands straight from HBM into registers -- one coalesced 128-bit load per
// operand, no LDS, no VALU -- and only the activations go through LDS.
//
// GEMM: each wave owns one 64-column slab and TM rows (TM/32 x 2 blocks of
// 32x32 int32 accumulators); WN waves side by side share the x rows through a
// double-buffered LDS ring, KS k-parts split K inside the workgroup.  The
// weight operands of a stage are loaded two stages ahead into a ring of three
// register sets; the x vectors of a stage two stages ahead too, spread over
// the k32 steps of the stage being computed.  The MFMA computes the transposed
// tile (weights as the row operand), so a lane ends up with four consecutive
// output columns per register quad: int32 results leave as 16-byte stores,
// fp16 results as 16-byte stores after one v_permlane32_swap per pair.
//
// GEMV (M <= 4, or M <= 2 when K > 2048): one workgroup per slab, waves splitting K, v_dot4
// int8 dot products on the same operand lines, partial sums meeting in LDS.
//
// Replaces matmul_w8a8_i32_custom + w8a8_dequant_custom and their host
// wrappers (src/csrc/lib/ops.cpp:1097-1133, 1173-1210) for weights packed by
// quantize_dense_weight_w8a8 (src/csrc/lib/quantized_weight.cpp:231-268).
#include <cstdlib>
#include <cstring>

#include "common.h"

namespace mcv {
namespace {

constexpr int kW8Block = 1024;        // bytes of one 32-column x 32-k operand line

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, static_cast<int>(bytes), 0x00020000);
}

__device__ __forceinline__ int xcd_tile(int b, int total) {
    const int per = total >> 3, rem = total & 7, x = b & 7, i = b >> 3;
    return x * per + (x < rem ? x : rem) + i;
}

__device__ __forceinline__ float scale_at(const void* p, int is16, int idx) {
    return is16 ? h2f(static_cast<const uint16_t*>(p)[idx]) : static_cast<const float*>(p)[idx];
}

template <int TM, int WN, int KS>
struct Cfg8 {
    static constexpr int NW = WN * KS;
    static constexpr int NT = 64 * NW;
    static_assert(NW == 4, "four waves");
    static constexpr int MB = TM / 32;
    static constexpr int BK = 128;                              // k bytes per stage (4 MFMA k32 steps)
    static constexpr int NSTEP = BK / 32;
    static constexpr int PITCH = BK + 16;                       // bytes per LDS row of the x tile
    static constexpr int kAThreads = 64 * WN;
    static constexpr int kAVec = TM * (BK / 16) / kAThreads;    // 16-byte x vectors per thread per stage
    static_assert(kAVec >= 1 && kAVec <= 8, "x staging registers");
    static constexpr int kBVec = 2 * NSTEP;                     // weight operand lines per wave per stage
    static constexpr int kAStage = TM * PITCH;
    static constexpr int kLdsBytes = KS * 2 * kAStage;
    // KS > 1: k-parts 1..KS-1 hand one 32-row block at a time to k-part 0
    static constexpr int kRedBytes = (KS - 1) * WN * 32 * 64 * 4;
    static constexpr int kLdsAlloc = kLdsBytes > kRedBytes ? kLdsBytes : kRedBytes;
};

template <int TM, int WN, int KS, int DEPTH, bool OUT_F16>
__global__ __launch_bounds__(64 * WN * KS) void w8a8_tiled_gemm_kernel(
    const int8_t* __restrict__ xq, const int8_t* __restrict__ w, int M, int K, int N, int KB, void* __restrict__ out,
    const void* __restrict__ xs, int xs16, const void* __restrict__ ws, int ws16, int nslab, int n_tiles,
    int total_tiles, int KT, int col_major) {
    using C = Cfg8<TM, WN, KS>;
    __shared__ __attribute__((aligned(16))) uint8_t lds[C::kLdsAlloc];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int kp = wave / WN;
    const int wn = wave - kp * WN;
    // Each XCD gets a contiguous run of tiles (xcd_tile); col_major orders
    // that run down the columns of tiles, so an XCD's L2 holds a few weight
    // slabs and re-reads of the smaller x operand cross XCDs instead.
    const int tile = xcd_tile(static_cast<int>(blockIdx.x), total_tiles);
    const int m_tiles = total_tiles / n_tiles;
    const int tm = col_major ? tile % m_tiles : tile / n_tiles;
    const int tn = col_major ? tile / m_tiles : tile - tm * n_tiles;
    const int m0 = tm * TM;
    const int slab = tn * WN + wn;
    const int kt0 = kp * KT;                   // first stage of this k-part

    uint8_t* As = lds + kp * 2 * C::kAStage;

    // x rows m0.. through a range-checked buffer: rows past M read as zero;
    // k past K within a row reads the next row, which meets zero weights.
    const int rows_here = M - m0 < TM ? M - m0 : TM;
    const __amdgpu_buffer_rsrc_t xr = rsrc(xq + static_cast<size_t>(m0) * K, static_cast<uint32_t>(rows_here) * K);
    // Weights: slabs past the end read as zero.
    const __amdgpu_buffer_rsrc_t wr = rsrc(w, static_cast<uint32_t>(nslab) * KB * 2 * kW8Block);
    const uint32_t wbase = (static_cast<uint32_t>(slab) * KB * 2) * kW8Block + lane * 16u;
    const int at = wn * 64 + lane;
    constexpr int kVecPerRow = C::BK / 16;

    struct Set {
        uint4 a[C::kAVec];
        int4_t b[C::kBVec];     // [k32 step][half]
    };
    constexpr int kItems = C::kAVec + C::kBVec;
    // Stages past this k-part's last are loaded from an offset beyond both
    // buffers: the loads still issue (no branch, so the waits stay exact) but
    // return zero without touching memory.
    constexpr uint32_t kNowhere = 0xFFFFFF00u;
    auto load_item = [&](int kt, Set& st, int it) {
        const bool live = kt < KT;
        const int k0 = (kt0 + kt) * C::BK;
        if (it < C::kAVec) {
            const int idx = at + it * C::kAThreads;
            const uint32_t off = live ? static_cast<uint32_t>((idx / kVecPerRow) * K + k0 + (idx % kVecPerRow) * 16)
                                      : kNowhere;
            st.a[it] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(xr, off, 0, 0));
        } else {
            const int b = it - C::kAVec;       // step * 2 + half
            const uint32_t off = live ? wbase + static_cast<uint32_t>((k0 / 32 + (b >> 1)) * 2 + (b & 1)) * kW8Block
                                      : kNowhere;
            st.b[b] = __builtin_bit_cast(int4_t, __builtin_amdgcn_raw_buffer_load_b128(wr, off, 0, 0));
        }
    };
    auto store_a = [&](int buf, const Set& st, int it) {
        const int idx = at + it * C::kAThreads;
        *reinterpret_cast<uint4*>(As + buf * C::kAStage + (idx / kVecPerRow) * C::PITCH + (idx % kVecPerRow) * 16) =
            st.a[it];
    };

    int16_t_v acc[C::MB][2];
#pragma unroll
    for (int i = 0; i < C::MB; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;

    // The fused epilogue's scales are loaded now, off the critical path: the
    // lane's 32 columns' weight scales (zero past N) and its rows' x scales.
    // Transposed blocks: register r of lane l holds row 32 i + l%32 and column
    // 32 j + 8 (r/4) + 4 (l/32) + r%4.
    // Buffer loads, so columns past N and rows past M read as zero with no
    // branch, and all of them are issued before any is used (a branch per
    // scale put a wait behind every fp16 load: 32 serial round trips).
    const int h = lane >> 5;
    float wsv[2][4][4];
    float xsv_all[C::MB];
    if constexpr (OUT_F16) {
        const __amdgpu_buffer_rsrc_t wsr = rsrc(ws, static_cast<uint32_t>(N) * (ws16 ? 2u : 4u));
        const __amdgpu_buffer_rsrc_t xsr = rsrc(xs, static_cast<uint32_t>(M) * (xs16 ? 2u : 4u));
        uint32_t wraw[2][4][4], xraw[C::MB];
        const uint32_t wsz = ws16 ? 2u : 4u, xsz = xs16 ? 2u : 4u;
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int g = 0; g < 4; ++g)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const uint32_t off = static_cast<uint32_t>(slab * kSlab + 32 * j + 8 * g + 4 * h + e) * wsz;
                    wraw[j][g][e] = ws16 ? __builtin_amdgcn_raw_buffer_load_b16(wsr, off, 0, 0)
                                         : __builtin_amdgcn_raw_buffer_load_b32(wsr, off, 0, 0);
                }
#pragma unroll
        for (int i = 0; i < C::MB; ++i) {
            const uint32_t off = static_cast<uint32_t>(m0 + 32 * i + (lane & 31)) * xsz;
            xraw[i] = xs16 ? __builtin_amdgcn_raw_buffer_load_b16(xsr, off, 0, 0)
                           : __builtin_amdgcn_raw_buffer_load_b32(xsr, off, 0, 0);
        }
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int g = 0; g < 4; ++g)
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    wsv[j][g][e] = ws16 ? h2f(static_cast<uint16_t>(wraw[j][g][e])) : __uint_as_float(wraw[j][g][e]);
#pragma unroll
        for (int i = 0; i < C::MB; ++i)
            xsv_all[i] = xs16 ? h2f(static_cast<uint16_t>(xraw[i])) : __uint_as_float(xraw[i]);
    }

    // Stage kt: weights from `cur`, x from LDS buffer kt&1.  During its k32
    // steps the x vectors of stage kt+1 (`nxt`, loaded earlier) move to the
    // other LDS buffer and stage kt+DEPTH is loaded into `fut`, the register
    // set stage kt-1 has just released.
    auto step = [&](int kt, Set& cur, Set& nxt, Set& fut) {
        const int kn = kt + DEPTH;
        const bool store = kt + 1 < KT;
        const uint8_t* A = As + (kt & 1) * C::kAStage + (lane & 31) * C::PITCH + (lane >> 5) * 16;
        int4_t af[2][C::MB];
#pragma unroll
        for (int i = 0; i < C::MB; ++i) af[0][i] = *reinterpret_cast<const int4_t*>(A + i * 32 * C::PITCH);
#pragma unroll
        for (int s = 0; s < C::NSTEP; ++s) {
            const int c = s & 1, n = c ^ 1;
            if (s + 1 < C::NSTEP) {
#pragma unroll
                for (int i = 0; i < C::MB; ++i)
                    af[n][i] = *reinterpret_cast<const int4_t*>(A + i * 32 * C::PITCH + (s + 1) * 32);
            }
#pragma unroll
            for (int i = 0; i < C::MB; ++i) {
                acc[i][0] = __builtin_amdgcn_mfma_i32_32x32x32_i8(cur.b[2 * s], af[c][i], acc[i][0], 0, 0, 0);
                acc[i][1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(cur.b[2 * s + 1], af[c][i], acc[i][1], 0, 0, 0);
            }
#pragma unroll
            for (int it = s * kItems / C::NSTEP; it < (s + 1) * kItems / C::NSTEP; ++it) {
                if (it < C::kAVec && store) store_a((kt + 1) & 1, nxt, it);
                load_item(kn, fut, it);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        __syncthreads();
    };

    // A ring of DEPTH + 1 register sets: stage kt lives in set kt % (DEPTH + 1).
    constexpr int R = DEPTH + 1;
    Set sets[R];
#pragma unroll
    for (int d = 0; d < DEPTH; ++d)
#pragma unroll
        for (int it = 0; it < kItems; ++it) load_item(d, sets[d], it);
#pragma unroll
    for (int it = 0; it < C::kAVec; ++it) store_a(0, sets[0], it);
    __syncthreads();
    int kt = 0;
    for (; kt + R <= KT; kt += R) {
#pragma unroll
        for (int u = 0; u < R; ++u) step(kt + u, sets[u], sets[(u + 1) % R], sets[(u + DEPTH) % R]);
    }
#pragma unroll
    for (int u = 0; u < R - 1; ++u)
        if (kt + u < KT) step(kt + u, sets[u], sets[(u + 1) % R], sets[(u + DEPTH) % R]);

    if constexpr (KS > 1) {
        int* red = reinterpret_cast<int*>(lds);
#pragma unroll
        for (int i = 0; i < C::MB; ++i) {
            if (kp > 0) {
                int* dst = red + ((kp - 1) * WN + wn) * 2 * 16 * 64 + lane;
#pragma unroll
                for (int j = 0; j < 2; ++j)
#pragma unroll
                    for (int r = 0; r < 16; ++r) dst[(j * 16 + r) * 64] = acc[i][j][r];
            }
            __syncthreads();
            if (kp == 0) {
#pragma unroll
                for (int p = 1; p < KS; ++p) {
                    const int* src = red + ((p - 1) * WN + wn) * 2 * 16 * 64 + lane;
#pragma unroll
                    for (int j = 0; j < 2; ++j)
#pragma unroll
                        for (int r = 0; r < 16; ++r) acc[i][j][r] += src[(j * 16 + r) * 64];
                }
            }
            __syncthreads();
        }
        if (kp > 0) return;
    }

    if constexpr (!OUT_F16) {
        int32_t* o = static_cast<int32_t*>(out);
        const bool vec_ok = (N & 3) == 0 && (reinterpret_cast<uintptr_t>(out) & 15) == 0;
#pragma unroll
        for (int i = 0; i < C::MB; ++i) {
            const int row = m0 + 32 * i + (lane & 31);
            if (row >= M) continue;
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const int col = slab * kSlab + 32 * j + 8 * g + 4 * h;
                    if (col >= N) continue;
                    int32_t* dst = o + static_cast<size_t>(row) * N + col;
                    if (vec_ok) {
                        *reinterpret_cast<int4_t*>(dst) = int4_t{acc[i][j][4 * g], acc[i][j][4 * g + 1],
                                                                 acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]};
                    } else {
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            if (col + e < N) dst[e] = acc[i][j][4 * g + e];
                    }
                }
        }
    } else {
        uint16_t* o = static_cast<uint16_t*>(out);
        const bool vec_ok = (N & 7) == 0 && (reinterpret_cast<uintptr_t>(out) & 15) == 0;
#pragma unroll
        for (int i = 0; i < C::MB; ++i) {
            const int row = m0 + 32 * i + (lane & 31);
            const float xsv = xsv_all[i];
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int g = 0; g < 4; g += 2) {
                    uint32_t p[4];
#pragma unroll
                    for (int d = 0; d < 2; ++d) {
                        auto deq = [&](int gg, int e) {
                            return f2h(__fmul_rn(__fmul_rn(static_cast<float>(acc[i][j][4 * gg + e]), wsv[j][gg][e]), xsv));
                        };
                        const uint32_t x0 = deq(g, 2 * d) | (uint32_t(deq(g, 2 * d + 1)) << 16);
                        const uint32_t x1 = deq(g + 1, 2 * d) | (uint32_t(deq(g + 1, 2 * d + 1)) << 16);
                        const auto sw = __builtin_amdgcn_permlane32_swap(x0, x1, false, false);
                        p[d] = sw[0];
                        p[2 + d] = sw[1];
                    }
                    const int col = slab * kSlab + 32 * j + 8 * g + 8 * h;
                    if (row >= M || col >= N) continue;
                    uint16_t* dst = o + static_cast<size_t>(row) * N + col;
                    if (vec_ok) {
                        *reinterpret_cast<uint4*>(dst) = make_uint4(p[0], p[1], p[2], p[3]);
                    } else {
#pragma unroll
                        for (int e = 0; e < 8; ++e)
                            if (col + e < N) dst[e] = static_cast<uint16_t>(p[e >> 1] >> (16 * (e & 1)));
                    }
                }
        }
    }
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
// MCV_W8GEMV="NW,HALVES,U" picks another instantiated variant (sweeps).
template <bool OUT_F16, bool DUAL>
int launch_w8a8_gemv(const int8_t* xq, int64_t M, int64_t K, int64_t N, const int8_t* w, const int8_t* w2, void* out,
                     const void* xs, int xs16, const void* ws, const void* ws2, int ws16, hipStream_t stream) {
    const int64_t nslab = ceil_div(N, kSlab);
    const int64_t KB = ceil_div(K, 128) * 4;
    if (nslab * KB * 2 * kW8Block >= (int64_t(1) << 32) || M * K >= (int64_t(1) << 32))
        return fail(MCV_ERR_SHAPE, "w8a8 tiled GEMV: weight or activation exceeds 4 GiB");
    const bool narrow = nslab < 128;
    int nw = narrow && KB <= 64 ? 8 : 16, halves = narrow ? 1 : 2, u = narrow && KB <= 64 ? 4 : 2;
    static const char* const e = std::getenv("MCV_W8GEMV");            // read once per process
    if (e != nullptr) {
        int a = 0, b = 0, c = 0;
        if (std::sscanf(e, "%d,%d,%d", &a, &b, &c) == 3) { nw = a; halves = b; u = c; }
    }
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
#define MCV_GEMV8(R) \
    MCV_GEMV8V(R, 16, 1, 4) MCV_GEMV8V(R, 8, 2, 4) MCV_GEMV8V(R, 8, 2, 1) MCV_GEMV8V(R, 16, 2, 2) MCV_GEMV8V(R, 8, 1, 4) \
    MCV_GEMV8V(R, 16, 1, 2) MCV_GEMV8V(R, 8, 2, 2)
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

struct Shape8 {
    int tm, wn, ks, depth;
};

template <bool F16>
using Gemm8Fn = void (*)(const int8_t*, const int8_t*, int, int, int, int, void*, const void*, int, const void*, int,
                         int, int, int, int, int);

template <bool F16>
Gemm8Fn<F16> pick8(const Shape8& s) {
#define MCV_S8(TM_, WN_, KS_, D_) \
    if (s.tm == TM_ && s.wn == WN_ && s.ks == KS_ && s.depth == D_) return w8a8_tiled_gemm_kernel<TM_, WN_, KS_, D_, F16>;
    MCV_S8(128, 2, 2, 2) MCV_S8(128, 4, 1, 2) MCV_S8(64, 4, 1, 2) MCV_S8(64, 2, 2, 2) MCV_S8(32, 2, 2, 2)
    MCV_S8(32, 1, 4, 2) MCV_S8(64, 4, 1, 3) MCV_S8(64, 4, 1, 4) MCV_S8(64, 2, 2, 3) MCV_S8(64, 2, 2, 4)
    MCV_S8(32, 2, 2, 3) MCV_S8(32, 2, 2, 4) MCV_S8(32, 1, 4, 3) MCV_S8(128, 4, 1, 3) MCV_S8(128, 2, 2, 3)
#undef MCV_S8
    return nullptr;
}

// Preference order from a sweep on MI355X (K=1024, N=3584, graph-replayed,
// column-major tile order): M=2048 128x256 tiles 15.7 us (64x256: 18.2);
// M=1024 64x256 10.0 us (128x256, 112 tiles: 13.4); M=256 the k-split 32x128
// tiles 7.3 us (64x256: 9.0).  Prefetching three stages ahead instead of two
// was 0.5-2 us slower at every size.
constexpr Shape8 kShapes8[] = {{128, 4, 1, 2}, {64, 4, 1, 2}, {64, 2, 2, 2}, {32, 2, 2, 2}, {32, 1, 4, 2}, {128, 2, 2, 2}};

// The first listed shape whose grid covers most of the 256 CUs, else the one
// with the most workgroups; MCV_W8GEMM_SHAPE="TM,WN,KS" overrides it.
Shape8 choose8(int64_t M, int64_t KT, int64_t nslab) {
    static const char* const e = std::getenv("MCV_W8GEMM_SHAPE");      // read once per process
    if (e != nullptr) {
        Shape8 s{0, 0, 0, 2};
        if (std::sscanf(e, "%d,%d,%d,%d", &s.tm, &s.wn, &s.ks, &s.depth) >= 3 && pick8<true>(s) && KT % s.ks == 0)
            return s;
    }
    Shape8 best{0, 0, 0, 2};
    int64_t best_tiles = -1;
    for (const Shape8& s : kShapes8) {
        if (KT % s.ks != 0) continue;
        const int64_t t = ceil_div(M, s.tm) * ceil_div(nslab, s.wn);
        if (t >= 200) return s;
        if (t > best_tiles) {
            best_tiles = t;
            best = s;
        }
    }
    return best;
}

}  // namespace

// Columns pad to 64 (a slab), k to 128 (a GEMM stage); padding is zero.
int64_t w8a8_tiled_bytes(int64_t K, int64_t N) {
    if (K <= 0 || N <= 0) return 0;
    return ceil_div(N, kSlab) * kSlab * ceil_div(K, 128) * 128;
}

int launch_w8a8_gemm_lds(const int8_t* xq, int64_t M, int64_t K, int64_t N, const int8_t* w, void* out, bool f16,
                         const void* xs, int xs16, const void* ws, int ws16, hipStream_t stream);

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
    if (M <= 2 || (M <= 4 && KB <= 64)) {
        return f16 ? launch_w8a8_gemv<true, false>(xq, M, K, N, w, nullptr, out, xs, xs16, ws, nullptr, ws16, stream)
                   : launch_w8a8_gemv<false, false>(xq, M, K, N, w, nullptr, out, xs, xs16, ws, nullptr, ws16, stream);
    }
    // M > 4: the LDS-staged GEMM (w8a8_gemm_lds.hip); MCV_W8GEMM_KERNEL=regs
    // keeps the register-operand kernel below (read once; comparisons).
    static const char* const which = std::getenv("MCV_W8GEMM_KERNEL");
    if (which == nullptr || std::strcmp(which, "regs") != 0)
        return launch_w8a8_gemm_lds(xq, M, K, N, w, out, f16, xs, xs16, ws, ws16, stream);
    const int64_t KT_all = KB / 4;                      // 128-k stages over the padded K
    const Shape8 s = choose8(M, KT_all, nslab);
    const int64_t n_tiles = ceil_div(nslab, s.wn);
    const int64_t total = ceil_div(M, s.tm) * n_tiles;
    if (total > 0x7fffffff) return fail(MCV_ERR_SHAPE, "w8a8 tiled: too many tiles");
    const int KT = static_cast<int>(KT_all / s.ks);
    const int KBs = static_cast<int>(KB);
    // Down the tile columns when x is the smaller operand (M < N); along the
    // tile rows otherwise.  MCV_W8GEMM_ORDER=0/1 overrides (tuning sweeps).
    int col_major = M < N ? 1 : 0;
    static const char* const order = std::getenv("MCV_W8GEMM_ORDER");  // read once per process
    if (order != nullptr) col_major = std::atoi(order) ? 1 : 0;
    if (f16)
        hipLaunchKernelGGL(pick8<true>(s), dim3(static_cast<unsigned>(total)), dim3(256), 0, stream, xq, w,
                           static_cast<int>(M), static_cast<int>(K), static_cast<int>(N), KBs, out, xs, xs16, ws, ws16,
                           static_cast<int>(nslab), static_cast<int>(n_tiles), static_cast<int>(total), KT, col_major);
    else
        hipLaunchKernelGGL(pick8<false>(s), dim3(static_cast<unsigned>(total)), dim3(256), 0, stream, xq, w,
                           static_cast<int>(M), static_cast<int>(K), static_cast<int>(N), KBs, out, xs, xs16, ws, ws16,
                           static_cast<int>(nslab), static_cast<int>(n_tiles), static_cast<int>(total), KT, col_major);
    return check_launch("w8a8_tiled_gemm_kernel");
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
