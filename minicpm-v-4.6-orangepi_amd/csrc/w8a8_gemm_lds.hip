// w8a8_gemm_lds.hip -- int8 x int8 -> int32 GEMM over the MFMA-tiled weight
// layout (MCV_W8_TILED), both operands staged through LDS by gfx950's
// direct-to-LDS loads, with the fused fp16 epilogue.  gfx950.
//
// acc[m][n] = sum_k xq[m][k] * w[k][n] (exact int32), optionally
// out = fp16 RNE((float(acc) * ws[n]) * xs[m]).
//
// Workgroup: 4 waves in a 2 x 2 arrangement over a BM x BN output tile, each
// wave BM/2 x BN/2 as 32 x 32 blocks of v_mfma_i32_32x32x32_i8.  K advances in
// stages of 128; a stage's x rows (BM x 128 bytes) and weight lines (BN/32
// column halves x 4 k32 blocks, 1 KiB each) are copied global -> LDS with
// buffer_load_dwordx4 ... lds (no VGPR staging: a wave-wide instruction moves
// 1 KiB into 1 KiB of LDS), NS stages in flight, one barrier per stage.
//   - x: row-major in LDS, 128 bytes per row, the 16-byte chunk index XORed
//     with bits 1..3 of the row: one ds_read_b128 pass serves 16 rows, two
//     per 256-byte bank window, so the row's parity picks the half and bits
//     1..3 must spread the 8 rows of each parity over the 8 chunks.  (XOR by
//     the row's low 3 bits left rows r and r + 8 on the same banks: 229K
//     bank-conflict cycles per M=1024 launch, a third of the LDS-active time.)  The XOR is applied by choosing
//     which global chunk each lane fetches (the LDS side of the copy is always
//     lane-linear).
//   - weights: the tiled layout already stores each 32-column x 32-k block
//     in operand order (lane l: column l%32, k-half l/32), so a line is
//     copied verbatim and read back with one ds_read_b128 at lane*16.
// Both operands of a k32 step come from LDS with conflict-free 16-byte reads;
// each is used by two MFMAs of the wave.  The MFMA computes the transposed
// tile (weights as the row operand), so a lane holds one output row and
// 4 consecutive columns per register quad: int32 results leave as 16-byte
// stores; fp16 ones, after one v_permlane32_swap per pair, pass through LDS
// and leave as non-temporal stores of whole 128-byte row lines.
//
// WR = 1 (the dispatch's 128 x 128 and 64 x 128 tiles): the four waves sit
// 4 x 1 instead, each over all BM rows of its own BN/4 columns, so its weight
// lines are read by no other wave; it loads them straight into a ring of NS
// register slots with ordinary buffer loads (in the copy slots, under the
// same vmcnt waits), the stage buffers hold x alone, and the fp16 tile passes
// through LDS whole so the stores still write whole row lines (M=1024: 7.86
// against 7.93 us).
//
// Each stage lives in its own __shared__ array, indexed by a compile-time
// constant after the stage loop is unrolled NS ways, so the waitcnt pass sees
// that the operand reads of stage s do not alias the copies in flight into
// the other stages and keeps them in flight.  The explicit s_waitcnt vmcnt
// before each barrier is the only wait on the copies; the barrier is a bare
// s_barrier (a __syncthreads fence would wait for every copy in flight).
// The copies of a stage are spread over the k32 steps of the one three
// stages earlier, step s+1's operands are read while step s's MFMAs run, and
// the barrier sits between the MFMAs of a stage's last step, so the next
// stage's first operands are read before the pipe drains.
//
// Replaces matmul_w8a8_i32_custom + w8a8_dequant_custom
// (src/csrc/custom_ops/op_kernel/matmul_w8a8_i32_custom.cpp:15-48,
// w8a8_dequant_custom.cpp:33-69) for weights packed by
// quantize_dense_weight_w8a8 (src/csrc/lib/quantized_weight.cpp:231-268).
#include <cstdio>
#include <cstdlib>
#include <string>

#include "common.h"

namespace mcv {
namespace {

constexpr int kLine = 1024;                 // one 32-column x 32-k operand line

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc_l(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, static_cast<int>(bytes), 0x00020000);
}

// 16 bytes per lane, global (buffer `r` at byte voff + soff) -> LDS at
// lds + 16 * lane.
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, uint8_t* lds, uint32_t voff, int soff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, lds, 16, voff, soff, 0, 0);
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

__device__ __forceinline__ int xcd_tile_l(int b, int total) {
    const int per = total >> 3, rem = total & 7, x = b & 7, i = b >> 3;
    return x * per + (x < rem ? x : rem) + i;
}

// WR = 0: the four waves sit 2 x 2 over the tile and both operands pass
// through LDS.  WR = 1: they sit 4 x 1 (each all BM rows of its BN/4
// columns), so a wave's weight lines are its own: it loads them with
// ordinary buffer loads into a ring of NS register slots (stage kt in slot
// kt % NS, a compile-time index once the stages are unrolled), in the same
// copy slots and under the same vmcnt waits as the x rows, and the stage
// buffers hold x alone.
template <int BM, int BN, int NS, int WR>
struct CfgL {
    static constexpr int BK = 128;                     // k bytes per stage
    static constexpr int A_BYTES = BM * BK;
    static constexpr int B_BYTES = WR ? 0 : BN * BK;
    static constexpr int STAGE = A_BYTES + B_BYTES;
    static constexpr int A_COPIES = A_BYTES / kLine;   // wave-wide 1 KiB copies per stage
    static constexpr int B_COPIES = B_BYTES / kLine;
    static_assert(A_COPIES % 4 == 0 && B_COPIES % 4 == 0, "copies split over four waves");
    static constexpr int PA = A_COPIES / 4;            // x copies per wave per stage
    static constexpr int PB = B_COPIES / 4;            // weight copies per wave per stage
    static constexpr int IB = WR ? BM / 32 : BM / 64;  // 32-row blocks per wave
    static constexpr int JB = WR ? BN / 128 : BN / 64; // 32-column blocks per wave
    static constexpr int PR = WR ? 4 * JB : 0;         // weight lines per wave per stage into registers
    static constexpr int P = PA + PB + PR;
    static_assert(IB >= 1 && JB >= 1 && NS >= 2 && NS <= 4, "tile shape");
    static_assert(WR == 0 || WR == 1, "WR");
    static constexpr int PF = 2;                       // weight stages prefetched per tile
    static constexpr int PFL = WR ? 4 * JB : PB;       // prefetched lines per wave per stage
    static_assert(P * (NS - 2) + PF * PFL < 64, "vmcnt");
};

// EPI: 0 int32 out; 4 | x-scale fp16 (1) | weight-scale fp16 (2): fp16 out
// through the fused epilogue with fp16 or fp32 scales.
template <int BM, int BN, int NS, int EPI, int WR>
__global__ __launch_bounds__(256) void w8a8_gemm_lds_kernel(
    const int8_t* __restrict__ xq, const int8_t* __restrict__ w, int M, int K, int N, int KB, void* __restrict__ out,
    const void* __restrict__ xs, const void* __restrict__ ws, int nslab, int n_tiles, int total_tiles, int KT,
    int xcd_m) {
    constexpr bool OUT_F16 = (EPI & 4) != 0;
    constexpr bool XS16 = (EPI & 1) != 0, WS16 = (EPI & 2) != 0;
    using C = CfgL<BM, BN, NS, WR>;
    __shared__ __attribute__((aligned(1024))) uint8_t lds0[C::STAGE];
    __shared__ __attribute__((aligned(1024))) uint8_t lds1[C::STAGE];
    __shared__ __attribute__((aligned(1024))) uint8_t lds2[NS > 2 ? C::STAGE : 16];
    __shared__ __attribute__((aligned(1024))) uint8_t lds3[NS > 3 ? C::STAGE : 16];
    __shared__ __attribute__((aligned(1024))) uint8_t sink[4 * kLine];   // prefetches land here, never read
    uint8_t* const bufs[4] = {lds0, lds1, lds2, lds3};

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = WR ? 0 : wave & 1, wn = WR ? wave : wave >> 1;
    constexpr int WROWS = WR ? BM : BM / 2, WCOLS = WR ? BN / 4 : BN / 2;   // a wave's share of the tile
    const int h = lane >> 5;

    // Workgroup b runs on XCD b % 8.  With xcd_m > 0 the tile grid is cut
    // into xcd_m x (8 / xcd_m) blocks, one per XCD, so each XCD's L2 sees
    // only its block's x rows and weight columns; otherwise the tiles of one
    // XCD form a contiguous run down the tile columns.  `rows` tiles of one
    // tile column share an XCD, and this tile is the `ri`-th of them.
    const int m_tiles = total_tiles / n_tiles;
    int tm, tn, rows, ri;
    if (xcd_m > 0) {
        const int xb_n = 8 / xcd_m, mr = m_tiles / xcd_m, nr = n_tiles / xb_n;
        const int xcd = static_cast<int>(blockIdx.x) & 7, i = static_cast<int>(blockIdx.x) >> 3;
        ri = i % mr;
        tm = (xcd / xb_n) * mr + ri;
        tn = (xcd % xb_n) * nr + i / mr;
        rows = mr;
    } else {
        const int tile = xcd_tile_l(static_cast<int>(blockIdx.x), total_tiles);
        tm = tile % m_tiles;
        tn = tile / m_tiles;
        rows = m_tiles;
        ri = tm;
    }
    const int m0 = tm * BM, n0 = tn * BN;
    const int slab0 = n0 / kSlab;

    // x rows m0..: rows past M read as zero; k past K within a row reads the
    // next row, which meets zero (padded) weights.
    const int rows_here = M - m0 < BM ? M - m0 : BM;
    const __amdgpu_buffer_rsrc_t xr = rsrc_l(xq + static_cast<size_t>(m0) * K, static_cast<uint32_t>(rows_here) * K);
    // weights: slabs past the last read as zero
    const __amdgpu_buffer_rsrc_t wr = rsrc_l(w, static_cast<uint32_t>(nslab) * KB * 2 * kLine);

    // This wave's copies of a stage: x copies wave*PA .. +PA (8 rows of 128
    // bytes each), weight lines wave*PB .. +PB.  Each lane's offset inside a
    // stage is fixed (computed once here); the stage's advance is one scalar
    // add for x and rides in the scalar offset for the weights, whose buffer
    // is padded to whole stages.  Stages past the last re-read the last stage
    // into a buffer that is never read again: every stage issues the same P
    // copies with no branch, so the vmcnt waits stay exact (a select compiled
    // into a branch makes the waitcnt pass wait for the next stage's copies
    // before this stage's operand reads), and every access stays in range.
    uint32_t xoff[C::PA], woff[C::PB ? C::PB : 1];
#pragma unroll
    for (int j = 0; j < C::PA; ++j) {
        const int row = (wave * C::PA + j) * 8 + (lane >> 3);
        xoff[j] = static_cast<uint32_t>(row * K + (((lane & 7) ^ ((row >> 1) & 7)) << 4));
    }
#pragma unroll
    for (int j = 0; j < C::PB; ++j) {
        const int bi = wave * C::PB + j;                               // (slab bi / 8, k32 block, half)
        woff[j] = (static_cast<uint32_t>(slab0 + (bi >> 3)) * KB * 2 + (bi & 7)) * kLine + lane * 16u;
    }
    // WR: the lane's offsets of this wave's weight lines (column block jb),
    // the k32 step and the stage in the scalar offset
    uint32_t wq_off[C::JB];
#pragma unroll
    for (int jb = 0; jb < C::JB; ++jb) {
        const int col = wn * WCOLS + 32 * jb;
        wq_off[jb] = (static_cast<uint32_t>(slab0 + (col >> 6)) * KB * 2 + ((col >> 5) & 1)) * kLine + lane * 16u;
    }
    int4_t rb[WR ? NS : 1][4][C::JB];
    auto issue_item = [&](int kt, uint8_t* dst, int it, int slot) {
        const int kc = kt < KT ? kt : KT - 1;
        if (it < C::PA) {
            dma16(xr, dst + (wave * C::PA + it) * kLine, xoff[it] + static_cast<uint32_t>(kc * C::BK), 0);
        } else if (WR) {
            const int j = it - C::PA, s = j / C::JB, jb = j % C::JB;
            rb[slot][s][jb] = __builtin_bit_cast(
                int4_t, __builtin_amdgcn_raw_buffer_load_b128(wr, wq_off[jb], (kc * 8 + 2 * s) * kLine, 0));
        } else {
            const int j = it - C::PA;
            dma16(wr, dst + C::A_BYTES + (wave * C::PB + j) * kLine, woff[j], kc * 8 * kLine);
        }
    };

    auto issue = [&](int kt, uint8_t* dst, int slot) {
#pragma unroll
        for (int it = 0; it < C::P; ++it) issue_item(kt, dst, it, slot);
    };

    // The fused epilogue's scales, as raw bits, issued before the first copy:
    // loads complete in issue order, so the first stage's wait covers them.
    // Register r of block (ib, jb) holds row wm*BM/2 + 32 ib + l%32 and column
    // wn*BN/2 + 32 jb + 8 (r/4) + 4 h + r%4.
    // Buffer loads: columns past N and rows past M read as zero with no branch,
    // so all of them issue back to back.  A lane's four consecutive weight
    // scales come in one load when N % 4 == 0 and the scales are aligned
    // (a quad is then wholly inside or wholly past N); otherwise one load per
    // scale.  Each gather instruction holds the address unit for the whole
    // wave, and these go ahead of the first stage's copies: 8 instead of 32
    // per wave brings the first stage in ~0.25 us sooner.  They are older
    // than every copy, so their number does not enter the vmcnt waits.
    uint32_t wraw[C::JB][4][4], xraw[C::IB];
    if constexpr (OUT_F16) {
        const __amdgpu_buffer_rsrc_t wsr = rsrc_l(ws, static_cast<uint32_t>(N) * (WS16 ? 2u : 4u));
        const __amdgpu_buffer_rsrc_t xsr = rsrc_l(xs, static_cast<uint32_t>(M) * (XS16 ? 2u : 4u));
        const bool quads = (N & 3) == 0 && (reinterpret_cast<uintptr_t>(ws) & (WS16 ? 7u : 15u)) == 0;
        if (quads) {
#pragma unroll
            for (int jb = 0; jb < C::JB; ++jb)
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const uint32_t n = static_cast<uint32_t>(n0 + wn * WCOLS + 32 * jb + 8 * g + 4 * h);
                    if constexpr (WS16) {
                        const auto v = __builtin_amdgcn_raw_buffer_load_b64(wsr, n * 2u, 0, 0);
                        wraw[jb][g][0] = v[0] & 0xFFFFu;
                        wraw[jb][g][1] = v[0] >> 16;
                        wraw[jb][g][2] = v[1] & 0xFFFFu;
                        wraw[jb][g][3] = v[1] >> 16;
                    } else {
                        const auto v = __builtin_amdgcn_raw_buffer_load_b128(wsr, n * 4u, 0, 0);
#pragma unroll
                        for (int e = 0; e < 4; ++e) wraw[jb][g][e] = v[e];
                    }
                }
        } else {
#pragma unroll
            for (int jb = 0; jb < C::JB; ++jb)
#pragma unroll
                for (int g = 0; g < 4; ++g)
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const uint32_t n = static_cast<uint32_t>(n0 + wn * WCOLS + 32 * jb + 8 * g + 4 * h + e);
                        if constexpr (WS16) wraw[jb][g][e] = __builtin_amdgcn_raw_buffer_load_b16(wsr, n * 2u, 0, 0);
                        else wraw[jb][g][e] = __builtin_amdgcn_raw_buffer_load_b32(wsr, n * 4u, 0, 0);
                    }
        }
#pragma unroll
        for (int ib = 0; ib < C::IB; ++ib) {
            const uint32_t m = static_cast<uint32_t>(m0 + wm * WROWS + 32 * ib + (lane & 31));
            if constexpr (XS16) xraw[ib] = __builtin_amdgcn_raw_buffer_load_b16(xsr, m * 2u, 0, 0);
            else xraw[ib] = __builtin_amdgcn_raw_buffer_load_b32(xsr, m * 4u, 0, 0);
        }
    }

    int16_t_v acc[C::IB][C::JB];
#pragma unroll
    for (int ib = 0; ib < C::IB; ++ib)
#pragma unroll
        for (int jb = 0; jb < C::JB; ++jb)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[ib][jb][r] = 0;

    // Operand addresses inside a stage (bytes), fixed per lane.
    int a_off[C::IB][4];
#pragma unroll
    for (int ib = 0; ib < C::IB; ++ib) {
        const int row = wm * WROWS + 32 * ib + (lane & 31);
#pragma unroll
        for (int s = 0; s < 4; ++s) a_off[ib][s] = (row * 8 + ((2 * s + h) ^ ((row >> 1) & 7))) * 16;
    }
    int b_off[C::JB][4];
#pragma unroll
    for (int jb = 0; jb < C::JB; ++jb) {
        const int col = wn * WCOLS + 32 * jb;
        const int sl = col >> 6, jh = (col >> 5) & 1;
#pragma unroll
        for (int s = 0; s < 4; ++s) b_off[jb][s] = C::A_BYTES + ((sl * 4 + s) * 2 + jh) * kLine + lane * 16;
    }

    // Operands of k32 step s, double-buffered: step s uses set s & 1.
    int4_t af[2][C::IB], bf[2][C::JB];
    auto read_ops = [&](const uint8_t* src, int s, int set, int slot) {
#pragma unroll
        for (int ib = 0; ib < C::IB; ++ib) af[set][ib] = *reinterpret_cast<const int4_t*>(src + a_off[ib][s]);
#pragma unroll
        for (int jb = 0; jb < C::JB; ++jb)
            bf[set][jb] = WR ? rb[slot][s][jb] : *reinterpret_cast<const int4_t*>(src + b_off[jb][s]);
    };
    constexpr int kNM = C::IB * C::JB;                 // MFMAs per k32 step
    constexpr int kNR = C::IB + (WR ? 0 : C::JB);      // LDS operand reads per k32 step
    auto mfmas = [&](int set, int lo, int hi) {
#pragma unroll
        for (int m = lo; m < hi; ++m) {
            const int ib = m / C::JB, jb = m % C::JB;
            acc[ib][jb] = __builtin_amdgcn_mfma_i32_32x32x32_i8(bf[set][jb], af[set][ib], acc[ib][jb], 0, 0, 0);
        }
    };

    // One stage from `cur`.  Steps 0-2 read step s+1's operands while step
    // s's MFMAs run and spread the copies of stage kt + NS - 1 into `prv`
    // (free since the last barrier) over the steps: a burst of copies stalls
    // the issuing wave, and with one wave per SIMD the MFMA pipe with it.
    // Each step is its own scheduling region laid out as (DS read, copy,
    // MFMA) groups.  Step 3 crosses into the next stage between its MFMAs:
    // wait for the next stage's copies (this wave's by vmcnt, everyone's by
    // the barrier, which also says every wave is done reading `cur`), then
    // read the next stage's step-0 operands from `nxt` before the last MFMAs.
    auto run_stage = [&](int kt, const uint8_t* cur, const uint8_t* nxt, uint8_t* prv, int u) {
#pragma unroll
        for (int s = 0; s < 3; ++s) {
            const int c = s & 1, n = c ^ 1;
            constexpr int kLo[4] = {0, C::P / 3, 2 * C::P / 3, C::P};
#pragma unroll
            for (int it = kLo[s]; it < kLo[s + 1]; ++it) issue_item(kt + NS - 1, prv, it, (u + NS - 1) % NS);
            read_ops(cur, s + 1, n, u);
            mfmas(c, 0, kNM);
            constexpr int kCp[3] = {kLo[1] - kLo[0], kLo[2] - kLo[1], kLo[3] - kLo[2]};
#pragma unroll
            for (int i = 0; i < kNM; ++i) {
                const int nr = kNR / kNM + (i < kNR % kNM ? 1 : 0);
                const int nc = kCp[s] / kNM + (i < kCp[s] % kNM ? 1 : 0);
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    if (r < nr) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);   // DS read
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    if (r < nc) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);   // copy
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                   // MFMA
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        mfmas(1, 0, (kNM + 1) / 2);
        __builtin_amdgcn_sched_barrier(0);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        wait_vmcnt<C::P * (NS - 2)>();
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        read_ops(nxt, 0, 0, (u + 1) % NS);
        mfmas(1, (kNM + 1) / 2, kNM);
        __builtin_amdgcn_sched_barrier(0);
    };

    // Stage kt lives in buffer kt % NS.  Prologue: stages 0 .. NS-2 (stage
    // NS-1 goes out during stage 0), then the first crossing.
#pragma unroll
    for (int d = 0; d < NS - 1; ++d) issue(d, bufs[d], d);
    // Weight prefetch.  The `rows` tiles of a tile column on one XCD read the
    // same weight lines in step with each other, so without it each line is
    // first asked for one ring depth ahead of its use and every stage waits
    // out an HBM miss (0.5 us per stage instead of 0.3 at K=1024, N=3584).
    // The ri-th of them asks now for stages NS - 1 + ri + f * rows (f < PF)
    // of its columns, into a sink nobody reads (together they cover stages
    // NS - 1 .. NS - 2 + PF * rows); when the loop gets there the lines are L2
    // hits.  (Asking two stages ahead of the ring instead, one line per wave
    // per stage, was too late: the misses take longer under this load.)  A
    // stage past the last asks for an offset past the buffer, which moves
    // nothing.  PF * PB copies per wave, always, so the vmcnt waits stay
    // exact.
#pragma unroll
    for (int f = 0; f < C::PF; ++f) {
        const int sp = NS - 1 + ri + f * rows;
        const uint32_t dead = static_cast<uint32_t>(sp >= KT) << 31;
        const int spc = sp < KT ? sp : KT - 1;
        if constexpr (WR) {
#pragma unroll
            for (int s = 0; s < 4; ++s)
#pragma unroll
                for (int jb = 0; jb < C::JB; ++jb)
                    dma16(wr, sink + wave * kLine, wq_off[jb] | dead, (spc * 8 + 2 * s) * kLine);
        } else {
#pragma unroll
            for (int j = 0; j < C::PB; ++j) dma16(wr, sink + wave * kLine, woff[j] | dead, spc * 8 * kLine);
        }
    }
    wait_vmcnt<C::P * (NS - 2) + C::PF * C::PFL>();
    __builtin_amdgcn_s_barrier();
    read_ops(bufs[0], 0, 0, 0);
    // Every stage runs the same body; the last ones copy the last stage
    // again and the last crossing reads operands that are never used.
    int kt = 0;
    for (; kt + NS <= KT; kt += NS) {
#pragma unroll
        for (int u = 0; u < NS; ++u) run_stage(kt + u, bufs[u], bufs[(u + 1) % NS], bufs[(u + NS - 1) % NS], u);
    }
    // (the tail leaves by `break`, so each tail stage is reached only from
    // the one before and the copy accounting stays exact)
#pragma unroll
    for (int u = 0; u < NS - 1; ++u) {
        if (kt + u >= KT) break;
        run_stage(kt + u, bufs[u], bufs[(u + 1) % NS], bufs[(u + NS - 1) % NS], u);
    }
    // no copy may land in LDS after the workgroup has left
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

    const int row_base = m0 + wm * WROWS;
    const int col_base = n0 + wn * WCOLS;
    if constexpr (!OUT_F16) {
        int32_t* o = static_cast<int32_t*>(out);
        const bool vec_ok = (N & 3) == 0 && (reinterpret_cast<uintptr_t>(out) & 15) == 0;
#pragma unroll
        for (int ib = 0; ib < C::IB; ++ib) {
            const int row = row_base + 32 * ib + (lane & 31);
            if (row >= M) continue;
#pragma unroll
            for (int jb = 0; jb < C::JB; ++jb)
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const int col = col_base + 32 * jb + 8 * g + 4 * h;
                    if (col >= N) continue;
                    int32_t* dst = o + static_cast<size_t>(row) * N + col;
                    if (vec_ok) {
                        *reinterpret_cast<int4_t*>(dst) = int4_t{acc[ib][jb][4 * g], acc[ib][jb][4 * g + 1],
                                                                 acc[ib][jb][4 * g + 2], acc[ib][jb][4 * g + 3]};
                    } else {
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            if (col + e < N) dst[e] = acc[ib][jb][4 * g + e];
                    }
                }
        }
    } else {
        float wsv[C::JB][4][4], xsv[C::IB];
#pragma unroll
        for (int jb = 0; jb < C::JB; ++jb)
#pragma unroll
            for (int g = 0; g < 4; ++g)
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    wsv[jb][g][e] = WS16 ? h2f(static_cast<uint16_t>(wraw[jb][g][e])) : __uint_as_float(wraw[jb][g][e]);
#pragma unroll
        for (int ib = 0; ib < C::IB; ++ib)
            xsv[ib] = XS16 ? h2f(static_cast<uint16_t>(xraw[ib])) : __uint_as_float(xraw[ib]);
        uint16_t* o = static_cast<uint16_t*>(out);
        const bool vec_ok = (N & 7) == 0 && (reinterpret_cast<uintptr_t>(out) & 15) == 0;
        auto deq = [&](int ib, int jb, int gg, int e) {
            return f2h(__fmul_rn(__fmul_rn(static_cast<float>(acc[ib][jb][4 * gg + e]), wsv[jb][gg][e]), xsv[ib]));
        };
        // 128 x 128 tiles (M=1024: 7.3 MB of output) stage it; 64 x 64 ones
        // (M=256) stayed 0.07 us faster with the direct stores below
        constexpr bool kStaged = BM * BN >= 128 * 128;
        if (kStaged && vec_ok) {
            // The wave's fp16 sub-tile goes through LDS (the stage buffers,
            // free once every wave is past the loop) so that each store
            // instruction writes whole 128-byte lines of output rows, with
            // non-temporal stores: full lines go to HBM while other tiles
            // still compute, and none wait in L2 for the end of the kernel.
            // Measured on MI355X (M=1024, K=1024, N=3584): 8.0-8.6 us per call
            // against 8.3-9.0 with the 16-byte-per-row stores straight from
            // registers; staged stores without the non-temporal hint 8.5;
            // non-temporal stores of the partial lines 11.2.
            if constexpr (WR) {
                // a wave's rows are only BN/4 columns wide: the whole tile
                // goes through LDS (row r in stage buffer r / RPA), then the
                // workgroup stores whole rows
                constexpr int RBT = BN * 2 + 16;                             // padded row bytes
                constexpr int RPA = C::STAGE / RBT < BM ? C::STAGE / RBT : BM;
                static_assert(RPA >= 8 && (BM + RPA - 1) / RPA <= NS, "epilogue staging space");
                auto srow = [&](int r) -> uint8_t* {
                    const int a = r / RPA;
                    return (a == 0 ? lds0 : a == 1 ? lds1 : a == 2 ? lds2 : lds3) + (r - a * RPA) * RBT;
                };
                __syncthreads();
#pragma unroll
                for (int ib = 0; ib < C::IB; ++ib)
#pragma unroll
                    for (int jb = 0; jb < C::JB; ++jb)
#pragma unroll
                        for (int g = 0; g < 4; g += 2) {
                            uint32_t p[4];
#pragma unroll
                            for (int d = 0; d < 2; ++d) {
                                const uint32_t x0 = deq(ib, jb, g, 2 * d) | (uint32_t(deq(ib, jb, g, 2 * d + 1)) << 16);
                                const uint32_t x1 =
                                    deq(ib, jb, g + 1, 2 * d) | (uint32_t(deq(ib, jb, g + 1, 2 * d + 1)) << 16);
                                const auto sw = __builtin_amdgcn_permlane32_swap(x0, x1, false, false);
                                p[d] = sw[0];
                                p[2 + d] = sw[1];
                            }
                            *reinterpret_cast<uint4*>(srow(32 * ib + (lane & 31)) +
                                                      (wn * WCOLS + 32 * jb + 8 * g + 8 * h) * 2) =
                                make_uint4(p[0], p[1], p[2], p[3]);
                        }
                __syncthreads();
                constexpr int CPR = BN / 8, RPI = 256 / CPR;            // 16-byte chunks per row, rows per pass
                static_assert(BM % RPI == 0, "row passes");
                const int cl = static_cast<int>(threadIdx.x) % CPR, rl = static_cast<int>(threadIdx.x) / CPR;
#pragma unroll
                for (int i = 0; i < BM / RPI; ++i) {
                    const int r = i * RPI + rl;
                    const int row = m0 + r, col = n0 + 8 * cl;
                    const uint4 v = *reinterpret_cast<const uint4*>(srow(r) + cl * 16);
                    if (row < M && col < N)
                        __builtin_nontemporal_store(int4_t{static_cast<int>(v.x), static_cast<int>(v.y),
                                                           static_cast<int>(v.z), static_cast<int>(v.w)},
                                                    reinterpret_cast<int4_t*>(o + static_cast<size_t>(row) * N + col));
                }
                return;
            } else {
                constexpr int SR = BM / 2, SC = BN / 2;
                constexpr int RB = SC * 2 + 16;                  // padded row bytes
                static_assert(((4 + NS - 1) / NS) * SR * RB <= C::STAGE, "epilogue staging space");
                const int wb = wave % NS;
                uint8_t* const st = (wb == 0 ? lds0 : wb == 1 ? lds1 : wb == 2 ? lds2 : lds3) + (wave / NS) * SR * RB;
                __syncthreads();
#pragma unroll
                for (int ib = 0; ib < C::IB; ++ib)
#pragma unroll
                    for (int jb = 0; jb < C::JB; ++jb)
#pragma unroll
                        for (int g = 0; g < 4; g += 2) {
                            uint32_t p[4];
#pragma unroll
                            for (int d = 0; d < 2; ++d) {
                                const uint32_t x0 = deq(ib, jb, g, 2 * d) | (uint32_t(deq(ib, jb, g, 2 * d + 1)) << 16);
                                const uint32_t x1 = deq(ib, jb, g + 1, 2 * d) | (uint32_t(deq(ib, jb, g + 1, 2 * d + 1)) << 16);
                                const auto sw = __builtin_amdgcn_permlane32_swap(x0, x1, false, false);
                                p[d] = sw[0];
                                p[2 + d] = sw[1];
                            }
                            *reinterpret_cast<uint4*>(st + (32 * ib + (lane & 31)) * RB + (32 * jb + 8 * g + 8 * h) * 2) =
                                make_uint4(p[0], p[1], p[2], p[3]);
                        }
                __syncthreads();
                constexpr int CPR = SC / 8, RPI = 64 / CPR;        // 16-byte chunks per row, rows per store
                const int cl = lane % CPR, rl = lane / CPR;
#pragma unroll
                for (int i = 0; i < SR / RPI; ++i) {
                    const int r = i * RPI + rl;
                    const int row = row_base + r, col = col_base + 8 * cl;
                    const uint4 v = *reinterpret_cast<const uint4*>(st + r * RB + cl * 16);
                    if (row < M && col < N)
                        __builtin_nontemporal_store(int4_t{static_cast<int>(v.x), static_cast<int>(v.y),
                                                           static_cast<int>(v.z), static_cast<int>(v.w)},
                                                    reinterpret_cast<int4_t*>(o + static_cast<size_t>(row) * N + col));
                }
                return;
            }
        }
        // 16-byte stores straight from registers: lane l holds 8 consecutive
        // columns of one row after one v_permlane32_swap per register pair;
        // element stores when N is not a multiple of 8 (or the output is
        // unaligned)
#pragma unroll
        for (int ib = 0; ib < C::IB; ++ib) {
            const int row = row_base + 32 * ib + (lane & 31);
#pragma unroll
            for (int jb = 0; jb < C::JB; ++jb) {
                if (vec_ok) {
#pragma unroll
                    for (int g = 0; g < 4; g += 2) {
                        uint32_t p[4];
#pragma unroll
                        for (int d = 0; d < 2; ++d) {
                            const uint32_t x0 = deq(ib, jb, g, 2 * d) | (uint32_t(deq(ib, jb, g, 2 * d + 1)) << 16);
                            const uint32_t x1 = deq(ib, jb, g + 1, 2 * d) | (uint32_t(deq(ib, jb, g + 1, 2 * d + 1)) << 16);
                            const auto sw = __builtin_amdgcn_permlane32_swap(x0, x1, false, false);
                            p[d] = sw[0];
                            p[2 + d] = sw[1];
                        }
                        const int col = col_base + 32 * jb + 8 * g + 8 * h;
                        if (row < M && col < N)
                            *reinterpret_cast<uint4*>(o + static_cast<size_t>(row) * N + col) =
                                make_uint4(p[0], p[1], p[2], p[3]);
                    }
                } else {
#pragma unroll
                    for (int g = 0; g < 4; ++g) {
                        const int col = col_base + 32 * jb + 8 * g + 4 * h;
                        if (row >= M) continue;
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            if (col + e < N) o[static_cast<size_t>(row) * N + col + e] = deq(ib, jb, g, e);
                    }
                }
            }
        }
    }
}

struct ShapeL {
    int bm, bn, ns;
    int wr = 0;
};

using GemmLFn = void (*)(const int8_t*, const int8_t*, int, int, int, int, void*, const void*, const void*, int, int,
                         int, int, int);

template <int EPI>
GemmLFn pick_epi(const ShapeL& s) {
#define MCV_L(BM_, BN_, NS_, WR_) \
    if (s.bm == BM_ && s.bn == BN_ && s.ns == NS_ && s.wr == WR_) return w8a8_gemm_lds_kernel<BM_, BN_, NS_, EPI, WR_>;
    MCV_L(128, 128, 3, 0) MCV_L(128, 128, 4, 0) MCV_L(64, 128, 4, 0) MCV_L(128, 64, 4, 0) MCV_L(64, 64, 4, 0)
    MCV_L(64, 64, 3, 0) MCV_L(128, 128, 3, 1) MCV_L(128, 128, 4, 1) MCV_L(64, 128, 4, 1)
#undef MCV_L
    return nullptr;
}

GemmLFn pick_l(const ShapeL& s, int epi) {
    switch (epi) {
        case 4: return pick_epi<4>(s);
        case 5: return pick_epi<5>(s);
        case 6: return pick_epi<6>(s);
        case 7: return pick_epi<7>(s);
        default: return pick_epi<0>(s);
    }
}

// Largest tiles first; the first shape whose grid covers most of the 256
// CUs, else the one with the most workgroups.  Measured on MI355X (K=1024,
// N=3584, 160 rotated weight sets, back to back, two passes of three timed
// regions): M=1024 128x128 with 3 stages and the weights in registers 7.85-7.90
// us (through LDS 7.91-7.95, 4 stages 8.26-8.37, 64x128 10.4-11.1, 64x64
// 11.9-12.2); M=256 64x64 4.72-4.75 us (64x128 6.0-6.15, 128x128 7.4-7.8),
// and with 3 stages 4.66-4.68 us (2 stages 5.38-5.43; 32x128 with the
// weights in registers 4.90-4.93 with 3 stages, 5.31-5.34 with 4).
ShapeL choose_l(int64_t M, int64_t N) {
    constexpr ShapeL kOrder[] = {{128, 128, 3, 1}, {64, 128, 4, 1}, {64, 64, 3, 0}};
    ShapeL best = kOrder[0];
    int64_t best_t = -1;
    for (const ShapeL& s : kOrder) {
        const int64_t t = ceil_div(M, s.bm) * ceil_div(N, s.bn);
        if (t >= 200) return s;
        if (t > best_t) {
            best_t = t;
            best = s;
        }
    }
    return best;
}

}  // namespace

// The kernel launch_w8a8_gemm_lds picks for M x N, as text (report labels).
std::string w8a8_gemm_lds_name(int64_t M, int64_t N, bool f16) {
    const ShapeL s = choose_l(M, N);
    char buf[128];
    // EPI as launched with fp32 scales (fp16 ones add 1 and 2)
    std::snprintf(buf, sizeof(buf), "w8a8_gemm_lds_kernel<%d, %d, %d, %d, %d> (%s, %lld workgroups)", s.bm, s.bn,
                  s.ns, f16 ? 4 : 0, s.wr, f16 ? "fused fp16 epilogue" : "int32 out",
                  (long long)(ceil_div(M, s.bm) * ceil_div(N, s.bn)));
    return buf;
}

namespace {

// xq [M][K] int8 (K % 16 == 0), w tiled; out int32 or fp16 [M][N], tile
// shape s.  Shapes were validated by the caller.
int launch_w8a8_gemm_lds_shape(const int8_t* xq, int64_t M, int64_t K, int64_t N, const int8_t* w, void* out, bool f16,
                               const void* xs, int xs16, const void* ws, int ws16, const ShapeL& s, hipStream_t stream) {
    const int64_t nslab = ceil_div(N, kSlab);
    const int64_t KB = ceil_div(K, 128) * 4;
    // (bit 31 of a weight offset marks a prefetch with nothing to fetch)
    if (nslab * KB * 2 * kLine >= (int64_t(1) << 31) || M * K >= (int64_t(1) << 32))
        return fail(MCV_ERR_SHAPE, "w8a8 GEMM: weight exceeds 2 GiB or activation 4 GiB");
    const int epi = f16 ? 4 | (xs16 ? 1 : 0) | (ws16 ? 2 : 0) : 0;
    const GemmLFn fn = pick_l(s, epi);
    if (fn == nullptr)
        return fail(MCV_ERR_INVALID_ARG, "w8a8 GEMM: no kernel for %d x %d tiles, %d stages, weights in registers %d",
                    s.bm, s.bn, s.ns, s.wr);
    const int64_t n_tiles = ceil_div(N, s.bn);
    const int64_t total = ceil_div(M, s.bm) * n_tiles;
    if (total > 0x7fffffff) return fail(MCV_ERR_SHAPE, "w8a8 GEMM: too many tiles");
    const int KT = static_cast<int>(KB / 4);
    // Tile order: a contiguous run of tiles per XCD, down the tile columns.
    // Cutting the grid into one 2-D block per XCD (the kernel's xcd_m > 0)
    // halves the x bytes each L2 sees but doubles the weight columns, which
    // come from HBM: slower at M = 1024 (8.7 against 8.4 us).
    const int xcd_m = 0;
    hipLaunchKernelGGL(fn, dim3(static_cast<unsigned>(total)),
                       dim3(256), 0, stream, xq, w, static_cast<int>(M), static_cast<int>(K), static_cast<int>(N),
                       static_cast<int>(KB), out, xs, ws, static_cast<int>(nslab), static_cast<int>(n_tiles),
                       static_cast<int>(total), KT, xcd_m);
    return check_launch("w8a8_gemm_lds_kernel");
}

}  // namespace

// As above with the dispatch's tile shape (choose_l).
int launch_w8a8_gemm_lds(const int8_t* xq, int64_t M, int64_t K, int64_t N, const int8_t* w, void* out, bool f16,
                         const void* xs, int xs16, const void* ws, int ws16, hipStream_t stream) {
    return launch_w8a8_gemm_lds_shape(xq, M, K, N, w, out, f16, xs, xs16, ws, ws16, choose_l(M, N), stream);
}

// Any built tile shape (tests and tuning; mcv_w8a8_gemm_lds).
int launch_w8a8_gemm_lds_cfg(const int8_t* xq, int64_t M, int64_t K, int64_t N, const int8_t* w, void* out, bool f16,
                             const void* xs, int xs16, const void* ws, int ws16, int bm, int bn, int ns, int wr,
                             hipStream_t stream) {
    ShapeL s{bm, bn, ns};
    s.wr = wr;
    return launch_w8a8_gemm_lds_shape(xq, M, K, N, w, out, f16, xs, xs16, ws, ws16, s, stream);
}

}  // namespace mcv
