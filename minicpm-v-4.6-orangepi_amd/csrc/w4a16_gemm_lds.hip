// w4a16_gemm_lds.hip -- W4A16 prefill GEMM (M > 1) on fp16 MFMA with both
// operands staged through LDS by gfx950's direct-to-LDS copies.
//
// out[M][N] = x[M][K] . W[K][N], W in the slab-64 int4 layout, fp32
// accumulation, fp16 RNE output.
//
// Workgroup: 4 waves, tile TM rows x 4 slabs (256 columns); wave w owns slab
// w of the tile over all TM rows: TM/32 x 2 blocks of
// v_mfma_f32_32x32x16_f16.  K advances in stages of 128 (one quantisation
// group, so a wave's scales and zeros are constant over a stage).  With
// KP = 2 the waves are 2 k-parts x 2 slabs (128-column tiles, twice the
// workgroups): a stage holds two groups, k-part p computes the p-th, and
// k-part 1 hands its partial tile to k-part 0 through LDS at the end.  Per
// stage:
//   - x rows (TM x 256 bytes) are copied global -> LDS with
//     buffer_load_dwordx4 ... lds, 4 rows per wave-wide 1 KiB copy; the
//     16-byte chunk index is XORed with the row's low 4 bits (by choosing
//     which global chunk each lane fetches), so the operand reads of 16 rows
//     at one k offset (one ds_read_b128 pass) cover all 64 banks.  Rows past
//     M read as zero.
//   - each wave copies its own slab's 4 packed chunks (32 k x 64 columns,
//     1 KiB each, contiguous in the slab layout) into LDS verbatim, and the
//     slab's zero and scale words of the group.
//   The copies of stage kt + NS - 1 are spread over the k16 steps of stage
//   kt, two or so per step: a burst of them stalls the issuing wave, and with
//   one wave per SIMD that idles the MFMA pipe.  Each lane's offset inside a
//   stage is fixed; the stage's advance rides in the scalar offset.
// Compute: per k16 step a wave reads TM/32 x-operands (one ds_read_b128 each)
// and turns one pair of packed words into the two 32-column weight operands:
// one v_permlane32_swap re-lanes lane-per-column words into the MFMA operand
// order (lanes 0-31 / 32-63 carry k-octets 0 / 1 of the same 32 columns),
// then (1024 + q) - (1024 + z) (exact, fp16 exponent trick) times the scale
// (one RNE) -- the same fp16 values mcv_w4a16_dequant materialises.  Step
// s+1's operands are produced while step s's MFMAs run.  One barrier per
// stage, placed between the MFMAs of the last step, after the explicit
// vmcnt wait that is the only wait on the copies (each stage is its own
// __shared__ array, indexed by compile-time constants, so the waitcnt pass
// keeps the other stages' copies in flight); the next stage's weights,
// zeros, scales and first x operands are read before the last MFMAs issue.
// The MFMA computes the transposed tile, so the epilogue writes 16 bytes per
// lane after one v_permlane32_swap per pair.
//
// What bounds it (MI355X, measured): the widening is ~31 VALU instructions
// per k16 step per wave (4 cycles each on a wave64) against 2 x TM/32 MFMAs
// of 32 cycles; about four VALU instructions hide under one MFMA, so 128-row
// tiles run near the MFMA rate and 32-row tiles are VALU-bound.  The copies
// themselves cost little once spread (0.6 us of 20 at M=2048 K=1024).
//
// The reference has no M > 1 quantised path: its prefill runs dense fp16
// aclnnMm through matmul_b_transposed (src/csrc/lib/decoder_layer.cpp:459-462,
// 656-659, 857-860; src/csrc/lib/ops.cpp:159-322).
#include <cstdlib>

#include "common.h"

namespace mcv {
namespace {

constexpr int kLineW = 1024;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc_w(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, static_cast<int>(bytes), 0x00020000);
}

// Direct global -> LDS copies of 16 / 4 bytes per lane at voff + soff.
__device__ __forceinline__ void dma16_w(__amdgpu_buffer_rsrc_t r, uint8_t* lds, uint32_t voff, int soff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, lds, 16, voff, soff, 0, 0);
}

__device__ __forceinline__ void dma4_w(__amdgpu_buffer_rsrc_t r, uint8_t* lds, uint32_t voff, int soff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, lds, 4, voff, soff, 0, 0);
}

template <int N>
__device__ __forceinline__ void wait_vmcnt_w() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

__device__ __forceinline__ int xcd_tile_w(int b, int total) {
    const int per = total >> 3, rem = total & 7, x = b & 7, i = b >> 3;
    return x * per + (x < rem ? x : rem) + i;
}

// TM rows per tile, NS stages in flight, KP k-parts: the four waves are KP
// k-parts x WN = 4 / KP slabs, and a stage covers KP quantisation groups,
// k-part p taking the p-th.
template <int TM, int NS, int KP>
struct CfgW {
    static constexpr int WN = 4 / KP;                      // slabs per tile
    static constexpr int BK = 128;                         // k per k-part per stage: one quantisation group
    static constexpr int ROW = BK * 2;                     // bytes of one x row per k-part per stage
    static constexpr int A_BYTES = KP * TM * ROW;          // x blocks of the KP k-parts
    static constexpr int B_BYTES = 4 * 4 * kLineW;         // each wave's 4 packed chunks
    static constexpr int ZS_BYTES = 4 * 512;               // per wave: 64 zero dwords, 64 scale dwords
    static constexpr int STAGE = A_BYTES + B_BYTES + ZS_BYTES;
    static constexpr int A_COPIES = A_BYTES / kLineW;      // 4 rows per copy
    static_assert(A_COPIES % 4 == 0, "x copies split over four waves");
    static constexpr int PA = A_COPIES / 4;
    static constexpr int PB = 4;                           // the wave's own slab chunks
    static constexpr int PS = 2;                           // zero and scale words
    static constexpr int P = PA + PB + PS;                 // vector-memory ops per wave per stage
    static constexpr int MB = TM / 32;
    static_assert(TM == 32 || TM == 64 || TM == 128, "TM");
    static_assert(KP == 1 || KP == 2, "KP");
    static_assert(NS >= 2 && NS <= 4 && P * (NS - 1) < 64, "stages");
    static_assert(NS * STAGE <= 160 * 1024, "LDS");
    static_assert(KP == 1 || WN * MB * 2 * 16 * 64 * 4 <= STAGE, "k-part reduction buffer");
};

template <int TM, int NS, int KP>
__global__ __launch_bounds__(256) void w4a16_gemm_lds_kernel(
    const uint16_t* __restrict__ x, const uint4* __restrict__ qw, const uint16_t* __restrict__ scales,
    const uint32_t* __restrict__ zeros, uint32_t zero_bias, uint16_t* __restrict__ out, int M, int K, int N,
    int nslab, int n_tiles, int total_tiles, int col_major, int xcd_m) {
    using C = CfgW<TM, NS, KP>;
    __shared__ __attribute__((aligned(1024))) uint8_t lds0[C::STAGE];
    __shared__ __attribute__((aligned(1024))) uint8_t lds1[C::STAGE];
    __shared__ __attribute__((aligned(1024))) uint8_t lds2[NS > 2 ? C::STAGE : 16];
    __shared__ __attribute__((aligned(1024))) uint8_t lds3[NS > 3 ? C::STAGE : 16];
    uint8_t* const bufs[4] = {lds0, lds1, lds2, lds3};

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int h = lane >> 5;
    // Workgroup b runs on XCD b % 8.  With xcd_m > 0 the tile grid is cut
    // into xcd_m x (8 / xcd_m) blocks, one per XCD, so each XCD's L2 sees
    // only its block's x rows and weight slabs; otherwise each XCD gets a
    // contiguous run of tiles, down the tile columns (col_major: an XCD holds
    // a few weight slabs, x rows cross XCDs) or along the rows.
    const int m_tiles = total_tiles / n_tiles;
    int tm, tn;
    if (xcd_m > 0) {
        const int xb_n = 8 / xcd_m, mr = m_tiles / xcd_m, nr = n_tiles / xb_n;
        const int xcd = static_cast<int>(blockIdx.x) & 7, i = static_cast<int>(blockIdx.x) >> 3;
        tm = (xcd / xb_n) * mr + i % mr;
        tn = (xcd % xb_n) * nr + i / mr;
    } else {
        const int tile = xcd_tile_w(static_cast<int>(blockIdx.x), total_tiles);
        tm = col_major ? tile % m_tiles : tile / n_tiles;
        tn = col_major ? tile / m_tiles : tile - tm * n_tiles;
    }
    const int m0 = tm * TM;
    const int kp = wave / C::WN;                           // k-part of this wave
    const int slab = tn * C::WN + (wave - kp * C::WN);
    const int Npad = nslab * kSlab;
    const int CK = K / kChunkK;
    const int KT = K / (C::BK * KP);                       // stages

    const int rows_here = M - m0 < TM ? M - m0 : TM;
    const __amdgpu_buffer_rsrc_t xr =
        rsrc_w(x + static_cast<size_t>(m0) * K, static_cast<uint32_t>(rows_here) * K * 2u);
    // a slab past the end reads as zero weights; its scale and zero words are
    // read as zero too (its columns are never stored)
    const __amdgpu_buffer_rsrc_t qr = rsrc_w(qw, static_cast<uint32_t>(nslab) * CK * kSlab * 16u);
    const __amdgpu_buffer_rsrc_t sr = rsrc_w(scales, static_cast<uint32_t>(K / kGroup) * Npad * 2u);
    const __amdgpu_buffer_rsrc_t zr = rsrc_w(zeros, static_cast<uint32_t>(K / kGroup) * (Npad >> 3) * 4u);
    const uint32_t qoff = static_cast<uint32_t>(slab) * CK * kSlab * 16u + lane * 16u;

    // The stage's vector-memory ops of this wave, all copies into LDS: x
    // rows, its slab's packed chunks, and the slab's group zero words (lanes
    // 0-7) and scales (lanes 0-31, two per dword).  Each lane's offset inside
    // a stage is fixed (computed once here); the stage's advance goes into
    // the scalar offset, so a copy costs no VALU work.  Stages past the last
    // re-read the last stage into a buffer that is never read again: every
    // stage issues the same P ops (the waits stay exact) and every access
    // stays inside its buffer.  Lanes with nothing to fetch get bit 31 set,
    // past the end of every buffer (all are below 2 GiB): they copy zeros.
    uint32_t xoff[C::PA];
#pragma unroll
    for (int j = 0; j < C::PA; ++j) {
        const int i = wave * C::PA + j;                    // copy i: k-part block i / (TM/4), 4 rows
        const int kb = i / (TM / 4);
        const int row = 4 * (i - kb * (TM / 4)) + (lane >> 4);
        xoff[j] = static_cast<uint32_t>(row * K + kb * C::BK) * 2u +
                  static_cast<uint32_t>((lane & 15) ^ (row & 15)) * 16u;
    }
    // The buffer range check covers the vector offset only (the group's
    // stride rides in the scalar offset), so a padding slab past nslab -- the
    // last tile's when nslab % WN != 0 -- must put its copies out of range by
    // the vector offset alone, like the idle lanes.
    const bool slab_live = slab < nslab;
    const uint32_t zoff =
        (static_cast<uint32_t>(slab) * 32u + lane * 4u) | (lane < 8 && slab_live ? 0u : 0x80000000u);
    const uint32_t soff =
        (static_cast<uint32_t>(slab) * 128u + lane * 4u) | (lane < 32 && slab_live ? 0u : 0x80000000u);
    // Copy `it` (0 .. P-1: x rows, packed chunks, zero words, scales) of
    // stage kt into dst.
    auto issue_item = [&](int kt, uint8_t* dst, int it) {
        const int kc = kt < KT ? kt : KT - 1;
        const int g = kc * KP + kp;                        // this wave's quantisation group
        if (it < C::PA) {
            dma16_w(xr, dst + (wave * C::PA + it) * kLineW, xoff[it], kc * KP * C::ROW);
        } else if (it < C::PA + C::PB) {
            const int c = it - C::PA;
            dma16_w(qr, dst + C::A_BYTES + (wave * 4 + c) * kLineW, qoff, (g * 4 + c) * kSlab * 16);
        } else if (it == C::PA + C::PB) {
            dma4_w(zr, dst + C::A_BYTES + C::B_BYTES + wave * 512, zoff, g * (Npad >> 3) * 4);
        } else {
            dma4_w(sr, dst + C::A_BYTES + C::B_BYTES + wave * 512 + 256, soff, g * Npad * 2);
        }
    };
    auto issue = [&](int kt, uint8_t* dst) {
#pragma unroll
        for (int it = 0; it < C::P; ++it) issue_item(kt, dst, it);
    };

    uint32_t vmagic;
    asm("v_mov_b32 %0, 0x64006400" : "=v"(vmagic));
    const uint32_t mlo = __builtin_amdgcn_readfirstlane(0x000F000Fu);
    const uint32_t zsh = (lane & 7) * 4;                   // c0 & 7 == c1 & 7 == lane & 7

    float16_t acc[C::MB][2];
#pragma unroll
    for (int i = 0; i < C::MB; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    // x operand of k16 step s, block i: row 32 i + l%32, 16-byte chunk
    // 2 s + l/32, XOR-swizzled by the row's low 4 bits (= l & 15); block i is
    // a constant 8 KiB further.
    int a_off[8];
#pragma unroll
    for (int s = 0; s < 8; ++s)
        a_off[s] = kp * TM * C::ROW + (lane & 31) * C::ROW + (((2 * s + h) ^ (lane & 15)) << 4);
    const int b_off = C::A_BYTES + wave * 4 * kLineW + lane * 16;
    const int z_off = C::A_BYTES + C::B_BYTES + wave * 512 + ((lane & 31) >> 3) * 4;
    const int s_off = C::A_BYTES + C::B_BYTES + wave * 512 + 256 + (lane & 31) * 2;

    // Operand state of the stage being computed: its packed chunks, the
    // zero and scale constants of the two operand columns, and double-
    // buffered x / weight operands (step s uses set s & 1).
    uint4 q[4];
    uint32_t zz0 = 0, zz1 = 0, ss0 = 0, ss1 = 0;
    half8_t af[2][C::MB], bf[2][2];
    auto widen = [&](int s, half8_t& b0, half8_t& b1) {
        const uint4& qc = q[s >> 1];
        const uint32_t w0 = (s & 1) ? qc.z : qc.x, w1 = (s & 1) ? qc.w : qc.y;
        // lanes 32-63 of octet 2t <-> lanes 0-31 of octet 2t+1
        const auto sw = __builtin_amdgcn_permlane32_swap(w0, w1, false, false);
        dequant_pair(sw[0], sw[1], zz0, ss0, zz1, ss1, mlo, vmagic, b0, b1);
    };
    auto read_a = [&](const uint8_t* src, int s, half8_t* dst) {
#pragma unroll
        for (int i = 0; i < C::MB; ++i) dst[i] = *reinterpret_cast<const half8_t*>(src + a_off[s] + i * 32 * C::ROW);
    };
    // A stage's LDS reads: weights, zero and scale words, step 0's x.
    auto head = [&](const uint8_t* src) {
#pragma unroll
        for (int c = 0; c < 4; ++c) q[c] = *reinterpret_cast<const uint4*>(src + b_off + c * kLineW);
        const uint32_t zw0 = *reinterpret_cast<const uint32_t*>(src + z_off);
        const uint32_t zw1 = *reinterpret_cast<const uint32_t*>(src + z_off + 16);
        const uint32_t sh0 = *reinterpret_cast<const uint16_t*>(src + s_off);
        const uint32_t sh1 = *reinterpret_cast<const uint16_t*>(src + s_off + 64);
        read_a(src, 0, af[0]);
        // zz = half2(1024 + z), ss = half2(s) of the two operand columns
        zz0 = (0x6400u + ((zw0 >> zsh) & 15u) + zero_bias) * 0x10001u;
        zz1 = (0x6400u + ((zw1 >> zsh) & 15u) + zero_bias) * 0x10001u;
        ss0 = sh0 * 0x10001u;
        ss1 = sh1 * 0x10001u;
    };
    constexpr int kNM = 2 * C::MB;                         // MFMAs per k16 step
    auto mfmas = [&](int cur, int lo, int hi) {
#pragma unroll
        for (int m = lo; m < hi; ++m) {
            const int i = m >> 1, j = m & 1;
            // weights as the row operand: the transposed 32x32 tile
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(bf[cur][j], af[cur][i], acc[i][j], 0, 0, 0);
        }
    };
    constexpr int kValuPerMfma = (31 + kNM - 1) / kNM;     // widening VALU ops per step: 31

    // One stage from `cur`.  Steps 0-6 produce step s+1's operands (LDS
    // reads, permlane + widening) while step s's MFMAs run, and spread the
    // copies of stage kt + NS - 1 into `prv` (free since the last barrier)
    // over the steps, a few per step: a burst of copies would stall this
    // wave's issue, and with it the MFMA pipe.  Each step is its own
    // scheduling region laid out as (DS read, copy, MFMA, VALU run) groups.
    // Step 7 crosses into the next stage between its MFMAs: wait for the next
    // stage's copies, barrier (every wave is also done reading `cur`), read
    // the next stage's head from `nxt`; the widening of the next step 0
    // follows the last MFMA.
    auto run_stage = [&](int kt, const uint8_t* cur, const uint8_t* nxt, uint8_t* prv) {
#pragma unroll
        for (int s = 0; s < 7; ++s) {
            const int c = s & 1, n = c ^ 1;
            constexpr int kLo[8] = {0, C::P * 1 / 7, C::P * 2 / 7, C::P * 3 / 7, C::P * 4 / 7, C::P * 5 / 7,
                                    C::P * 6 / 7, C::P};
#pragma unroll
            for (int it = kLo[s]; it < kLo[s + 1]; ++it) issue_item(kt + NS - 1, prv, it);
            read_a(cur, s + 1, af[n]);
            widen(s + 1, bf[n][0], bf[n][1]);
            mfmas(c, 0, kNM);
#pragma unroll
            for (int i = 0; i < kNM; ++i) {
                if (i < C::MB) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);   // DS read
                if (i < kLo[s + 1] - kLo[s]) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);   // copy
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                  // MFMA
                __builtin_amdgcn_sched_group_barrier(0x002, kValuPerMfma, 0);       // VALU
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        mfmas(1, 0, (kNM + 1) / 2);
        __builtin_amdgcn_sched_barrier(0);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        wait_vmcnt_w<C::P * (NS - 2)>();
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        head(nxt);
        mfmas(1, (kNM + 1) / 2, kNM);
        __builtin_amdgcn_sched_barrier(0);
        widen(0, bf[0][0], bf[0][1]);
    };

    // Prologue: stages 0 .. NS-2; stage NS-1 goes out during stage 0.
#pragma unroll
    for (int d = 0; d < NS - 1; ++d) issue(d, bufs[d]);
    wait_vmcnt_w<C::P * (NS - 2)>();
    __builtin_amdgcn_s_barrier();
    head(bufs[0]);
    widen(0, bf[0][0], bf[0][1]);
    // Every stage runs the same body; the last ones copy nothing (stage >=
    // KT) and the last crossing reads a stale head that is never used.
    int kt = 0;
    for (; kt + NS <= KT; kt += NS) {
#pragma unroll
        for (int u = 0; u < NS; ++u) run_stage(kt + u, bufs[u], bufs[(u + 1) % NS], bufs[(u + NS - 1) % NS]);
    }
    // (the tail leaves by `break`, so each tail stage is reached only from
    // the one before and the copy accounting stays exact)
#pragma unroll
    for (int u = 0; u < NS - 1; ++u) {
        if (kt + u >= KT) break;
        run_stage(kt + u, bufs[u], bufs[(u + 1) % NS], bufs[(u + NS - 1) % NS]);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

    // k-part 1 hands its partial tile to k-part 0 through LDS (the stage
    // buffers are free once every wave is past the loop); fp32 adds, in the
    // same order for every element.
    if constexpr (KP == 2) {
        float* red = reinterpret_cast<float*>(lds0) + lane;
        const int wn = wave - kp * C::WN;
        __syncthreads();
        if (kp == 1) {
#pragma unroll
            for (int i = 0; i < C::MB; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
#pragma unroll
                    for (int r = 0; r < 16; ++r) red[(((wn * C::MB + i) * 2 + j) * 16 + r) * 64] = acc[i][j][r];
        }
        __syncthreads();
        if (kp == 1) return;
#pragma unroll
        for (int i = 0; i < C::MB; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[i][j][r] += red[(((wn * C::MB + i) * 2 + j) * 16 + r) * 64];
    }

    // Transposed 32x32 blocks: register r of lane l holds output row
    // 32 i + l%32 and column 32 j + 8 (r/4) + 4 (l/32) + r%4.  Swapping the
    // upper lanes of quad g with the lower lanes of quad g+1 leaves lane l with
    // the 8 consecutive columns 32 j + 8 g + 8 (l/32), g even: one 16-byte store.
    const bool vec_ok = (N & 7) == 0 && (reinterpret_cast<uintptr_t>(out) & 15) == 0;
    auto pack = [&](int i, int j, int g, uint32_t (&p)[4]) {
#pragma unroll
        for (int d = 0; d < 2; ++d) {
            const uint32_t x0 = f2h(acc[i][j][4 * g + 2 * d]) | (uint32_t(f2h(acc[i][j][4 * g + 2 * d + 1])) << 16);
            const uint32_t x1 = f2h(acc[i][j][4 * g + 4 + 2 * d]) | (uint32_t(f2h(acc[i][j][4 * g + 5 + 2 * d])) << 16);
            const auto sw = __builtin_amdgcn_permlane32_swap(x0, x1, false, false);
            p[d] = sw[0];
            p[2 + d] = sw[1];
        }
    };
    if (vec_ok) {
        // The wave's TM x 64 fp16 block goes through LDS so that each store
        // instruction writes whole 128-byte lines of output rows, with
        // non-temporal stores: full lines go to HBM while other tiles still
        // compute, and none wait in L2 for the end of the kernel (MI355X,
        // M=2048 K=1024 N=3584: 20.8-21.2 against 21.2-22.0 us with 16 bytes
        // per row per store straight from registers; the two-k-part shapes
        // measured the same either way).  One k-part:
        // the stage buffers, after a barrier (every wave past the loop).  Two
        // k-parts: lds1, untouched since the reduction's first barrier (the
        // waves of k-part 1 have left, so there is no second barrier).
        constexpr int RB = kSlab * 2 + 16;                 // padded row bytes
        constexpr int REGION = TM * RB;
        static_assert(KP == 1 ? ((4 + NS - 1) / NS) * REGION <= C::STAGE : C::WN * REGION <= C::STAGE,
                      "epilogue staging space");
        uint8_t* st;
        if constexpr (KP == 1) {
            __syncthreads();
            const int wb = wave % NS;
            st = (wb == 0 ? lds0 : wb == 1 ? lds1 : wb == 2 ? lds2 : lds3) + (wave / NS) * REGION;
        } else {
            st = lds1 + (wave - kp * C::WN) * REGION;
        }
#pragma unroll
        for (int i = 0; i < C::MB; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int g = 0; g < 4; g += 2) {
                    uint32_t p[4];
                    pack(i, j, g, p);
                    *reinterpret_cast<uint4*>(st + (32 * i + (lane & 31)) * RB + (32 * j + 8 * g + 8 * h) * 2) =
                        make_uint4(p[0], p[1], p[2], p[3]);
                }
        // the wave reads back only its own block: its LDS writes are done
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
        for (int it = 0; it < TM / 8; ++it) {
            const int r = it * 8 + (lane >> 3);
            const int row = m0 + r, col = slab * kSlab + 8 * (lane & 7);
            const uint4 v = *reinterpret_cast<const uint4*>(st + r * RB + (lane & 7) * 16);
            if (row < M && col < N)
                __builtin_nontemporal_store(int4_t{static_cast<int>(v.x), static_cast<int>(v.y), static_cast<int>(v.z),
                                                   static_cast<int>(v.w)},
                                            reinterpret_cast<int4_t*>(out + static_cast<size_t>(row) * N + col));
        }
        return;
    }
    // N not a multiple of 8 (or an unaligned output): element stores
#pragma unroll
    for (int i = 0; i < C::MB; ++i) {
        const int row = m0 + 32 * i + (lane & 31);
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int g = 0; g < 4; g += 2) {
                uint32_t p[4];
                pack(i, j, g, p);
                const int col = slab * kSlab + 32 * j + 8 * g + 8 * h;
                if (row >= M || col >= N) continue;
                uint16_t* dst = out + static_cast<size_t>(row) * N + col;
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    if (col + e < N) dst[e] = static_cast<uint16_t>(p[e >> 1] >> (16 * (e & 1)));
            }
    }
}

struct ShapeW {
    int tm, ns, kp;
};

using GemmWFn = void (*)(const uint16_t*, const uint4*, const uint16_t*, const uint32_t*, uint32_t, uint16_t*, int,
                         int, int, int, int, int, int, int);

GemmWFn pick_w(const ShapeW& s) {
#define MCV_W(TM_, NS_, KP_) \
    if (s.tm == TM_ && s.ns == NS_ && s.kp == KP_) return w4a16_gemm_lds_kernel<TM_, NS_, KP_>;
    MCV_W(128, 2, 1) MCV_W(128, 3, 1) MCV_W(64, 2, 1) MCV_W(64, 3, 1) MCV_W(32, 3, 1) MCV_W(64, 2, 2) MCV_W(64, 3, 2)
    MCV_W(32, 3, 2)
#undef MCV_W
    return nullptr;
}

}  // namespace

// The LDS kernel's shape for M x K x N, or -1 when the register-staged
// kernel is the better choice.  Measured on MI355X (graph-replayed, 300
// rotated weight sets of random data, microseconds per call; register-staged
// kernel in brackets): M=2048 K=1024 N=3584 TM=128 22.5 (26.6); M=1024
// K=1024 N=3584 TM=64 14.7 (17.9); M=512 K=1024 N=3584 TM=32 11.7 (12.0).
// With 32-row tiles each widened weight operand feeds only two MFMAs and the
// VALU work (about 31 instructions per k16 step) dominates; with N=1024 the
// grid is too small for tall single-k-part tiles, so 64-row tiles split K
// over two k-parts of two waves (KP=2, 128-column tiles): M=2048 K=3584
// N=1024 24.0 (30.7), M=512 K=1024 N=3584 9.8 (12.1).  Three stages in
// flight: with two, the copies of stage kt + 1 go out during stage kt and the
// last of them has a k16 step or two to land before the next barrier waits
// for it (M=1024: 15.4 against 14.7 us; M=2048 K=1024: equal with random
// data, 1 us slower with constant data).  So: the first of 128-row, 64-row,
// 64-row-two-k-parts tiles whose grid still covers most of the 256 CUs, else
// -1, except at a short K (below).  MCV_W4LDS_SHAPE="TM,NS,KP" forces a
// shape (read once per process; tuning sweeps).
int choose_w4a16_lds(int64_t M, int64_t K, int64_t N, int* tm, int* ns, int* kp) {
    static const char* const e = std::getenv("MCV_W4LDS_SHAPE");
    ShapeW s{0, 0, 1};
    if (e != nullptr && std::sscanf(e, "%d,%d,%d", &s.tm, &s.ns, &s.kp) >= 2 && pick_w(s) &&
        K % (int64_t(kGroup) * s.kp) == 0) {
        *tm = s.tm;
        *ns = s.ns;
        *kp = s.kp;
        return 0;
    }
    constexpr ShapeW kOrder[] = {{128, 3, 1}, {64, 3, 1}, {64, 3, 2}};
    for (const ShapeW& c : kOrder) {
        if (K % (int64_t(kGroup) * c.kp) != 0) continue;
        if (ceil_div(M, c.tm) * ceil_div(ceil_div(N, kSlab), 4 / c.kp) >= 200) {
            *tm = c.tm;
            *ns = c.ns;
            *kp = c.kp;
            return 0;
        }
    }
    // No tall tile fills the chip: at a short K, 32-row tiles over two
    // k-parts still beat the register-staged kernel, whatever their grid
    // (graph-replayed, rotated weights, us per call, register-staged kernel
    // in brackets): M=128 K=1024 N=3584 7.4 (8.05); M=256 7.8 (9.8); M=192
    // 7.6 (14.0); M=64 7.2 (8.8); M=128 N=6144 7.8 (14.2); M=128 K=1024
    // N=1024 6.7 (7.9); M=128 K=2048 N=2048 10.1 (10.4).  At K=3584 they
    // lose: M=128 N=1024 14.5 against 10.9 for the register kernel's K split,
    // M=512 15.3 against 14.4.
    if (M >= 32 && K <= 2048 && K % (int64_t(kGroup) * 2) == 0) {
        *tm = 32;
        *ns = 3;
        *kp = 2;
        return 0;
    }
    return -1;
}

int launch_w4a16_gemm_lds(const void* x, int64_t M, int64_t K, int64_t N, const void* qw, const void* scales,
                          const void* zeros, int zero_bias, void* out, int tm, int ns, int kp, hipStream_t stream) {
    const ShapeW s{tm, ns, kp};
    GemmWFn fn = pick_w(s);
    if (fn == nullptr || K % (int64_t(kGroup) * kp) != 0)
        return fail(MCV_ERR_INVALID_ARG, "w4a16 GEMM: no LDS kernel for TM=%d NS=%d KP=%d, K=%lld", tm, ns, kp,
                    (long long)K);
    const int wn = 4 / kp;                                 // slabs per tile
    const int64_t nslab = ceil_div(N, kSlab);
    const int64_t n_tiles = ceil_div(nslab, wn);
    const int64_t total = ceil_div(M, tm) * n_tiles;
    // Tile order: the XCD blocking with the fewest bytes of x and weights per
    // XCD when the tile grid splits evenly, else a contiguous run per XCD,
    // down the tile columns when M < N.  MCV_W4GEMM_ORDER=0/1 forces the
    // run along the rows / columns (read once per process).
    int col_major = M < N ? 1 : 0, xcd_m = 0;
    static const char* const order = std::getenv("MCV_W4GEMM_ORDER");
    if (order != nullptr) {
        col_major = std::atoi(order) ? 1 : 0;
    } else {
        const int64_t m_tiles = ceil_div(M, tm);
        int64_t best = -1;
        for (int a = 1; a <= 8; a *= 2) {
            if (m_tiles % a != 0 || n_tiles % (8 / a) != 0) continue;
            const int64_t bytes = (m_tiles / a) * tm * K * 2 + (n_tiles / (8 / a)) * wn * kSlab * K / 2;
            if (best < 0 || bytes < best) {
                best = bytes;
                xcd_m = a;
            }
        }
    }
    // Buffer offsets are 32-bit: x inside one row tile, the packed weight.
    if (total > 0x7fffffff || K > (int64_t(1) << 22) || K * nslab * kSlab / 2 >= (int64_t(1) << 31) ||
        int64_t(tm) * K * 2 >= (int64_t(1) << 31))
        return fail(MCV_ERR_SHAPE, "w4a16 GEMM: problem too large (M=%lld N=%lld)", (long long)M, (long long)N);
    hipLaunchKernelGGL(fn, dim3(static_cast<unsigned>(total)), dim3(256), 0, stream, static_cast<const uint16_t*>(x),
                       static_cast<const uint4*>(qw), static_cast<const uint16_t*>(scales),
                       static_cast<const uint32_t*>(zeros), static_cast<uint32_t>(zero_bias), static_cast<uint16_t*>(out),
                       static_cast<int>(M), static_cast<int>(K), static_cast<int>(N), static_cast<int>(nslab),
                       static_cast<int>(n_tiles), static_cast<int>(total), col_major, xcd_m);
    return check_launch("w4a16_gemm_lds_kernel");
}

}  // namespace mcv
