// w4a16_gemm_sk.hip -- W4A16 prefill GEMM (M > 1) on fp16 MFMA, half-slab
// waves, K split across workgroups with the reduction inside the same launch.
//
// out[M][N] = x[M][K] . W[K][N], W in the slab-64 int4 layout, fp32
// accumulation, fp16 RNE output.
//
// Workgroup: NWV x KW waves; wave w owns the 32-column half-slab w % NWV of
// the tile (columns 32 (w % NWV) .. + 31) over all TM rows, for k-part
// w / NWV: TM/32 blocks of v_mfma_f32_32x32x16_f16, so every widened weight
// operand feeds TM/32 MFMAs (the widening is ~15 VALU per k16 step per wave,
// the same per MFMA as a full-slab wave over the same rows).  Tile TM x
// 32 NWV.  Each wave reads all TM x-rows of every k16 step from LDS, twice
// the LDS reads per MFMA of a full-slab wave: gfx950's LDS serves them
// (measured ds_read_b128 throughput ~340 GB/s per CU from four waves, ~500
// from eight, against ~100 GB/s per CU that the whole kernel needs).
//
// K advances in stages of KG quantisation groups (128 k each; a lane's scale
// and zero are constant over a group).  With KW = 2 (KG = 2) k-part j takes
// group j of every stage and the two partial sums meet in LDS after the
// loop: the copies of a stage then come from eight waves, two per SIMD, so
// one wave's MFMAs run while the other issues copies (MI355X: an LDS-DMA
// load from a wave that also issues MFMAs holds that wave ~90 ns; a second
// wave on the SIMD hides it).  Per stage, the waves copy global -> LDS with
// gfx950's direct-to-LDS buffer loads (no VGPR staging; staging through
// registers measured no faster), P copies per wave of 1 KiB (or 4 B per
// lane for zero and scale words), spread over the k16 steps of the stage
// NS - 1 earlier:
//   - x rows (TM x 256 KG bytes), 4 / KG rows per copy, the 16-byte chunk
//     index XORed with the row's low 4 bits (by choosing which global chunk
//     each lane fetches), so one ds_read_b128 pass over 16 rows at one k
//     offset covers all banks; rows past M read as zero;
//   - the packed chunks of the tile's slabs (32 k x 64 columns, 1 KiB each,
//     contiguous in the slab layout) verbatim;
//   - the slabs' zero words (lanes 0-7) and scales (lanes 0-31, two per
//     dword) of the stage's groups.
// A lane of half-slab h reads column 32 h + l%32 of its slab: per 32-k chunk
// the two 4-byte words of its k-octet parity (l/32) -- a pair of chunks in one
// ds_read_b128 (the half-waves read one chunk each) and two v_permlane32_swap
// (a lane-per-word read, 16 bytes apart, costs ~12 bank-conflict cycles) --
// eight words per group, one per k16 step, each widened into the 8-value
// fp16 operand RNE((q - z) * s) -- the values mcv_w4a16_dequant materialises
// ((1024 + q) - (1024 + z) exact through the fp16 exponent, times s, one
// rounding).
//
// WR = 1: the packed chunks, zero words and scales skip LDS.  A wave's
// weight columns are its own (no other wave of the tile reads them), so each
// wave fetches them with ordinary buffer loads into a ring of NS register
// slots, stage kt in slot kt % NS (a compile-time index: the stages are
// unrolled NS at a time), issued in the same copy slots and covered by the
// same vmcnt wait as the x rows; the stage buffers then hold x alone.  At
// MI355X this measured 0-9 % faster on 64- and 32-row tiles and the same on
// 128 x 256 (whose LDS path stays).
//
// K split (S > 1): workgroup (tile, p) runs the stages [p U/S, (p+1) U/S)
// of the U = G/KG stages over K (S need not divide U).
// Each writes its fp32 partial tile (after the k-parts' sum) to the
// workspace with device-scope
// stores (written through to the point of coherence of all XCDs; a plain
// store plus one device-scope release, an L2 write-back, measured 1.5-2x
// slower on MI355X), waits for them, and adds 1 to the tile's arrival
// counter (device-scope atomic); the
// workgroup that sees S - 1 is the last: it resets the counter to 0 for the
// next call, reads the other partials with device-scope loads and adds all S
// in split order p = 0, 1, ..., S-1 (its own from registers at its place),
// so the sum -- and the output -- is the same whichever workgroup is last.
// No workgroup waits for another, so any grid size works.  The counters
// start zero-filled once and every call leaves them zero; they sit in a
// fixed region at the start of the workspace (kSkCounterBytes, one per tile,
// at most kSkMaxSplitTiles tiles), and the partials after it, so one
// workspace serves calls of every shape without new clearing.
//
// Output: fp16 through LDS, whole tile rows per store instruction,
// non-temporal (full lines go straight to HBM while other tiles compute).
//
// The reference has no M > 1 quantised path: its prefill runs dense fp16
// aclnnMm through matmul_b_transposed (src/csrc/lib/decoder_layer.cpp:459-462,
// 656-659, 857-860; src/csrc/lib/ops.cpp:159-322).
#include <cmath>

#include "common.h"
#include "w4a16_gemm_sk.h"

namespace mcv {
namespace {

constexpr int kLine = 1024;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc_s(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, static_cast<int>(bytes), 0x00020000);
}

__device__ __forceinline__ void dma16_s(__amdgpu_buffer_rsrc_t r, uint8_t* lds, uint32_t voff, int soff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, lds, 16, voff, soff, 0, 0);
}

__device__ __forceinline__ void dma4_s(__amdgpu_buffer_rsrc_t r, uint8_t* lds, uint32_t voff, int soff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, lds, 4, voff, soff, 0, 0);
}

template <int N>
__device__ __forceinline__ void wait_vmcnt_s() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Linear work index of workgroup b: b runs on XCD b % 8, so each XCD gets a
// contiguous run of the linear order.
__device__ __forceinline__ int xcd_run(int b, int total) {
    const int per = total >> 3, rem = total & 7, x = b & 7, i = b >> 3;
    return x * per + (x < rem ? x : rem) + i;
}

template <int TM, int NWV, int NS, int KG, int KW, int WR>
struct CfgS {
    static constexpr int WS = NWV / 2;                   // slabs per tile
    static constexpr int TN = 32 * NWV;                  // columns per tile
    static constexpr int NWT = NWV * KW;                 // waves: NWV half-slabs x KW k-parts
    static constexpr int MB = TM / 32;                   // 32-row blocks per wave
    static constexpr int RP = 256 * KG;                  // bytes of one x row per stage (KG groups of 128 k)
    static constexpr int GW = KG / KW;                   // groups of a stage per wave
    static constexpr int STEPS = 8 * GW;                 // k16 steps per stage per wave
    static constexpr int A_BYTES = TM * RP;              // x rows
    static constexpr int B_BYTES = WR ? 0 : WS * 4 * KG * kLine;   // packed chunks, per slab group-major
    static constexpr int Z_OFF = A_BYTES + B_BYTES;      // per group and slab: 8 zero words at +0, 32 scale words at +256
    static constexpr int STAGE = Z_OFF + (WR ? 0 : KG * WS * 512);
    // copy items of a stage, spread evenly over all NWT waves
    static constexpr int PA = (TM * RP / kLine) / NWT;   // x rows, 1 KiB each
    static constexpr int PB = WR ? 0 : (4 * KG * WS) / NWT;   // packed chunks, 1 KiB each
    static constexpr int PZ = WR ? 0 : (2 * KG * WS) / NWT;   // zero words or scales of one (group, slab)
    // WR: each wave loads its own part of the stage's weights into registers
    // instead (per group: two chunk pairs, the zero word, the scale)
    static constexpr int PR = WR ? 4 * GW : 0;
    static constexpr int P = PA + PB + PZ + PR;
    // after the K loop each wave owns OB of the tile's MB row blocks of its
    // half-slab (k-part kp owns blocks kp * OB ..), the KW partial sums added
    static constexpr int OB = MB >= KW ? MB / KW : 1;
    static_assert(TM == 32 || TM == 64 || TM == 128, "TM");
    static_assert(NWV == 2 || NWV == 4 || NWV == 8, "NWV");
    static_assert(KG == 1 || KG == 2, "KG");
    static_assert(KW == 1 || (KW == 2 && KG == 2 && NWV <= 4), "KW: each k-part takes one group of a stage");
    static_assert(PA * NWT * kLine == TM * RP && (WR || (PB * NWT == 4 * KG * WS && PZ * NWT == 2 * KG * WS)),
                  "copies split evenly over the waves");
    static_assert(WR || ((4 * KG) % (PB ? PB : 1) == 0 && KG % (PZ ? PZ : 1) == 0 && PB > 0 && PZ > 0),
                  "a wave's chunk copies share one slab, its zero/scale copies one kind");
    static_assert(WR == 0 || WR == 1, "WR");
    static_assert(NS >= 2 && NS <= 4 && P * (NS - 1) < 64, "stages");
    static_assert(NS * STAGE <= 160 * 1024, "LDS");
    static constexpr int RB = TN * 2 + 16;               // padded bytes of one staged output row
    // staged output rows per stage buffer: whole 32-row blocks where a buffer
    // holds one (a wave's rows then share a buffer), else what fits
    static constexpr int R32 = (STAGE / RB) / 32 * 32;
    static constexpr int RPA = R32 >= 32 ? (R32 < TM ? R32 : TM) : (STAGE / RB < TM ? STAGE / RB : TM);
    static_assert(RPA >= 8 && (TM + RPA - 1) / RPA <= NS, "epilogue staging space");
    static_assert(KW == 1 || NWV * MB * 16 * 64 * 4 <= STAGE, "k-part exchange space");
};

template <int TM, int NWV, int NS, int KG, int KW, int WR>
__global__ __launch_bounds__(64 * NWV * KW) void w4a16_gemm_sk_kernel(
    const uint16_t* __restrict__ x, const uint4* __restrict__ qw, const uint16_t* __restrict__ scales,
    const uint32_t* __restrict__ zeros, uint32_t zero_bias, uint16_t* __restrict__ out, int M, int K, int N,
    int nslab, int m_tiles, int n_tiles, int S, int order, uint8_t* __restrict__ ws, uint32_t ws_bytes) {
    using C = CfgS<TM, NWV, NS, KG, KW, WR>;
    __shared__ __attribute__((aligned(1024))) uint8_t lds0[C::STAGE];
    __shared__ __attribute__((aligned(1024))) uint8_t lds1[C::STAGE];
    __shared__ __attribute__((aligned(1024))) uint8_t lds2[NS > 2 ? C::STAGE : 16];
    __shared__ __attribute__((aligned(1024))) uint8_t lds3[NS > 3 ? C::STAGE : 16];
    __shared__ int last_flag;
    uint8_t* const bufs[4] = {lds0, lds1, lds2, lds3};

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // 0 .. NWT-1: copies
    const int hw = wave % NWV;                           // half-slab of the tile: compute and output
    const int kp = wave / NWV;                           // k-part: groups kp * GW .. of every stage
    const int h = lane >> 5;

    // (tile, split): the split index is the slowest, then the tile order --
    // along the rows (order 0), down the tile columns (1: x rows shared
    // within an XCD's run), or down the columns of groups of `order` tile
    // rows (>= 2: an XCD's run then covers a block of tile rows and columns).
    const int tiles = m_tiles * n_tiles;
    const int lin = xcd_run(static_cast<int>(blockIdx.x), tiles * S);
    const int p = lin / tiles;
    const int tile = lin - p * tiles;
    int tm, tn;
    if (order >= 2) {
        const int grp = tile / (order * n_tiles), first = grp * order;
        const int rows = m_tiles - first < order ? m_tiles - first : order;
        const int t = tile - grp * order * n_tiles;
        tm = first + t % rows;
        tn = t / rows;
    } else if (order == 1) {
        tm = tile % m_tiles;
        tn = tile / m_tiles;
    } else {
        tm = tile / n_tiles;
        tn = tile - tm * n_tiles;
    }
    const int m0 = tm * TM;
    const int Npad = nslab * kSlab;
    const int CK = K / kChunkK;
    const int G = K / kGroup;
    // split p takes stages [p U / S, (p+1) U / S) of the U = G / KG stages
    // over all of K (S need not divide U: the splits differ by one stage)
    const int U = G / KG;
    const int u0 = static_cast<int>(int64_t(p) * U / S);
    const int g0 = u0 * KG;
    const int KT = static_cast<int>(int64_t(p + 1) * U / S) - u0;   // stages of this split

    const int rows_here = M - m0 < TM ? M - m0 : TM;
    const __amdgpu_buffer_rsrc_t xr =
        rsrc_s(x + static_cast<size_t>(m0) * K, static_cast<uint32_t>(rows_here) * K * 2u);
    const __amdgpu_buffer_rsrc_t qr = rsrc_s(qw, static_cast<uint32_t>(nslab) * CK * kSlab * 16u);
    const __amdgpu_buffer_rsrc_t sr = rsrc_s(scales, static_cast<uint32_t>(G) * Npad * 2u);
    const __amdgpu_buffer_rsrc_t zr = rsrc_s(zeros, static_cast<uint32_t>(G) * (Npad >> 3) * 4u);

    // This wave's copies of a stage, each lane's offset fixed here; the
    // stage's advance rides in the scalar offset.  The buffer range check
    // covers the vector offset alone, so anything with nothing to fetch (idle
    // lanes, padding slabs past nslab) gets bit 31 set: out of range, reads
    // zero.  Stages past the last re-read the last stage into a buffer that is
    // never read again, so every stage issues the same P copies and the vmcnt
    // waits stay exact.
    uint32_t xoff[C::PA];
#pragma unroll
    for (int j = 0; j < C::PA; ++j) {
        // copy j of this wave: 4 / KG rows of RP bytes
        constexpr int kRowsPerCopy = kLine / C::RP, kLanesPerRow = 64 / kRowsPerCopy;
        const int row = kRowsPerCopy * (wave * C::PA + j) + lane / kLanesPerRow;
        const int chunk = lane % kLanesPerRow;
        xoff[j] = static_cast<uint32_t>(row * K) * 2u + static_cast<uint32_t>(chunk ^ (row & 15)) * 16u;
    }
    // chunk items wave * PB .. + PB - 1 of the stage's 4 KG WS: slab t / (4 KG),
    // chunk t % (4 KG) of that slab's stage (group c / 4, 32-k chunk c % 4)
    const int bitem = wave * C::PB;
    const int bslab_t = bitem / (4 * KG);
    const int bslab = tn * C::WS + bslab_t;
    const bool bslab_live = bslab < nslab;
    const uint32_t qoff = (static_cast<uint32_t>(bslab) * CK * kSlab * 16u + lane * 16u) | (bslab_live ? 0u : 0x80000000u);
    const int bchunk = bitem % (4 * KG);
    // zero/scale items wave * PZ .. + PZ - 1 of the stage's 2 KG WS: slab
    // t / (2 KG), then zero words (kind 0) or scales (kind 1), then group
    const int zitem = wave * C::PZ;
    const int zslab_t = zitem / (2 * KG);
    const int zslab = tn * C::WS + zslab_t;
    const bool zslab_live = zslab < nslab;
    const bool zkind = (zitem % (2 * KG)) / KG == 0;
    const int zgrp = zitem % KG;                         // first group of this wave's items
    const uint32_t zsoff = zkind ? ((static_cast<uint32_t>(zslab) * 32u + lane * 4u) | (lane < 8 && zslab_live ? 0u : 0x80000000u))
                                 : ((static_cast<uint32_t>(zslab) * 128u + lane * 4u) | (lane < 32 && zslab_live ? 0u : 0x80000000u));
    const int zsstride = zkind ? (Npad >> 3) * 4 : Npad * 2;
    const __amdgpu_buffer_rsrc_t zsr = zkind ? zr : sr;
    const int zsdst = C::Z_OFF + zslab_t * 512 + (zkind ? 0 : 256);   // + group * WS * 512

    // WR: this wave's weights of stage kt land in register slot kt % NS (the
    // slot index is a compile-time constant wherever the stages are unrolled):
    // per group j of its part, chunk pairs (4j, 4j+1) and (4j+2, 4j+3) of
    // its column -- the lower half-wave fetches the first chunk of a pair,
    // the upper half the second, as the LDS path's ds_read_b128 does -- plus
    // the column's zero word and scale.  Padding slabs get bit 31 (read zero).
    const int col = 32 * (hw & 1) + (lane & 31);         // this lane's column inside its slab
    const int wslab = tn * C::WS + (hw >> 1);
    const uint32_t wdead = wslab < nslab ? 0u : 0x80000000u;
    const uint32_t wq_off = (static_cast<uint32_t>(wslab) * CK * kSlab * 16u + h * 1024u + col * 16u) | wdead;
    const uint32_t wz_off = (static_cast<uint32_t>(wslab) * 32u + (col >> 3) * 4u) | wdead;
    const uint32_t ws_off = (static_cast<uint32_t>(wslab) * 128u + col * 2u) | wdead;
    uint4 rq[WR ? NS : 1][2 * C::GW];
    uint32_t rz[WR ? NS : 1][C::GW], rs[WR ? NS : 1][C::GW];

    auto issue_item = [&](int kt, uint8_t* dst, int it, int slot) {
        const int kc = kt < KT ? kt : KT - 1;
        const int g = g0 + kc * KG;                      // the stage's first group
        if (it < C::PA) {
            dma16_s(xr, dst + (wave * C::PA + it) * kLine, xoff[it], g * 256);
        } else if (WR) {
            const int r = it - C::PA, j = r / 4, kind = r % 4;
            const int grp = g + kp * C::GW + j;
            if (kind < 2)
                rq[slot][2 * j + kind] = __builtin_bit_cast(
                    uint4, __builtin_amdgcn_raw_buffer_load_b128(qr, wq_off, (grp * 4 + 2 * kind) * kSlab * 16, 0));
            else if (kind == 2)
                rz[slot][j] = __builtin_amdgcn_raw_buffer_load_b32(zr, wz_off, grp * (Npad >> 3) * 4, 0);
            else
                rs[slot][j] = __builtin_amdgcn_raw_buffer_load_b16(sr, ws_off, grp * Npad * 2, 0);
        } else if (it < C::PA + C::PB) {
            const int c = bchunk + (it - C::PA);
            dma16_s(qr, dst + C::A_BYTES + (bslab_t * 4 * KG + c) * kLine, qoff, (g * 4 + c) * kSlab * 16);
        } else {
            const int j = zgrp + (it - C::PA - C::PB);   // group j of the stage
            dma4_s(zsr, dst + zsdst + j * C::WS * 512, zsoff, (g + j) * zsstride);
        }
    };
    auto issue = [&](int kt, uint8_t* dst, int slot) {
#pragma unroll
        for (int it = 0; it < C::P; ++it) issue_item(kt, dst, it, slot);
    };

    uint32_t vmagic;
    asm("v_mov_b32 %0, 0x64006400" : "=v"(vmagic));
    const uint32_t mlo = __builtin_amdgcn_readfirstlane(0x000F000Fu);
    const uint32_t zsh = (col & 7) * 4;

    float16_t acc[C::MB];
#pragma unroll
    for (int i = 0; i < C::MB; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][r] = 0.f;

    // x operand of this wave's k16 step s (step 8 kp GW + s of the stage),
    // block i: row 32 i + l%32, 16-byte chunk 2 (8 kp GW + s) + l/32,
    // XOR-swizzled by the row's low 4 bits; block i is 32 rows on.
    int a_off[C::STEPS];
#pragma unroll
    for (int s = 0; s < C::STEPS; ++s)
        a_off[s] = (lane & 31) * C::RP + (((2 * (8 * kp * C::GW + s) + h) ^ (lane & 15)) << 4);
    // the lane's two words of chunk c: word h (k-octet 4c + h) and word 2 + h;
    // this wave's chunks start at group kp GW of its slab's stage
    const int b_off = C::A_BYTES + ((hw >> 1) * 4 * KG + 4 * kp * C::GW + h) * kLine + col * 16;
    const int z_off = C::Z_OFF + kp * C::GW * C::WS * 512 + (hw >> 1) * 512 + (col >> 3) * 4;
    const int s_off = C::Z_OFF + kp * C::GW * C::WS * 512 + (hw >> 1) * 512 + 256 + col * 2;

    uint32_t q[C::STEPS];                                // the wave's words of a stage, one per k16 step
    uint32_t zza[C::GW], ssa[C::GW];                     // per group of the wave's part of a stage
#pragma unroll
    for (int j = 0; j < C::GW; ++j) zza[j] = ssa[j] = 0;
    half8_t af[2][C::MB], bf[2];
    auto widen = [&](int s, half8_t& b) {
        const uint32_t w = q[s];
        const uint32_t zz = zza[s / 8], ss = ssa[s / 8];
        uint32_t t[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) t[j] = and_or_b32(j ? w >> (4 * j) : w, mlo, vmagic);
        half2_t d[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) d[j] = as_h2(t[j]) - as_h2(zz);
#pragma unroll
        for (int j = 0; j < 4; ++j) d[j] = d[j] * as_h2(ss);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            b[2 * j] = d[j][0];
            b[2 * j + 1] = d[j][1];
        }
    };
    auto read_a = [&](const uint8_t* src, int s, half8_t* dst) {
#pragma unroll
        for (int i = 0; i < C::MB; ++i) dst[i] = *reinterpret_cast<const half8_t*>(src + a_off[s] + i * 32 * C::RP);
    };
    auto head = [&](const uint8_t* src, int slot) {
        // Chunks c, c+1 (c even) in one conflict-free ds_read_b128: the lower
        // half-wave reads column col of chunk c, the upper half of chunk c+1;
        // two lane-half swaps then leave each lane its k-octet parity's words
        // (h and 2 + h) of both chunks.
#pragma unroll
        for (int c = 0; c < 4 * C::GW; c += 2) {
            const uint4 w = WR ? rq[slot][c / 2] : *reinterpret_cast<const uint4*>(src + b_off + c * kLine);
            const auto s0 = __builtin_amdgcn_permlane32_swap(w.x, w.y, false, false);
            const auto s2 = __builtin_amdgcn_permlane32_swap(w.z, w.w, false, false);
            q[2 * c] = s0[0];                            // word h of chunk c
            q[2 * c + 2] = s0[1];                        // word h of chunk c + 1
            q[2 * c + 1] = s2[0];                        // word 2 + h of chunk c
            q[2 * c + 3] = s2[1];                        // word 2 + h of chunk c + 1
        }
        uint32_t zw[C::GW], sh[C::GW];
#pragma unroll
        for (int j = 0; j < C::GW; ++j) {
            zw[j] = WR ? rz[slot][j] : *reinterpret_cast<const uint32_t*>(src + z_off + j * C::WS * 512);
            sh[j] = WR ? rs[slot][j] & 0xffffu : *reinterpret_cast<const uint16_t*>(src + s_off + j * C::WS * 512);
        }
        read_a(src, 0, af[0]);
#pragma unroll
        for (int j = 0; j < C::GW; ++j) {
            zza[j] = (0x6400u + ((zw[j] >> zsh) & 15u) + zero_bias) * 0x10001u;
            ssa[j] = sh[j] * 0x10001u;
        }
    };
    auto mfmas = [&](int cur, int lo, int hi) {
#pragma unroll
        for (int i = lo; i < hi; ++i)
            acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(bf[cur], af[cur][i], acc[i], 0, 0, 0);
    };
    constexpr int kV = (15 + C::MB - 1) / C::MB;         // widening VALU per MFMA

    // One stage from `cur`: steps 0-6 produce step s+1's operands while step
    // s's MFMAs run and spread the copies of stage kt + NS - 1 into `prv`
    // (free since the last barrier); step 7 crosses into the next stage
    // between its MFMAs (wait for the copies, barrier, the next stage's head).
    auto run_stage = [&](int kt, const uint8_t* cur, const uint8_t* nxt, uint8_t* prv, int u) {
#pragma unroll
        for (int s = 0; s < C::STEPS - 1; ++s) {
            const int c = s & 1, n = c ^ 1;
            // copies of this step: [lo, hi) of the stage's P, spread evenly
            const int lo = C::P * s / (C::STEPS - 1), hi = C::P * (s + 1) / (C::STEPS - 1);
#pragma unroll
            for (int it = lo; it < hi; ++it) issue_item(kt + NS - 1, prv, it, (u + NS - 1) % NS);
            read_a(cur, s + 1, af[n]);
            widen(s + 1, bf[n]);
            mfmas(c, 0, C::MB);
#pragma unroll
            for (int i = 0; i < C::MB; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);                  // DS read
                if (i < hi - lo) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);   // copy
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                  // MFMA
                __builtin_amdgcn_sched_group_barrier(0x002, kV, 0);                 // VALU
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        static_assert(C::STEPS % 2 == 0, "the last step uses operand set 1");
        mfmas(1, 0, (C::MB + 1) / 2);
        __builtin_amdgcn_sched_barrier(0);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        wait_vmcnt_s<C::P * (NS - 2)>();
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        head(nxt, (u + 1) % NS);
        mfmas(1, (C::MB + 1) / 2, C::MB);
        __builtin_amdgcn_sched_barrier(0);
        widen(0, bf[0]);
    };

#pragma unroll
    for (int d = 0; d < NS - 1; ++d) issue(d, bufs[d], d);
    wait_vmcnt_s<C::P * (NS - 2)>();
    __builtin_amdgcn_s_barrier();
    head(bufs[0], 0);
    widen(0, bf[0]);
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
    // no copy may land in LDS after this point (the stage buffers are reused)
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

    // ---- The wave's owned row blocks ib0 .. ib0 + OB - 1 of half-slab hw
    // (all MB with one k-part).  With KW k-parts the partial sums meet in
    // LDS: k-part 0's + k-part 1's, the same sum whichever wave adds it.
    const int ib0 = KW > 1 && C::MB >= KW ? kp * C::OB : 0;
    const bool owns = KW == 1 || C::MB >= KW || kp == 0;
    float16_t own[C::OB];
    if constexpr (KW == 1) {
#pragma unroll
        for (int i = 0; i < C::MB; ++i) own[i] = acc[i];
    } else {
        // [half-slab][block][register quad][lane] float4 in the first stage buffer
        auto roff = [&](int i, int rq) { return ((hw * C::MB + i) * 4 + rq) * 1024 + lane * 16; };
        __syncthreads();                                 // every wave is past its last operand read
#pragma unroll
        for (int i = 0; i < C::MB; ++i) {
            const bool mine = owns && i >= ib0 && i < ib0 + C::OB;
            if (!mine)
#pragma unroll
                for (int rq = 0; rq < 4; ++rq)
                    *reinterpret_cast<float4*>(lds0 + roff(i, rq)) =
                        make_float4(acc[i][4 * rq], acc[i][4 * rq + 1], acc[i][4 * rq + 2], acc[i][4 * rq + 3]);
        }
        __syncthreads();
#pragma unroll
        for (int ii = 0; ii < C::OB; ++ii) {
            const int i = ib0 + ii;
#pragma unroll
            for (int rq = 0; rq < 4; ++rq) {
                const float4 o = *reinterpret_cast<const float4*>(lds0 + roff(i, rq));
                own[ii][4 * rq] = acc[i][4 * rq] + o.x;
                own[ii][4 * rq + 1] = acc[i][4 * rq + 1] + o.y;
                own[ii][4 * rq + 2] = acc[i][4 * rq + 2] + o.z;
                own[ii][4 * rq + 3] = acc[i][4 * rq + 3] + o.w;
            }
        }
    }

    if (S > 1) {
        // ---- K split: publish this split's partial tile, the last arriver adds all S.
        // Partial layout per (tile, split): [half-slab][block i][register quad rq][lane] float4.
        constexpr uint32_t kPart = TM * C::TN * 4;
        const __amdgpu_buffer_rsrc_t wr = rsrc_s(ws, ws_bytes);
        unsigned* const counters = reinterpret_cast<unsigned*>(ws);
        const uint32_t base = kSkCounterBytes + static_cast<uint32_t>(tile * S) * kPart;
        const uint32_t lo = (static_cast<uint32_t>(hw) * C::MB * 4 + ib0 * 4) * 1024u + lane * 16u;
#pragma unroll
        for (int i = 0; i < C::OB; ++i)
#pragma unroll
            for (int rq = 0; rq < 4; ++rq) {
                if (!owns) continue;
                const int4_t v = {__float_as_int(own[i][4 * rq]), __float_as_int(own[i][4 * rq + 1]),
                                  __float_as_int(own[i][4 * rq + 2]), __float_as_int(own[i][4 * rq + 3])};
                // device scope (sc1): written through to where every XCD reads it
                __builtin_amdgcn_raw_buffer_store_b128(v, wr, lo + (i * 4 + rq) * 1024u, base + p * kPart, 16);
            }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if (threadIdx.x == 0) {
            const unsigned old = __hip_atomic_fetch_add(counters + tile, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const int last = old == static_cast<unsigned>(S - 1);
            if (last) __hip_atomic_store(counters + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            last_flag = last;
        }
        __syncthreads();
        if (!last_flag) return;
        // sum in split order 0 .. S-1, this split's own partial from
        // registers.  The loads of a batch of partials go out together (one
        // round trip to where the device-scope stores landed per batch, not
        // per partial), then the batch is added in order; the batch is as
        // large as the registers allow (4 partials of a 32-row block, 2 of
        // two blocks, 1 of four).
        constexpr int kBatch = C::OB >= 4 ? 1 : (C::OB == 2 ? 2 : 4);
        float16_t sum[C::OB];
        for (int q0 = 0; q0 < S && owns; q0 += kBatch) {
            float16_t got[kBatch][C::OB];
#pragma unroll
            for (int b = 0; b < kBatch; ++b) {
                const int q2 = q0 + b;
                if (q2 >= S || q2 == p) continue;
#pragma unroll
                for (int i = 0; i < C::OB; ++i)
#pragma unroll
                    for (int rq = 0; rq < 4; ++rq) {
                        const int4_t t = __builtin_amdgcn_raw_buffer_load_b128(wr, lo + (i * 4 + rq) * 1024u,
                                                                               base + q2 * kPart, 16);
#pragma unroll
                        for (int e = 0; e < 4; ++e) got[b][i][4 * rq + e] = __int_as_float(t[e]);
                    }
            }
#pragma unroll
            for (int b = 0; b < kBatch; ++b) {
                const int q2 = q0 + b;
                if (q2 >= S) break;
#pragma unroll
                for (int i = 0; i < C::OB; ++i)
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const float v = q2 == p ? own[i][r] : got[b][i][r];
                        sum[i][r] = q2 == 0 ? v : sum[i][r] + v;
                    }
            }
        }
        if (owns)
#pragma unroll
            for (int i = 0; i < C::OB; ++i) own[i] = sum[i];
    }

    // ---- fp16 epilogue.  Owned block ii (row block ib0 + ii): register r of
    // lane l holds output row 32 (ib0 + ii) + l%32 and column 8 (r/4) +
    // 4 (l/32) + r%4 of the half-slab's 32; swapping the upper lanes of quad g
    // with the lower lanes of quad g+1 leaves lane l with the 8 consecutive
    // columns 8 g + 8 (l/32), g even.
    auto pack = [&](int ii, int g, uint32_t (&pk)[4]) {
#pragma unroll
        for (int d = 0; d < 2; ++d) {
            const uint32_t x0 = f2h(own[ii][4 * g + 2 * d]) | (uint32_t(f2h(own[ii][4 * g + 2 * d + 1])) << 16);
            const uint32_t x1 = f2h(own[ii][4 * g + 4 + 2 * d]) | (uint32_t(f2h(own[ii][4 * g + 5 + 2 * d])) << 16);
            const auto sw = __builtin_amdgcn_permlane32_swap(x0, x1, false, false);
            pk[d] = sw[0];
            pk[2 + d] = sw[1];
        }
    };
    const int n0 = tn * C::TN;
    const bool vec_ok = (N & 7) == 0 && (reinterpret_cast<uintptr_t>(out) & 15) == 0;
    if (vec_ok) {
        // the whole tile through LDS (the stage buffers: every wave is past
        // its last operand read after this barrier), then whole rows per
        // store instruction, non-temporal
        __syncthreads();
        // staged row r lives in stage buffer r / RPA (separate arrays)
        auto srow = [&](int r) -> uint8_t* {
            const int a = r / C::RPA;
            return (a == 0 ? lds0 : a == 1 ? lds1 : a == 2 ? lds2 : lds3) + (r - a * C::RPA) * C::RB;
        };
#pragma unroll
        for (int ii = 0; ii < C::OB; ++ii)
#pragma unroll
            for (int g = 0; g < 4; g += 2) {
                if (!owns) continue;
                uint32_t pk[4];
                pack(ii, g, pk);
                *reinterpret_cast<uint4*>(srow(32 * (ib0 + ii) + (lane & 31)) + (32 * hw + 8 * g + 8 * h) * 2) =
                    make_uint4(pk[0], pk[1], pk[2], pk[3]);
            }
        __syncthreads();
        constexpr int CPR = C::TN / 8;                   // 16-byte chunks per row
        constexpr int RPI = 64 * C::NWT / CPR;           // rows per workgroup-wide pass
        static_assert(TM % RPI == 0, "row passes");
        const int cl = static_cast<int>(threadIdx.x) % CPR, rl = static_cast<int>(threadIdx.x) / CPR;
#pragma unroll
        for (int it = 0; it < TM / RPI; ++it) {
            const int r = it * RPI + rl;
            const int row = m0 + r, c0 = n0 + 8 * cl;
            const uint4 v = *reinterpret_cast<const uint4*>(srow(r) + cl * 16);
            if (row < M && c0 < N)
                __builtin_nontemporal_store(int4_t{static_cast<int>(v.x), static_cast<int>(v.y), static_cast<int>(v.z),
                                                   static_cast<int>(v.w)},
                                            reinterpret_cast<int4_t*>(out + static_cast<size_t>(row) * N + c0));
        }
        return;
    }
    // N not a multiple of 8 (or an unaligned output): element stores
#pragma unroll
    for (int ii = 0; ii < C::OB; ++ii) {
        if (!owns) break;
        const int row = m0 + 32 * (ib0 + ii) + (lane & 31);
#pragma unroll
        for (int g = 0; g < 4; g += 2) {
            uint32_t pk[4];
            pack(ii, g, pk);
            const int c0 = n0 + 32 * hw + 8 * g + 8 * h;
            if (row >= M || c0 >= N) continue;
            uint16_t* dst = out + static_cast<size_t>(row) * N + c0;
#pragma unroll
            for (int e = 0; e < 8; ++e)
                if (c0 + e < N) dst[e] = static_cast<uint16_t>(pk[e >> 1] >> (16 * (e & 1)));
        }
    }
}

using SkFn = void (*)(const uint16_t*, const uint4*, const uint16_t*, const uint32_t*, uint32_t, uint16_t*, int, int,
                      int, int, int, int, int, int, uint8_t*, uint32_t);

#define MCV_SK_SHAPES(X)                                                                                   \
    X(128, 8, 3, 1, 1, 0) X(128, 4, 3, 1, 1, 0) X(64, 8, 3, 1, 1, 0) X(64, 4, 3, 1, 1, 0) X(32, 4, 3, 1, 1, 0)   \
    X(64, 4, 3, 2, 1, 0) X(32, 4, 3, 2, 1, 0) X(64, 4, 3, 2, 2, 0) X(32, 4, 3, 2, 2, 0) X(128, 8, 4, 1, 1, 1)   \
    X(64, 4, 3, 1, 1, 1) X(64, 4, 3, 2, 2, 1) X(64, 4, 4, 2, 2, 1) X(32, 4, 3, 1, 1, 1) X(32, 4, 3, 2, 1, 1)   \
    X(32, 4, 3, 2, 2, 1) X(32, 2, 3, 1, 1, 1) X(32, 2, 3, 2, 2, 1) X(64, 2, 3, 2, 2, 1) X(32, 2, 4, 2, 2, 1)   \
    X(128, 2, 3, 1, 1, 1) X(128, 2, 2, 2, 2, 1) X(64, 2, 3, 1, 1, 1)

SkFn pick_sk(int tm, int nwv, int ns, int kg, int kw, int wr) {
#define MCV_SK_PICK(a, b, c, d, e, f) \
    if (tm == a && nwv == b && ns == c && kg == d && kw == e && wr == f) return w4a16_gemm_sk_kernel<a, b, c, d, e, f>;
    MCV_SK_SHAPES(MCV_SK_PICK)
#undef MCV_SK_PICK
    return nullptr;
}

}  // namespace

int64_t w4a16_sk_tiles(int64_t M, int64_t N, const SkConfig& c) {
    return ceil_div(M, c.tm) * ceil_div(ceil_div(N, kSlab), c.nwv / 2);
}

int64_t w4a16_sk_workspace_bytes(int64_t M, int64_t N, const SkConfig& c) {
    if (c.splits <= 1) return 0;
    const int64_t tiles = w4a16_sk_tiles(M, N, c);
    return kSkCounterBytes + tiles * c.splits * int64_t(c.tm) * (32 * c.nwv) * 4;
}

bool w4a16_sk_config_valid(int64_t M, int64_t K, int64_t N, const SkConfig& c) {
    return pick_sk(c.tm, c.nwv, c.ns, c.kg, c.kw, c.wr) != nullptr && c.splits >= 1 && c.splits <= 64 && K % kGroup == 0 &&
           (K / kGroup) % c.kg == 0 && c.splits <= K / kGroup / c.kg &&
           (c.splits == 1 || w4a16_sk_tiles(M, N, c) <= kSkMaxSplitTiles);
}

int launch_w4a16_gemm_sk(const void* x, int64_t M, int64_t K, int64_t N, const void* qw, const void* scales,
                         const void* zeros, int zero_bias, void* out, const SkConfig& c, void* ws, int64_t ws_bytes,
                         hipStream_t stream) {
    SkFn fn = pick_sk(c.tm, c.nwv, c.ns, c.kg, c.kw, c.wr);
    if (fn == nullptr || !w4a16_sk_config_valid(M, K, N, c))
        return fail(MCV_ERR_INVALID_ARG,
                    "w4a16 GEMM: no kernel for TM=%d waves=%d NS=%d KG=%d KW=%d WR=%d S=%d at M=%lld K=%lld N=%lld (KG must "
                    "divide K/128, S be at most K/128/KG, and a split needs at most %d tiles)",
                    c.tm, c.nwv, c.ns, c.kg, c.kw, c.wr, c.splits, (long long)M, (long long)K, (long long)N,
                    kSkMaxSplitTiles);
    const int64_t nslab = ceil_div(N, kSlab);
    const int64_t m_tiles = ceil_div(M, c.tm), n_tiles = ceil_div(nslab, c.nwv / 2);
    const int64_t total = m_tiles * n_tiles * c.splits;
    const int64_t need = w4a16_sk_workspace_bytes(M, N, c);
    if (c.splits > 1 && (ws == nullptr || ws_bytes < need || (reinterpret_cast<uintptr_t>(ws) & 255) != 0))
        return fail(MCV_ERR_INVALID_ARG, "w4a16 GEMM: the K split needs a 256-byte aligned workspace of %lld bytes",
                    (long long)need);
    // Buffer offsets are 32-bit: x inside one row tile, the packed weight,
    // the workspace.
    if (total > 0x7fffffff || K > (int64_t(1) << 22) || K * nslab * kSlab / 2 >= (int64_t(1) << 31) ||
        int64_t(c.tm) * K * 2 >= (int64_t(1) << 31) || need >= (int64_t(1) << 31))
        return fail(MCV_ERR_SHAPE, "w4a16 GEMM: problem too large (M=%lld N=%lld)", (long long)M, (long long)N);
    // Each XCD takes a contiguous run of the tile order.  Down the columns,
    // an XCD's tiles share few weight columns but need (nearly) every x row;
    // along the rows, the reverse; so the order goes down the columns only
    // when x is the smaller operand (every XCD re-reads it from beyond its
    // L2 instead of the weights).  MI355X, M=2048 K=1024 N=3584 (x 4.2 MB,
    // weights 2.3 MB): the column order fetched 36 MB per call.  Where x is
    // the larger operand, groups of g tile rows taken down their columns
    // give each XCD a block of rows and columns instead of whole rows
    // (interleaved A/B, medians of 12 regions: M=2048 K=1024 19.23 against
    // 19.35-19.53 us along the rows, M=2048 K=3584 20.66 against 20.80-21.17,
    // M=512 K=3584 10.61 against 10.69-10.72; where x is the smaller operand
    // the column order stays ahead: M=512 K=1024 8.67 against 8.72).
    const int64_t x_bytes = M * K * 2, w_bytes = K * N / 2 + (K / kGroup) * N * 5 / 2;
    int order = c.order == 2 || (c.order == 0 && x_bytes < w_bytes) ? 1 : 0;
    if ((c.order == 3 || (c.order == 0 && x_bytes >= w_bytes)) && m_tiles >= 2) {
        // groups of g tile rows, g balancing an XCD run's x rows (g of them)
        // against its weight columns (run / g): g = sqrt(run * col / row)
        const double run = double(m_tiles * n_tiles) / 8.0;
        const double row = double(c.tm) * K * 2, col = double(c.nwv / 2) * (double(w_bytes) / nslab);
        int g = static_cast<int>(std::lround(std::sqrt(run * col / row)));
        order = g < 2 ? 2 : (g > m_tiles ? static_cast<int>(m_tiles) : g);
    }
    hipLaunchKernelGGL(fn, dim3(static_cast<unsigned>(total)), dim3(64 * c.nwv * c.kw), 0, stream,
                       static_cast<const uint16_t*>(x), static_cast<const uint4*>(qw),
                       static_cast<const uint16_t*>(scales), static_cast<const uint32_t*>(zeros),
                       static_cast<uint32_t>(zero_bias), static_cast<uint16_t*>(out), static_cast<int>(M),
                       static_cast<int>(K), static_cast<int>(N), static_cast<int>(nslab), static_cast<int>(m_tiles),
                       static_cast<int>(n_tiles), c.splits, order, static_cast<uint8_t*>(ws),
                       static_cast<uint32_t>(c.splits > 1 ? need : 0));
    return check_launch("w4a16_gemm_sk_kernel");
}

}  // namespace mcv

using namespace mcv;

extern "C" {

int64_t mcv_w4a16_gemm_sk_workspace_bytes(int64_t M, int64_t N, int tm, int waves, int splits) {
    if (M <= 0 || N <= 0 || tm <= 0 || waves <= 0 || splits <= 0) return 0;
    return w4a16_sk_workspace_bytes(M, N, SkConfig{tm, waves, 3, splits});
}

int mcv_w4a16_gemm_sk(const void* x, int64_t M, int64_t K, int64_t N, const void* qw, const void* scales,
                      const void* zeros, int zero_bias, void* out, int tm, int waves, int stages,
                      int groups_per_stage, int k_parts, int weights_in_registers, int tile_order, int splits,
                      void* workspace, int64_t workspace_bytes, mcv_stream_t stream) {
    if (!x || !out || !qw || !scales || !zeros) return fail(MCV_ERR_INVALID_ARG, "mcv_w4a16_gemm_sk: null pointer");
    if (zero_bias != 0 && zero_bias != 1) return fail(MCV_ERR_INVALID_ARG, "mcv_w4a16_gemm_sk: zero_bias must be 0 or 1");
    if (K <= 0 || K % kGroup != 0 || M <= 0 || M > (int64_t(1) << 30) || N <= 0 || N > (int64_t(1) << 30))
        return fail(MCV_ERR_SHAPE, "mcv_w4a16_gemm_sk: bad shape (M=%lld K=%lld N=%lld)", (long long)M, (long long)K,
                    (long long)N);
    if (reinterpret_cast<uintptr_t>(x) % 16 != 0) return fail(MCV_ERR_INVALID_ARG, "mcv_w4a16_gemm_sk: x must be 16-byte aligned");
    int rc = require_device();
    if (rc != MCV_OK) return rc;
    if (tile_order < 0 || tile_order > 3)
        return fail(MCV_ERR_INVALID_ARG, "mcv_w4a16_gemm_sk: tile_order must be 0, 1, 2 or 3 (%d)", tile_order);
    return launch_w4a16_gemm_sk(x, M, K, N, qw, scales, zeros, zero_bias, out,
                                SkConfig{tm, waves, stages, splits, groups_per_stage, k_parts, weights_in_registers,
                                         tile_order},
                                workspace, workspace_bytes,
                                static_cast<hipStream_t>(stream));
}

}  // extern "C"
