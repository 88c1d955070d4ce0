// w4a16_gemm_sk.hip -- W4A16 prefill GEMM (M > 1) on fp16 MFMA, half-slab
// waves, K split across workgroups with the reduction inside the same launch.
//
// out[M][N] = x[M][K] . W[K][N], W in the slab-64 int4 layout, fp32
// accumulation, fp16 RNE output.
//
// Workgroup: NWV waves; wave w owns the 32-column half-slab w of the tile
// (columns 32 w .. 32 w + 31) over all TM rows: TM/32 blocks of
// v_mfma_f32_32x32x16_f16, so every widened weight operand feeds TM/32 MFMAs
// (the widening is ~15 VALU per k16 step per wave, the same per MFMA as a
// full-slab wave over the same rows).  Tile TM x 32 NWV.  Each wave reads all
// TM x-rows of every k16 step from LDS, twice the LDS reads per MFMA of a
// full-slab wave: gfx950's LDS serves them (measured ds_read_b128 throughput
// ~340 GB/s per CU from four waves, ~500 from eight, against ~100 GB/s per CU
// that the whole kernel needs).
//
// K advances in stages of 128 (one quantisation group, so a lane's scale and
// zero are constant over a stage).  Per stage, every wave copies global ->
// LDS with gfx950's direct-to-LDS buffer loads (no VGPR staging), P copies
// of 1 KiB (or 4 B per lane for zero and scale words), spread over the k16
// steps of the stage NS - 1 earlier:
//   - x rows (TM x 256 bytes), 4 rows per copy, the 16-byte chunk index XORed
//     with the row's low 4 bits (by choosing which global chunk each lane
//     fetches), so one ds_read_b128 pass over 16 rows at one k offset covers
//     all banks; rows past M read as zero;
//   - the packed chunks of the tile's slabs (32 k x 64 columns, 1 KiB each,
//     contiguous in the slab layout) verbatim;
//   - the slabs' zero words (lanes 0-7) and scales (lanes 0-31, two per
//     dword) of the stage's group.
// A lane of half-slab h reads column 32 h + l%32 of its slab: per 32-k chunk
// the two 4-byte words of its k-octet parity (l/32) with one ds_read2_b32,
// eight words per stage, one per k16 step, each widened into the 8-value
// fp16 operand RNE((q - z) * s) -- the values mcv_w4a16_dequant materialises
// ((1024 + q) - (1024 + z) exact through the fp16 exponent, times s, one
// rounding).
//
// K split (S > 1): workgroup (tile, p) runs k-groups [p G/S, (p+1) G/S).
// Each writes its fp32 partial tile to the workspace with device-scope
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

template <int TM, int NWV, int NS>
struct CfgS {
    static constexpr int WS = NWV / 2;                   // slabs per tile
    static constexpr int TN = 32 * NWV;                  // columns per tile
    static constexpr int MB = TM / 32;                   // 32-row blocks per wave
    static constexpr int A_BYTES = TM * 256;             // x rows, 128 k of fp16
    static constexpr int B_BYTES = WS * 4 * kLine;       // packed chunks
    static constexpr int Z_OFF = A_BYTES + B_BYTES;      // per slab: 8 zero words at +0, 32 scale words at +256
    static constexpr int STAGE = Z_OFF + WS * 512;
    static constexpr int PA = (TM / 4) / NWV;            // x copies per wave per stage
    static constexpr int PB = (4 * WS) / NWV;            // chunk copies per wave: 2
    static constexpr int PZ = (2 * WS) / NWV;            // zero-or-scale copies per wave: 1
    static constexpr int P = PA + PB + PZ;
    static_assert(TM == 32 || TM == 64 || TM == 128, "TM");
    static_assert(NWV == 4 || NWV == 8, "NWV");
    static_assert(PA * NWV == TM / 4 && PB == 2 && PZ == 1, "copies split evenly over the waves");
    static_assert(NS >= 2 && NS <= 4 && P * (NS - 1) < 64, "stages");
    static_assert(NS * STAGE <= 160 * 1024, "LDS");
    static constexpr int RB = TN * 2 + 16;               // padded bytes of one staged output row
    static constexpr int RPA = (STAGE / RB) / 32 * 32 < TM ? (STAGE / RB) / 32 * 32 : TM;   // staged rows per stage buffer
    static_assert(RPA >= 32 && (TM + RPA - 1) / RPA <= NS, "epilogue staging space");
};

template <int TM, int NWV, int NS>
__global__ __launch_bounds__(64 * NWV) void w4a16_gemm_sk_kernel(
    const uint16_t* __restrict__ x, const uint4* __restrict__ qw, const uint16_t* __restrict__ scales,
    const uint32_t* __restrict__ zeros, uint32_t zero_bias, uint16_t* __restrict__ out, int M, int K, int N,
    int nslab, int m_tiles, int n_tiles, int S, int col_major, uint8_t* __restrict__ ws, uint32_t ws_bytes) {
    using C = CfgS<TM, NWV, NS>;
    __shared__ __attribute__((aligned(1024))) uint8_t lds0[C::STAGE];
    __shared__ __attribute__((aligned(1024))) uint8_t lds1[C::STAGE];
    __shared__ __attribute__((aligned(1024))) uint8_t lds2[NS > 2 ? C::STAGE : 16];
    __shared__ __attribute__((aligned(1024))) uint8_t lds3[NS > 3 ? C::STAGE : 16];
    __shared__ int last_flag;
    uint8_t* const bufs[4] = {lds0, lds1, lds2, lds3};

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int h = lane >> 5;

    // (tile, split): the split index is the slowest, then the tile order --
    // down the tile columns (col_major, x rows shared within an XCD's run) or
    // along the rows.
    const int tiles = m_tiles * n_tiles;
    const int lin = xcd_run(static_cast<int>(blockIdx.x), tiles * S);
    const int p = lin / tiles;
    const int tile = lin - p * tiles;
    const int tm = col_major ? tile % m_tiles : tile / n_tiles;
    const int tn = col_major ? tile / m_tiles : tile - tm * n_tiles;
    const int m0 = tm * TM;
    const int Npad = nslab * kSlab;
    const int CK = K / kChunkK;
    const int G = K / kGroup;
    const int g0 = static_cast<int>(int64_t(p) * G / S);
    const int KT = static_cast<int>(int64_t(p + 1) * G / S) - g0;   // stages of this split

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
        const int row = 4 * (wave * C::PA + j) + (lane >> 4);
        xoff[j] = static_cast<uint32_t>(row * K) * 2u + static_cast<uint32_t>((lane & 15) ^ (row & 15)) * 16u;
    }
    // chunks 2 (wave & 1), +1 of slab wave / 2 (PB = 2: the slab's four chunks
    // over its two waves)
    const int bslab = tn * C::WS + (wave >> 1);
    const bool bslab_live = bslab < nslab;
    const uint32_t qoff = (static_cast<uint32_t>(bslab) * CK * kSlab * 16u + lane * 16u) | (bslab_live ? 0u : 0x80000000u);
    const int bchunk = 2 * (wave & 1);
    // zero words (even wave) or scales (odd wave) of slab wave / 2
    const bool zkind = (wave & 1) == 0;
    const uint32_t zsoff = zkind ? ((static_cast<uint32_t>(bslab) * 32u + lane * 4u) | (lane < 8 && bslab_live ? 0u : 0x80000000u))
                                 : ((static_cast<uint32_t>(bslab) * 128u + lane * 4u) | (lane < 32 && bslab_live ? 0u : 0x80000000u));
    const int zsstride = zkind ? (Npad >> 3) * 4 : Npad * 2;
    const __amdgpu_buffer_rsrc_t zsr = zkind ? zr : sr;
    const int zsdst = C::Z_OFF + (wave >> 1) * 512 + (zkind ? 0 : 256);

    auto issue_item = [&](int kt, uint8_t* dst, int it) {
        const int kc = kt < KT ? kt : KT - 1;
        const int g = g0 + kc;
        if (it < C::PA) {
            dma16_s(xr, dst + (wave * C::PA + it) * kLine, xoff[it], g * 256);
        } else if (it < C::PA + C::PB) {
            const int c = bchunk + (it - C::PA);
            dma16_s(qr, dst + C::A_BYTES + ((wave >> 1) * 4 + c) * kLine, qoff, (g * 4 + c) * kSlab * 16);
        } else {
            dma4_s(zsr, dst + zsdst, zsoff, g * zsstride);
        }
    };
    auto issue = [&](int kt, uint8_t* dst) {
#pragma unroll
        for (int it = 0; it < C::P; ++it) issue_item(kt, dst, it);
    };

    uint32_t vmagic;
    asm("v_mov_b32 %0, 0x64006400" : "=v"(vmagic));
    const uint32_t mlo = __builtin_amdgcn_readfirstlane(0x000F000Fu);
    const int col = 32 * (wave & 1) + (lane & 31);       // this lane's column inside its slab
    const uint32_t zsh = (col & 7) * 4;

    float16_t acc[C::MB];
#pragma unroll
    for (int i = 0; i < C::MB; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][r] = 0.f;

    // x operand of k16 step s, block i: row 32 i + l%32, 16-byte chunk
    // 2 s + l/32, XOR-swizzled by the row's low 4 bits; block i is 8 KiB on.
    int a_off[8];
#pragma unroll
    for (int s = 0; s < 8; ++s) a_off[s] = (lane & 31) * 256 + (((2 * s + h) ^ (lane & 15)) << 4);
    // the lane's two words of chunk c: word h (k-octet 4c + h) and word 2 + h
    const int b_off = C::A_BYTES + (wave >> 1) * 4 * kLine + col * 16 + h * 4;
    const int z_off = C::Z_OFF + (wave >> 1) * 512 + (col >> 3) * 4;
    const int s_off = C::Z_OFF + (wave >> 1) * 512 + 256 + col * 2;

    uint32_t q[8];                                       // the stage's eight words, one per k16 step
    uint32_t zz = 0, ss = 0;
    half8_t af[2][C::MB], bf[2];
    auto widen = [&](int s, half8_t& b) {
        const uint32_t w = q[s];
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
        for (int i = 0; i < C::MB; ++i) dst[i] = *reinterpret_cast<const half8_t*>(src + a_off[s] + i * 32 * 256);
    };
    auto head = [&](const uint8_t* src) {
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const uint32_t* wp = reinterpret_cast<const uint32_t*>(src + b_off + c * kLine);
            q[2 * c] = wp[0];
            q[2 * c + 1] = wp[2];
        }
        const uint32_t zw = *reinterpret_cast<const uint32_t*>(src + z_off);
        const uint32_t sh = *reinterpret_cast<const uint16_t*>(src + s_off);
        read_a(src, 0, af[0]);
        zz = (0x6400u + ((zw >> zsh) & 15u) + zero_bias) * 0x10001u;
        ss = sh * 0x10001u;
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
    auto run_stage = [&](int kt, const uint8_t* cur, const uint8_t* nxt, uint8_t* prv) {
#pragma unroll
        for (int s = 0; s < 7; ++s) {
            const int c = s & 1, n = c ^ 1;
            constexpr int kLo[8] = {0, C::P * 1 / 7, C::P * 2 / 7, C::P * 3 / 7, C::P * 4 / 7, C::P * 5 / 7,
                                    C::P * 6 / 7, C::P};
#pragma unroll
            for (int it = kLo[s]; it < kLo[s + 1]; ++it) issue_item(kt + NS - 1, prv, it);
            read_a(cur, s + 1, af[n]);
            widen(s + 1, bf[n]);
            mfmas(c, 0, C::MB);
#pragma unroll
            for (int i = 0; i < C::MB; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);                  // DS read
                if (i < kLo[s + 1] - kLo[s]) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);   // copy
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                  // MFMA
                __builtin_amdgcn_sched_group_barrier(0x002, kV, 0);                 // VALU
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        mfmas(1, 0, (C::MB + 1) / 2);
        __builtin_amdgcn_sched_barrier(0);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        wait_vmcnt_s<C::P * (NS - 2)>();
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        head(nxt);
        mfmas(1, (C::MB + 1) / 2, C::MB);
        __builtin_amdgcn_sched_barrier(0);
        widen(0, bf[0]);
    };

#pragma unroll
    for (int d = 0; d < NS - 1; ++d) issue(d, bufs[d]);
    wait_vmcnt_s<C::P * (NS - 2)>();
    __builtin_amdgcn_s_barrier();
    head(bufs[0]);
    widen(0, bf[0]);
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
    // no copy may land in LDS after this point (the stage buffers are reused)
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

    if (S > 1) {
        // ---- K split: publish this split's partial tile, the last arriver adds all S.
        // Partial layout per (tile, split): [wave][block i][register quad rq][lane] float4.
        constexpr uint32_t kPart = TM * C::TN * 4;
        const __amdgpu_buffer_rsrc_t wr = rsrc_s(ws, ws_bytes);
        unsigned* const counters = reinterpret_cast<unsigned*>(ws);
        const uint32_t base = kSkCounterBytes + static_cast<uint32_t>(tile * S) * kPart;
        const uint32_t lo = (static_cast<uint32_t>(wave) * C::MB * 4) * 1024u + lane * 16u;
#pragma unroll
        for (int i = 0; i < C::MB; ++i)
#pragma unroll
            for (int rq = 0; rq < 4; ++rq) {
                const int4_t v = {__float_as_int(acc[i][4 * rq]), __float_as_int(acc[i][4 * rq + 1]),
                                  __float_as_int(acc[i][4 * rq + 2]), __float_as_int(acc[i][4 * rq + 3])};
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
        // registers; the next partial's loads are in flight while the
        // current one is added
        auto fetch = [&](int q2, float16_t (&dst)[C::MB]) {
            if (q2 == p) {
#pragma unroll
                for (int i = 0; i < C::MB; ++i) dst[i] = acc[i];
                return;
            }
#pragma unroll
            for (int i = 0; i < C::MB; ++i)
#pragma unroll
                for (int rq = 0; rq < 4; ++rq) {
                    const int4_t t =
                        __builtin_amdgcn_raw_buffer_load_b128(wr, lo + (i * 4 + rq) * 1024u, base + q2 * kPart, 16);
#pragma unroll
                    for (int e = 0; e < 4; ++e) dst[i][4 * rq + e] = __int_as_float(t[e]);
                }
        };
        float16_t sum[C::MB], cur[C::MB], nxt[C::MB];
        fetch(0, cur);
        for (int q2 = 0; q2 < S; ++q2) {
            if (q2 + 1 < S) fetch(q2 + 1, nxt);
#pragma unroll
            for (int i = 0; i < C::MB; ++i) {
                if (q2 == 0) {
                    sum[i] = cur[i];
                } else {
#pragma unroll
                    for (int r = 0; r < 16; ++r) sum[i][r] += cur[i][r];
                }
                cur[i] = nxt[i];
            }
        }
#pragma unroll
        for (int i = 0; i < C::MB; ++i) acc[i] = sum[i];
    }

    // ---- fp16 epilogue.  Block i: register r of lane l holds output row
    // 32 i + l%32 and column 8 (r/4) + 4 (l/32) + r%4 of the wave's 32;
    // swapping the upper lanes of quad g with the lower lanes of quad g+1
    // leaves lane l with the 8 consecutive columns 8 g + 8 (l/32), g even.
    auto pack = [&](int i, int g, uint32_t (&pk)[4]) {
#pragma unroll
        for (int d = 0; d < 2; ++d) {
            const uint32_t x0 = f2h(acc[i][4 * g + 2 * d]) | (uint32_t(f2h(acc[i][4 * g + 2 * d + 1])) << 16);
            const uint32_t x1 = f2h(acc[i][4 * g + 4 + 2 * d]) | (uint32_t(f2h(acc[i][4 * g + 5 + 2 * d])) << 16);
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
        for (int i = 0; i < C::MB; ++i)
#pragma unroll
            for (int g = 0; g < 4; g += 2) {
                uint32_t pk[4];
                pack(i, g, pk);
                *reinterpret_cast<uint4*>(srow(32 * i + (lane & 31)) + (32 * wave + 8 * g + 8 * h) * 2) =
                    make_uint4(pk[0], pk[1], pk[2], pk[3]);
            }
        __syncthreads();
        constexpr int CPR = C::TN / 8;                   // 16-byte chunks per row
        constexpr int RPI = 64 * NWV / CPR;              // rows per workgroup-wide pass
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
    for (int i = 0; i < C::MB; ++i) {
        const int row = m0 + 32 * i + (lane & 31);
#pragma unroll
        for (int g = 0; g < 4; g += 2) {
            uint32_t pk[4];
            pack(i, g, pk);
            const int c0 = n0 + 32 * wave + 8 * g + 8 * h;
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

#define MCV_SK_SHAPES(X) X(128, 8, 3) X(128, 4, 3) X(64, 8, 3) X(64, 4, 3) X(32, 4, 3)

SkFn pick_sk(int tm, int nwv, int ns) {
#define MCV_SK_PICK(a, b, c) \
    if (tm == a && nwv == b && ns == c) return w4a16_gemm_sk_kernel<a, b, c>;
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
    return pick_sk(c.tm, c.nwv, c.ns) != nullptr && c.splits >= 1 && c.splits <= 64 && K % kGroup == 0 &&
           (K / kGroup) % c.splits == 0 && (c.splits == 1 || w4a16_sk_tiles(M, N, c) <= kSkMaxSplitTiles);
}

int launch_w4a16_gemm_sk(const void* x, int64_t M, int64_t K, int64_t N, const void* qw, const void* scales,
                         const void* zeros, int zero_bias, void* out, const SkConfig& c, void* ws, int64_t ws_bytes,
                         hipStream_t stream) {
    SkFn fn = pick_sk(c.tm, c.nwv, c.ns);
    if (fn == nullptr || !w4a16_sk_config_valid(M, K, N, c))
        return fail(MCV_ERR_INVALID_ARG,
                    "w4a16 GEMM: no split-K kernel for TM=%d waves=%d NS=%d S=%d at M=%lld K=%lld N=%lld (S must divide "
                    "K/128, and a split needs at most %d tiles)",
                    c.tm, c.nwv, c.ns, c.splits, (long long)M, (long long)K, (long long)N, kSkMaxSplitTiles);
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
    const int col_major = M < N ? 1 : 0;
    hipLaunchKernelGGL(fn, dim3(static_cast<unsigned>(total)), dim3(64 * c.nwv), 0, stream,
                       static_cast<const uint16_t*>(x), static_cast<const uint4*>(qw),
                       static_cast<const uint16_t*>(scales), static_cast<const uint32_t*>(zeros),
                       static_cast<uint32_t>(zero_bias), static_cast<uint16_t*>(out), static_cast<int>(M),
                       static_cast<int>(K), static_cast<int>(N), static_cast<int>(nslab), static_cast<int>(m_tiles),
                       static_cast<int>(n_tiles), c.splits, col_major, static_cast<uint8_t*>(ws),
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
                      const void* zeros, int zero_bias, void* out, int tm, int waves, int stages, int splits,
                      void* workspace, int64_t workspace_bytes, mcv_stream_t stream) {
    if (!x || !out || !qw || !scales || !zeros) return fail(MCV_ERR_INVALID_ARG, "mcv_w4a16_gemm_sk: null pointer");
    if (zero_bias != 0 && zero_bias != 1) return fail(MCV_ERR_INVALID_ARG, "mcv_w4a16_gemm_sk: zero_bias must be 0 or 1");
    if (K <= 0 || K % kGroup != 0 || M <= 0 || M > (int64_t(1) << 30) || N <= 0 || N > (int64_t(1) << 30))
        return fail(MCV_ERR_SHAPE, "mcv_w4a16_gemm_sk: bad shape (M=%lld K=%lld N=%lld)", (long long)M, (long long)K,
                    (long long)N);
    if (reinterpret_cast<uintptr_t>(x) % 16 != 0) return fail(MCV_ERR_INVALID_ARG, "mcv_w4a16_gemm_sk: x must be 16-byte aligned");
    int rc = require_device();
    if (rc != MCV_OK) return rc;
    return launch_w4a16_gemm_sk(x, M, K, N, qw, scales, zeros, zero_bias, out, SkConfig{tm, waves, stages, splits},
                                workspace, workspace_bytes, static_cast<hipStream_t>(stream));
}

}  // extern "C"
