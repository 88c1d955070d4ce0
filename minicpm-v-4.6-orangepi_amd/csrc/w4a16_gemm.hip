// w4a16_gemm.hip -- W4A16 prefill GEMM (M > 1) on fp16 MFMA, gfx950.
//
// out[M][N] = x[M][K] . W[K][N], W in the slab-64 int4 layout.
//
// Each wave owns one 64-column slab and TM rows (a TM x 64 tile, TM/32 x 2
// blocks of v_mfma_f32_32x32x16_f16 with fp32 accumulation).  A workgroup is
// four waves: WN waves side by side along N share the x rows, KS groups of
// them split K (KS > 1 sums the partial tiles through LDS at the end).
//
//   B (weights) stay packed until the MFMA needs them.  A wave reads its
//   slab's 16-byte lane chunks -- one contiguous 1 KiB line per 32 k -- parks
//   them in its own LDS ring (so no register lives across stages) and turns
//   them into MFMA B operands in registers.  The slab layout gives lane l
//   column l; the 32x32x16 operand wants lanes 0-31 / 32-63 to carry k-octets
//   0 / 1 of the SAME 32 columns.  One v_permlane32_swap per pair of packed
//   words (octets 2t and 2t+1) exchanges the upper half of the first with the
//   lower half of the second: afterwards the first word is the operand of
//   columns 0-31 and the second that of columns 32-63, still as nibbles.  They
//   are then widened with the fp16 exponent trick ((1024 + q) - (1024 + z) is
//   exact) and multiplied by the scale once (RNE): the same fp16 values
//   mcv_w4a16_dequant materialises.  Weights are dequantised once per
//   workgroup (KS > 1) or once per wave column (WN waves never share a slab).
//   A (activations) go global -> registers -> LDS through a buffer resource
//   whose range check zero-fills rows past M, and are read back as 16-byte
//   operand runs; the 272-byte row pitch keeps those reads conflict-free.
//   Both rings are double buffered with one barrier per 128-k stage (one
//   quantisation group, so a wave's scales and zeros are constant over it):
//   stage kt+1's global loads are in flight while stage kt's MFMAs run.
//
// Tiles are numbered so that each XCD (workgroups go to the 8 XCDs round
// robin) receives a contiguous run of tile rows: the x rows and slabs it reads
// stay in its own L2.
//
// The reference has no M > 1 quantised path: its prefill runs dense fp16
// aclnnMm through matmul_b_transposed (src/csrc/lib/decoder_layer.cpp:459-462,
// 656-659, 857-860; src/csrc/lib/ops.cpp:159-322).
#include <algorithm>
#include <cstdlib>
#include <cstring>

#include "common.h"

namespace mcv {

int launch_w4a16_gemv(const void* x, int64_t M, int64_t K, int64_t N, const void* qw, const void* scales,
                      const void* zeros, int zero_bias, void* out, hipStream_t stream);
int choose_w4a16_lds(int64_t M, int64_t K, int64_t N, int* tm, int* ns, int* kp);
int launch_w4a16_gemm_lds(const void* x, int64_t M, int64_t K, int64_t N, const void* qw, const void* scales,
                          const void* zeros, int zero_bias, void* out, int tm, int ns, int kp, hipStream_t stream);

namespace {


// Workgroup b of `total` is dispatched to XCD b % 8; hand XCD x the
// contiguous logical range [x * per + min(x, rem), ...).
__device__ __forceinline__ int xcd_tile(int b, int total) {
    const int per = total >> 3, rem = total & 7, x = b & 7, i = b >> 3;
    return x * per + (x < rem ? x : rem) + i;
}

// Raw buffer resource over `bytes` bytes from `base`: loads at offsets past
// the end return zero (gfx9 dword 3 = 0x00020000).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, static_cast<int>(bytes), 0x00020000);
}

// TM rows per wave, WN waves along N (one slab each), KS k-parts, BK k per
// stage, DEPTH stages of global prefetch (register staging sets).
template <int TM, int WN, int KS, int BK, int DEPTH>
struct Cfg {
    static constexpr int NW = WN * KS;                          // waves per workgroup
    static constexpr int NT = 64 * NW;
    static_assert(NW == 4 || NW == 8, "four or eight waves");
    static_assert(TM == 32 || TM == 64 || TM == 128, "TM");
    static_assert(BK == 64 || BK == 128, "BK");
    static_assert(DEPTH == 1 || DEPTH == 2, "DEPTH");
    static constexpr int MB = TM / 32;                          // 32-row MFMA blocks per wave
    static constexpr int NCH = BK / kChunkK;                    // packed chunks per stage
    static constexpr int NSTEP = BK / 16;                       // k16 MFMA steps per stage
    static constexpr int PITCH = BK + 8;                        // halves per LDS row of the x tile
    static constexpr int kAThreads = 64 * WN;                   // threads loading one k-part's x tile
    static constexpr int kAVec = TM * (BK / 8) / kAThreads;     // 16-byte vectors per thread per stage
    static_assert(kAVec >= 1 && kAVec <= 8, "x staging registers");
    static constexpr int kAStage = TM * PITCH * 2;              // bytes of one x stage buffer
    static constexpr int kBStage = (NCH + 1) * 64 * 16;         // bytes of one wave's weight stage
    static constexpr int kBOff = KS * 2 * kAStage;
    static constexpr int kLdsBytes = kBOff + NW * 2 * kBStage;
    static_assert(kLdsBytes <= 160 * 1024, "LDS");
    // KS > 1: k-parts 1..KS-1 hand one 32-row block at a time to k-part 0.
    static_assert(KS == 1 || (KS - 1) * WN * 32 * 64 * 4 <= kLdsBytes, "reduction buffer");
};

template <int TM, int WN, int KS, int BK, int DEPTH>
__global__ __launch_bounds__(64 * WN * KS) void w4a16_gemm_kernel(
    const uint16_t* __restrict__ x, const uint4* __restrict__ qw, const uint16_t* __restrict__ scales,
    const uint32_t* __restrict__ zeros, uint32_t zero_bias, uint16_t* __restrict__ out, int M, int K, int N,
    int nslab, int n_tiles, int total_tiles, int col_major, int kx, float* __restrict__ part) {
    using C = Cfg<TM, WN, KS, BK, DEPTH>;
    __shared__ __attribute__((aligned(16))) uint8_t lds[C::kLdsBytes];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int kp = wave / WN;                  // k-part of this wave
    const int wn = wave - kp * WN;             // slab position inside the workgroup
    // Each XCD gets a contiguous run of tiles; col_major orders the run down
    // the columns of tiles (an XCD's L2 then holds a few weight slabs and the
    // x rows are what crosses XCDs), row-major along the rows.
    // kx > 1: each tile's K is cut into kx contiguous ranges of whole stage
    // sets (one BK stage per k-part), one workgroup each, and the fp32
    // partial tiles go to part[split][M][N] for the reduction kernel
    const int ts = xcd_tile(static_cast<int>(blockIdx.x), total_tiles * kx);
    const int tile = ts / kx, sx = ts - tile * kx;
    const int m_tiles = total_tiles / n_tiles;
    const int tm = col_major ? tile % m_tiles : tile / n_tiles;
    const int tn = col_major ? tile / m_tiles : tile - tm * n_tiles;
    const int m0 = tm * TM;
    const int slab = tn * WN + wn;
    const int Npad = nslab * kSlab;
    const int CK = K / kChunkK;                // packed chunks per slab
    const int T = K / (BK * KS);               // stage sets of all of K
    const int t0 = static_cast<int>(int64_t(sx) * T / kx);
    const int KT = static_cast<int>(int64_t(sx + 1) * T / kx) - t0;   // stages of this split's k-parts
    const int kbeg = (t0 * KS + kp * KT) * BK;

    uint8_t* As = lds + kp * 2 * C::kAStage;                  // this k-part's two x stage buffers
    uint8_t* Bs = lds + C::kBOff + wave * 2 * C::kBStage;     // this wave's two weight stage buffers

    // ---- x tile rows m0.. of this k-part: kAVec 16-byte vectors per thread.
    // Rows past M read as zero through the buffer resource's range check.
    const int rows_here = M - m0 < TM ? M - m0 : TM;
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(x + static_cast<size_t>(m0) * K, static_cast<uint32_t>(rows_here) * K * 2u);
    const int at = wn * 64 + lane;
    constexpr int kVecPerRow = BK / 8;
    struct Staging {
        uint4 a[C::kAVec];     // x vectors of one stage
        uint4 b[C::NCH + 1];   // packed weight chunks + raw (zero, zero, scale, scale) words
    };
    auto load_a = [&](int kt, Staging& st) {
        const int k0 = kbeg + kt * BK;
#pragma unroll
        for (int i = 0; i < C::kAVec; ++i) {
            const int idx = at + i * C::kAThreads;
            const uint32_t off = static_cast<uint32_t>((idx / kVecPerRow) * K + k0 + (idx % kVecPerRow) * 8) * 2u;
            st.a[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(xr, off, 0, 0));
        }
    };
    auto store_a = [&](int buf, const Staging& st) {
        uint8_t* dst = As + buf * C::kAStage;
#pragma unroll
        for (int i = 0; i < C::kAVec; ++i) {
            const int idx = at + i * C::kAThreads;
            *reinterpret_cast<uint4*>(dst + ((idx / kVecPerRow) * C::PITCH + (idx % kVecPerRow) * 8) * 2) = st.a[i];
        }
    };

    // ---- weights: NCH chunks of this wave's slab per stage, plus the zero
    // and scale words of the two columns this lane's operands carry.
    const int c0 = slab * kSlab + (lane & 31);   // column of the first operand (columns 0-31)
    const int c1 = c0 + 32;                      // column of the second operand (columns 32-63)
    // Buffer resources: a slab past the end reads as zero weights; its
    // scale/zero words may be any in-range values (its columns are never
    // stored).
    const __amdgpu_buffer_rsrc_t qr = make_rsrc(qw, static_cast<uint32_t>(nslab) * CK * kSlab * 16u);
    const __amdgpu_buffer_rsrc_t sr = make_rsrc(scales, static_cast<uint32_t>(K / kGroup) * Npad * 2u);
    const __amdgpu_buffer_rsrc_t zr = make_rsrc(zeros, static_cast<uint32_t>(K / kGroup) * (Npad >> 3) * 4u);
    const uint32_t qoff = (static_cast<uint32_t>(slab) * CK * kSlab + lane) * 16u;
    auto load_b = [&](int kt, Staging& st) {
        const int k0 = kbeg + kt * BK;
        const uint32_t g = static_cast<uint32_t>(k0 / kGroup);
#pragma unroll
        for (int c = 0; c < C::NCH; ++c)
            st.b[c] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                                                    qr, qoff + static_cast<uint32_t>(k0 / kChunkK + c) * kSlab * 16u, 0, 0));
        // Raw words only: deriving the operand constants here would make
        // the wave wait for this stage's loads before the current MFMAs.
        const uint32_t zrow = g * static_cast<uint32_t>(Npad >> 3) * 4u;
        const uint32_t srow = g * static_cast<uint32_t>(Npad) * 2u;
        st.b[C::NCH] = make_uint4(__builtin_amdgcn_raw_buffer_load_b32(zr, zrow + (c0 >> 3) * 4u, 0, 0),
                                  __builtin_amdgcn_raw_buffer_load_b32(zr, zrow + (c1 >> 3) * 4u, 0, 0),
                                  __builtin_amdgcn_raw_buffer_load_b16(sr, srow + c0 * 2u, 0, 0),
                                  __builtin_amdgcn_raw_buffer_load_b16(sr, srow + c1 * 2u, 0, 0));
    };
    auto store_b = [&](int buf, const Staging& st) {
        uint4* dst = reinterpret_cast<uint4*>(Bs + buf * C::kBStage) + lane;
#pragma unroll
        for (int c = 0; c <= C::NCH; ++c) dst[c * 64] = st.b[c];
    };
    // Item-wise forms of the four above (items: kAVec x vectors, NCH weight
    // chunks, one raw word quad), so a stage's traffic can be spread over the
    // k16 steps of the previous stage.
    constexpr int kItems = C::kAVec + C::NCH + 1;
    auto load_item = [&](int kt, Staging& st, int it) {
        const int k0 = kbeg + kt * BK;
        if (it < C::kAVec) {
            const int idx = at + it * C::kAThreads;
            const uint32_t off = static_cast<uint32_t>((idx / kVecPerRow) * K + k0 + (idx % kVecPerRow) * 8) * 2u;
            st.a[it] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(xr, off, 0, 0));
        } else if (it < C::kAVec + C::NCH) {
            const int c = it - C::kAVec;
            st.b[c] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                                                    qr, qoff + static_cast<uint32_t>(k0 / kChunkK + c) * kSlab * 16u, 0, 0));
        } else {
            const uint32_t g = static_cast<uint32_t>(k0 / kGroup);
            const uint32_t zrow = g * static_cast<uint32_t>(Npad >> 3) * 4u;
            const uint32_t srow = g * static_cast<uint32_t>(Npad) * 2u;
            st.b[C::NCH] = make_uint4(__builtin_amdgcn_raw_buffer_load_b32(zr, zrow + (c0 >> 3) * 4u, 0, 0),
                                      __builtin_amdgcn_raw_buffer_load_b32(zr, zrow + (c1 >> 3) * 4u, 0, 0),
                                      __builtin_amdgcn_raw_buffer_load_b16(sr, srow + c0 * 2u, 0, 0),
                                      __builtin_amdgcn_raw_buffer_load_b16(sr, srow + c1 * 2u, 0, 0));
        }
    };
    auto store_item = [&](int buf, const Staging& st, int it) {
        if (it < C::kAVec) {
            const int idx = at + it * C::kAThreads;
            *reinterpret_cast<uint4*>(As + buf * C::kAStage + ((idx / kVecPerRow) * C::PITCH + (idx % kVecPerRow) * 8) * 2) =
                st.a[it];
        } else {
            const int c = it - C::kAVec;
            (reinterpret_cast<uint4*>(Bs + buf * C::kBStage) + lane)[c * 64] = st.b[c];
        }
    };

    uint32_t vmagic;
    asm("v_mov_b32 %0, 0x64006400" : "=v"(vmagic));
    const uint32_t mlo = __builtin_amdgcn_readfirstlane(0x000F000Fu);

    float16_t acc[C::MB][2];
#pragma unroll
    for (int i = 0; i < C::MB; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    // One stage = NSTEP k16 steps.  Step s+1's x operands (LDS reads) and
    // weight operands (permlane + widening, VALU) are produced while step s's
    // MFMAs run: each step is its own scheduling region, laid out as (DS
    // read, MFMA, VALU run) groups so the VALU work issues in the MFMA shadow
    // and the reads are in flight a full step before their use.
    constexpr int kNM = 2 * C::MB;                               // MFMAs per step
    constexpr int kValuPerMfma = (31 + kNM - 1) / kNM;           // widening VALU ops per step: 31
    auto compute = [&](int buf, auto&& per_step) {
        const uint8_t* A = As + buf * C::kAStage + ((lane & 31) * C::PITCH + (lane >> 5) * 8) * 2;
        const uint4* B = reinterpret_cast<const uint4*>(Bs + buf * C::kBStage) + lane;
        uint4 q[C::NCH];
#pragma unroll
        for (int c = 0; c < C::NCH; ++c) q[c] = B[c * 64];
        const uint4 raw = B[C::NCH * 64];
        // zz = half2(1024 + z), ss = half2(s) for the two operand columns
        const uint32_t zsh = (lane & 7) * 4;   // c0 & 7 == c1 & 7 == lane & 7
        const uint4 zs = make_uint4((0x6400u + ((raw.x >> zsh) & 15u) + zero_bias) * 0x10001u,
                                    (0x6400u + ((raw.y >> zsh) & 15u) + zero_bias) * 0x10001u,
                                    (raw.z & 0xffffu) * 0x10001u, (raw.w & 0xffffu) * 0x10001u);
        auto widen = [&](int s, half8_t& b0, half8_t& b1) {
            const int c = s >> 1, t = s & 1;
            const uint32_t words[4] = {q[c].x, q[c].y, q[c].z, q[c].w};
            // lanes 32-63 of octet 2t <-> lanes 0-31 of octet 2t+1
            const auto sw = __builtin_amdgcn_permlane32_swap(words[2 * t], words[2 * t + 1], false, false);
            dequant_pair(sw[0], sw[1], zs.x, zs.z, zs.y, zs.w, mlo, vmagic, b0, b1);
        };
        half8_t af[2][C::MB], bf[2][2];
#pragma unroll
        for (int i = 0; i < C::MB; ++i) af[0][i] = *reinterpret_cast<const half8_t*>(A + i * 32 * C::PITCH * 2);
        widen(0, bf[0][0], bf[0][1]);
#pragma unroll
        for (int s = 0; s < C::NSTEP; ++s) {
            const int cur = s & 1, nxt = cur ^ 1;
            if (s + 1 < C::NSTEP) {
#pragma unroll
                for (int i = 0; i < C::MB; ++i)
                    af[nxt][i] = *reinterpret_cast<const half8_t*>(A + (i * 32 * C::PITCH + (s + 1) * 16) * 2);
                widen(s + 1, bf[nxt][0], bf[nxt][1]);
            }
#pragma unroll
            for (int i = 0; i < C::MB; ++i) {
                // weights as the row operand: the block is the transposed
                // 32x32 tile (output column x output row), see the epilogue
                acc[i][0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(bf[cur][0], af[cur][i], acc[i][0], 0, 0, 0);
                acc[i][1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(bf[cur][1], af[cur][i], acc[i][1], 0, 0, 0);
            }
            per_step(s);
            if (s + 1 < C::NSTEP) {
#pragma unroll
                for (int i = 0; i < kNM; ++i) {
                    if (i < C::MB) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);   // DS read
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                  // MFMA
                    __builtin_amdgcn_sched_group_barrier(0x002, kValuPerMfma, 0);       // VALU
                }
            }
            __builtin_amdgcn_sched_barrier(0);   // one scheduling region per k16 step
        }
    };

    Staging s0, s1;
    if constexpr (DEPTH == 2) {
        // Two register staging sets alternate, so a stage's loads are issued
        // two stages before they are needed.  The reload is unconditional
        // (the last two stages re-read the final stage): with a single path
        // the waitcnt pass counts exactly and the store of `other` waits only
        // for `other`'s own loads.  LDS is double buffered, one barrier per
        // stage.
        load_a(0, s0);
        load_b(0, s0);
        load_a(KT > 1 ? 1 : 0, s1);
        load_b(KT > 1 ? 1 : 0, s1);
        store_a(0, s0);
        store_b(0, s0);
        __syncthreads();
        // The reload of `mine` and the LDS store of `other` are spread over
        // the k16 steps so they issue under the MFMAs.
        auto step = [&](int kt, Staging& mine, Staging& other) {
            const int kn = kt + 2 < KT ? kt + 2 : KT - 1;
            const bool store = kt + 1 < KT;
            const int nb = (kt + 1) & 1;
            compute(kt & 1, [&](int s) {
#pragma unroll
                for (int it = s * kItems / C::NSTEP; it < (s + 1) * kItems / C::NSTEP; ++it) {
                    if (store) store_item(nb, other, it);
                    load_item(kn, mine, it);
                }
            });
            __syncthreads();
        };
        int kt = 0;
        for (; kt + 1 < KT; kt += 2) {
            step(kt, s0, s1);
            step(kt + 1, s1, s0);
        }
        if (kt < KT) step(kt, s0, s1);
    } else {
        // One staging set: stage kt+1's loads fly while stage kt computes
        // (with eight waves a second wave per SIMD covers the rest).
        load_a(0, s0);
        load_b(0, s0);
        store_a(0, s0);
        store_b(0, s0);
        __syncthreads();
        for (int kt = 0; kt < KT; ++kt) {
            const int kn = kt + 1 < KT ? kt + 1 : KT - 1;
            load_a(kn, s0);
            load_b(kn, s0);
            compute(kt & 1, [](int) {});
            if (kt + 1 < KT) {
                store_a((kt + 1) & 1, s0);
                store_b((kt + 1) & 1, s0);
            }
            __syncthreads();
        }
    }

    // ---- k-parts 1..KS-1 hand their partial tiles to k-part 0 through LDS,
    // one 32-row block at a time (the stage buffers are free by now).
    if constexpr (KS > 1) {
        float* red = reinterpret_cast<float*>(lds);
#pragma unroll
        for (int i = 0; i < C::MB; ++i) {
            if (kp > 0) {
                float* dst = red + ((kp - 1) * WN + wn) * 2 * 16 * 64 + lane;
#pragma unroll
                for (int j = 0; j < 2; ++j)
#pragma unroll
                    for (int r = 0; r < 16; ++r) dst[(j * 16 + r) * 64] = acc[i][j][r];
            }
            __syncthreads();
            if (kp == 0) {
#pragma unroll
                for (int p = 1; p < KS; ++p) {
                    const float* src = red + ((p - 1) * WN + wn) * 2 * 16 * 64 + lane;
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

    if (part != nullptr) {
        // the split's fp32 partial tile: register quad g of block (i, j) is
        // four consecutive columns of one row
        float* const pd = part + static_cast<size_t>(sx) * M * N;
        const bool vec4 = (N & 3) == 0 && (reinterpret_cast<uintptr_t>(part) & 15) == 0;
#pragma unroll
        for (int i = 0; i < C::MB; ++i) {
            const int row = m0 + 32 * i + (lane & 31);
            if (row >= M) continue;
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const int col = slab * kSlab + 32 * j + 8 * g + 4 * (lane >> 5);
                    if (col >= N) continue;
                    float* dst = pd + static_cast<size_t>(row) * N + col;
                    if (vec4) {
                        *reinterpret_cast<float4*>(dst) =
                            make_float4(acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]);
                    } else {
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            if (col + e < N) dst[e] = acc[i][j][4 * g + e];
                    }
                }
        }
        return;
    }

    // Transposed 32x32 blocks: register r of lane l holds output row
    // 32 i + l%32 and column 32 j + 8 (r/4) + 4 (l/32) + r%4 -- four
    // consecutive columns per register quad.  Swapping the upper lanes of quad
    // g with the lower lanes of quad g+1 leaves lane l with the 8 consecutive
    // columns 32 j + 8 g + 8 (l/32), g even: one 16-byte store.
    const bool vec_ok = (N & 7) == 0 && (reinterpret_cast<uintptr_t>(out) & 15) == 0;
#pragma unroll
    for (int i = 0; i < C::MB; ++i) {
        const int row = m0 + 32 * i + (lane & 31);
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int g = 0; g < 4; g += 2) {
                uint32_t p[4];
#pragma unroll
                for (int d = 0; d < 2; ++d) {
                    const uint32_t x0 = f2h(acc[i][j][4 * g + 2 * d]) | (uint32_t(f2h(acc[i][j][4 * g + 2 * d + 1])) << 16);
                    const uint32_t x1 = f2h(acc[i][j][4 * g + 4 + 2 * d]) | (uint32_t(f2h(acc[i][j][4 * g + 5 + 2 * d])) << 16);
                    const auto sw = __builtin_amdgcn_permlane32_swap(x0, x1, false, false);
                    p[d] = sw[0];
                    p[2 + d] = sw[1];
                }
                const int col = slab * kSlab + 32 * j + 8 * g + 8 * (lane >> 5);
                if (row >= M || col >= N) continue;
                uint16_t* dst = out + static_cast<size_t>(row) * N + col;
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

// out = fp16 RNE of the KX partial tiles added in split order, four
// elements per thread (the same order on every call: deterministic).  KX is
// a compile-time count so every partial's load is issued before the first
// add.
template <int KX>
__global__ __launch_bounds__(256) void w4a16_splitk_reduce_kernel(const float* __restrict__ part, int64_t mn,
                                                                 uint16_t* __restrict__ out) {
    const int64_t i0 = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) * 4;
    if (i0 >= mn) return;
    if (i0 + 4 <= mn && (mn & 3) == 0 && (reinterpret_cast<uintptr_t>(out) & 7) == 0) {
        float4 v[KX];
#pragma unroll
        for (int s = 0; s < KX; ++s) v[s] = *reinterpret_cast<const float4*>(part + static_cast<size_t>(s) * mn + i0);
        float4 a = v[0];
#pragma unroll
        for (int s = 1; s < KX; ++s) {
            a.x += v[s].x;
            a.y += v[s].y;
            a.z += v[s].z;
            a.w += v[s].w;
        }
        *reinterpret_cast<uint2*>(out + i0) =
            make_uint2(f2h(a.x) | (uint32_t(f2h(a.y)) << 16), f2h(a.z) | (uint32_t(f2h(a.w)) << 16));
        return;
    }
    for (int64_t i = i0; i < i0 + 4 && i < mn; ++i) {
        float a = part[i];
#pragma unroll
        for (int s = 1; s < KX; ++s) a += part[static_cast<size_t>(s) * mn + i];
        out[i] = f2h(a);
    }
}

using ReduceFn = void (*)(const float*, int64_t, uint16_t*);

ReduceFn pick_reduce(int kx) {
    switch (kx) {
        case 2: return w4a16_splitk_reduce_kernel<2>;
        case 3: return w4a16_splitk_reduce_kernel<3>;
        case 4: return w4a16_splitk_reduce_kernel<4>;
        case 5: return w4a16_splitk_reduce_kernel<5>;
        case 6: return w4a16_splitk_reduce_kernel<6>;
        case 7: return w4a16_splitk_reduce_kernel<7>;
        default: return w4a16_splitk_reduce_kernel<8>;
    }
}

struct Shape {
    int tm, wn, ks, bk, depth;
    int waves() const { return wn * ks; }
};

using GemmFn = void (*)(const uint16_t*, const uint4*, const uint16_t*, const uint32_t*, uint32_t, uint16_t*, int,
                        int, int, int, int, int, int, int, float*);

#define MCV_W4_SHAPES(X)                                                                              \
    X(128, 4, 1, 128, 2) X(128, 4, 2, 64, 1) X(64, 4, 2, 64, 1) X(64, 2, 4, 64, 1) X(64, 2, 2, 128, 2) \
    X(64, 4, 1, 128, 2) X(32, 4, 1, 128, 2) X(32, 2, 2, 128, 2) X(32, 1, 4, 128, 2) X(32, 2, 4, 64, 1)

GemmFn pick(const Shape& s) {
#define MCV_PICK(a, b, c, d, e) \
    if (s.tm == a && s.wn == b && s.ks == c && s.bk == d && s.depth == e) return w4a16_gemm_kernel<a, b, c, d, e>;
    MCV_W4_SHAPES(MCV_PICK)
#undef MCV_PICK
    return nullptr;
}

constexpr Shape kShapes[] = {
#define MCV_LIST(a, b, c, d, e) {a, b, c, d, e},
    MCV_W4_SHAPES(MCV_LIST)
#undef MCV_LIST
};

int64_t tiles_of(const Shape& s, int64_t M, int64_t nslab) {
    return ceil_div(M, s.tm) * ceil_div(nslab, s.wn);
}

// The first listed shape (largest tiles first) whose grid covers most of the
// 256 CUs; failing that, the shape with the most workgroups.
// MCV_W4GEMM_SHAPE="TM,WN,KS,BK,DEPTH" overrides it for tuning sweeps.
Shape choose_shape(int64_t M, int64_t K, int64_t nslab) {
    static const char* const e = std::getenv("MCV_W4GEMM_SHAPE");      // read once per process
    if (e != nullptr) {
        Shape s{0, 0, 0, 0, 0};
        if (std::sscanf(e, "%d,%d,%d,%d,%d", &s.tm, &s.wn, &s.ks, &s.bk, &s.depth) == 5 && pick(s) &&
            K % (int64_t(s.bk) * s.ks) == 0)
            return s;
    }
    Shape best{0, 0, 0, 0, 0};
    int64_t best_tiles = -1;
    for (const Shape& s : kShapes) {
        if (K % (int64_t(s.bk) * s.ks) != 0) continue;
        const int64_t t = tiles_of(s, M, nslab);
        if (t >= 200) return s;
        if (t > best_tiles) {
            best_tiles = t;
            best = s;
        }
    }
    return best;
}

// Workgroups per tile along K.  A grid far below the 256 CUs (few rows, long
// K: M=128, K=3584, N=1024 gives 64 tiles) streams each tile's weights and x
// rows through one CU; cutting K into kx ranges puts kx CUs on every tile,
// at the cost of kx fp32 partial tiles and a reduction launch.  Up to 8
// ways, toward 200 workgroups, with at most 8 MB of partial tiles.
// MCV_W4GEMM_SPLITK=n (1..8) forces n ways where the grid is small (read
// once per process; tuning sweeps).
int splitk_ways(const Shape& s, int64_t M, int64_t K, int64_t N) {
    const int64_t t = tiles_of(s, M, ceil_div(N, kSlab));
    if (t >= 128) return 1;
    static const int forced = [] {
        const char* const e = std::getenv("MCV_W4GEMM_SPLITK");
        const int v = e != nullptr ? std::atoi(e) : 0;
        return v >= 1 && v <= 8 ? v : 0;
    }();
    const int64_t want = forced > 0 ? forced : ceil_div(200, t);
    int64_t kx = std::min<int64_t>({want, 8, K / (int64_t(s.bk) * s.ks)});
    while (kx > 1 && kx * M * N * 4 > (int64_t(8) << 20)) --kx;
    return static_cast<int>(kx < 1 ? 1 : kx);
}

// Few rows: the GEMV streams the weights once per row and still beats the
// MFMA GEMM, whose tile count is M/TM * N/TN, until the output reaches about
// 64K elements (MI355X, graph-replayed, rotated weights: K=1024 N=3584 M=16
// 5.7 us against 7.0; K=3584 N=1024 M=48 12.4 against 12.5; K=1024 N=6144
// crosses over near M=11).
bool w4a16_prefers_gemv(int64_t M, int64_t N) { return M >= 1 && (M < 8 || M * N < 65536); }

// The LDS-staged kernel (w4a16_gemm_lds.hip) where its tall tiles fill the
// chip, the register-staged one otherwise; MCV_W4GEMM_KERNEL=regs forces the
// latter (read once per process).
bool w4a16_uses_lds(int64_t M, int64_t K, int64_t N, int* tm, int* ns, int* kp) {
    static const bool regs_only = [] {
        const char* const e = std::getenv("MCV_W4GEMM_KERNEL");
        return e != nullptr && std::strcmp(e, "regs") == 0;
    }();
    return !regs_only && choose_w4a16_lds(M, K, N, tm, ns, kp) == 0;
}

}  // namespace

// Bytes of workspace the register-staged path would use for M x K x N (0:
// no K split, or the LDS kernel or the GEMV takes the shape).
int64_t w4a16_gemm_workspace_bytes(int64_t M, int64_t K, int64_t N) {
    if (M < 1 || K <= 0 || N <= 0 || K % kGroup != 0 || w4a16_prefers_gemv(M, N)) return 0;
    int tm = 0, ns = 0, kp = 1;
    if (w4a16_uses_lds(M, K, N, &tm, &ns, &kp)) return 0;
    const Shape s = choose_shape(M, K, ceil_div(N, kSlab));
    const int kx = splitk_ways(s, M, K, N);
    return kx > 1 ? int64_t(kx) * M * N * 4 : 0;
}

int launch_w4a16_gemm_mfma(const void* x, int64_t M, int64_t K, int64_t N, const void* qw, const void* scales,
                           const void* zeros, int zero_bias, void* out, hipStream_t stream, void* ws = nullptr,
                           int64_t ws_bytes = 0) {
    if (!x || !out || !qw || !scales || !zeros) return fail(MCV_ERR_INVALID_ARG, "mcv_w4a16_gemm_mfma: null pointer");
    if (zero_bias != 0 && zero_bias != 1) return fail(MCV_ERR_INVALID_ARG, "mcv_w4a16_gemm_mfma: zero_bias must be 0 or 1");
    if (K <= 0 || K % kGroup != 0 || K > (int64_t(1) << 24))
        return fail(MCV_ERR_SHAPE, "mcv_w4a16_gemm_mfma: K must be a positive multiple of 128 (K=%lld)", (long long)K);
    if (N <= 0 || N > (int64_t(1) << 30) || M <= 0 || M > (int64_t(1) << 30))
        return fail(MCV_ERR_SHAPE, "mcv_w4a16_gemm_mfma: bad M/N (M=%lld N=%lld)", (long long)M, (long long)N);
    if (reinterpret_cast<uintptr_t>(x) % 16 != 0) return fail(MCV_ERR_INVALID_ARG, "mcv_w4a16_gemm_mfma: x must be 16-byte aligned");
    int rc = require_device();
    if (rc != MCV_OK) return rc;
    int tm = 0, ns = 0, kp = 1;
    if (w4a16_uses_lds(M, K, N, &tm, &ns, &kp))
        return launch_w4a16_gemm_lds(x, M, K, N, qw, scales, zeros, zero_bias, out, tm, ns, kp, stream);
    const int64_t nslab = ceil_div(N, kSlab);
    const Shape s = choose_shape(M, K, nslab);
    // Tile order, measured (MI355X, graph-replayed): down the tile columns
    // for M=2048, K=1024, N=3584 (23.4 us against 24.5 along the rows), along
    // the rows for M=2048, K=3584, N=1024 (25.8 against 28.5); even at M=128
    // and 512.  So: column-major when M < N.  MCV_W4GEMM_ORDER=0/1 overrides.
    int col_major = M < N ? 1 : 0;
    static const char* const order = std::getenv("MCV_W4GEMM_ORDER");  // read once per process
    if (order != nullptr) col_major = std::atoi(order) ? 1 : 0;
    const int64_t n_tiles = ceil_div(nslab, s.wn);
    const int64_t total = ceil_div(M, s.tm) * n_tiles;
    // a K split only into a caller's workspace that holds all of it
    int kx = ws != nullptr ? splitk_ways(s, M, K, N) : 1;
    if (kx > 1 && (ws_bytes < int64_t(kx) * M * N * 4 || (reinterpret_cast<uintptr_t>(ws) & 15) != 0)) kx = 1;
    // Buffer offsets are 32-bit: x inside one row tile (TM * K * 2 bytes) and
    // the packed weight (K * Npad / 2 bytes).
    if (total * kx > 0x7fffffff || K > (int64_t(1) << 22) || K * nslab * kSlab / 2 >= (int64_t(1) << 32))
        return fail(MCV_ERR_SHAPE, "mcv_w4a16_gemm_mfma: problem too large (M=%lld N=%lld)", (long long)M, (long long)N);
    float* const part = kx > 1 ? static_cast<float*>(ws) : nullptr;
    hipLaunchKernelGGL(pick(s), dim3(static_cast<unsigned>(total * kx)), dim3(64 * s.waves()), 0, stream,
                       static_cast<const uint16_t*>(x), static_cast<const uint4*>(qw),
                       static_cast<const uint16_t*>(scales), static_cast<const uint32_t*>(zeros),
                       static_cast<uint32_t>(zero_bias), static_cast<uint16_t*>(out), static_cast<int>(M),
                       static_cast<int>(K), static_cast<int>(N), static_cast<int>(nslab), static_cast<int>(n_tiles),
                       static_cast<int>(total), col_major, kx, part);
    if (kx == 1) return check_launch("w4a16_gemm_kernel");
    if ((rc = check_launch("w4a16_gemm_kernel")) != MCV_OK) return rc;
    const int64_t mn = M * N;
    hipLaunchKernelGGL(pick_reduce(kx), dim3(static_cast<unsigned>(ceil_div(ceil_div(mn, 4), 256))), dim3(256), 0,
                       stream, part, mn, static_cast<uint16_t*>(out));
    return check_launch("w4a16_splitk_reduce_kernel");
}

}  // namespace mcv

using namespace mcv;

extern "C" {

int mcv_w4a16_gemm_mfma(const void* x, int64_t M, int64_t K, int64_t N, const void* qw, const void* scales,
                        const void* zeros, int zero_bias, void* out, mcv_stream_t stream) {
    return launch_w4a16_gemm_mfma(x, M, K, N, qw, scales, zeros, zero_bias, out, static_cast<hipStream_t>(stream));
}

int64_t mcv_w4a16_gemm_workspace_bytes(int64_t M, int64_t K, int64_t N) { return w4a16_gemm_workspace_bytes(M, K, N); }

// mcv_w4a16_gemm with a caller-owned workspace, which lets the MFMA path
// split K across workgroups where the tile grid is small.
int mcv_w4a16_gemm_ws(const void* x, int64_t M, int64_t K, int64_t N, const void* qw, const void* scales,
                      const void* zeros, int zero_bias, void* out, void* workspace, int64_t workspace_bytes,
                      mcv_stream_t stream) {
    if (w4a16_prefers_gemv(M, N))
        return launch_w4a16_gemv(x, M, K, N, qw, scales, zeros, zero_bias, out, static_cast<hipStream_t>(stream));
    return launch_w4a16_gemm_mfma(x, M, K, N, qw, scales, zeros, zero_bias, out, static_cast<hipStream_t>(stream),
                                  workspace, workspace_bytes);
}

// Decode-sized M streams the weights once per row through the GEMV; larger M
// goes to the MFMA kernel, which reuses each dequantised operand across rows.
int mcv_w4a16_gemm(const void* x, int64_t M, int64_t K, int64_t N, const void* qw, const void* scales,
                   const void* zeros, int zero_bias, void* out, mcv_stream_t stream) {
    if (w4a16_prefers_gemv(M, N))
        return launch_w4a16_gemv(x, M, K, N, qw, scales, zeros, zero_bias, out, static_cast<hipStream_t>(stream));
    return launch_w4a16_gemm_mfma(x, M, K, N, qw, scales, zeros, zero_bias, out, static_cast<hipStream_t>(stream));
}

}  // extern "C"
