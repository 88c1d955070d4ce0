// w4a16_gemm.hip -- the W4A16 matmul dispatch for any M, gfx950.
//
// out[M][N] = x[M][K] . W[K][N], W in the slab-64 int4 layout.  Decode-sized
// M streams the weights through the GEMV (w4a16_gemv.hip), one grid row per
// activation row; larger M runs the half-slab MFMA GEMM (w4a16_gemm_sk.hip),
// which reuses each widened weight operand across TM rows, in the tile shape
// and K split picked here.
//
// The reference has no M > 1 quantised path: its matmul_w4a16 is M = 1 only
// (src/csrc/lib/ops.cpp:1030-1095) and its prefill runs dense fp16 aclnnMm
// through matmul_b_transposed (src/csrc/lib/decoder_layer.cpp:459-462,
// 656-659, 857-860; src/csrc/lib/ops.cpp:159-322).
#include <cstdio>
#include <string>

#include "common.h"
#include "w4a16_gemm_sk.h"

namespace mcv {

int launch_w4a16_gemv(const void* x, int64_t M, int64_t K, int64_t N, const void* qw, const void* scales,
                      const void* zeros, int zero_bias, void* out, hipStream_t stream);
int gemv_ksplit(int64_t G, int64_t blocks);

namespace {

// Few rows: the GEMV streams the weights once per row and still beats the
// MFMA GEMM, whose tile count is M/TM * N/TN, until the output reaches about
// 64K elements (MI355X, rotated weights: K=1024 N=3584 M=16 5.7 us against
// 7.0; K=3584 N=1024 M=48 12.4 against 12.5; K=1024 N=6144 crosses over near
// M=11).
bool w4a16_prefers_gemv(int64_t M, int64_t N) { return M >= 1 && (M < 8 || M * N < 65536); }

// The GEMM's configuration for M x K x N.  First the largest tile whose grid
// gives 200-256 workgroups, one tile each (a workgroup per CU): 128 x 256
// (eight waves), 64 x 128, 64 x 64, 32 x 128, 32 x 64; past 256, the largest
// that reaches 200 other than 64 x 64.  Failing that (few rows and N =
// 1024-like widths), with a workspace, K is split across workgroups on 32 x 64
// tiles: the most ways that keep the grid within one workgroup per CU and
// leave each workgroup at least 7 quantisation groups on average (splits are
// cut in whole stages, so they differ by at most one) -- the partial tiles'
// exchange costs ~1-2 us, which a shorter loop does not pay back.  A
// tile of four half-slabs takes two k-parts (eight waves, two groups per
// stage) when its workgroups' group count is even and at least 8 (64-row
// tiles) or 14 (32-row tiles); the 32 x 64 and 64 x 64 tiles (two
// half-slabs) whenever K/128 is even: two waves per SIMD cover each other's
// copy issue.  The 64-
// and 32-row tiles load their weights, zeros and scales straight into
// registers (each wave's columns are its own; LDS then stages x only): 0-9 %
// faster than staging them in LDS in two sweeps, never slower; the 128 x 256
// tile measured the same either way and keeps the LDS path.  Measured on
// MI355X (rotated weights, us per call, back to back; the same launch varies
// by up to +-7 % from one 200-launch region to the next on the long shapes):
// M=2048 K=1024 N=3584 128x256 20.0-20.6 (64x128 24-25); M=2048 K=3584 N=1024
// 64x128 two k-parts 19.6-22.3 (LDS weights 20.1-21.6, one k-part 21.6-22.6);
// M=512 K=1024 N=3584 64x128 two k-parts 8.3-8.5 (32x64 10.0-11.6); M=512
// K=3584 N=1024 32x64 two k-parts 10.1 (32x128 split 2 ways 11.4-12.1, 64x64
// split 2 ways 10.8); M=128 K=1024 N=3584 32x64 two k-parts 5.5 (one k-part
// 6.6, 32x128 6.7-7.0); M=128 K=3584 N=1024 32x64 split 2 ways, two k-parts
// 7.96 (3 ways 7.93, 2 ways 8.8; one k-part 4 ways 9.7; 32x128 split 4 ways
// 9.6-9.8); M=64 K=3584 N=1024 32x64 split 4 ways 7.2 (3 ways 7.4, 8 ways
// 8.0); M=128 K=2048 N=1024 2 ways 7.1 (3 ways 6.85); 64x64 two
// k-parts against 32x128 at 224-256 tiles: M=256 K=1024 N=3584 6.6 / 7.3,
// M=1024 K=3584 N=1024 13.9 / 15.6, M=512 K=1024 N=2048 6.5 / 7.1, M=1024
// K=2048 N=1024 9.3 / 9.9, M=512 K=3584 N=2048 14.1 / 15.9; at 288-384
// tiles 64x64 is 0.1-2 us slower.  Against the
// rule before the 32 x 64 tile, over M = 48..512 and (K, N) = (1024, 3584),
// (3584, 1024), (1024, 6144), (1024, 2048), (2048, 1024): 10-25 % faster
// where it changes the configuration, except 0.05-0.15 us slower where its
// grid passes 256 workgroups (M = 96-192 at N = 3584-6144).
SkConfig choose_gemm(int64_t M, int64_t K, int64_t N, bool can_split) {
    constexpr SkConfig kOne[] = {{128, 8, 3, 1}, {64, 4, 3, 1}, {64, 2, 3, 1}, {32, 4, 3, 1}, {32, 2, 3, 1}};
    const int64_t G = K / kGroup;
    auto finish = [&](SkConfig c) {
        if (G % 2 == 0 && (c.nwv == 2 || (c.nwv == 4 && ((c.tm == 64 && G >= 8) || (c.tm == 32 && G >= 14)))))
            c.kg = c.kw = 2;
        c.wr = c.tm != 128;
        return c;
    };
    // one tile per workgroup and one workgroup per CU where a tile fits that
    // (200-256 tiles); else the largest tile that still covers most CUs,
    // 64 x 64 aside (past 256 tiles it trails 32 x 128 by 5-20 %)
    for (const SkConfig& c : kOne) {
        const int64_t t = w4a16_sk_tiles(M, N, c);
        if (t >= 200 && t <= 256) return finish(c);
    }
    for (const SkConfig& c : kOne)
        if (w4a16_sk_tiles(M, N, c) >= 200 && !(c.tm == 64 && c.nwv == 2)) return finish(c);
    SkConfig c{32, 2, 3, 1};
    const int64_t tiles = w4a16_sk_tiles(M, N, c);
    if (!can_split || tiles > kSkMaxSplitTiles) return finish(c);
    // the K split: the most ways within 256 workgroups that leave at least 7
    // groups per workgroup on average, cut in whole stages (two groups each
    // where K/128 is even)
    const int64_t U = G % 2 == 0 ? G / 2 : G;
    for (int64_t s = 2; s <= U && s <= 64; ++s)
        if (tiles * s <= 256 && G >= 7 * s) c.splits = static_cast<int>(s);
    return finish(c);
}

int check_gemm_args(const void* x, int64_t M, int64_t K, int64_t N, const void* qw, const void* scales,
                    const void* zeros, int zero_bias, const void* out, const char* who) {
    if (!x || !out || !qw || !scales || !zeros) return fail(MCV_ERR_INVALID_ARG, "%s: null pointer", who);
    if (zero_bias != 0 && zero_bias != 1) return fail(MCV_ERR_INVALID_ARG, "%s: zero_bias must be 0 or 1", who);
    if (K <= 0 || K % kGroup != 0 || K > (int64_t(1) << 24))
        return fail(MCV_ERR_SHAPE, "%s: K must be a positive multiple of 128 (K=%lld)", who, (long long)K);
    if (N <= 0 || N > (int64_t(1) << 30) || M <= 0 || M > (int64_t(1) << 30))
        return fail(MCV_ERR_SHAPE, "%s: bad M/N (M=%lld N=%lld)", who, (long long)M, (long long)N);
    if (reinterpret_cast<uintptr_t>(x) % 16 != 0) return fail(MCV_ERR_INVALID_ARG, "%s: x must be 16-byte aligned", who);
    return require_device();
}

// The MFMA GEMM with the configuration above; a split only into a caller's
// workspace that holds it (else unsplit).
int launch_w4a16_gemm_mfma(const void* x, int64_t M, int64_t K, int64_t N, const void* qw, const void* scales,
                           const void* zeros, int zero_bias, void* out, hipStream_t stream, void* ws,
                           int64_t ws_bytes) {
    int rc = check_gemm_args(x, M, K, N, qw, scales, zeros, zero_bias, out, "mcv_w4a16_gemm_mfma");
    if (rc != MCV_OK) return rc;
    SkConfig c = choose_gemm(M, K, N, ws != nullptr);
    if (c.splits > 1 && (ws_bytes < w4a16_sk_workspace_bytes(M, N, c) || (reinterpret_cast<uintptr_t>(ws) & 255) != 0))
        c = choose_gemm(M, K, N, false);
    return launch_w4a16_gemm_sk(x, M, K, N, qw, scales, zeros, zero_bias, out, c, ws, ws_bytes, stream);
}

thread_local std::string g_kernel_name;

}  // namespace

}  // namespace mcv

using namespace mcv;

extern "C" {

int mcv_w4a16_gemm_mfma(const void* x, int64_t M, int64_t K, int64_t N, const void* qw, const void* scales,
                        const void* zeros, int zero_bias, void* out, mcv_stream_t stream) {
    return launch_w4a16_gemm_mfma(x, M, K, N, qw, scales, zeros, zero_bias, out, static_cast<hipStream_t>(stream),
                                  nullptr, 0);
}

int64_t mcv_w4a16_gemm_workspace_bytes(int64_t M, int64_t K, int64_t N) {
    if (M < 1 || K <= 0 || N <= 0 || K % kGroup != 0 || w4a16_prefers_gemv(M, N)) return 0;
    return w4a16_sk_workspace_bytes(M, N, choose_gemm(M, K, N, true));
}

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
    return launch_w4a16_gemm_mfma(x, M, K, N, qw, scales, zeros, zero_bias, out, static_cast<hipStream_t>(stream),
                                  nullptr, 0);
}

const char* mcv_w4a16_gemm_kernel_name(int64_t M, int64_t K, int64_t N, int with_workspace) {
    char buf[160];
    if (M < 1 || K <= 0 || N <= 0 || K % kGroup != 0) {
        g_kernel_name = "none (bad shape)";
    } else if (w4a16_prefers_gemv(M, N)) {
        std::snprintf(buf, sizeof(buf), "w4a16_gemv_kernel<%d, 1, 0> (grid %lld x %lld)",
                      gemv_ksplit(K / kGroup, ceil_div(N, kSlab) * M), (long long)ceil_div(N, kSlab), (long long)M);
        g_kernel_name = buf;
    } else {
        const SkConfig c = choose_gemm(M, K, N, with_workspace != 0);
        std::snprintf(buf, sizeof(buf), "w4a16_gemm_sk_kernel<%d, %d, %d, %d, %d, %d> (K split %d ways, %lld workgroups)%s",
                      c.tm, c.nwv, c.ns, c.kg, c.kw, c.wr, c.splits, (long long)(w4a16_sk_tiles(M, N, c) * c.splits),
                      w4a16_sk_config_valid(M, K, N, c) ? "" : " NOT BUILT");
        g_kernel_name = buf;
    }
    return g_kernel_name.c_str();
}

}  // extern "C"
