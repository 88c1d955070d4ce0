// w4a16_gemm_sk.h -- launch interface of the half-slab W4A16 GEMM with an
// in-launch K split (w4a16_gemm_sk.hip), shared with the dispatcher.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace mcv {

// Tile TM rows x 32 * nwv columns (nwv half-slabs of 32 columns), ns stages
// in flight, K split `splits` ways across workgroups, kg quantisation groups
// (128 k each) per stage (kg must divide the groups of every split:
// K / 128 / splits), kw k-parts: nwv * kw waves, k-part j taking group j of
// every stage (kw = 2 needs kg = 2), their sums added in LDS at the end.
struct SkConfig {
    int tm;
    int nwv;
    int ns;
    int splits;
    int kg = 1;
    int kw = 1;
    int wr = 0;             // 1: each wave loads its weights, zeros and scales into registers (LDS holds x only)
    int order = 0;          // tile order: 0 by operand bytes (2 or 3), 1 along the rows, 2 down the
                            // columns, 3 down the columns of groups of tile rows
};

// The workspace starts with the tile arrival counters, a fixed region for
// every shape (so calls of different shapes may share one workspace), then
// the partial tiles.  A split call may have at most kSkMaxSplitTiles tiles.
constexpr int kSkMaxSplitTiles = 1024;
constexpr uint32_t kSkCounterBytes = kSkMaxSplitTiles * 4;

int64_t w4a16_sk_tiles(int64_t M, int64_t N, const SkConfig& c);
// Workspace bytes of a call (0 without a split): tile arrival counters
// (zero-filled once, left zero by every call) and the fp32 partial tiles.
int64_t w4a16_sk_workspace_bytes(int64_t M, int64_t N, const SkConfig& c);
bool w4a16_sk_config_valid(int64_t M, int64_t K, int64_t N, const SkConfig& c);
int launch_w4a16_gemm_sk(const void* x, int64_t M, int64_t K, int64_t N, const void* qw, const void* scales,
                         const void* zeros, int zero_bias, void* out, const SkConfig& c, void* ws, int64_t ws_bytes,
                         hipStream_t stream);

}  // namespace mcv
