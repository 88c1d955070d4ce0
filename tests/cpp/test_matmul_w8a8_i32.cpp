// Exact int8 x int8 -> int32 against the CPU dot product, as the reference's
// test (tests/test_matmul_w8a8_i32.cpp: K=1024, N=3584, mt19937(0), U{-8..7}),
// plus an M=256 case and the extreme-value corner |acc| = 2^24.
#include "minicpmv/hip_context.h"
#include "minicpmv/ops.h"
#include "test_common.h"

#include <random>

using namespace minicpmv;

static int run(HipContext& ctx, int M, int K, int N, int lo, int hi, bool extreme) {
    std::mt19937 rng(0);
    std::uniform_int_distribution<int> xd(lo, hi), wd(lo, hi);
    std::vector<int8_t> hx(static_cast<size_t>(M) * K), hw(static_cast<size_t>(K) * N);
    for (auto& v : hx) v = static_cast<int8_t>(xd(rng));
    for (auto& v : hw) v = static_cast<int8_t>(wd(rng));
    if (extreme) {
        for (int k = 0; k < K; ++k) hx[k] = -128, hw[static_cast<size_t>(k) * N] = -128;
    }
    Tensor x({M, K}, DType::Int8), w({K, N}, DType::Int8), out({M, N}, DType::Int32);
    x.copy_from_host(hx.data(), hx.size());
    w.copy_from_host(hw.data(), hw.size());
    out.allocate();
    matmul_w8a8_i32(x, w, out, ctx.stream());
    std::vector<int32_t> ho(static_cast<size_t>(M) * N);
    out.copy_to_host(ho.data(), ho.size() * 4);
    int bad = 0;
    for (int m = 0; m < M; ++m)
        for (int n = 0; n < N; ++n) {
            int32_t ref = 0;
            for (int k = 0; k < K; ++k) ref += int32_t(hx[m * K + k]) * int32_t(hw[static_cast<size_t>(k) * N + n]);
            if (ho[static_cast<size_t>(m) * N + n] != ref) ++bad;
        }
    std::printf("W8A8 i32 M=%d K=%d N=%d mismatches=%d\n", M, K, N, bad);
    return bad != 0;
}

int main() {
    HipContext ctx(0);
    int rc = run(ctx, 1, 1024, 3584, -8, 7, false);
    rc |= run(ctx, 256, 1024, 512, -128, 127, false);
    rc |= run(ctx, 4, 1024, 64, -128, 127, true);
    return rc;
}
