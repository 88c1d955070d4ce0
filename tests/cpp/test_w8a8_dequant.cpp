// The reference's deterministic dequant test (tests/test_w8a8_dequant.cpp:42-63):
// acc[i] = i - 1024, ws[i] = f2h(0.01 + (i % 7) * 0.001), xs = f2h(0.02),
// N = 3584; pass if max |out - acc * xs * ws| < 0.02.  Also checks that the
// fused GEMM epilogue equals this epilogue bit for bit.
#include "minicpmv/hip_context.h"
#include "minicpmv/ops.h"
#include "test_common.h"

#include <cmath>

using namespace minicpmv;

int main() {
    HipContext ctx(0);
    constexpr int N = 3584;
    std::vector<int32_t> hacc(N);
    std::vector<uint16_t> hws(N);
    for (int i = 0; i < N; ++i) {
        hacc[i] = i - 1024;
        hws[i] = t::f2h(0.01f + static_cast<float>(i % 7) * 0.001f);
    }
    std::vector<uint16_t> hxs(1, t::f2h(0.02f));
    Tensor acc({1, N}, DType::Int32);
    acc.copy_from_host(hacc.data(), hacc.size() * 4);
    Tensor xs({1}, DType::Float16);
    xs.copy_from_host(hxs.data(), 2);
    Tensor ws({N}, DType::Float16);
    ws.copy_from_host(hws.data(), hws.size() * 2);
    Tensor out({1, N}, DType::Float16);
    out.allocate();
    w8a8_dequant(acc, xs, ws, out, ctx.stream());
    std::vector<uint16_t> ho(N);
    out.copy_to_host(ho.data(), ho.size() * 2);
    float max_abs = 0.0f;
    int exact_bad = 0;
    for (int i = 0; i < N; ++i) {
        const float ref = static_cast<float>(hacc[i]) * t::h2f(hxs[0]) * t::h2f(hws[i]);
        max_abs = std::max(max_abs, std::fabs(ref - t::h2f(ho[i])));
        volatile float e = static_cast<float>(hacc[i]) * t::h2f(hws[i]);
        volatile float e2 = e * t::h2f(hxs[0]);
        if (t::f2h_rne(e2) != ho[i]) ++exact_bad;
    }
    std::printf("W8A8 dequant max_abs_diff=%.6f exact_mismatches=%d\n", max_abs, exact_bad);
    return (max_abs < 0.02f && exact_bad == 0) ? 0 : 1;
}
