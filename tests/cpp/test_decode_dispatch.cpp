// matmul_decode_dispatch (src/csrc/lib/decoder_layer.cpp:226-244) and the
// MINICPM_W8A8_DECODE policy (decoder_layer.cpp:19-25, language_model.cpp:19-41).
//   test_decode_dispatch policy   -- CPU only: prints the policy decisions
//   test_decode_dispatch dispatch -- GPU: checks which branch ran by comparing
//                                    with the direct operator outputs
#include "minicpmv/decode_dispatch.h"
#include "minicpmv/hip_context.h"
#include "minicpmv/ops.h"
#include "test_common.h"

#include <cmath>
#include <random>

using namespace minicpmv;

static int policy() {
    std::printf("layers=%d enabled=%d", int(w8a8_decode_enabled_for_layers()), int(w8a8_decode_enabled()));
    for (const char* tkn : {"mlp", "linear_qkv", "linear_z", "linear_out", "full_q", "full_k", "full_v", "full_o", "lm_head"})
        std::printf(" %s=%d", tkn, int(w8a8_policy_allows(tkn)));
    std::printf("\n");
    return 0;
}

static std::vector<uint16_t> d2h(const Tensor& t) {
    std::vector<uint16_t> h(t.numel());
    t.copy_to_host(h.data(), h.size() * 2);
    return h;
}

static int dispatch() {
    HipContext ctx(0);
    constexpr int64_t K = 1024, N = 512;
    std::mt19937 rng(5);
    std::normal_distribution<float> wn(0.f, 0.02f), xn(0.f, 1.f);
    std::vector<uint16_t> w(static_cast<size_t>(K * N)), hx(K);
    for (auto& v : w) v = t::f2h_rne(wn(rng));
    for (auto& v : hx) v = t::f2h_rne(xn(rng));
    W4A16QuantizedWeight q4 = quantize_w4a16_synthetic(w.data(), K, N);
    W8A8QuantizedWeight w8 = quantize_w8a8_host(w.data(), K, N);
    Tensor dense({K, N}, DType::Float16);
    dense.copy_from_host(w.data(), w.size() * 2);
    Tensor x({1, K}, DType::Float16);
    x.copy_from_host(hx.data(), K * 2);
    Tensor out({1, N}, DType::Float16), a({1, N}, DType::Float16), b({1, N}, DType::Float16), c({1, N}, DType::Float16);
    out.allocate(); a.allocate(); b.allocate(); c.allocate();

    matmul_w4a16(x, q4, a, ctx.stream());
    Tensor xq({1, K}, DType::Int8), xs({1}, DType::Float32);
    xq.allocate(); xs.allocate();
    w8a8_quantize(x, xq, xs, ctx.stream());
    matmul_w8a8(xq, xs, w8, b, ctx.stream());
    matmul_b_transposed(x, dense, c, ctx.stream());

    matmul_decode_dispatch(x, &dense, &q4, &w8, out, ctx.stream());
    const bool want_w8 = w8a8_decode_enabled_for_layers();
    const auto ho = d2h(out);
    const bool is_w8 = ho == d2h(b), is_q4 = ho == d2h(a);
    matmul_decode_dispatch(x, &dense, nullptr, nullptr, out, ctx.stream());
    const bool dense_ok = d2h(out) == d2h(c);
    // dense vs CPU fp32
    const auto hc = d2h(c);
    double max_abs = 0;
    for (int64_t n = 0; n < N; ++n) {
        float ref = 0.f;
        for (int64_t k = 0; k < K; ++k) ref += t::h2f(hx[k]) * t::h2f(w[k * N + n]);
        max_abs = std::max(max_abs, double(std::fabs(ref - t::h2f(hc[n]))));
    }
    // the [N, K] layout of the dense weight gives the same product
    std::vector<uint16_t> wt(static_cast<size_t>(K * N));
    for (int64_t k = 0; k < K; ++k)
        for (int64_t n = 0; n < N; ++n) wt[n * K + k] = w[k * N + n];
    Tensor dense_nk({N, K}, DType::Float16);
    dense_nk.copy_from_host(wt.data(), wt.size() * 2);
    matmul_b_transposed(x, dense_nk, out, ctx.stream());
    const auto hnk = d2h(out);
    double nk_diff = 0;
    for (int64_t n = 0; n < N; ++n) nk_diff = std::max(nk_diff, double(std::fabs(t::h2f(hnk[n]) - t::h2f(hc[n]))));
    std::printf("dispatch: want_w8=%d took_w8=%d took_q4=%d dense_ok=%d dense_max_abs=%.2e nk_vs_kn=%.2e\n", int(want_w8),
                int(is_w8), int(is_q4), int(dense_ok), max_abs, nk_diff);
    const bool ok = (want_w8 ? is_w8 : is_q4) && dense_ok && max_abs < 1e-2 && nk_diff < 2e-3;
    return ok ? 0 : 1;
}

int main(int argc, char** argv) {
    const std::string mode = argc > 1 ? argv[1] : "policy";
    if (mode == "policy") return policy();
    return dispatch();
}
