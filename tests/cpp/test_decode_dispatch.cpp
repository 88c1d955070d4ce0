// matmul_decode_dispatch (src/csrc/lib/decoder_layer.cpp:226-244) and the
// MINICPM_W8A8_DECODE policy (decoder_layer.cpp:19-25, language_model.cpp:19-41).
//   test_decode_dispatch policy   -- CPU only: prints the policy decisions
//   test_decode_dispatch dispatch -- GPU: the branch the reference takes, with
//       the W8A8 branch bit-exact against the oracle's composition of the
//       reference's steps (w8a8_quantize -> matmul_w8a8_i32 -> w8a8_dequant
//       with the fp16 x_scale and the truncated fp16 w_scale); the M > 1
//       rules; and a HIP graph holding the W8A8 branch and the device-token
//       lm_head, replayed with eager work in between, equal to eager calls.
#include "mcv_oracle.h"
#include "minicpmv/decode_dispatch.h"
#include "minicpmv/hip_context.h"
#include "minicpmv/lm_head.h"
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

// The reference's W8A8 decode projection on the CPU: per-tensor activation
// quantisation, exact int32 products, dequant with the fp16 x_scale and the
// truncated fp16 w_scale, all by the oracle.
static std::vector<uint16_t> oracle_w8a8(const std::vector<uint16_t>& hx, const std::vector<uint16_t>& w, int64_t M,
                                         int64_t K, int64_t N) {
    std::vector<int8_t> xq(static_cast<size_t>(M * K)), wq(static_cast<size_t>(K * N));
    std::vector<float> xs32(M), ws32(N), xs(M), ws(N);
    std::vector<uint16_t> xs16(M), ws16(N), out(static_cast<size_t>(M * N));
    std::vector<int32_t> acc(static_cast<size_t>(M * N));
    or_w8a8_quantize_act(hx.data(), M, K, xq.data(), xs32.data(), xs16.data());
    or_w8a8_quantize_weight(w.data(), K, N, wq.data(), ws32.data(), ws16.data());
    or_gemm_i32(xq.data(), wq.data(), M, K, N, acc.data(), 0);
    for (int64_t m = 0; m < M; ++m) xs[m] = or_h2f(xs16[m]);
    for (int64_t n = 0; n < N; ++n) ws[n] = or_h2f(ws16[n]);
    or_w8a8_dequant(acc.data(), xs.data(), ws.data(), M, N, out.data());
    return out;
}

static int dispatch() {
    HipContext ctx(0);
    hipStream_t st = ctx.stream();
    constexpr int64_t K = 1024, N = 512, M2 = 3;
    std::mt19937 rng(5);
    std::normal_distribution<float> wn(0.f, 0.02f), xn(0.f, 1.f);
    std::vector<uint16_t> w(static_cast<size_t>(K * N)), hx(K), hx2(static_cast<size_t>(M2 * K));
    for (auto& v : w) v = t::f2h_rne(wn(rng));
    for (auto& v : hx) v = t::f2h_rne(xn(rng));
    for (auto& v : hx2) v = t::f2h_rne(xn(rng));
    W4A16QuantizedWeight q4 = quantize_w4a16_synthetic(w.data(), K, N);
    W8A8QuantizedWeight w8 = quantize_w8a8_host(w.data(), K, N);
    Tensor dense({K, N}, DType::Float16);
    dense.copy_from_host(w.data(), w.size() * 2);
    Tensor x({1, K}, DType::Float16), x2({M2, K}, DType::Float16);
    x.copy_from_host(hx.data(), K * 2);
    x2.copy_from_host(hx2.data(), hx2.size() * 2);
    Tensor out({1, N}, DType::Float16), a({1, N}, DType::Float16), c({1, N}, DType::Float16);
    out.allocate(); a.allocate(); c.allocate();

    matmul_w4a16(x, q4, a, st);
    matmul_b_transposed(x, dense, c, st);
    const bool want_w8 = w8a8_decode_enabled_for_layers();
    DecodeScratch scratch;

    // M = 1: the reference's priority
    matmul_decode_dispatch(x, &dense, &q4, &w8, out, st, scratch);
    const auto ho = d2h(out);
    const auto want8 = oracle_w8a8(hx, w, 1, K, N);
    const bool w8_exact = ho == want8, is_q4 = ho == d2h(a);
    int w8_mismatch = 0;
    for (int64_t n = 0; n < N; ++n) w8_mismatch += ho[n] != want8[n];
    matmul_decode_dispatch(x, &dense, nullptr, nullptr, out, st);
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
    matmul_b_transposed(x, dense_nk, out, st);
    const auto hnk = d2h(out);
    double nk_diff = 0;
    for (int64_t n = 0; n < N; ++n) nk_diff = std::max(nk_diff, double(std::fabs(t::h2f(hnk[n]) - t::h2f(hc[n]))));

    // M > 1: the reference takes the dense weight whenever it exists; with no
    // dense weight the quantised objects serve every row (W4A16 first).
    Tensor o2({M2, N}, DType::Float16), d2({M2, N}, DType::Float16), q2({M2, N}, DType::Float16);
    o2.allocate(); d2.allocate(); q2.allocate();
    matmul_b_transposed(x2, dense, d2, st);
    matmul_w4a16(x2, q4, q2, st);
    matmul_decode_dispatch(x2, &dense, &q4, &w8, o2, st, scratch);
    const bool m2_dense = d2h(o2) == d2h(d2);
    matmul_decode_dispatch(x2, nullptr, &q4, &w8, o2, st, scratch);
    const bool m2_q4 = d2h(o2) == d2h(q2);
    bool m2_w8 = true;
    if (want_w8) {
        matmul_decode_dispatch(x2, nullptr, nullptr, &w8, o2, st, scratch);
        m2_w8 = d2h(o2) == oracle_w8a8(hx2, w, M2, K, N);       // per-row scales, same steps
    }

    std::printf("dispatch: want_w8=%d w8_exact=%d (mismatches %d) took_q4=%d dense_ok=%d dense_max_abs=%.2e "
                "nk_vs_kn=%.2e m2_dense=%d m2_q4=%d m2_w8=%d\n",
                int(want_w8), int(w8_exact), w8_mismatch, int(is_q4), int(dense_ok), max_abs, nk_diff, int(m2_dense),
                int(m2_q4), int(m2_w8));
    bool ok = (want_w8 ? w8_exact : is_q4) && dense_ok && max_abs < 1e-2 && nk_diff < 2e-3 && m2_dense && m2_q4 && m2_w8;

    // A HIP graph of the decode-time calls: the dispatcher's W8A8 branch (its
    // scratch already allocated by the eager calls above) and the
    // device-token lm_head.  Replays with eager launches and host reads in
    // between must reproduce the eager outputs every time.
    if (want_w8) {
        constexpr int64_t V = 5000, NV = 5056;
        std::vector<uint16_t> wv(static_cast<size_t>(K * NV));
        for (auto& v : wv) v = t::f2h_rne(wn(rng));
        LmHeadW4A16 head = make_lm_head_w4a16(quantize_w4a16_synthetic(wv.data(), K, NV), V);
        Tensor lg({1, V}, DType::Float16), lg_eager({1, V}, DType::Float16);
        lg.allocate(); lg_eager.allocate();
        matmul_decode_dispatch(x, &dense, &q4, &w8, out, st, scratch);
        lm_head_argmax_w4a16(x, head, &lg_eager, st);
        const auto eager_out = d2h(out), eager_lg = d2h(lg_eager);
        const int64_t eager_tok = lm_head_read_token(head, st);
        hipGraph_t graph = nullptr;
        hipGraphExec_t exec = nullptr;
        check_hip(hipStreamBeginCapture(st, hipStreamCaptureModeGlobal), "hipStreamBeginCapture");
        matmul_decode_dispatch(x, &dense, &q4, &w8, out, st, scratch);
        lm_head_argmax_w4a16(x, head, &lg, st);
        check_hip(hipStreamEndCapture(st, &graph), "hipStreamEndCapture");
        check_hip(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0), "hipGraphInstantiate");
        int good = 0;
        for (int rep = 0; rep < 4; ++rep) {
            Tensor junk({1, N}, DType::Float16);
            junk.allocate();
            matmul_decode_dispatch(x, &dense, nullptr, nullptr, junk, st);   // eager work between replays
            check_hip(hipMemsetAsync(out.data(), 0xff, out.size_bytes(), st), "hipMemsetAsync");
            check_hip(hipGraphLaunch(exec, st), "hipGraphLaunch");
            const int64_t tok = lm_head_read_token(head, st);
            good += d2h(out) == eager_out && d2h(lg) == eager_lg && tok == eager_tok;
        }
        check_hip(hipGraphExecDestroy(exec), "hipGraphExecDestroy");
        check_hip(hipGraphDestroy(graph), "hipGraphDestroy");
        std::printf("graph: %d of 4 replays equal to the eager calls (token %lld)\n", good, (long long)eager_tok);
        ok = ok && good == 4;
    }
    return ok ? 0 : 1;
}

int main(int argc, char** argv) {
    const std::string mode = argc > 1 ? argv[1] : "policy";
    if (mode == "policy") return policy();
    return dispatch();
}
