// Greedy lm_head over a W4A16 vocabulary projection, with the final RMSNorm
// (lm_head_greedy semantics, src/csrc/lib/language_model.cpp:412-482), against
// a CPU reference: RMSNorm in fp32 -> fp16, the group formula over the
// unpacked (q - z), fp16 logits, first-maximum scan.  Plus: exact ties pick
// the first index, the workspace is reusable, the W8A8 variant's logits are
// bit-exact against the oracle's composition of the reference's steps
// (language_model.cpp:434-467: fp16 x_scale, truncated fp16 w_scale), and a
// give-up of the device-token route's bounded wait -- forced from the host
// through the library's test hook, which has the poller expect a tag no key
// carries -- yields token -1, the status word and a thrown error, after which
// the head works again.
#include "mcv_oracle.h"
#include "mcv_quant.h"
#include "minicpmv/hip_context.h"
#include "minicpmv/lm_head.h"
#include "minicpmv/ops.h"
#include "test_common.h"

#include <cmath>
#include <random>

using namespace minicpmv;

int main() {
    HipContext ctx(0);
    constexpr int64_t K = 1024, N = 20000, V = 19997, G = K / 128;
    constexpr int order[8] = {0, 2, 4, 6, 1, 3, 5, 7};
    std::mt19937 rng(11);
    std::normal_distribution<float> wn(0.f, 0.02f), xn(0.f, 1.f);
    std::vector<uint16_t> w(static_cast<size_t>(K * N));
    for (auto& v : w) v = t::f2h_rne(wn(rng));
    for (int64_t k = 0; k < K; ++k) w[k * N + 777] = w[k * N + 4321];   // two identical columns
    std::vector<int32_t> qweight(static_cast<size_t>(K * N / 8)), qzeros(static_cast<size_t>(G * N / 8));
    std::vector<uint16_t> scales(static_cast<size_t>(G * N));
    if (mcv_w4a16_quantize_host(w.data(), K, N, qweight.data(), qzeros.data(), scales.data(), 0) != 0) return 1;
    std::vector<int8_t> w8(static_cast<size_t>(K * N));
    for (int64_t k = 0; k < K; ++k)
        for (int64_t j = 0; j < N / 8; ++j)
            for (int s = 0; s < 8; ++s) {
                const int q = (static_cast<uint32_t>(qweight[k * (N / 8) + j]) >> (4 * s)) & 15;
                const int z = (static_cast<uint32_t>(qzeros[(k / 128) * (N / 8) + j]) >> (4 * s)) & 15;
                w8[k * N + j * 8 + order[s]] = static_cast<int8_t>(q - z);
            }
    LmHeadW4A16 head = make_lm_head_w4a16(pack_w4a16_awq(qweight.data(), qzeros.data(), scales.data(), K, N), V);

    std::vector<uint16_t> hx(K), hg(K);
    for (auto& v : hx) v = t::f2h_rne(xn(rng));
    for (auto& v : hg) v = t::f2h_rne(1.0f + 0.1f * xn(rng));
    Tensor x({1, K}, DType::Float16), gamma({K}, DType::Float16);
    x.copy_from_host(hx.data(), K * 2);
    gamma.copy_from_host(hg.data(), K * 2);
    const double eps = 1e-6;

    // CPU reference
    float ss = 0.f;
    for (int64_t i = 0; i < K; ++i) ss += t::h2f(hx[i]) * t::h2f(hx[i]);
    const float rstd = 1.0f / std::sqrt(ss / K + static_cast<float>(eps));
    std::vector<uint16_t> xn16(K);
    for (int64_t i = 0; i < K; ++i) xn16[i] = t::f2h_rne((t::h2f(hx[i]) * rstd) * t::h2f(hg[i]));
    std::vector<float> logits(V);
    for (int64_t n = 0; n < V; ++n) {
        float acc = 0.f;
        for (int64_t g = 0; g < G; ++g) {
            float part = 0.f;
            for (int64_t kk = 0; kk < 128; ++kk) part += t::h2f(xn16[g * 128 + kk]) * static_cast<float>(w8[(g * 128 + kk) * N + n]);
            acc += part * t::h2f(scales[g * N + n]);
        }
        logits[n] = acc;
    }
    int64_t best = 0;
    float bv = -INFINITY, second = -INFINITY;
    for (int64_t n = 0; n < V; ++n) {
        const float v = t::h2f(t::f2h_rne(logits[n]));
        if (v > bv) { second = bv; bv = v; best = n; }
        else if (v > second) second = v;
    }
    int rc = 0;
    const int64_t tok = lm_head_greedy_w4a16(x, &gamma, eps, head, ctx.stream());
    std::printf("W4A16 lm_head token=%lld cpu=%lld margin=%.4f\n", (long long)tok, (long long)best, bv - second);
    if (bv - second > 1e-2f && tok != best) rc = 1;
    if (lm_head_greedy_w4a16(x, &gamma, eps, head, ctx.stream()) != tok) rc = 1;    // workspace reusable

    // tie: make column 777 / 4321 the maximum by pointing x along them
    Tensor lg({1, V}, DType::Float16);
    lg.allocate();
    std::vector<uint16_t> hx2(K);
    for (int64_t k = 0; k < K; ++k) hx2[k] = t::f2h_rne(static_cast<float>(w8[k * N + 4321]));
    Tensor x2({1, K}, DType::Float16);
    x2.copy_from_host(hx2.data(), K * 2);
    lm_head_argmax_w4a16(x2, head, &lg, ctx.stream());
    std::vector<uint16_t> hl(V);
    lg.copy_to_host(hl.data(), V * 2);
    int64_t tok2 = 0;
    head.token.copy_to_host(&tok2, 8);
    int64_t scan = 0;
    float sv = -INFINITY;
    for (int64_t n = 0; n < V; ++n) {
        const float v = ((hl[n] & 0x7c00u) == 0) ? 0.f : t::h2f(hl[n]);
        if (v > sv) { sv = v; scan = n; }
    }
    std::printf("tie case token=%lld scan=%lld logit[777]=%.3f logit[4321]=%.3f\n", (long long)tok2, (long long)scan,
                t::h2f(hl[777]), t::h2f(hl[4321]));
    if (tok2 != scan || hl[777] != hl[4321] || tok2 != 777) rc = 1;

    // W8A8 head on the same fp16 weights: per-channel int8 + per-token int8
    W8A8QuantizedWeight wq8 = quantize_w8a8_host(w.data(), K, N);
    LmHeadW8A8 h8 = make_lm_head_w8a8(wq8, V);
    const int64_t t8 = lm_head_greedy_w8a8(x, &gamma, eps, h8, ctx.stream());
    {
        // the oracle's composition over the kernel's own normed row
        std::vector<uint16_t> normed(K), got(V);
        h8.normed.copy_to_host(normed.data(), K * 2);
        h8.logits.copy_to_host(got.data(), V * 2);
        std::vector<int8_t> xq(K), wq(static_cast<size_t>(K * N));
        float xs32 = 0.f;
        uint16_t xs16 = 0;
        std::vector<float> ws32(N), ws(N);
        std::vector<uint16_t> ws16(N), want(N);
        std::vector<int32_t> acc(N);
        or_w8a8_quantize_act(normed.data(), 1, K, xq.data(), &xs32, &xs16);
        or_w8a8_quantize_weight(w.data(), K, N, wq.data(), ws32.data(), ws16.data());
        or_gemm_i32(xq.data(), wq.data(), 1, K, N, acc.data(), 0);
        for (int64_t n = 0; n < N; ++n) ws[n] = or_h2f(ws16[n]);
        const float xs = or_h2f(xs16);
        or_w8a8_dequant(acc.data(), &xs, ws.data(), 1, N, want.data());
        int bad = 0;
        for (int64_t n = 0; n < V; ++n) bad += got[n] != want[n];
        const int64_t want_tok = or_argmax_f16(want.data(), V);
        std::printf("W8A8 lm_head token=%lld oracle=%lld logit mismatches=%d\n", (long long)t8, (long long)want_tok, bad);
        if (bad != 0 || t8 != want_tok) rc = 1;
        if (bv - second > 5e-2f && t8 != best) rc = 1;
        // an [K, N] weight takes the separate argmax over the logits: the same token and logits
        W8A8QuantizedWeight wq8kn = quantize_w8a8_host(w.data(), K, N, MCV_W8_KN);
        LmHeadW8A8 h8kn = make_lm_head_w8a8(wq8kn, V);
        const int64_t t8kn = lm_head_greedy_w8a8(x, &gamma, eps, h8kn, ctx.stream());
        std::vector<uint16_t> got_kn(V);
        h8kn.logits.copy_to_host(got_kn.data(), V * 2);
        std::printf("W8A8 lm_head [K, N] weight token=%lld\n", (long long)t8kn);
        if (t8kn != t8 || got_kn != got) rc = 1;
    }

    // Give-up of the device-token route: the poller expects a tag no key
    // carries.  The kernel still ends (bounded wait), writes token -1 and sets
    // the status word; the next call throws and resets the workspace, after
    // which the head works again.
    {
        lm_head_argmax_w4a16(x2, head, nullptr, ctx.stream());
        const int64_t before = lm_head_read_token(head, ctx.stream());
        uint32_t gen[2] = {0, 0};
        check_hip(hipMemcpy(gen, head.workspace.data(), 8, hipMemcpyDeviceToHost), "hipMemcpy");
        mcv_testing_lm_head_skew_poll(1);
        lm_head_argmax_w4a16(x2, head, nullptr, ctx.stream());
        check_hip(hipStreamSynchronize(ctx.stream()), "hipStreamSynchronize");
        mcv_testing_lm_head_skew_poll(0);
        int64_t sentinel = 0;
        check_hip(hipMemcpy(&sentinel, head.token.data(), 8, hipMemcpyDeviceToHost), "hipMemcpy");
        uint32_t ws_flag = 0;
        check_hip(hipMemcpy(&ws_flag, head.workspace.data(), 4, hipMemcpyDeviceToHost), "hipMemcpy");
        const bool status = head.status.gave_up();
        bool threw = false;
        try {
            lm_head_argmax_w4a16(x2, head, nullptr, ctx.stream());
        } catch (const std::runtime_error& e) {
            threw = std::string(e.what()).find("gave up") != std::string::npos;
        }
        lm_head_argmax_w4a16(x2, head, nullptr, ctx.stream());      // the workspace was reset: works again
        const int64_t after = lm_head_read_token(head, ctx.stream());
        std::printf("give-up: generation %u, token %lld, workspace flag %u, status %d, threw %d, recovered %d\n",
                    gen[1], (long long)sentinel, ws_flag, int(status), int(threw), int(after == before));
        if (sentinel != -1 || ws_flag == 0 || !status || !threw || after != before || before != 777) rc = 1;
    }
    return rc;
}
