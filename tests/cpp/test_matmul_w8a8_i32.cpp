// Exact int8 x int8 -> int32 against the CPU dot product, as the reference's
// test (tests/test_matmul_w8a8_i32.cpp: K=1024, N=3584, mt19937(0), U{-8..7}),
// plus an M=256 case and the extreme-value corner |acc| = 2^24.
#include "mcv_oracle.h"
#include "minicpmv/hip_context.h"
#include "minicpmv/ops.h"
#include "test_common.h"

#include <algorithm>
#include <cstdlib>
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

// The W8A8 decode MLP block: one launch (tiled weights) == the four-launch
// sequence, bit for bit, in both precisions; with the reference's precision
// (fp16 activation scales, truncated fp16 weight scales) also == the oracle's
// composition of the reference's steps (decoder_layer.cpp:1022-1046:
// w8a8_quantize, matmul_w8a8_i32 + w8a8_dequant for gate and up, silu_mul,
// the same for down).  silu_mul's exp is the one step whose last bit the host
// libm and the device may round differently, so the composition runs that
// step through the device's silu_mul (pinned against the oracle within one
// fp16 ulp elsewhere) and everything else through the oracle.  Finally a
// give-up of the kernel's bounded waits, forced from the host, is reported.
static int run_mlp(HipContext& ctx, int H, int I) {
    std::mt19937 rng(H + I);
    std::normal_distribution<float> nd(0.0f, 1.0f);
    auto host = [&](int K, int N, float sd) {
        std::vector<uint16_t> h(static_cast<size_t>(K) * N);
        for (auto& v : h) v = t::f2h(nd(rng) * sd);
        return h;
    };
    auto dev = [](const std::vector<uint16_t>& h, int K, int N) {
        Tensor w({K, N}, DType::Float16);
        w.copy_from_host(h.data(), h.size() * 2);
        return w;
    };
    const auto hg = host(H, I, 0.02f), hu = host(H, I, 0.02f), hd = host(I, H, 0.02f), hx = host(1, H, 1.0f);
    Tensor gd = dev(hg, H, I), ud = dev(hu, H, I), dd = dev(hd, I, H), xt = dev(hx, 1, H);
    W8A8QuantizedWeight g = quantize_dense_weight_w8a8(gd), u = quantize_dense_weight_w8a8(ud),
                        d = quantize_dense_weight_w8a8(dd);
    int rc = 0;
    std::vector<uint16_t> ref16;
    for (bool f32 : {false, true}) {
        DecodeMlpW8A8 one = make_decode_mlp_w8a8(g, u, d, f32);
        Tensor y1({1, H}, DType::Float16), y2({1, H}, DType::Float16);
        y1.allocate();
        y2.allocate();
        for (int rep = 0; rep < 3; ++rep) mlp_w8a8(xt, one, y1, ctx.stream());
        DecodeMlpW8A8 four = make_decode_mlp_w8a8(g, u, d, f32);
        four.one_launch = false;
        mlp_w8a8(xt, four, y2, ctx.stream());
        std::vector<uint16_t> h1(H), h2(H);
        y1.copy_to_host(h1.data(), h1.size() * 2);
        y2.copy_to_host(h2.data(), h2.size() * 2);
        uint32_t err = 1;
        one.workspace.copy_to_host(&err, 4);
        std::printf("W8A8 decode MLP H=%d I=%d %s scales: one_launch=%d bit-identical=%d give-up flag=%u\n", H, I,
                    f32 ? "fp32" : "fp16 (reference)", one.one_launch ? 1 : 0, h1 == h2 ? 1 : 0, err);
        if (!(one.one_launch && h1 == h2 && err == 0)) rc = 1;
        if (!f32) ref16 = h1;
    }
    // the oracle's composition at the reference's precision
    auto proj = [&](const std::vector<uint16_t>& xrow, int K, const std::vector<uint16_t>& w, int N) {
        std::vector<int8_t> xq(K), wq(static_cast<size_t>(K) * N);
        float xs32 = 0.f;
        uint16_t xs16 = 0;
        std::vector<float> ws32(N), ws(N);
        std::vector<uint16_t> ws16(N), out(N);
        std::vector<int32_t> acc(N);
        or_w8a8_quantize_act(xrow.data(), 1, K, xq.data(), &xs32, &xs16);
        or_w8a8_quantize_weight(w.data(), K, N, wq.data(), ws32.data(), ws16.data());
        or_gemm_i32(xq.data(), wq.data(), 1, K, N, acc.data(), 0);
        for (int n = 0; n < N; ++n) ws[n] = or_h2f(ws16[n]);
        const float xs = or_h2f(xs16);
        or_w8a8_dequant(acc.data(), &xs, ws.data(), 1, N, out.data());
        return out;
    };
    const auto gate = proj(hx, H, hg, I), up = proj(hx, H, hu, I);
    Tensor gt = dev(gate, 1, I), ut = dev(up, 1, I), at({1, I}, DType::Float16);
    at.allocate();
    silu_mul(gt, ut, at, ctx.stream());
    std::vector<uint16_t> act(I), act_o(I);
    at.copy_to_host(act.data(), act.size() * 2);
    or_silu_mul(gate.data(), up.data(), I, act_o.data());
    int silu_ulps = 0;
    for (int i = 0; i < I; ++i) silu_ulps = std::max(silu_ulps, std::abs(int(act[i]) - int(act_o[i])));
    const auto want = proj(act, I, hd, H);
    int bad = 0;
    for (int n = 0; n < H; ++n) bad += want[n] != ref16[n];
    std::printf("W8A8 decode MLP vs oracle composition (reference precision): mismatches=%d (device vs host silu "
                "within %d fp16 ulp)\n", bad, silu_ulps);
    if (bad != 0 || silu_ulps > 1) rc = 1;

    // give-up: every call counter but workgroup 0's ahead, so workgroup 0
    // (a phase-2 workgroup) polls for a tag that never comes; bounded, so the
    // kernel ends, the status word is set, the next call throws and resets
    {
        DecodeMlpW8A8 one = make_decode_mlp_w8a8(g, u, d);
        Tensor y({1, H}, DType::Float16);
        y.allocate();
        std::vector<uint32_t> ahead(1023, 77u);
        check_hip(hipMemcpy(static_cast<uint8_t*>(one.workspace.data()) + 65 * 4, ahead.data(), ahead.size() * 4,
                            hipMemcpyHostToDevice),
                  "hipMemcpy");
        mlp_w8a8(xt, one, y, ctx.stream());
        ctx.synchronize();
        const bool status = one.status.gave_up();
        bool threw = false;
        try {
            mlp_w8a8(xt, one, y, ctx.stream());
        } catch (const std::runtime_error& e) {
            threw = std::string(e.what()).find("gave up") != std::string::npos;
        }
        mlp_w8a8(xt, one, y, ctx.stream());
        std::vector<uint16_t> hy(H);
        y.copy_to_host(hy.data(), hy.size() * 2);
        std::printf("W8A8 decode MLP give-up: status %d, threw %d, exact after reset %d\n", int(status), int(threw),
                    int(hy == ref16));
        if (!status || !threw || hy != ref16) rc = 1;
    }
    return rc;
}

int main() {
    HipContext ctx(0);
    int rc = run_mlp(ctx, 1024, 3584);
    rc |= run(ctx, 1, 1024, 3584, -8, 7, false);
    rc |= run(ctx, 256, 1024, 512, -128, 127, false);
    rc |= run(ctx, 4, 1024, 64, -128, 127, true);
    return rc;
}
