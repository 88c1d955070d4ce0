// W4A16 M=1 against the CPU reference on the gate_proj shape K=1024 N=3584,
// with the inputs of the reference's test (tests/test_matmul_w4a16.cpp:173-241:
// mt19937(0); x ~ U[-0.3, 0.3], w8 ~ U{-8..7}, s ~ U[0.001, 0.02], truncating
// fp16 encode).  Runs both device formats: the reference's int8 tile format
// through the 4-argument matmul_w4a16, and the nibble-packed slab-64 format
// (w8 = q - 8 packed as AutoAWQ with zero 8) through the weight overload.
#include "minicpmv/hip_context.h"
#include "minicpmv/ops.h"
#include "minicpmv/quantized_weight.h"
#include "test_common.h"

#include <algorithm>
#include <cmath>
#include <random>

using namespace minicpmv;

static int64_t tile_len_for(int64_t N) {
    const int64_t block = (N + 7) / 8, tiles = (block + 447) / 448;
    return std::max<int64_t>(16, ((block + tiles - 1) / tiles + 15) / 16 * 16);
}

// The reference's pack_w4a16_weight (src/csrc/lib/quantized_weight.cpp:48-73), to build its format.
static std::vector<int8_t> tile_pack(const std::vector<int8_t>& w, int64_t K, int64_t N, int64_t tile) {
    const int64_t G = K / 128, block = (N + 7) / 8, tpb = (block + tile - 1) / tile;
    std::vector<int8_t> p(static_cast<size_t>(G * 8 * tpb * 128 * tile), 0);
    for (int64_t g = 0; g < G; ++g)
        for (int64_t b = 0; b < 8; ++b) {
            const int64_t valid = std::max<int64_t>(0, std::min<int64_t>(block, N - b * block));
            for (int64_t t2 = 0; t2 < tpb; ++t2) {
                const int64_t tv = std::max<int64_t>(0, std::min<int64_t>(tile, valid - t2 * tile));
                const size_t base = static_cast<size_t>((((g * 8 + b) * tpb + t2) * 128) * tile);
                for (int64_t kk = 0; kk < 128; ++kk)
                    for (int64_t i = 0; i < tv; ++i)
                        p[base + kk * tile + i] = w[(g * 128 + kk) * N + b * block + t2 * tile + i];
            }
        }
    return p;
}

int main() {
    HipContext ctx(0);
    constexpr int K = 1024, N = 3584, G = 128, NG = K / G;
    std::mt19937 rng(0);
    std::uniform_real_distribution<float> xd(-0.3f, 0.3f);
    std::uniform_int_distribution<int> wd(-8, 7);
    std::uniform_real_distribution<float> sd(0.001f, 0.02f);
    std::vector<uint16_t> hx(K);
    for (auto& v : hx) v = t::f2h(xd(rng));
    std::vector<int8_t> hw(static_cast<size_t>(K) * N);
    for (auto& v : hw) v = static_cast<int8_t>(wd(rng));
    std::vector<uint16_t> hs(NG * N);
    for (auto& v : hs) v = t::f2h(sd(rng));

    std::vector<float> ref(N, 0.0f);
    for (int g = 0; g < NG; ++g)
        for (int n = 0; n < N; ++n) {
            float partial = 0.0f;
            for (int kk = 0; kk < G; ++kk) partial += t::h2f(hx[g * G + kk]) * static_cast<float>(hw[(g * G + kk) * N + n]);
            ref[n] += partial * t::h2f(hs[g * N + n]);
        }

    Tensor x({1, K}, DType::Float16);
    x.copy_from_host(hx.data(), hx.size() * 2);
    Tensor s({NG, N}, DType::Float16);
    s.copy_from_host(hs.data(), hs.size() * 2);
    Tensor out({1, N}, DType::Float16);
    out.allocate();

    auto check = [&](const char* what) {
        std::vector<uint16_t> ho(N);
        out.copy_to_host(ho.data(), ho.size() * 2);
        float max_abs = 0.0f;
        int big = 0;
        for (int n = 0; n < N; ++n) {
            const float d = std::fabs(ref[n] - t::h2f(ho[n]));
            max_abs = std::max(max_abs, d);
            if (d > 0.1f) ++big;
        }
        std::printf("%s K=%d N=%d max_abs_diff=%.5f large(>0.1)=%d\n", what, K, N, max_abs, big);
        return big == 0 && max_abs <= 2e-2f;
    };

    // 1) the reference's own device format
    const int64_t tile = tile_len_for(N);
    std::vector<int8_t> packed = tile_pack(hw, K, N, tile);
    Tensor w({static_cast<int64_t>(packed.size() / tile), tile}, DType::Int8);
    w.copy_from_host(packed.data(), packed.size());
    matmul_w4a16(x, w, s, out, ctx.stream());
    if (!check("tile-int8")) return 1;

    // 2) nibble-packed: q = w8 + 8 in AutoAWQ packing, zero-point 8
    constexpr int order[8] = {0, 2, 4, 6, 1, 3, 5, 7};
    std::vector<int32_t> qweight(static_cast<size_t>(K) * N / 8), qzeros(static_cast<size_t>(NG) * N / 8, 0);
    for (int k = 0; k < K; ++k)
        for (int j = 0; j < N / 8; ++j) {
            uint32_t word = 0;
            for (int sl = 0; sl < 8; ++sl) word |= static_cast<uint32_t>(hw[k * N + j * 8 + order[sl]] + 8) << (4 * sl);
            qweight[k * (N / 8) + j] = static_cast<int32_t>(word);
        }
    for (auto& z : qzeros) z = static_cast<int32_t>(0x88888888u);
    W4A16QuantizedWeight q4 = pack_w4a16_awq(qweight.data(), qzeros.data(), hs.data(), K, N);
    matmul_w4a16(x, q4, out, ctx.stream());
    if (!check("slab64-nibbles")) return 1;

    // 3) the decode MLP block over the same gate/up weight and a [N, K] down
    // projection: one launch == gate+up+silu*mul then the down GEMV, bit for bit
    {
        std::vector<int32_t> dq(static_cast<size_t>(N) * K / 8), dz(static_cast<size_t>(N / G) * K / 8);
        std::vector<uint16_t> ds(static_cast<size_t>(N / G) * K);
        std::uniform_int_distribution<int> qd(0, 15);
        for (auto& v : dq) {
            uint32_t word = 0;
            for (int sl = 0; sl < 8; ++sl) word |= static_cast<uint32_t>(qd(rng)) << (4 * sl);
            v = static_cast<int32_t>(word);
        }
        for (auto& v : dz) v = static_cast<int32_t>(0x77777777u);
        for (auto& v : ds) v = t::f2h(sd(rng));
        W4A16QuantizedWeight down = pack_w4a16_awq(dq.data(), dz.data(), ds.data(), N, K);
        DecodeMlpW4A16 mlp = make_decode_mlp_w4a16(q4, q4, down);
        Tensor y1({1, K}, DType::Float16), y2({1, K}, DType::Float16), act({1, N}, DType::Float16);
        y1.allocate();
        y2.allocate();
        act.allocate();
        for (int rep = 0; rep < 3; ++rep) mlp_w4a16(x, mlp, y1, ctx.stream());
        mlp_gate_up_silu_w4a16(x, q4, q4, act, ctx.stream());
        matmul_w4a16(act, down, y2, ctx.stream());
        std::vector<uint16_t> h1(K), h2(K);
        y1.copy_to_host(h1.data(), h1.size() * 2);
        y2.copy_to_host(h2.data(), h2.size() * 2);
        uint32_t err = 1;
        mlp.workspace.copy_to_host(&err, 4);
        std::printf("decode MLP one_launch=%d bit-identical=%d give-up flag=%u\n", mlp.one_launch ? 1 : 0,
                    h1 == h2 ? 1 : 0, err);
        if (!mlp.one_launch || h1 != h2 || err != 0) return 1;

        // A give-up of the one-launch kernel's bounded waits, forced from the
        // host: every call counter but workgroup 0's (u32 words 65..1087 of
        // the workspace) set ahead, so workgroup 0 -- a phase-2 workgroup --
        // never sees the tag it polls for.  The kernel still ends; the status
        // word turns non-zero without a synchronisation; the next call
        // throws, resets the workspace, and the call after that is exact again.
        std::vector<uint32_t> ahead(1023, 77u);
        check_hip(hipMemcpy(static_cast<uint8_t*>(mlp.workspace.data()) + 65 * 4, ahead.data(), ahead.size() * 4,
                            hipMemcpyHostToDevice),
                  "hipMemcpy");
        mlp_w4a16(x, mlp, y1, ctx.stream());
        ctx.synchronize();
        uint32_t ws_flag = 0;
        mlp.workspace.copy_to_host(&ws_flag, 4);
        const bool status = mlp.status.gave_up();
        bool threw = false;
        try {
            mlp_w4a16(x, mlp, y1, ctx.stream());
        } catch (const std::runtime_error& e) {
            threw = std::string(e.what()).find("gave up") != std::string::npos;
        }
        mlp_w4a16(x, mlp, y1, ctx.stream());
        y1.copy_to_host(h1.data(), h1.size() * 2);
        check_wait_status(mlp, ctx.stream());              // no give-up since the reset: no throw
        std::printf("decode MLP give-up: workspace flag %u, status %d, threw %d, exact after reset %d\n", ws_flag,
                    int(status), int(threw), int(h1 == h2));
        if (ws_flag == 0 || !status || !threw || h1 != h2) return 1;

        // The K split across workgroups into a caller-owned workspace, on the
        // down projection's shape (K=3584, N=1024) at M = 128: within fp16
        // rounding of the unsplit kernel (the C-ABI without a workspace; only
        // the fp32 summation order differs), the same bits on every call, the
        // workspace allocated once.
        constexpr int MR = 128;
        Tensor a({MR, N}, DType::Float16), o1({MR, K}, DType::Float16), o2({MR, K}, DType::Float16), wsp;
        a.allocate();
        o1.allocate();
        o2.allocate();
        std::vector<uint16_t> ha(static_cast<size_t>(MR) * N), r1(static_cast<size_t>(MR) * K), r2(r1.size()),
            r3(r1.size());
        for (auto& v : ha) v = t::f2h(xd(rng));
        a.copy_from_host(ha.data(), ha.size() * 2);
        check_mcv(mcv_w4a16_gemm(a.data(), MR, down.K, down.N, down.w_int8.data(), down.scales.data(),
                                 down.zeros.data(), down.zero_bias, o1.data(), ctx.stream()),
                  "unsplit GEMM");
        matmul_w4a16(a, down, o2, ctx.stream(), wsp);
        const int64_t nb = mcv_w4a16_gemm_workspace_bytes(MR, N, K);
        const void* const first = wsp.data();
        o1.copy_to_host(r1.data(), r1.size() * 2);
        o2.copy_to_host(r2.data(), r2.size() * 2);
        matmul_w4a16(a, down, o2, ctx.stream(), wsp);
        o2.copy_to_host(r3.data(), r3.size() * 2);
        double worst = 0.0;
        for (size_t i = 0; i < r1.size(); ++i) {
            const double u = t::h2f(r1[i]), v = t::h2f(r2[i]);
            worst = std::max(worst, std::fabs(u - v) / (std::fabs(u) + 1e-2));
        }
        std::printf("split-K M=%d: workspace %lld bytes (allocated %zu), max rel diff vs unsplit %.2e, repeat %d, "
                    "reused %d\n", MR, static_cast<long long>(nb), wsp.numel(), worst, int(r2 == r3),
                    int(wsp.data() == first));
        if (nb <= 0 || static_cast<int64_t>(wsp.numel()) < nb || worst > 2e-3 || r2 != r3 || wsp.data() != first)
            return 1;
    }

    // 4) shape validation mirrors the reference's host wrapper
    try {
        Tensor bad({2, K}, DType::Float16);
        bad.allocate();
        matmul_w4a16(bad, w, s, out, ctx.stream());
        std::printf("expected a shape error\n");
        return 1;
    } catch (const std::runtime_error& e) {
        std::printf("rejected as expected: %s\n", e.what());
    }
    return 0;
}
