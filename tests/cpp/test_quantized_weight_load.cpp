// Loader: AutoAWQ and GPTQ checkpoints written to a safetensors file load
// through load_w4a16_quantized_weight (GPTQ chosen by the presence of g_idx,
// quantized_weight.cpp:212-214), and the loaded weight multiplies like the CPU
// reference formula on the unpacked (q - z).  Also checks the dequantised
// int8 values bit for bit against a host unpack.  W8A8: checkpoint [N, K]
// F16 / BF16 weights quantise in one host pass to the same bytes as the
// reference's transpose + quantize_dense_weight_w8a8, and pre-quantised I8
// weights with F32 / F16 scales load to the tiled layout and multiply exactly.
#include "minicpmv/hip_context.h"
#include "minicpmv/ops.h"
#include "minicpmv/quantized_weight.h"
#include "test_common.h"

#include <cmath>
#include <cstring>
#include <random>

using namespace minicpmv;

static int check(HipContext& ctx, const W4A16QuantizedWeight& w, const std::vector<int8_t>& w8,
                 const std::vector<uint16_t>& scales, const char* what) {
    const int64_t K = w.K, N = w.N;
    std::mt19937 rng(7);
    std::normal_distribution<float> nd(0.f, 1.f);
    std::vector<uint16_t> hx(static_cast<size_t>(K));
    for (auto& v : hx) v = t::f2h_rne(nd(rng));
    Tensor x({1, K}, DType::Float16);
    x.copy_from_host(hx.data(), hx.size() * 2);
    Tensor out({1, N}, DType::Float16);
    out.allocate();
    matmul_w4a16(x, w, out, ctx.stream());
    std::vector<uint16_t> ho(static_cast<size_t>(N));
    out.copy_to_host(ho.data(), ho.size() * 2);
    double num = 0, den = 0, max_abs = 0;
    for (int64_t n = 0; n < N; ++n) {
        float ref = 0.f;
        for (int64_t g = 0; g < K / 128; ++g) {
            float part = 0.f;
            for (int64_t kk = 0; kk < 128; ++kk) part += t::h2f(hx[g * 128 + kk]) * static_cast<float>(w8[(g * 128 + kk) * N + n]);
            ref += part * t::h2f(scales[g * N + n]);
        }
        const double d = std::fabs(ref - t::h2f(ho[n]));
        max_abs = std::max(max_abs, d);
        num += d * d;
        den += double(ref) * ref;
    }
    bool exact = true;
    if (w.dense_kn.numel() > 0) {
        // kept dense (an act-order block spans more than 16 levels): every
        // value is RNE(w8 * scale of its k / 128 group)
        std::vector<uint16_t> hd(static_cast<size_t>(K * N));
        w.dense_kn.copy_to_host(hd.data(), hd.size() * 2);
        for (int64_t k = 0; k < K; ++k)
            for (int64_t n = 0; n < N; ++n)
                exact &= hd[k * N + n] ==
                         t::f2h_rne(static_cast<float>(w8[k * N + n]) * t::h2f(scales[(k / 128) * N + n]));
    } else {
        Tensor wi8({K, N}, DType::Int8);
        wi8.allocate();
        w4a16_dequant(w, nullptr, &wi8, ctx.stream());
        std::vector<int8_t> hw8(static_cast<size_t>(K * N));
        wi8.copy_to_host(hw8.data(), hw8.size());
        exact = hw8 == w8;
    }
    std::printf("%s K=%lld N=%lld max_abs=%.2e rel_l2=%.2e dequant_exact=%d\n", what, (long long)K, (long long)N, max_abs,
                std::sqrt(num / den), int(exact));
    return (max_abs <= 2e-2 && std::sqrt(num / den) <= 1e-3 && exact) ? 0 : 1;
}


// bf16 -> fp16 as the reference loads checkpoint tensors (weights.cpp:25-33)
static uint16_t bf16_to_f16(uint16_t bf) {
    const uint32_t x = static_cast<uint32_t>(bf) << 16;
    const uint32_t sign = (x >> 16) & 0x8000u;
    const int32_t e = static_cast<int32_t>((x >> 23) & 0xffu) - 112;
    if (e <= 0) return static_cast<uint16_t>(sign);
    if (e >= 31) return static_cast<uint16_t>(sign | 0x7c00u);
    return static_cast<uint16_t>(sign | (static_cast<uint32_t>(e) << 10) | ((x & 0x7fffffu) >> 13));
}

template <typename T>
static std::vector<T> host_copy(const Tensor& t) {
    std::vector<T> v(t.size_bytes() / sizeof(T));
    t.copy_to_host(v.data(), t.size_bytes());
    return v;
}

static int check_w8a8(HipContext& ctx, const std::string& dir) {
    constexpr int64_t N = 208, K = 384;
    std::mt19937 rng(11);
    std::normal_distribution<float> nd(0.f, 0.02f);
    std::vector<uint16_t> w_nk(static_cast<size_t>(N * K)), bf_nk(static_cast<size_t>(N * K));
    for (auto& v : w_nk) v = t::f2h_rne(nd(rng));
    for (auto& v : bf_nk) {
        const float f = nd(rng);
        uint32_t bits;
        std::memcpy(&bits, &f, 4);
        v = static_cast<uint16_t>(bits >> 16);
    }
    std::uniform_int_distribution<int> qd(-128, 127);
    std::vector<int8_t> q_nk(static_cast<size_t>(N * K));
    for (auto& v : q_nk) v = static_cast<int8_t>(qd(rng));
    std::vector<float> s_f32(static_cast<size_t>(N));
    std::vector<uint16_t> s_f16(static_cast<size_t>(N));
    for (int64_t n = 0; n < N; ++n) {
        s_f32[n] = 0.001f + 0.0001f * static_cast<float>(n % 13);
        s_f16[n] = t::f2h_rne(s_f32[n]);
    }
    const std::string p = dir + "/mcv_w8a8.safetensors";
    t::write_safetensors(p, {{"a.weight", "F16", {N, K}, t::bytes_of(w_nk)},
                             {"b.weight", "BF16", {N, K}, t::bytes_of(bf_nk)},
                             {"c.weight", "I8", {N, K}, t::bytes_of(q_nk)},
                             {"c.weight_scale", "F32", {N}, t::bytes_of(s_f32)},
                             {"d.weight", "I8", {N, K}, t::bytes_of(q_nk)},
                             {"d.weight_scale", "F16", {N, 1}, t::bytes_of(s_f16)}});
    WeightsIndex idx(p);
    int rc = 0;
    if (has_w8a8_quantized_weight(idx, "a") || !has_w8a8_quantized_weight(idx, "c") ||
        !has_w8a8_quantized_weight(idx, "d")) {
        std::printf("has_w8a8_quantized_weight wrong\n");
        rc = 1;
    }
    // dense sources: the same bytes and scales as transpose + quantize_dense_weight_w8a8
    for (int src = 0; src < 2; ++src) {
        std::vector<uint16_t> kn(static_cast<size_t>(K * N));
        for (int64_t n = 0; n < N; ++n)
            for (int64_t k = 0; k < K; ++k) kn[k * N + n] = src ? bf16_to_f16(bf_nk[n * K + k]) : w_nk[n * K + k];
        const W8A8QuantizedWeight ref = quantize_w8a8_host(kn.data(), K, N, MCV_W8_TILED);
        const W8A8QuantizedWeight got = load_w8a8_quantized_weight(idx, src ? "b" : "a");
        const bool same = host_copy<int8_t>(ref.w_int8) == host_copy<int8_t>(got.w_int8) &&
                          host_copy<uint32_t>(ref.w_scale_f32) == host_copy<uint32_t>(got.w_scale_f32) &&
                          host_copy<uint16_t>(ref.w_scale) == host_copy<uint16_t>(got.w_scale) &&
                          got.layout == MCV_W8_TILED && got.K == K && got.N == N;
        std::printf("W8A8 %s checkpoint == transpose + quantize: %d\n", src ? "BF16" : "F16", int(same));
        if (!same) rc = 1;
        const W8A8QuantizedWeight kn_w = load_w8a8_quantized_weight(idx, src ? "b" : "a", MCV_W8_KN);
        const W8A8QuantizedWeight kn_ref = quantize_w8a8_host(kn.data(), K, N, MCV_W8_KN);
        if (host_copy<int8_t>(kn_w.w_int8) != host_copy<int8_t>(kn_ref.w_int8)) {
            std::printf("W8A8 [K, N] layout differs\n");
            rc = 1;
        }
    }
    // pre-quantised I8: exact int32 products through the tiled GEMM and GEMV
    for (const char* name : {"c", "d"}) {
        const W8A8QuantizedWeight w = load_w8a8_quantized_weight(idx, name);
        const std::vector<float> sc = host_copy<float>(w.w_scale_f32);
        bool scales_ok = true;
        for (int64_t n = 0; n < N; ++n)
            scales_ok &= name[0] == 'c' ? sc[n] == s_f32[n] : sc[n] == t::h2f(s_f16[n]);
        for (int64_t M : {3, 70}) {
            std::vector<int8_t> hx(static_cast<size_t>(M * K));
            for (auto& v : hx) v = static_cast<int8_t>(qd(rng));
            Tensor x({M, K}, DType::Int8);
            x.copy_from_host(hx.data(), hx.size());
            Tensor acc({M, N}, DType::Int32);
            acc.allocate();
            matmul_w8a8_i32(x, w, acc, ctx.stream());
            const std::vector<int32_t> ha = host_copy<int32_t>(acc);
            bool exact = true;
            for (int64_t m = 0; m < M; ++m)
                for (int64_t n = 0; n < N; ++n) {
                    int32_t r = 0;
                    for (int64_t k = 0; k < K; ++k) r += int32_t(hx[m * K + k]) * int32_t(q_nk[n * K + k]);
                    exact &= r == ha[m * N + n];
                }
            std::printf("W8A8 I8 checkpoint %s M=%lld: int32 exact %d, scales %d\n", name, (long long)M, int(exact),
                        int(scales_ok));
            if (!exact || !scales_ok) rc = 1;
        }
    }
    return rc;
}

int main(int argc, char** argv) {
    HipContext ctx(0);
    const std::string dir = argc > 1 ? argv[1] : "/tmp";
    constexpr int64_t K = 512, N = 200, G = K / 128;
    constexpr int order[8] = {0, 2, 4, 6, 1, 3, 5, 7};
    std::mt19937 rng(3);
    std::uniform_int_distribution<int> nib(0, 15);
    std::uniform_real_distribution<float> sd(0.001f, 0.01f);
    std::vector<uint8_t> q(static_cast<size_t>(K * N)), z(static_cast<size_t>(G * N));
    for (auto& v : q) v = static_cast<uint8_t>(nib(rng));
    for (auto& v : z) v = static_cast<uint8_t>(nib(rng));
    std::vector<uint16_t> scales(static_cast<size_t>(G * N));
    for (auto& v : scales) v = t::f2h_rne(sd(rng));
    int rc = 0;

    // AutoAWQ: qweight [K, N/8], qzeros [G, N/8], column order within a word
    std::vector<int32_t> aq(static_cast<size_t>(K * N / 8)), az(static_cast<size_t>(G * N / 8));
    for (int64_t k = 0; k < K; ++k)
        for (int64_t j = 0; j < N / 8; ++j) {
            uint32_t w = 0;
            for (int s = 0; s < 8; ++s) w |= uint32_t(q[k * N + j * 8 + order[s]]) << (4 * s);
            aq[k * (N / 8) + j] = static_cast<int32_t>(w);
        }
    for (int64_t g = 0; g < G; ++g)
        for (int64_t j = 0; j < N / 8; ++j) {
            uint32_t w = 0;
            for (int s = 0; s < 8; ++s) w |= uint32_t(z[g * N + j * 8 + order[s]]) << (4 * s);
            az[g * (N / 8) + j] = static_cast<int32_t>(w);
        }
    std::vector<int8_t> w8(static_cast<size_t>(K * N));
    for (int64_t k = 0; k < K; ++k)
        for (int64_t n = 0; n < N; ++n) w8[k * N + n] = static_cast<int8_t>(int(q[k * N + n]) - int(z[(k / 128) * N + n]));
    const std::string pa = dir + "/mcv_awq.safetensors";
    t::write_safetensors(pa, {{"m.proj.qweight", "I32", {K, N / 8}, t::bytes_of(aq)},
                              {"m.proj.qzeros", "I32", {G, N / 8}, t::bytes_of(az)},
                              {"m.proj.scales", "F16", {G, N}, t::bytes_of(scales)}});
    WeightsIndex ia(pa);
    if (!has_w4a16_quantized_weight(ia, "m.proj") || has_w4a16_quantized_weight(ia, "m.other")) rc = 1;
    rc |= check(ctx, load_w4a16_quantized_weight(ia, "m.proj"), w8, scales, "AWQ");

    // GPTQ v1: qweight [K/8, N] along K, qzeros [G, N/8] natural order storing zero - 1
    std::vector<int32_t> gq(static_cast<size_t>(K / 8 * N)), gz(static_cast<size_t>(G * N / 8));
    for (int64_t k0 = 0; k0 < K / 8; ++k0)
        for (int64_t n = 0; n < N; ++n) {
            uint32_t w = 0;
            for (int i = 0; i < 8; ++i) w |= uint32_t(q[(k0 * 8 + i) * N + n]) << (4 * i);
            gq[k0 * N + n] = static_cast<int32_t>(w);
        }
    for (int64_t g = 0; g < G; ++g)
        for (int64_t j = 0; j < N / 8; ++j) {
            uint32_t w = 0;
            for (int s = 0; s < 8; ++s) w |= uint32_t(z[g * N + j * 8 + s] & 15u) << (4 * s);
            gz[g * (N / 8) + j] = static_cast<int32_t>(w);
        }
    std::vector<int8_t> w8g(static_cast<size_t>(K * N));
    for (int64_t k = 0; k < K; ++k)
        for (int64_t n = 0; n < N; ++n) w8g[k * N + n] = static_cast<int8_t>(int(q[k * N + n]) - (int(z[(k / 128) * N + n]) + 1));
    std::vector<int32_t> gidx(static_cast<size_t>(K));
    for (int64_t k = 0; k < K; ++k) gidx[k] = static_cast<int32_t>(k / 128);
    const std::string pg = dir + "/mcv_gptq.safetensors";
    t::write_safetensors(pg, {{"m.proj.qweight", "I32", {K / 8, N}, t::bytes_of(gq)},
                              {"m.proj.qzeros", "I32", {G, N / 8}, t::bytes_of(gz)},
                              {"m.proj.g_idx", "I32", {K}, t::bytes_of(gidx)},
                              {"m.proj.scales", "F16", {G, N}, t::bytes_of(scales)}});
    WeightsIndex ig(pg);
    rc |= check(ctx, load_w4a16_quantized_weight(ig, "m.proj"), w8g, scales, "GPTQ");

    // act-order g_idx (quantized_weight.cpp:98-117): row k's zero comes from
    // group g_idx[k], its scale stays that of group k / 128.  Stored zeros 6
    // and 7 alternate by group and the nibbles stay below 15, so every
    // 128-row block's values fit one common zero (16 levels).
    std::swap(gidx[0], gidx[K - 1]);
    std::swap(gidx[5], gidx[K / 2 + 3]);
    std::vector<int32_t> gq2(gq.size()), gz2(gz.size());
    for (size_t i = 0; i < gq.size(); ++i) gq2[i] = static_cast<int32_t>(static_cast<uint32_t>(gq[i]) & 0x77777777u);
    for (int64_t g = 0; g < G; ++g)
        for (int64_t j = 0; j < N / 8; ++j) gz2[g * (N / 8) + j] = static_cast<int32_t>(g % 2 ? 0x77777777u : 0x66666666u);
    for (int64_t k = 0; k < K; ++k)
        for (int64_t n = 0; n < N; ++n)
            w8g[k * N + n] = static_cast<int8_t>(int(q[k * N + n] & 7u) - (6 + int(gidx[k] % 2) + 1));
    t::write_safetensors(pg, {{"m.proj.qweight", "I32", {K / 8, N}, t::bytes_of(gq2)},
                              {"m.proj.qzeros", "I32", {G, N / 8}, t::bytes_of(gz2)},
                              {"m.proj.g_idx", "I32", {K}, t::bytes_of(gidx)},
                              {"m.proj.scales", "F16", {G, N}, t::bytes_of(scales)}});
    WeightsIndex ig2(pg);
    rc |= check(ctx, load_w4a16_quantized_weight(ig2, "m.proj"), w8g, scales, "GPTQ act-order");

    // act-order rows drawn from zero-1 and zero-16 groups (stored zeros 0 and
    // 15) with the full nibble range: the blocks' values span 31 levels, which
    // one 4-bit zero per block cannot hold, so the loader keeps the weight as
    // its dense fp16 values and matmul_w4a16 runs a dense GEMM over it
    std::vector<int32_t> gz3(gz.size()), gidx3(static_cast<size_t>(K));
    for (int64_t g = 0; g < G; ++g)
        for (int64_t j = 0; j < N / 8; ++j) gz3[g * (N / 8) + j] = static_cast<int32_t>(g % 2 ? 0xFFFFFFFFu : 0u);
    for (int64_t k = 0; k < K; ++k) gidx3[k] = static_cast<int32_t>(k % 2);
    for (int64_t k = 0; k < K; ++k)
        for (int64_t n = 0; n < N; ++n) w8g[k * N + n] = static_cast<int8_t>(int(q[k * N + n]) - (k % 2 ? 16 : 1));
    t::write_safetensors(pg, {{"m.proj.qweight", "I32", {K / 8, N}, t::bytes_of(gq)},
                              {"m.proj.qzeros", "I32", {G, N / 8}, t::bytes_of(gz3)},
                              {"m.proj.g_idx", "I32", {K}, t::bytes_of(gidx3)},
                              {"m.proj.scales", "F16", {G, N}, t::bytes_of(scales)}});
    WeightsIndex ig3(pg);
    const W4A16QuantizedWeight wd = load_w4a16_quantized_weight(ig3, "m.proj");
    if (wd.dense_kn.numel() != static_cast<size_t>(K * N) || wd.w_int8.numel() != 0) {
        std::printf("GPTQ act-order, 31 levels: not kept dense\n");
        rc |= 1;
    }
    rc |= check(ctx, wd, w8g, scales, "GPTQ act-order, 31 levels (dense)");
    rc |= check_w8a8(ctx, dir);
    return rc;
}
