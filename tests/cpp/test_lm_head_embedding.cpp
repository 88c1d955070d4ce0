// GPU: the lm_head built from the tied token embedding of a checkpoint.  A
// synthetic safetensors file holds model.language_model.embed_tokens.weight
// [248094, 1024] (F16, and a BF16 copy); load_lm_head_w4a16 /
// load_lm_head_w8a8 turn it into the padded vocabulary projection in one
// host pass (what language_model.cpp:170,238-270 builds as 16 transposed,
// zero-padded chunks), and lm_head_greedy_w4a16 / _w8a8 run it.  Checked
// against the oracle over the same padded, transposed matrix: W4A16 logits
// within the fp16 tolerance and the argmax of the device's own logits exact
// (the oracle's token too when its margin is clear); W8A8 logits and token
// bit-exact at the reference's precision (fp16 activation scale, truncated
// fp16 weight scale).
#include "mcv_oracle.h"
#include "mcv_quant.h"
#include "minicpmv/hip_context.h"
#include "minicpmv/lm_head.h"
#include "minicpmv/ops.h"
#include "minicpmv/weights.h"
#include "test_common.h"

#include <cmath>
#include <cstdio>

using namespace minicpmv;

namespace {

// splitmix64: a fast reproducible stream for 254M synthetic weights
struct Mix {
    uint64_t s;
    uint64_t next() {
        uint64_t z = (s += 0x9e3779b97f4a7c15ull);
        z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
        z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
        return z ^ (z >> 31);
    }
    // roughly N(0, sd): the sum of four uniforms, centred and scaled
    float normalish(float sd) {
        const uint64_t r = next();
        float a = 0.f;
        for (int i = 0; i < 4; ++i) a += static_cast<float>((r >> (16 * i)) & 0xffff) * (1.0f / 65536.0f);
        return (a - 2.0f) * 1.7320508f * sd;
    }
};

}  // namespace

int main(int argc, char** argv) {
    const std::string dir = argc > 1 ? argv[1] : "/tmp";
    HipContext ctx(0);
    constexpr int64_t V = 248094, H = 1024, G = H / 128;
    const int64_t N = (V + 63) / 64 * 64;
    const char* name = "model.language_model.embed_tokens.weight";
    std::vector<uint16_t> emb(static_cast<size_t>(V * H));
    Mix mix{2024};
    for (auto& v : emb) v = t::f2h_rne(mix.normalish(0.02f));
    std::vector<uint16_t> emb_bf(static_cast<size_t>(V * H));
    for (size_t i = 0; i < emb.size(); ++i) {           // bf16 bits of the same values (truncated)
        float f = t::h2f(emb[i]);
        uint32_t u;
        std::memcpy(&u, &f, 4);
        emb_bf[i] = static_cast<uint16_t>(u >> 16);
    }
    const std::string path = dir + "/mcv_embed.safetensors";
    t::write_safetensors(path, {{name, "F16", {V, H}, t::bytes_of(emb)},
                                {"bf16.embed_tokens.weight", "BF16", {V, H}, t::bytes_of(emb_bf)}});
    WeightsIndex index(path);

    std::vector<uint16_t> hx(H);
    for (auto& v : hx) v = t::f2h_rne(mix.normalish(1.0f));
    Tensor x({1, H}, DType::Float16);
    x.copy_from_host(hx.data(), H * 2);

    // the oracle's [H, N] projection: the embedding transposed, zero columns from V
    std::vector<uint16_t> pad(static_cast<size_t>(H * N), 0);
    for (int64_t v = 0; v < V; ++v)
        for (int64_t k = 0; k < H; ++k) pad[k * N + v] = emb[v * H + k];
    int rc = 0;

    // ---- W4A16
    {
        W4A16QuantizedWeight w = load_lm_head_w4a16(index, name, V);
        if (w.K != H || w.N != N) rc = 1;
        std::vector<int32_t> qw(static_cast<size_t>(H * (N / 8))), qz(static_cast<size_t>(G * (N / 8)));
        std::vector<uint16_t> sc(static_cast<size_t>(G * N));
        or_quantize_int4_awq(pad.data(), H, N, qw.data(), qz.data(), sc.data());
        std::vector<int8_t> w8(static_cast<size_t>(H * N));
        or_unpack_awq(qw.data(), qz.data(), H, N, w8.data());
        std::vector<float> ref(N);
        or_w4a16_matmul(hx.data(), w8.data(), sc.data(), 1, H, N, ref.data(), 0);
        std::vector<uint16_t> ref16(V);
        for (int64_t n = 0; n < V; ++n) ref16[n] = or_f2h_rne(ref[n]);
        const int64_t want = or_argmax_f16(ref16.data(), V);
        float best = -INFINITY, second = -INFINITY;
        for (int64_t n = 0; n < V; ++n) {
            if (ref[n] > best) { second = best; best = ref[n]; }
            else if (ref[n] > second) second = ref[n];
        }
        LmHeadW4A16 head = make_lm_head_w4a16(std::move(w), V);
        const int64_t tok = lm_head_greedy_w4a16(x, nullptr, 1e-6, head, ctx.stream());
        Tensor lg({1, V}, DType::Float16);
        lg.allocate();
        lm_head_argmax_w4a16(x, head, &lg, ctx.stream());
        const int64_t tok_dev = lm_head_read_token(head, ctx.stream());
        std::vector<uint16_t> got(V);
        lg.copy_to_host(got.data(), V * 2);
        double max_abs = 0, num = 0, den = 0;
        for (int64_t n = 0; n < V; ++n) {
            const double d = static_cast<double>(t::h2f(got[n])) - ref[n];
            max_abs = std::max(max_abs, std::fabs(d));
            num += d * d;
            den += static_cast<double>(ref[n]) * ref[n];
        }
        const double rel = std::sqrt(num / den);
        const int64_t scan = or_argmax_f16(got.data(), V);
        std::printf("W4A16 lm_head from the embedding: token=%lld device-route=%lld argmax(device logits)=%lld "
                    "oracle=%lld margin=%.4f max_abs=%.3e rel_l2=%.3e\n",
                    (long long)tok, (long long)tok_dev, (long long)scan, (long long)want, best - second, max_abs, rel);
        if (max_abs > 2e-2 || rel > 1e-3 || tok != scan || tok_dev != scan) rc = 1;
        if (best - second > 2e-2f && tok != want) rc = 1;
    }

    // ---- W8A8 (tiled and [K, N]), from the F16 tensor and from the BF16 copy
    // (converted as the reference loads bf16: weights.cpp:25-33)
    auto w8_oracle = [&](const std::vector<uint16_t>& e16, std::vector<uint16_t>& want) {
        std::vector<uint16_t> p16(static_cast<size_t>(H * N), 0);
        for (int64_t v = 0; v < V; ++v)
            for (int64_t k = 0; k < H; ++k) p16[k * N + v] = e16[v * H + k];
        std::vector<int8_t> wq(static_cast<size_t>(H * N));
        std::vector<float> ws32(N), ws(N);
        std::vector<uint16_t> ws16(N);
        or_w8a8_quantize_weight(p16.data(), H, N, wq.data(), ws32.data(), ws16.data());
        std::vector<int8_t> xq(H);
        float xs32 = 0.f;
        uint16_t xs16 = 0;
        or_w8a8_quantize_act(hx.data(), 1, H, xq.data(), &xs32, &xs16);
        std::vector<int32_t> acc(N);
        or_gemm_i32(xq.data(), wq.data(), 1, H, N, acc.data(), 0);
        for (int64_t n = 0; n < N; ++n) ws[n] = or_h2f(ws16[n]);
        const float xs = or_h2f(xs16);
        want.assign(N, 0);
        or_w8a8_dequant(acc.data(), &xs, ws.data(), 1, N, want.data());
        return or_argmax_f16(want.data(), V);
    };
    {
        std::vector<uint16_t> emb_bf16(emb_bf.size());
        or_bf16_to_f16_trunc_array(emb_bf.data(), static_cast<int64_t>(emb_bf.size()), emb_bf16.data());
        for (int from_bf : {0, 1}) {
            std::vector<uint16_t> want;
            const int64_t want_tok = w8_oracle(from_bf ? emb_bf16 : emb, want);
            const char* src = from_bf ? "bf16.embed_tokens.weight" : name;
            for (int layout : {MCV_W8_TILED, MCV_W8_KN}) {
                W8A8QuantizedWeight w8 = load_lm_head_w8a8(index, src, V, layout);
                LmHeadW8A8 h8 = make_lm_head_w8a8(w8, V);
                const int64_t tok = lm_head_greedy_w8a8(x, nullptr, 1e-6, h8, ctx.stream());
                std::vector<uint16_t> got(V);
                h8.logits.copy_to_host(got.data(), V * 2);
                int bad = 0;
                for (int64_t n = 0; n < V; ++n) bad += got[n] != want[n];
                std::printf("W8A8 lm_head from %s (%s): token=%lld oracle=%lld logit mismatches=%d\n", src,
                            layout == MCV_W8_TILED ? "tiled" : "[K, N]", (long long)tok, (long long)want_tok, bad);
                if (bad != 0 || tok != want_tok) rc = 1;
            }
        }
    }
    std::remove(path.c_str());
    std::printf("%s\n", rc ? "FAILED" : "ok");
    return rc;
}
