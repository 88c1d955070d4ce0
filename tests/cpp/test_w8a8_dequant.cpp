// GPU: the W8A8 epilogue of the C++ surface (w8a8_dequant) against the
// reference's deterministic dequant vectors, held in
// tests/golden/w8a8_dequant_reference.npz (the fixture of
// tests/test_w8a8_dequant.cpp:42-63); the pytest wrapper unpacks them into
// raw little-endian files in the directory given as argv[1]:
//   acc.i32  int32 [N]   accumulators
//   ws.f16   fp16  [N]   per-channel weight scales
//   xs.f16   fp16  [1]   the row's activation scale
//   out.f16  fp16  [N]   the expected fp16 outputs
// Three passes:
//   1. the fixture row, fp16 scales: every output bit-identical to out.f16,
//      and within the fixture's own tolerance (0.02) of acc * xs * ws;
//   2. a 4-row batch made from the fixture row (row r's accumulators rotated
//      by 97 r columns, its scale xs * {1, 1/2, 2, 1/4}), so a wrong row
//      stride, row scale or column pairing shows: bit-exact against the
//      oracle's epilogue, which must itself reproduce out.f16 on row 0;
//   3. the same batch with fp32 scales (the widened fp16 values), bit-exact
//      against the oracle with the same floats.
#include "mcv_oracle.h"
#include "minicpmv/hip_context.h"
#include "minicpmv/ops.h"
#include "test_common.h"

#include <cmath>
#include <fstream>

using namespace minicpmv;

namespace {

template <typename T>
std::vector<T> read_raw(const std::string& path) {
    std::ifstream f(path, std::ios::binary | std::ios::ate);
    if (!f) {
        std::fprintf(stderr, "cannot open %s\n", path.c_str());
        std::exit(2);
    }
    const std::streamsize n = f.tellg();
    std::vector<T> v(static_cast<size_t>(n) / sizeof(T));
    f.seekg(0);
    f.read(reinterpret_cast<char*>(v.data()), static_cast<std::streamsize>(v.size() * sizeof(T)));
    return v;
}

int count_diff(const std::vector<uint16_t>& a, const std::vector<uint16_t>& b) {
    int d = 0;
    for (size_t i = 0; i < a.size(); ++i) d += a[i] != b[i];
    return d;
}

// One w8a8_dequant call over [rows, N] with the given scale tensors; returns the fp16 bits.
std::vector<uint16_t> dequant(const std::vector<int32_t>& acc, int64_t rows, int64_t n, const Tensor& xs,
                              const Tensor& ws, hipStream_t stream) {
    Tensor a({rows, n}, DType::Int32);
    a.copy_from_host(acc.data(), acc.size() * sizeof(int32_t));
    Tensor out({rows, n}, DType::Float16);
    out.allocate();
    w8a8_dequant(a, xs, ws, out, stream);
    std::vector<uint16_t> h(static_cast<size_t>(rows * n));
    out.copy_to_host(h.data(), h.size() * 2);
    return h;
}

}  // namespace

int main(int argc, char** argv) {
    if (argc < 2) {
        std::fprintf(stderr, "usage: %s <dir with acc.i32 ws.f16 xs.f16 out.f16>\n", argv[0]);
        return 2;
    }
    const std::string dir = argv[1];
    const auto acc = read_raw<int32_t>(dir + "/acc.i32");
    const auto ws16 = read_raw<uint16_t>(dir + "/ws.f16");
    const auto xs16 = read_raw<uint16_t>(dir + "/xs.f16");
    const auto want = read_raw<uint16_t>(dir + "/out.f16");
    const int64_t N = static_cast<int64_t>(acc.size());
    if (N == 0 || ws16.size() != acc.size() || want.size() != acc.size() || xs16.size() != 1) {
        std::fprintf(stderr, "fixture sizes disagree\n");
        return 2;
    }
    HipContext ctx(0);
    int rc = 0;

    // ---- 1: the fixture row as it stands
    Tensor xs1({1}, DType::Float16);
    xs1.copy_from_host(xs16.data(), 2);
    Tensor ws({N}, DType::Float16);
    ws.copy_from_host(ws16.data(), ws16.size() * 2);
    const auto got1 = dequant(acc, 1, N, xs1, ws, ctx.stream());
    double worst = 0.0;
    for (int64_t n = 0; n < N; ++n) {
        const double exact = static_cast<double>(acc[n]) * t::h2f(xs16[0]) * t::h2f(ws16[n]);
        worst = std::max(worst, std::fabs(exact - static_cast<double>(t::h2f(got1[n]))));
    }
    const int bad1 = count_diff(got1, want);
    std::printf("fixture row: %d of %lld outputs differ from the fixture, max |out - acc*xs*ws| = %.5f\n", bad1,
                (long long)N, worst);
    if (bad1 != 0 || !(worst < 0.02)) rc = 1;

    // ---- 2 and 3: a 4-row batch built from the fixture row
    constexpr int64_t R = 4;
    const float row_mul[R] = {1.0f, 0.5f, 2.0f, 0.25f};
    std::vector<int32_t> accb(static_cast<size_t>(R * N));
    std::vector<uint16_t> xsb16(R);
    std::vector<float> xsb(R), wsf(N);
    for (int64_t r = 0; r < R; ++r) {
        for (int64_t n = 0; n < N; ++n) accb[r * N + n] = acc[(n + 97 * r) % N];
        xsb[r] = t::h2f(xs16[0]) * row_mul[r];              // powers of two: exact in fp16
        xsb16[r] = t::f2h_rne(xsb[r]);
    }
    for (int64_t n = 0; n < N; ++n) wsf[n] = t::h2f(ws16[n]);
    std::vector<uint16_t> ref(static_cast<size_t>(R * N));
    or_w8a8_dequant(accb.data(), xsb.data(), wsf.data(), R, N, ref.data());
    const int oracle_row0 = count_diff(std::vector<uint16_t>(ref.begin(), ref.begin() + N), want);
    std::printf("oracle epilogue on row 0: %d outputs differ from the fixture\n", oracle_row0);
    if (oracle_row0 != 0) rc = 1;

    Tensor xs16b({R}, DType::Float16);
    xs16b.copy_from_host(xsb16.data(), R * 2);
    const int bad2 = count_diff(dequant(accb, R, N, xs16b, ws, ctx.stream()), ref);
    Tensor xs32({R}, DType::Float32);
    xs32.copy_from_host(xsb.data(), R * 4);
    Tensor ws32({N}, DType::Float32);
    ws32.copy_from_host(wsf.data(), wsf.size() * 4);
    const int bad3 = count_diff(dequant(accb, R, N, xs32, ws32, ctx.stream()), ref);
    std::printf("4-row batch: %d (fp16 scales) and %d (fp32 scales) of %lld outputs differ from the oracle\n", bad2,
                bad3, (long long)(R * N));
    if (bad2 != 0 || bad3 != 0) rc = 1;

    std::printf("%s\n", rc ? "FAILED" : "ok");
    return rc;
}
