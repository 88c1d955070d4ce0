// host_pack.cpp -- host half of the C-ABI: error state, packed sizes, the
// AWQ/GPTQ -> slab-64 packers, the inverse unpacker and the host W8A8 weight
// quantiser.  No device calls in this file.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <mutex>
#include <thread>
#include <unordered_map>
#include <vector>

#include "common.h"

namespace mcv {

std::string& last_error() {
    static thread_local std::string msg;
    return msg;
}

int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    last_error() = buf;
    return code;
}

int check_launch(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(MCV_ERR_HIP, "%s: kernel launch failed: %s", what, hipGetErrorString(e));
    return MCV_OK;
}

int require_device() {
    static std::mutex mu;
    static std::unordered_map<int, int> verdict;
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return fail(MCV_ERR_NO_DEVICE, "no HIP device: %s", hipGetErrorString(e));
    std::lock_guard<std::mutex> lock(mu);
    auto it = verdict.find(dev);
    if (it == verdict.end()) {
        hipDeviceProp_t prop;
        e = hipGetDeviceProperties(&prop, dev);
        if (e != hipSuccess) return fail(MCV_ERR_NO_DEVICE, "hipGetDeviceProperties(%d): %s", dev, hipGetErrorString(e));
        int v = std::strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? MCV_OK : MCV_ERR_NO_DEVICE;
        it = verdict.emplace(dev, v).first;
        if (v != MCV_OK) return fail(v, "device %d is %s; this library is built for gfx950 only", dev, prop.gcnArchName);
    }
    if (it->second != MCV_OK) return fail(it->second, "device %d is not gfx950", dev);
    return MCV_OK;
}

namespace {

// Position of k-offset j (0..7) inside a packed word: nibble slot inv[j], so
// that slot s holds k-offset order[s] = {0,2,4,6,1,3,5,7}[s].  With this order
// one AND-OR of the word with 0x000F000F / 0x00F000F0 (and of the word shifted
// right by 8) yields half2 pairs of consecutive k.
constexpr int kSlotOfK[8] = {0, 4, 1, 5, 2, 6, 3, 7};
// AutoAWQ's column order inside a word (quantized_weight.cpp:17).
constexpr int kAwqOrder[8] = {0, 2, 4, 6, 1, 3, 5, 7};

bool shape_ok(int64_t K, int64_t N) {
    return K > 0 && N > 0 && K % kGroup == 0 && K <= (int64_t(1) << 24) && N <= (int64_t(1) << 30);
}

struct Slab64Writer {
    int64_t K, N, Npad, C, G;
    uint32_t* qw;
    uint16_t* sc;
    uint32_t* zr;
    Slab64Writer(int64_t K_, int64_t N_, void* qw_, uint16_t* sc_, uint32_t* zr_)
        : K(K_), N(N_), Npad(ceil_div(N_, kSlab) * kSlab), C(K_ / kChunkK), G(K_ / kGroup),
          qw(static_cast<uint32_t*>(qw_)), sc(sc_), zr(zr_) {
        std::memset(qw, 0, static_cast<size_t>(Npad) * static_cast<size_t>(K) / 2);
        std::memset(sc, 0, static_cast<size_t>(G) * static_cast<size_t>(Npad) * 2);
        std::memset(zr, 0, static_cast<size_t>(G) * static_cast<size_t>(Npad) / 2);
    }
    void put_q(int64_t k, int64_t n, uint32_t q) {
        const int64_t slab = n / kSlab, lane = n % kSlab, c = k / kChunkK, w = (k % kChunkK) / 8;
        const size_t idx = static_cast<size_t>(((slab * C + c) * kSlab + lane) * 4 + w);
        qw[idx] |= (q & 15u) << (4 * kSlotOfK[k % 8]);
    }
    void put_z(int64_t g, int64_t n, uint32_t z) {
        zr[static_cast<size_t>(g * (Npad / 8) + n / 8)] |= (z & 15u) << (4 * (n % 8));
    }
    void put_s(int64_t g, int64_t n, uint16_t s) { sc[static_cast<size_t>(g * Npad + n)] = s; }
};

}  // namespace
}  // namespace mcv

using namespace mcv;

extern "C" {

const char* mcv_last_error(void) { return last_error().c_str(); }

const char* mcv_version(void) { return "mcv-quant 0.1 (gfx950)"; }

int64_t mcv_w4a16_packed_weight_bytes(int64_t K, int64_t N) {
    if (!shape_ok(K, N)) return 0;
    return ceil_div(N, kSlab) * kSlab * K / 2;
}
int64_t mcv_w4a16_packed_scale_bytes(int64_t K, int64_t N) {
    if (!shape_ok(K, N)) return 0;
    return (K / kGroup) * ceil_div(N, kSlab) * kSlab * 2;
}
int64_t mcv_w4a16_packed_zero_bytes(int64_t K, int64_t N) {
    if (!shape_ok(K, N)) return 0;
    return (K / kGroup) * ceil_div(N, kSlab) * kSlab / 2;
}

int mcv_w4a16_pack_awq(const int32_t* qweight, const int32_t* qzeros, const uint16_t* scales,
                       int64_t K, int64_t N, void* qw_out, uint16_t* scales_out, uint32_t* zeros_out) {
    if (!qweight || !qzeros || !scales || !qw_out || !scales_out || !zeros_out)
        return fail(MCV_ERR_INVALID_ARG, "mcv_w4a16_pack_awq: null pointer");
    if (!shape_ok(K, N) || N % 8 != 0)
        return fail(MCV_ERR_SHAPE, "mcv_w4a16_pack_awq: need K %% 128 == 0 and N %% 8 == 0 (K=%lld N=%lld)",
                    (long long)K, (long long)N);
    Slab64Writer wr(K, N, qw_out, scales_out, zeros_out);
    const int64_t np = N / 8, G = K / kGroup;
    for (int64_t k = 0; k < K; ++k)
        for (int64_t j = 0; j < np; ++j) {
            const uint32_t word = static_cast<uint32_t>(qweight[k * np + j]);
            for (int s = 0; s < 8; ++s) wr.put_q(k, j * 8 + kAwqOrder[s], word >> (4 * s));
        }
    for (int64_t g = 0; g < G; ++g)
        for (int64_t j = 0; j < np; ++j) {
            const uint32_t word = static_cast<uint32_t>(qzeros[g * np + j]);
            for (int s = 0; s < 8; ++s) wr.put_z(g, j * 8 + kAwqOrder[s], word >> (4 * s));
        }
    for (int64_t g = 0; g < G; ++g)
        for (int64_t n = 0; n < N; ++n) wr.put_s(g, n, scales[g * N + n]);
    return MCV_OK;
}

int mcv_w4a16_pack_gptq(const int32_t* qweight, const int32_t* qzeros, const int32_t* g_idx,
                        const uint16_t* scales, int64_t K, int64_t N, int64_t groups,
                        void* qw_out, uint16_t* scales_out, uint32_t* zeros_out) {
    if (!qweight || !qzeros || !scales || !qw_out || !scales_out || !zeros_out)
        return fail(MCV_ERR_INVALID_ARG, "mcv_w4a16_pack_gptq: null pointer");
    if (!shape_ok(K, N) || N % 8 != 0 || groups * kGroup != K)
        return fail(MCV_ERR_SHAPE, "mcv_w4a16_pack_gptq: need K %% 128 == 0, N %% 8 == 0, groups*128 == K "
                    "(K=%lld N=%lld groups=%lld)", (long long)K, (long long)N, (long long)groups);
    bool act_order = false;
    if (g_idx) {
        for (int64_t k = 0; k < K; ++k) {
            if (g_idx[k] < 0 || g_idx[k] >= groups)
                return fail(MCV_ERR_SHAPE, "mcv_w4a16_pack_gptq: g_idx out of range (g_idx[%lld]=%d, groups=%lld)",
                            (long long)k, g_idx[k], (long long)groups);
            act_order |= g_idx[k] != k / kGroup;
        }
    }
    Slab64Writer wr(K, N, qw_out, scales_out, zeros_out);
    auto nib_q = [&](int64_t k, int64_t n) {
        return static_cast<int>((static_cast<uint32_t>(qweight[(k / 8) * N + n]) >> (4 * (k % 8))) & 15u);
    };
    // zero of row k (stored zero - 1, :112); its group is g_idx[k] (:107)
    auto zero_of = [&](int64_t gz, int64_t n) {
        return static_cast<int>((static_cast<uint32_t>(qzeros[gz * (N / 8) + n / 8]) >> (4 * (n % 8))) & 15u) + 1;
    };
    if (!act_order) {
        for (int64_t k0 = 0; k0 < K / 8; ++k0)
            for (int64_t n = 0; n < N; ++n) {
                const uint32_t word = static_cast<uint32_t>(qweight[k0 * N + n]);
                for (int i = 0; i < 8; ++i) wr.put_q(k0 * 8 + i, n, word >> (4 * i));
            }
        for (int64_t g = 0; g < groups; ++g)
            for (int64_t n = 0; n < N; ++n) {
                const uint32_t word = static_cast<uint32_t>(qzeros[g * (N / 8) + n / 8]);
                wr.put_z(g, n, word >> (4 * (n % 8)));
                wr.put_s(g, n, scales[g * N + n]);
            }
        return MCV_OK;
    }
    // Act-order: the reference takes row k's zero from group g_idx[k] but
    // keeps the scales by position, group k / 128 (:101-117 build
    // w8 = q - zero[g_idx[k]]; pack_w4a16_weight and the kernel scale the
    // 128-row group k / 128).  The slab layout has one zero per (k / 128,
    // column); every w8 value is kept exact by storing, per (group, column),
    // the common zero c and nibbles q - zero[g_idx[k]] + c:
    //   - the rows' zeros agree (every sym=True checkpoint): c = that zero,
    //     the nibbles unchanged;
    //   - otherwise c = max(1, -min w8), which needs max w8 + c <= 15 (16
    //     levels); a (group, column) whose w8 span more is refused.
    for (int64_t g = 0; g < groups; ++g)
        for (int64_t n = 0; n < N; ++n) {
            const int z0 = zero_of(g_idx[g * kGroup], n);
            bool same = true;
            int lo = 99, hi = -99;
            for (int64_t k = g * kGroup; k < (g + 1) * kGroup; ++k) {
                const int z = zero_of(g_idx[k], n);
                same &= z == z0;
                const int w8 = nib_q(k, n) - z;
                lo = w8 < lo ? w8 : lo;
                hi = w8 > hi ? w8 : hi;
            }
            const int c = same ? z0 : (-lo > 1 ? -lo : 1);
            if (c + hi > 15 || c + lo < 0 || c > 16)
                return fail(MCV_ERR_UNSUPPORTED,
                            "mcv_w4a16_pack_gptq: act-order zero points of group %lld, column %lld put its int4 "
                            "values on %d levels (w8 in [%d, %d]); at most 16 fit one zero per group",
                            (long long)g, (long long)n, hi - lo + 1, lo, hi);
            for (int64_t k = g * kGroup; k < (g + 1) * kGroup; ++k)
                wr.put_q(k, n, static_cast<uint32_t>(nib_q(k, n) - zero_of(g_idx[k], n) + c));
            wr.put_z(g, n, static_cast<uint32_t>(c - 1));
            wr.put_s(g, n, scales[g * N + n]);
        }
    return MCV_OK;
}

int mcv_w4a16_unpack_host(const void* qw, const uint16_t* scales, const uint32_t* zeros, int zero_bias,
                          int64_t K, int64_t N, uint8_t* q_kn, uint8_t* zeff_gn, uint16_t* scales_gn) {
    if (!qw || !scales || !zeros) return fail(MCV_ERR_INVALID_ARG, "mcv_w4a16_unpack_host: null pointer");
    if (!shape_ok(K, N)) return fail(MCV_ERR_SHAPE, "mcv_w4a16_unpack_host: bad shape");
    if (zero_bias != 0 && zero_bias != 1) return fail(MCV_ERR_INVALID_ARG, "zero_bias must be 0 or 1");
    const int64_t Npad = ceil_div(N, kSlab) * kSlab, C = K / kChunkK, G = K / kGroup;
    const uint32_t* w = static_cast<const uint32_t*>(qw);
    if (q_kn) {
        for (int64_t k = 0; k < K; ++k)
            for (int64_t n = 0; n < N; ++n) {
                const int64_t slab = n / kSlab, lane = n % kSlab, c = k / kChunkK, wi = (k % kChunkK) / 8;
                const uint32_t word = w[((slab * C + c) * kSlab + lane) * 4 + wi];
                q_kn[k * N + n] = static_cast<uint8_t>((word >> (4 * kSlotOfK[k % 8])) & 15u);
            }
    }
    for (int64_t g = 0; g < G; ++g)
        for (int64_t n = 0; n < N; ++n) {
            if (zeff_gn)
                zeff_gn[g * N + n] = static_cast<uint8_t>(((zeros[g * (Npad / 8) + n / 8] >> (4 * (n % 8))) & 15u) + zero_bias);
            if (scales_gn) scales_gn[g * N + n] = scales[g * Npad + n];
        }
    return MCV_OK;
}

}  // extern "C"

// ------------------------------------------------------ host W8A8 quantiser --
namespace {

float h2f_host(uint16_t h) {
    const uint32_t sign = (static_cast<uint32_t>(h) & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    uint32_t bits;
    if (e == 0) {
        if (m == 0) { bits = sign; }
        else {
            const float v = static_cast<float>(m) * 5.9604644775390625e-08f;  // m * 2^-24, exact
            return sign ? -v : v;
        }
    } else if (e == 31) {
        bits = sign | 0x7f800000u | (m << 13);
    } else {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

// IEEE round-to-nearest-even fp32 -> fp16 with subnormals.
uint16_t f2h_rne_host(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u, ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return static_cast<uint16_t>(sign | (ax > 0x7f800000u ? 0x7e00u : 0x7c00u));
    const int32_t e = static_cast<int32_t>(ax >> 23) - 127;
    if (e > 15) return static_cast<uint16_t>(sign | 0x7c00u);
    if (e >= -14) {
        const uint32_t frac = ax & 0x7fffffu, q = frac >> 13, rem = frac & 0x1fffu;
        uint32_t r = (static_cast<uint32_t>(e + 15) << 10) + q;
        if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) ++r;   // a carry into the exponent is correct
        return static_cast<uint16_t>(sign | r);
    }
    if (ax == 0) return static_cast<uint16_t>(sign);
    const int32_t shift = -e - 1;                // value / 2^-24 = significand >> shift
    if (shift > 25) return static_cast<uint16_t>(sign);
    const uint32_t mant = (ax & 0x7fffffu) | 0x800000u;
    uint32_t q = mant >> shift;
    const uint32_t rem = mant & ((1u << shift) - 1), half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1u))) ++q;
    return static_cast<uint16_t>(sign | q);
}

// Truncating encode with underflow to signed zero, as the reference stores the
// W8A8 weight scale (quantized_weight.cpp:186-195, :253).
uint16_t f2h_trunc_host(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const int32_t e = static_cast<int32_t>((x >> 23) & 0xffu) - 112;
    if (e <= 0) return static_cast<uint16_t>(sign);
    if (e >= 31) return static_cast<uint16_t>(sign | 0x7c00u);
    return static_cast<uint16_t>(sign | (static_cast<uint32_t>(e) << 10) | ((x & 0x7fffffu) >> 13));
}

// Clamp, then round half away from zero (quantized_weight.cpp:197-202).  The
// volatile stores keep each fp32 operation separately rounded.  A NaN product
// (an inf weight times the zero inverse of an inf scale) passes both clamps
// and becomes 0: the value the reference's float-to-int conversion gives it
// on aarch64 and x86-64 alike (there the cast itself is undefined).
int8_t quantize_i8_host(float v, float inv) {
    volatile float q = v * inv;
    float t = q;
    if (t != t) return 0;
    if (t > 127.0f) t = 127.0f;
    if (t < -128.0f) t = -128.0f;
    volatile float r = t >= 0.0f ? t + 0.5f : t - 0.5f;
    return static_cast<int8_t>(static_cast<float>(r));
}

}  // namespace

namespace {
// Byte offset of w[k][n] in MCV_W8_TILED for a weight with Kp / 32 k-blocks
// per 64-column slab (include/mcv_quant.h).
inline int64_t tiled_offset(int64_t k, int64_t n, int64_t kblocks) {
    const int64_t l = (n % 32) + 32 * ((k % 32) / 16);
    return ((((n / 64) * kblocks + k / 32) * 2 + (n % 64) / 32) * 64 + l) * 16 + (k % 16);
}
}  // namespace

extern "C" int64_t mcv_w8a8_tiled_bytes(int64_t K, int64_t N) {
    if (K <= 0 || N <= 0 || K > (int64_t(1) << 30) || N > (int64_t(1) << 30)) return 0;
    return ceil_div(N, kSlab) * kSlab * ceil_div(K, 128) * 128;
}

extern "C" int mcv_w8a8_pack_tiled_host(const int8_t* q_kn, int64_t K, int64_t N, int8_t* tiled) {
    if (!q_kn || !tiled) return fail(MCV_ERR_INVALID_ARG, "mcv_w8a8_pack_tiled_host: null pointer");
    const int64_t bytes = mcv_w8a8_tiled_bytes(K, N);
    if (bytes == 0) return fail(MCV_ERR_SHAPE, "mcv_w8a8_pack_tiled_host: bad shape K=%lld N=%lld", (long long)K, (long long)N);
    std::memset(tiled, 0, static_cast<size_t>(bytes));
    const int64_t kblocks = ceil_div(K, 128) * 4;
    for (int64_t k = 0; k < K; ++k)
        for (int64_t n = 0; n < N; ++n) tiled[tiled_offset(k, n, kblocks)] = q_kn[k * N + n];
    return MCV_OK;
}

extern "C" int mcv_w8a8_quantize_weight_host(const uint16_t* w_kn, int64_t K, int64_t N, int8_t* q,
                                             int out_layout, float* scale_f32, uint16_t* scale_f16) {
    if (!w_kn || !q || !scale_f32) return fail(MCV_ERR_INVALID_ARG, "mcv_w8a8_quantize_weight_host: null pointer");
    if (K <= 0 || N <= 0) return fail(MCV_ERR_SHAPE, "mcv_w8a8_quantize_weight_host: K and N must be positive");
    if (out_layout != MCV_W8_KN && out_layout != MCV_W8_NK && out_layout != MCV_W8_TILED)
        return fail(MCV_ERR_INVALID_ARG, "mcv_w8a8_quantize_weight_host: bad layout %d", out_layout);
    if (out_layout == MCV_W8_TILED && mcv_w8a8_tiled_bytes(K, N) == 0)
        return fail(MCV_ERR_SHAPE, "mcv_w8a8_quantize_weight_host: K=%lld N=%lld too large for MCV_W8_TILED",
                    (long long)K, (long long)N);
    const int64_t kblocks = ceil_div(K, 128) * 4;
    if (out_layout == MCV_W8_TILED) std::memset(q, 0, static_cast<size_t>(mcv_w8a8_tiled_bytes(K, N)));
    for (int64_t n = 0; n < N; ++n) {
        float max_abs = 0.0f;
        for (int64_t k = 0; k < K; ++k) max_abs = std::max(max_abs, std::fabs(h2f_host(w_kn[k * N + n])));
        float scale = max_abs / 127.0f;
        if (scale < 0.00000001f) scale = 0.00000001f;
        const float inv = 1.0f / scale;
        scale_f32[n] = scale;
        if (scale_f16) scale_f16[n] = f2h_trunc_host(scale);
        for (int64_t k = 0; k < K; ++k) {
            const int8_t v = quantize_i8_host(h2f_host(w_kn[k * N + n]), inv);
            if (out_layout == MCV_W8_KN) q[k * N + n] = v;
            else if (out_layout == MCV_W8_NK) q[n * K + k] = v;
            else q[tiled_offset(k, n, kblocks)] = v;
        }
    }
    return MCV_OK;
}

namespace {

// bf16 -> fp16 exactly as the reference loads bf16 checkpoint tensors
// (src/csrc/lib/weights.cpp:25-33): exponent rebias, top mantissa bits kept,
// below the fp16 normal range -> signed zero, above it (NaN too) -> signed inf.
uint16_t bf16_to_f16_trunc_host(uint16_t bf) {
    const uint32_t x = static_cast<uint32_t>(bf) << 16;
    const uint32_t sign = (x >> 16) & 0x8000u;
    const int32_t e = static_cast<int32_t>((x >> 23) & 0xffu) - 112;
    if (e <= 0) return static_cast<uint16_t>(sign);
    if (e >= 31) return static_cast<uint16_t>(sign | 0x7c00u);
    return static_cast<uint16_t>(sign | (static_cast<uint32_t>(e) << 10) | ((x & 0x7fffffu) >> 13));
}

// Runs fn(n0, n1) over [0, N) split into contiguous ranges on up to 16 threads.
template <typename Fn>
void parallel_columns(int64_t N, int64_t work_per_column, Fn fn) {
    int nt = static_cast<int>(std::thread::hardware_concurrency());
    if (nt < 1) nt = 1;
    if (nt > 16) nt = 16;
    if (N * work_per_column < (int64_t(1) << 18)) nt = 1;            // small: not worth the threads
    if (nt == 1) {
        fn(int64_t(0), N);
        return;
    }
    std::vector<std::thread> th;
    for (int t = 0; t < nt; ++t) {
        const int64_t n0 = N * t / nt, n1 = N * (t + 1) / nt;
        if (n1 > n0) th.emplace_back(fn, n0, n1);
    }
    for (auto& x : th) x.join();
}

}  // namespace

extern "C" int mcv_w8a8_pack_tiled_nk_host(const int8_t* q_nk, int64_t K, int64_t N, int8_t* tiled) {
    if (!q_nk || !tiled) return fail(MCV_ERR_INVALID_ARG, "mcv_w8a8_pack_tiled_nk_host: null pointer");
    const int64_t bytes = mcv_w8a8_tiled_bytes(K, N);
    if (bytes == 0) return fail(MCV_ERR_SHAPE, "mcv_w8a8_pack_tiled_nk_host: bad shape K=%lld N=%lld", (long long)K, (long long)N);
    std::memset(tiled, 0, static_cast<size_t>(bytes));
    const int64_t kblocks = ceil_div(K, 128) * 4;
    parallel_columns(N, K, [&](int64_t n0, int64_t n1) {
        for (int64_t n = n0; n < n1; ++n)
            for (int64_t k = 0; k < K; ++k) tiled[tiled_offset(k, n, kblocks)] = q_nk[n * K + k];
    });
    return MCV_OK;
}

extern "C" int mcv_w8a8_quantize_weight_nk_pad_host(const uint16_t* w_nk, int src_dtype, int64_t K, int64_t N_src,
                                                    int64_t N, int8_t* q, int out_layout, float* scale_f32,
                                                    uint16_t* scale_f16) {
    const char* who = "mcv_w8a8_quantize_weight_nk_pad_host";
    if (!w_nk || !q || !scale_f32) return fail(MCV_ERR_INVALID_ARG, "%s: null pointer", who);
    if (K <= 0 || N <= 0 || N_src <= 0 || N_src > N)
        return fail(MCV_ERR_SHAPE, "%s: need K > 0 and 0 < N_src <= N (K=%lld N_src=%lld N=%lld)", who, (long long)K,
                    (long long)N_src, (long long)N);
    if (src_dtype != MCV_SRC_F16 && src_dtype != MCV_SRC_BF16)
        return fail(MCV_ERR_INVALID_ARG, "%s: bad source dtype %d", who, src_dtype);
    if (out_layout != MCV_W8_KN && out_layout != MCV_W8_NK && out_layout != MCV_W8_TILED)
        return fail(MCV_ERR_INVALID_ARG, "%s: bad layout %d", who, out_layout);
    if (out_layout == MCV_W8_TILED && mcv_w8a8_tiled_bytes(K, N) == 0)
        return fail(MCV_ERR_SHAPE, "%s: K=%lld N=%lld too large for MCV_W8_TILED", who, (long long)K, (long long)N);
    const int64_t kblocks = ceil_div(K, 128) * 4;
    if (out_layout == MCV_W8_TILED) std::memset(q, 0, static_cast<size_t>(mcv_w8a8_tiled_bytes(K, N)));
    const bool bf = src_dtype == MCV_SRC_BF16;
    // Output channel n is row n of the checkpoint's [N][K]: the same values,
    // the same per-channel formula as the [K][N] quantiser above.  Channels
    // from N_src on are zero columns (scale floored at 1e-8, every q zero),
    // what the quantiser makes of the zero padding the reference appends.
    parallel_columns(N, K, [&](int64_t n0, int64_t n1) {
        std::vector<float> row(static_cast<size_t>(K));
        for (int64_t n = n0; n < n1; ++n) {
            const uint16_t* src = w_nk + n * K;
            float max_abs = 0.0f;
            for (int64_t k = 0; k < K; ++k) {
                row[k] = n < N_src ? h2f_host(bf ? bf16_to_f16_trunc_host(src[k]) : src[k]) : 0.0f;
                max_abs = std::max(max_abs, std::fabs(row[k]));
            }
            float scale = max_abs / 127.0f;
            if (scale < 0.00000001f) scale = 0.00000001f;
            const float inv = 1.0f / scale;
            scale_f32[n] = scale;
            if (scale_f16) scale_f16[n] = f2h_trunc_host(scale);
            for (int64_t k = 0; k < K; ++k) {
                const int8_t v = quantize_i8_host(row[k], inv);
                if (out_layout == MCV_W8_KN) q[k * N + n] = v;
                else if (out_layout == MCV_W8_NK) q[n * K + k] = v;
                else q[tiled_offset(k, n, kblocks)] = v;
            }
        }
    });
    return MCV_OK;
}

extern "C" int mcv_w8a8_quantize_weight_nk_host(const uint16_t* w_nk, int src_dtype, int64_t K, int64_t N, int8_t* q,
                                                int out_layout, float* scale_f32, uint16_t* scale_f16) {
    return mcv_w8a8_quantize_weight_nk_pad_host(w_nk, src_dtype, K, N, N, q, out_layout, scale_f32, scale_f16);
}

namespace {

// The build's synthetic int4 quantiser for one (group, column): the 128
// values v[0..127] -> scale bits, zero, and the 128 nibbles q[].
void quantize_group_int4(const float* v, uint16_t* s16_out, uint32_t* z_out, uint8_t* q) {
    float lo = INFINITY, hi = -INFINITY;
    for (int kk = 0; kk < kGroup; ++kk) {
        lo = v[kk] < lo ? v[kk] : lo;
        hi = v[kk] > hi ? v[kk] : hi;
    }
    float range = hi - lo;
    if (range < 1e-5f) range = 1e-5f;
    const uint16_t s16 = f2h_rne_host(range / 15.0f);
    const float sc = h2f_host(s16);
    // clamp(x, 0, 15) with NaN -> 0 (a group holding an inf, e.g. a bf16
    // value beyond the fp16 range, divides inf by inf)
    float zf = std::nearbyint(-lo / sc);
    zf = zf > 0.0f ? (zf > 15.0f ? 15.0f : zf) : 0.0f;
    for (int kk = 0; kk < kGroup; ++kk) {
        float qf = std::nearbyint(v[kk] / sc) + zf;
        qf = qf > 0.0f ? (qf > 15.0f ? 15.0f : qf) : 0.0f;
        q[kk] = static_cast<uint8_t>(qf);
    }
    *s16_out = s16;
    *z_out = static_cast<uint32_t>(zf);
}

}  // namespace

extern "C" int mcv_w4a16_quantize_nk_host(const uint16_t* w_nk, int src_dtype, int64_t K, int64_t N_src, int64_t N,
                                          int32_t* qweight, int32_t* qzeros, uint16_t* scales, int nthreads) {
    const char* who = "mcv_w4a16_quantize_nk_host";
    if (!w_nk || !qweight || !qzeros || !scales) return fail(MCV_ERR_INVALID_ARG, "%s: null pointer", who);
    if (K <= 0 || K % kGroup != 0 || N <= 0 || N % 8 != 0 || N_src <= 0 || N_src > N)
        return fail(MCV_ERR_SHAPE, "%s: need K %% 128 == 0, N %% 8 == 0 and 0 < N_src <= N (K=%lld N_src=%lld N=%lld)",
                    who, (long long)K, (long long)N_src, (long long)N);
    if (src_dtype != MCV_SRC_F16 && src_dtype != MCV_SRC_BF16)
        return fail(MCV_ERR_INVALID_ARG, "%s: bad source dtype %d", who, src_dtype);
    const bool bf = src_dtype == MCV_SRC_BF16;
    const int64_t np = N / 8, G = K / kGroup;
    constexpr int order[8] = {0, 2, 4, 6, 1, 3, 5, 7};
    int nt = nthreads > 0 ? nthreads : static_cast<int>(std::thread::hardware_concurrency());
    if (nt < 1) nt = 1;
    if (nt > 64) nt = 64;
    // Each worker owns a contiguous range of 8-column words: disjoint outputs.
    // Column n is row n of the [N_src][K] source (zero from N_src on).
    auto work = [&](int64_t j0, int64_t j1) {
        std::vector<float> col(static_cast<size_t>(K));
        uint8_t q[8][kGroup];
        uint32_t z[8];
        for (int64_t j = j0; j < j1; ++j) {
            for (int64_t g = 0; g < G; ++g) {
                uint32_t zword = 0;
                for (int sl = 0; sl < 8; ++sl) {
                    const int64_t n = j * 8 + order[sl];
                    const uint16_t* src = w_nk + n * K + g * kGroup;
                    for (int kk = 0; kk < kGroup; ++kk)
                        col[kk] = n < N_src ? h2f_host(bf ? bf16_to_f16_trunc_host(src[kk]) : src[kk]) : 0.0f;
                    quantize_group_int4(col.data(), &scales[g * N + n], &z[sl], q[sl]);
                    zword |= z[sl] << (4 * sl);
                }
                qzeros[g * np + j] = static_cast<int32_t>(zword);
                for (int kk = 0; kk < kGroup; ++kk) {
                    uint32_t word = 0;
                    for (int sl = 0; sl < 8; ++sl) word |= static_cast<uint32_t>(q[sl][kk]) << (4 * sl);
                    qweight[(g * kGroup + kk) * np + j] = static_cast<int32_t>(word);
                }
            }
        }
    };
    if (nt == 1 || np < 64) {
        work(0, np);
    } else {
        std::vector<std::thread> th;
        const int64_t per = ceil_div(np, nt);
        for (int t = 0; t < nt; ++t) {
            const int64_t j0 = t * per, j1 = std::min<int64_t>(np, j0 + per);
            if (j0 < j1) th.emplace_back(work, j0, j1);
        }
        for (auto& t : th) t.join();
    }
    return MCV_OK;
}

extern "C" int mcv_w4a16_quantize_host(const uint16_t* w_kn, int64_t K, int64_t N, int32_t* qweight, int32_t* qzeros,
                                       uint16_t* scales, int nthreads) {
    if (!w_kn || !qweight || !qzeros || !scales) return fail(MCV_ERR_INVALID_ARG, "mcv_w4a16_quantize_host: null pointer");
    if (K <= 0 || N <= 0 || K % kGroup != 0 || N % 8 != 0)
        return fail(MCV_ERR_SHAPE, "mcv_w4a16_quantize_host: need K %% 128 == 0 and N %% 8 == 0 (K=%lld N=%lld)",
                    (long long)K, (long long)N);
    const int64_t np = N / 8, G = K / kGroup;
    constexpr int order[8] = {0, 2, 4, 6, 1, 3, 5, 7};
    int nt = nthreads > 0 ? nthreads : static_cast<int>(std::thread::hardware_concurrency());
    if (nt < 1) nt = 1;
    if (nt > 64) nt = 64;
    // Each worker owns a contiguous range of 8-column words: disjoint outputs.
    auto work = [&](int64_t j0, int64_t j1) {
        float col[kGroup];
        uint8_t q[8][kGroup];
        for (int64_t g = 0; g < G; ++g)
            for (int64_t j = j0; j < j1; ++j) {
                uint32_t zword = 0;
                for (int s = 0; s < 8; ++s) {
                    const int64_t n = j * 8 + order[s];
                    for (int kk = 0; kk < kGroup; ++kk) col[kk] = h2f_host(w_kn[(g * kGroup + kk) * N + n]);
                    uint32_t z = 0;
                    quantize_group_int4(col, &scales[g * N + n], &z, q[s]);
                    zword |= z << (4 * s);
                }
                qzeros[g * np + j] = static_cast<int32_t>(zword);
                for (int kk = 0; kk < kGroup; ++kk) {
                    uint32_t word = 0;
                    for (int s = 0; s < 8; ++s) word |= static_cast<uint32_t>(q[s][kk]) << (4 * s);
                    qweight[(g * kGroup + kk) * np + j] = static_cast<int32_t>(word);
                }
            }
    };
    if (nt == 1 || np < 64) {
        work(0, np);
    } else {
        std::vector<std::thread> th;
        const int64_t per = ceil_div(np, nt);
        for (int t = 0; t < nt; ++t) {
            const int64_t j0 = t * per, j1 = std::min<int64_t>(np, j0 + per);
            if (j0 < j1) th.emplace_back(work, j0, j1);
        }
        for (auto& t : th) t.join();
    }
    return MCV_OK;
}

// GPTQ act-order weights whose 128-row blocks a single 4-bit zero cannot
// hold: the dense fp16 weight, each element the reference's int8 value
// q - zero[g_idx[k]] (quantized_weight.cpp:98-117) times the scale of group
// k / 128, rounded once to fp16 (the value the slab path widens to).  The
// product of an integer in [-16, 15] and an fp16 scale is exact in fp32, so
// the one rounding is f2h_rne_host's.
extern "C" int mcv_w4a16_dequant_gptq_host(const int32_t* qweight, const int32_t* qzeros, const int32_t* g_idx,
                                           const uint16_t* scales, int64_t K, int64_t N, int64_t groups,
                                           uint16_t* w_kn) {
    if (!qweight || !qzeros || !scales || !w_kn) return fail(MCV_ERR_INVALID_ARG, "mcv_w4a16_dequant_gptq_host: null pointer");
    if (K <= 0 || N <= 0 || K % kGroup != 0 || N % 8 != 0 || groups * kGroup != K || K > (int64_t(1) << 24) ||
        N > (int64_t(1) << 24))
        return fail(MCV_ERR_SHAPE, "mcv_w4a16_dequant_gptq_host: need K %% 128 == 0, N %% 8 == 0, groups*128 == K "
                    "(K=%lld N=%lld groups=%lld)", (long long)K, (long long)N, (long long)groups);
    if (g_idx)
        for (int64_t k = 0; k < K; ++k)
            if (g_idx[k] < 0 || g_idx[k] >= groups)
                return fail(MCV_ERR_SHAPE, "mcv_w4a16_dequant_gptq_host: g_idx out of range (g_idx[%lld]=%d)",
                            (long long)k, g_idx[k]);
    for (int64_t k = 0; k < K; ++k) {
        const int64_t gz = g_idx ? g_idx[k] : k / kGroup, gs = k / kGroup;
        for (int64_t n = 0; n < N; ++n) {
            const int q = static_cast<int>((static_cast<uint32_t>(qweight[(k / 8) * N + n]) >> (4 * (k % 8))) & 15u);
            const int z = static_cast<int>((static_cast<uint32_t>(qzeros[gz * (N / 8) + n / 8]) >> (4 * (n % 8))) & 15u) + 1;
            w_kn[k * N + n] = f2h_rne_host(static_cast<float>(q - z) * h2f_host(scales[gs * N + n]));
        }
    }
    return MCV_OK;
}
