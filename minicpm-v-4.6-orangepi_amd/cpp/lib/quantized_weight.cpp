// quantized_weight.cpp -- W4A16 / W8A8 weight objects over the C-ABI packers.
#include "minicpmv/quantized_weight.h"

#include "mcv_quant.h"
#include "minicpmv/hip_context.h"

#include <cstring>
#include <stdexcept>
#include <vector>

namespace minicpmv {
namespace {

W4A16QuantizedWeight upload_packed(const std::vector<uint8_t>& qw, const std::vector<uint16_t>& sc,
                                   const std::vector<uint32_t>& zr, int64_t K, int64_t N, int zero_bias) {
    const int64_t npad = (N + 63) / 64 * 64;
    W4A16QuantizedWeight out;
    out.K = K;
    out.N = N;
    out.group_size = MCV_W4_GROUP;
    out.zero_bias = zero_bias;
    out.w_int8 = Tensor({static_cast<int64_t>(qw.size())}, DType::UInt8);
    out.w_int8.copy_from_host(qw.data(), qw.size());
    out.scales = Tensor({K / MCV_W4_GROUP, npad}, DType::Float16);
    out.scales.copy_from_host(sc.data(), sc.size() * 2);
    out.zeros = Tensor({K / MCV_W4_GROUP, npad / 8}, DType::Int32);
    out.zeros.copy_from_host(zr.data(), zr.size() * 4);
    return out;
}

struct PackedHost {
    std::vector<uint8_t> qw;
    std::vector<uint16_t> sc;
    std::vector<uint32_t> zr;
};

PackedHost alloc_packed(int64_t K, int64_t N) {
    const int64_t wb = mcv_w4a16_packed_weight_bytes(K, N);
    if (wb == 0) throw std::runtime_error("W4A16 weight shape must have K a positive multiple of 128");
    PackedHost p;
    p.qw.resize(static_cast<size_t>(wb));
    p.sc.resize(static_cast<size_t>(mcv_w4a16_packed_scale_bytes(K, N) / 2));
    p.zr.resize(static_cast<size_t>(mcv_w4a16_packed_zero_bytes(K, N) / 4));
    return p;
}

template <typename T>
const T* typed(const WeightsIndex& index, const std::string& name, DType want, const char* what) {
    const TensorInfo& info = index.at(name);
    if (info.dtype != want) throw std::runtime_error(std::string("unexpected ") + what + " tensor dtype for " + name);
    return reinterpret_cast<const T*>(index.host_data(name));
}

}  // namespace

bool has_w4a16_quantized_weight(const WeightsIndex& index, const std::string& base) {
    return index.contains(base + ".qweight") && index.contains(base + ".qzeros") && index.contains(base + ".scales");
}

W4A16QuantizedWeight pack_w4a16_awq(const int32_t* qweight, const int32_t* qzeros, const uint16_t* scales, int64_t K,
                                    int64_t N) {
    PackedHost p = alloc_packed(K, N);
    check_mcv(mcv_w4a16_pack_awq(qweight, qzeros, scales, K, N, p.qw.data(), p.sc.data(), p.zr.data()),
              "pack_w4a16_awq");
    return upload_packed(p.qw, p.sc, p.zr, K, N, 0);
}

W4A16QuantizedWeight pack_w4a16_gptq(const int32_t* qweight, const int32_t* qzeros, const int32_t* g_idx,
                                     const uint16_t* scales, int64_t K, int64_t N, int64_t groups) {
    PackedHost p = alloc_packed(K, N);
    const int rc =
        mcv_w4a16_pack_gptq(qweight, qzeros, g_idx, scales, K, N, groups, p.qw.data(), p.sc.data(), p.zr.data());
    if (rc == MCV_ERR_UNSUPPORTED) {
        // an act-order block spans more than 16 levels: the dense fp16 weight
        std::vector<uint16_t> w(static_cast<size_t>(K * N));
        check_mcv(mcv_w4a16_dequant_gptq_host(qweight, qzeros, g_idx, scales, K, N, groups, w.data()),
                  "pack_w4a16_gptq (dense)");
        W4A16QuantizedWeight out;
        out.K = K;
        out.N = N;
        out.group_size = MCV_W4_GROUP;
        out.zero_bias = 1;
        out.dense_kn = Tensor({K, N}, DType::Float16);
        out.dense_kn.copy_from_host(w.data(), w.size() * 2);
        return out;
    }
    check_mcv(rc, "pack_w4a16_gptq");
    return upload_packed(p.qw, p.sc, p.zr, K, N, 1);
}

// GPTQ when `base.g_idx` exists, AutoAWQ otherwise (quantized_weight.cpp:212-228).
W4A16QuantizedWeight load_w4a16_quantized_weight(const WeightsIndex& index, const std::string& base) {
    const TensorInfo& qi = index.at(base + ".qweight");
    const TensorInfo& zi = index.at(base + ".qzeros");
    const TensorInfo& si = index.at(base + ".scales");
    if (qi.shape.size() != 2 || zi.shape.size() != 2 || si.shape.size() != 2)
        throw std::runtime_error("unexpected W4A16 tensor ranks for " + base);
    const auto* qw = typed<int32_t>(index, base + ".qweight", DType::Int32, "qweight");
    const auto* qz = typed<int32_t>(index, base + ".qzeros", DType::Int32, "qzeros");
    const auto* sc = typed<uint16_t>(index, base + ".scales", DType::Float16, "scales");
    if (index.contains(base + ".g_idx")) {
        const TensorInfo& gi = index.at(base + ".g_idx");
        const auto* g = typed<int32_t>(index, base + ".g_idx", DType::Int32, "g_idx");
        const int64_t K = qi.shape[0] * 8, N = qi.shape[1], groups = si.shape[0];
        if (gi.shape.size() != 1 || gi.shape[0] != K || si.shape[1] != N || zi.shape[0] != groups ||
            zi.shape[1] * 8 != N || groups * MCV_W4_GROUP != K)
            throw std::runtime_error("unexpected GPTQ tensor shapes for " + base);
        return pack_w4a16_gptq(qw, qz, g, sc, K, N, groups);
    }
    const int64_t K = qi.shape[0], N = qi.shape[1] * 8, groups = si.shape[0];
    if (zi.shape != std::vector<int64_t>{groups, qi.shape[1]} || si.shape != std::vector<int64_t>{groups, N} ||
        groups * MCV_W4_GROUP != K)
        throw std::runtime_error("unexpected AWQ tensor shapes for " + base);
    return pack_w4a16_awq(qw, qz, sc, K, N);
}

W4A16QuantizedWeight quantize_w4a16_synthetic(const uint16_t* w_kn, int64_t K, int64_t N) {
    if (K <= 0 || N <= 0 || K % MCV_W4_GROUP != 0 || N % 8 != 0)
        throw std::runtime_error("quantize_w4a16_synthetic: need K % 128 == 0 and N % 8 == 0");
    std::vector<int32_t> qweight(static_cast<size_t>(K * N / 8)), qzeros(static_cast<size_t>(K / MCV_W4_GROUP * N / 8));
    std::vector<uint16_t> scales(static_cast<size_t>(K / MCV_W4_GROUP * N));
    check_mcv(mcv_w4a16_quantize_host(w_kn, K, N, qweight.data(), qzeros.data(), scales.data(), 0),
              "quantize_w4a16_synthetic");
    return pack_w4a16_awq(qweight.data(), qzeros.data(), scales.data(), K, N);
}

W8A8QuantizedWeight quantize_w8a8_host(const uint16_t* w_kn, int64_t K, int64_t N, int layout) {
    if (K <= 0 || N <= 0 || (N % 16) != 0)
        throw std::runtime_error("W8A8 dense weight shape must have positive K and N multiple of 16");
    if (layout != MCV_W8_TILED && layout != MCV_W8_KN)
        throw std::runtime_error("quantize_dense_weight_w8a8: layout must be MCV_W8_TILED or MCV_W8_KN");
    const int64_t bytes = layout == MCV_W8_TILED ? mcv_w8a8_tiled_bytes(K, N) : K * N;
    std::vector<int8_t> q(static_cast<size_t>(bytes));
    std::vector<float> s32(static_cast<size_t>(N));
    std::vector<uint16_t> s16(static_cast<size_t>(N));
    check_mcv(mcv_w8a8_quantize_weight_host(w_kn, K, N, q.data(), layout, s32.data(), s16.data()),
              "quantize_dense_weight_w8a8");
    W8A8QuantizedWeight out;
    out.K = K;
    out.N = N;
    out.layout = layout;
    out.w_int8 = layout == MCV_W8_TILED ? Tensor({bytes}, DType::Int8) : Tensor({K, N}, DType::Int8);
    out.w_int8.copy_from_host(q.data(), q.size());
    out.w_scale = Tensor({N}, DType::Float16);
    out.w_scale.copy_from_host(s16.data(), s16.size() * 2);
    out.w_scale_f32 = Tensor({N}, DType::Float32);
    out.w_scale_f32.copy_from_host(s32.data(), s32.size() * 4);
    return out;
}

// quantized_weight.cpp:231-268: the fp16 [K, N] weight comes back to the host
// once, is quantised per output channel, and goes up as int8 + scales.
W8A8QuantizedWeight quantize_dense_weight_w8a8(const Tensor& weight_kn) {
    if (weight_kn.dtype() != DType::Float16 || weight_kn.shape().size() != 2)
        throw std::runtime_error("W8A8 dense weight source must be fp16 [K, N]");
    const int64_t K = weight_kn.shape()[0], N = weight_kn.shape()[1];
    if (K <= 0 || N <= 0 || (N % 16) != 0)
        throw std::runtime_error("W8A8 dense weight shape must have positive K and N multiple of 16");
    std::vector<uint16_t> h(static_cast<size_t>(K * N));
    weight_kn.copy_to_host(h.data(), h.size() * 2);
    return quantize_w8a8_host(h.data(), K, N);
}

namespace {

W8A8QuantizedWeight upload_w8a8(const std::vector<int8_t>& q, const std::vector<float>& s32,
                                const std::vector<uint16_t>& s16, int64_t K, int64_t N, int layout) {
    W8A8QuantizedWeight out;
    out.K = K;
    out.N = N;
    out.layout = layout;
    out.w_int8 = layout == MCV_W8_TILED ? Tensor({static_cast<int64_t>(q.size())}, DType::Int8) : Tensor({K, N}, DType::Int8);
    out.w_int8.copy_from_host(q.data(), q.size());
    out.w_scale = Tensor({N}, DType::Float16);
    out.w_scale.copy_from_host(s16.data(), s16.size() * 2);
    out.w_scale_f32 = Tensor({N}, DType::Float32);
    out.w_scale_f32.copy_from_host(s32.data(), s32.size() * 4);
    return out;
}

// IEEE fp16 -> fp32 bits (exact, subnormals included).
uint32_t f16_to_f32_bits(uint16_t h) {
    const uint32_t sign = static_cast<uint32_t>(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    if (e == 0x1f) return sign | 0x7f800000u | (m << 13);
    if (e == 0) {
        if (m == 0) return sign;
        e = 113;                                   // normalise the subnormal
        while ((m & 0x400u) == 0) { m <<= 1; --e; }
        return sign | (e << 23) | ((m & 0x3ffu) << 13);
    }
    return sign | ((e + 112u) << 23) | (m << 13);
}

// The reference's stored fp16 copy of a W8A8 scale: truncating encode,
// underflow to signed zero (src/csrc/lib/quantized_weight.cpp:186-195).
uint16_t f32_to_f16_trunc(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const int32_t e = static_cast<int32_t>((x >> 23) & 0xffu) - 112;
    if (e <= 0) return static_cast<uint16_t>(sign);
    if (e >= 31) return static_cast<uint16_t>(sign | 0x7c00u);
    return static_cast<uint16_t>(sign | (static_cast<uint32_t>(e) << 10) | ((x & 0x7fffffu) >> 13));
}

float scale_value(const uint8_t* p, DType dt, int64_t i) {
    uint32_t bits = 0;
    uint16_t h = 0;
    switch (dt) {
        case DType::Float32: std::memcpy(&bits, p + 4 * i, 4); break;
        case DType::BFloat16: std::memcpy(&h, p + 2 * i, 2); bits = static_cast<uint32_t>(h) << 16; break;
        case DType::Float16: std::memcpy(&h, p + 2 * i, 2); bits = f16_to_f32_bits(h); break;
        default: throw std::runtime_error("W8A8 weight_scale must be F32, F16 or BF16");
    }
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

}  // namespace

bool has_w8a8_quantized_weight(const WeightsIndex& index, const std::string& base) {
    return index.contains(base + ".weight") && index.contains(base + ".weight_scale") &&
           index.at(base + ".weight").dtype == DType::Int8;
}

W8A8QuantizedWeight load_w8a8_quantized_weight(const WeightsIndex& index, const std::string& base, int layout) {
    if (layout != MCV_W8_TILED && layout != MCV_W8_KN)
        throw std::runtime_error("load_w8a8_quantized_weight: layout must be MCV_W8_TILED or MCV_W8_KN");
    const TensorInfo& wi = index.at(base + ".weight");
    if (wi.shape.size() != 2) throw std::runtime_error("W8A8 weight " + base + " must be 2-D [N, K]");
    const int64_t N = wi.shape[0], K = wi.shape[1];
    if (K <= 0 || N <= 0 || (N % 16) != 0)
        throw std::runtime_error("W8A8 weight " + base + " needs positive K and N multiple of 16");
    const int64_t bytes = layout == MCV_W8_TILED ? mcv_w8a8_tiled_bytes(K, N) : K * N;
    std::vector<int8_t> q(static_cast<size_t>(bytes));
    std::vector<float> s32(static_cast<size_t>(N));
    std::vector<uint16_t> s16(static_cast<size_t>(N));
    const uint8_t* src = index.host_data(base + ".weight");
    if (wi.dtype == DType::Int8) {
        // pre-quantised: int8 [N, K] plus one scale per output channel
        const TensorInfo& si = index.at(base + ".weight_scale");
        int64_t sn = 1;
        for (int64_t d : si.shape) sn *= d;
        if (sn != N) throw std::runtime_error("W8A8 weight_scale of " + base + " must hold N values");
        const uint8_t* sp = index.host_data(base + ".weight_scale");
        for (int64_t n = 0; n < N; ++n) {
            s32[n] = scale_value(sp, si.dtype, n);
            s16[n] = f32_to_f16_trunc(s32[n]);
        }
        const int8_t* qn = reinterpret_cast<const int8_t*>(src);
        if (layout == MCV_W8_TILED) {
            check_mcv(mcv_w8a8_pack_tiled_nk_host(qn, K, N, q.data()), "load_w8a8_quantized_weight");
        } else {
            for (int64_t n = 0; n < N; ++n)
                for (int64_t k = 0; k < K; ++k) q[k * N + n] = qn[n * K + k];
        }
    } else if (wi.dtype == DType::Float16 || wi.dtype == DType::BFloat16) {
        // dense checkpoint weight: quantised in one host pass (no transpose, no device round trip)
        check_mcv(mcv_w8a8_quantize_weight_nk_host(reinterpret_cast<const uint16_t*>(src),
                                                   wi.dtype == DType::BFloat16 ? MCV_SRC_BF16 : MCV_SRC_F16, K, N,
                                                   q.data(), layout, s32.data(), s16.data()),
                  "load_w8a8_quantized_weight");
    } else {
        throw std::runtime_error("W8A8 weight " + base + " must be I8 (with weight_scale), F16 or BF16");
    }
    return upload_w8a8(q, s32, s16, K, N, layout);
}

namespace {

// The tied embedding [vocab, hidden] (F16 or BF16) of the checkpoint: its
// host bytes, hidden size and source dtype, checked against `vocab`.
struct EmbeddingSource {
    const uint16_t* data;
    int64_t V;
    int64_t H;
    int src_dtype;
};

EmbeddingSource embedding_source(const WeightsIndex& index, const std::string& name, int64_t vocab) {
    const TensorInfo& info = index.at(name);
    if (info.shape.size() != 2) throw std::runtime_error("lm_head embedding " + name + " must be 2-D [vocab, hidden]");
    if (info.dtype != DType::Float16 && info.dtype != DType::BFloat16)
        throw std::runtime_error("lm_head embedding " + name + " must be F16 or BF16");
    const int64_t V = info.shape[0], H = info.shape[1];
    if (vocab != V) throw std::runtime_error("lm_head embedding " + name + " has " + std::to_string(V) +
                                             " rows, expected vocab " + std::to_string(vocab));
    if (H <= 0 || H % MCV_W4_GROUP != 0)
        throw std::runtime_error("lm_head embedding hidden size must be a positive multiple of 128");
    return {reinterpret_cast<const uint16_t*>(index.host_data(name)), V, H,
            info.dtype == DType::BFloat16 ? MCV_SRC_BF16 : MCV_SRC_F16};
}

}  // namespace

W4A16QuantizedWeight load_lm_head_w4a16(const WeightsIndex& index, const std::string& name, int64_t vocab) {
    const EmbeddingSource e = embedding_source(index, name, vocab);
    const int64_t N = (e.V + 63) / 64 * 64;
    std::vector<int32_t> qweight(static_cast<size_t>(e.H * (N / 8)));
    std::vector<int32_t> qzeros(static_cast<size_t>((e.H / MCV_W4_GROUP) * (N / 8)));
    std::vector<uint16_t> scales(static_cast<size_t>((e.H / MCV_W4_GROUP) * N));
    check_mcv(mcv_w4a16_quantize_nk_host(e.data, e.src_dtype, e.H, e.V, N, qweight.data(), qzeros.data(),
                                         scales.data(), 0),
              "load_lm_head_w4a16");
    return pack_w4a16_awq(qweight.data(), qzeros.data(), scales.data(), e.H, N);
}

W8A8QuantizedWeight load_lm_head_w8a8(const WeightsIndex& index, const std::string& name, int64_t vocab, int layout) {
    if (layout != MCV_W8_TILED && layout != MCV_W8_KN)
        throw std::runtime_error("load_lm_head_w8a8: layout must be MCV_W8_TILED or MCV_W8_KN");
    const EmbeddingSource e = embedding_source(index, name, vocab);
    const int64_t N = (e.V + 63) / 64 * 64;
    const int64_t bytes = layout == MCV_W8_TILED ? mcv_w8a8_tiled_bytes(e.H, N) : e.H * N;
    std::vector<int8_t> q(static_cast<size_t>(bytes));
    std::vector<float> s32(static_cast<size_t>(N));
    std::vector<uint16_t> s16(static_cast<size_t>(N));
    check_mcv(mcv_w8a8_quantize_weight_nk_pad_host(e.data, e.src_dtype, e.H, e.V, N, q.data(), layout, s32.data(),
                                                   s16.data()),
              "load_lm_head_w8a8");
    return upload_w8a8(q, s32, s16, e.H, N, layout);
}

}  // namespace minicpmv
