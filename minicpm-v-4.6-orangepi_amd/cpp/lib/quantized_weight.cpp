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
    check_mcv(mcv_w4a16_pack_gptq(qweight, qzeros, g_idx, scales, K, N, groups, p.qw.data(), p.sc.data(), p.zr.data()),
              "pack_w4a16_gptq");
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

}  // namespace minicpmv
