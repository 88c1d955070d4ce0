// quantized_weight.h -- W4A16 / W8A8 weight objects and their loaders.
//
// Mirrors src/csrc/include/minicpmv/quantized_weight.h:11-28.  Additive
// changes, all behind the same names:
//   - W4A16QuantizedWeight keeps the int4 nibbles packed on the device in the
//     gfx950 slab-64 layout (include/mcv_quant.h) instead of widening them to
//     int8 (q - z): `w_int8` holds those packed bytes, and the zero-points
//     travel as `zeros` (+ `zero_bias`) rather than being folded in.
//   - W8A8QuantizedWeight also keeps the fp32 per-channel scale; `w_scale` is
//     the reference's truncated fp16 copy (quantized_weight.cpp:253).  Its
//     `w_int8` is stored in `layout`: MCV_W8_TILED (MFMA operand lines, what
//     quantize_dense_weight_w8a8 produces) or the reference's [K, N].
//   - N need not be a multiple of 128 (the reference's load requires it,
//     quantized_weight.cpp:215-217); AutoAWQ/GPTQ packing needs N % 8 == 0.
#pragma once

#include "mcv_quant.h"
#include "minicpmv/tensor.h"
#include "minicpmv/weights.h"

#include <cstdint>
#include <string>

namespace minicpmv {

struct W4A16QuantizedWeight {
    Tensor w_int8;          // UInt8 [packed bytes]: slab-64 nibbles
    Tensor scales;          // Float16 [K/128, Npad]
    Tensor zeros;           // Int32 [K/128, Npad/8]: 4-bit zero-points
    int64_t K{0};
    int64_t N{0};
    int64_t group_size{128};
    int zero_bias{0};       // 0: AutoAWQ / synthetic, 1: GPTQ v1 (stored zero - 1)
    // Float16 [K, N], set instead of the three tensors above for a GPTQ
    // act-order weight whose 128-row blocks span more than 16 levels (no
    // 4-bit zero per block holds them): the exact dequantised values, run by
    // matmul_w4a16 as a dense fp16 GEMM; the fused W4A16 entry points refuse it
    Tensor dense_kn;
};

struct W8A8QuantizedWeight {
    Tensor w_int8;          // Int8: [K, N] (MCV_W8_KN) or flat MCV_W8_TILED bytes
    Tensor w_scale;         // Float16 [N], truncating encode of the fp32 scale
    Tensor w_scale_f32;     // Float32 [N]
    int64_t K{0};
    int64_t N{0};
    int layout{MCV_W8_KN};  // mcv_w8_layout
};

bool has_w4a16_quantized_weight(const WeightsIndex& index, const std::string& base);
W4A16QuantizedWeight load_w4a16_quantized_weight(const WeightsIndex& index, const std::string& base);
W8A8QuantizedWeight quantize_dense_weight_w8a8(const Tensor& weight_kn);

// Host tensors -> device weight (no device round trip).
W4A16QuantizedWeight pack_w4a16_awq(const int32_t* qweight, const int32_t* qzeros, const uint16_t* scales,
                                    int64_t K, int64_t N);
W4A16QuantizedWeight pack_w4a16_gptq(const int32_t* qweight, const int32_t* qzeros, const int32_t* g_idx,
                                     const uint16_t* scales, int64_t K, int64_t N, int64_t groups);
// Build-defined synthetic int4 quantiser (mcv_w4a16_quantize_host) applied to
// fp16 [K, N] host weights, then packed.
W4A16QuantizedWeight quantize_w4a16_synthetic(const uint16_t* w_kn, int64_t K, int64_t N);
// `layout` MCV_W8_TILED (default) or MCV_W8_KN.
W8A8QuantizedWeight quantize_w8a8_host(const uint16_t* w_kn, int64_t K, int64_t N, int layout = MCV_W8_TILED);

// W8A8 weights straight from a checkpoint, no device round trip and no host
// transpose: `base.weight` [N, K] either I8 with `base.weight_scale` ([N],
// F32 / F16 / BF16; a pre-quantised checkpoint, which the reference cannot
// read -- its loader has no I8, weights.cpp:15-23) or F16 / BF16 (quantised on
// the host exactly as load_matmul_weight_transposed + quantize_dense_weight_w8a8
// do, language_model.cpp:84-105,190-231).
bool has_w8a8_quantized_weight(const WeightsIndex& index, const std::string& base);
W8A8QuantizedWeight load_w8a8_quantized_weight(const WeightsIndex& index, const std::string& base,
                                               int layout = MCV_W8_TILED);

// The lm_head's vocabulary projection from the tied token embedding, read
// from the checkpoint (`name`, e.g. "model.language_model.embed_tokens.weight",
// [vocab, hidden] F16 or BF16, bf16 converted as the reference loads it) in
// one host pass: the embedding's rows become the projection's columns,
// padded with zero columns to N = vocab rounded up to 64 (the reference
// transposes it into 16384-wide chunks, the last padded with zero columns,
// language_model.cpp:170,238-270).  W4A16: the build's synthetic int4
// quantiser per (group, column) -- the reference has no int4 lm_head.  W8A8:
// the reference's per-channel quantiser (quantize_dense_weight_w8a8 of each
// chunk, language_model.cpp:264-266), bit-identical to it; the zero columns get
// the 1e-8 scale floor and q = 0.  Columns from vocab on are ignored by the
// lm_head entry points (vocab is passed to them).
W4A16QuantizedWeight load_lm_head_w4a16(const WeightsIndex& index, const std::string& name, int64_t vocab);
W8A8QuantizedWeight load_lm_head_w8a8(const WeightsIndex& index, const std::string& name, int64_t vocab,
                                      int layout = MCV_W8_TILED);

}  // namespace minicpmv
