// decode_dispatch.h -- per-projection choice between W8A8, W4A16 and dense.
//
// Mirrors matmul_decode_dispatch and its helpers
// (src/csrc/lib/decoder_layer.cpp:19-25, 205-244) and the lm_head policy of
// src/csrc/lib/language_model.cpp:19-41.
#pragma once

#include "minicpmv/quantized_weight.h"
#include "minicpmv/tensor.h"

#include <hip/hip_runtime_api.h>

#include <string>

namespace minicpmv {

// MINICPM_W8A8_DECODE as read by the decoder layers: set and not "0"/"false"
// (an empty string counts as enabled, decoder_layer.cpp:19-25).
bool w8a8_decode_enabled_for_layers();
// The language-model reading of the same variable (language_model.cpp:19-41):
// unset/empty/"0"/"false" off; "1"/"selective" lm_head only; "all" everything;
// anything else a substring match on the projection token.
std::string w8a8_decode_mode();
bool w8a8_decode_enabled();
bool w8a8_policy_allows(const char* token);

bool w8a8_weight_ready(const W8A8QuantizedWeight* w8_weight);

// x_int8 [1, K] + x_scale -> out fp16 [1, N] through the fused W8A8 kernel
// (the reference's matmul_w8a8_i32 + w8a8_dequant, decoder_layer.cpp:216-224).
// The epilogue uses the scales in x_scale's dtype: an fp16 x_scale (what the
// reference's w8a8_quantize stores) pairs with the truncated fp16 w_scale,
// exactly the reference's arithmetic; fp32 with the fp32 weight scale.
void matmul_decode_w8a8_prequant(const Tensor& x_int8, const Tensor& x_scale, const W8A8QuantizedWeight& w8_weight,
                                 Tensor& out, hipStream_t stream);

// Device scratch of the dispatcher: the W8A8 branch's quantised row and its
// fp16 scale, and the W4A16 GEMM's K-split workspace (fp32 partial tiles and
// their arrival counters).  Grown (allocated) only when a call needs more than
// it holds, so a decode loop allocates on its first call and never again.
// One stream at a time.
struct DecodeScratch {
    Tensor x_int8;       // Int8 [capacity]
    Tensor x_scale;      // Float16 [rows capacity]
    Tensor gemm_ws;      // Int8 [bytes], see matmul_w4a16's workspace overload
    // Makes room for an [M, K] activation (reallocates only on growth).
    void reserve(int64_t M, int64_t K);
};

// The reference's choice (decoder_layer.cpp:226-244): W8A8 when enabled and
// present and x is [1, K] (an fp16 activation scale and the truncated fp16
// weight scale, as the reference's w8a8_quantize / w8a8_dequant use them);
// else W4A16 when present and x is [1, K]; else the dense weight.  Beyond the
// reference, which would dereference a null dense weight there: with no dense
// weight, the quantised objects serve M > 1 rows too (W4A16 through the MFMA
// GEMM, W8A8 with per-row scales).  `scratch` holds the W8A8 temporaries.
void matmul_decode_dispatch(const Tensor& x, const Tensor* dense_weight, const W4A16QuantizedWeight* quant_weight,
                            const W8A8QuantizedWeight* w8_weight, Tensor& out, hipStream_t stream,
                            DecodeScratch& scratch);
// The reference's signature: the scratch is this thread's, one per (device,
// stream), so dispatches on two streams never share temporaries.
void matmul_decode_dispatch(const Tensor& x, const Tensor* dense_weight, const W4A16QuantizedWeight* quant_weight,
                            const W8A8QuantizedWeight* w8_weight, Tensor& out, hipStream_t stream);

}  // namespace minicpmv
