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

// x_int8 [1, K] + x_scale -> out fp16 [1, N] through the fused W8A8 kernel.
void matmul_decode_w8a8_prequant(const Tensor& x_int8, const Tensor& x_scale, const W8A8QuantizedWeight& w8_weight,
                                 Tensor& out, hipStream_t stream);

// W8A8 when enabled and present, else W4A16 when present, else dense.  The
// quantised branches serve any M here (the reference takes them at M = 1 only).
void matmul_decode_dispatch(const Tensor& x, const Tensor* dense_weight, const W4A16QuantizedWeight* quant_weight,
                            const W8A8QuantizedWeight* w8_weight, Tensor& out, hipStream_t stream);

}  // namespace minicpmv
