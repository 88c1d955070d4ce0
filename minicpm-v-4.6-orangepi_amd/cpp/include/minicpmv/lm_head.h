// lm_head.h -- greedy lm_head over a W4A16 (or W8A8) vocabulary projection.
//
// Replaces lm_head_greedy (src/csrc/lib/language_model.cpp:412-482): final
// RMSNorm, then -- instead of 16 chunk matmuls, 16 blocking D2H copies and a
// host scan -- one GEMV with the argmax folded into it.  Same tie rule: the
// first maximum wins, fp16 subnormals compare as zero, NaN never wins.  The
// head objects own every buffer a call needs, so calls allocate nothing.
#pragma once

#include "minicpmv/hip_context.h"
#include "minicpmv/quantized_weight.h"
#include "minicpmv/tensor.h"

#include <hip/hip_runtime_api.h>

#include <cstdint>

namespace minicpmv {

struct LmHeadW4A16 {
    W4A16QuantizedWeight weight;   // [hidden, >= vocab]
    int64_t vocab{0};
    Tensor workspace;              // zero-filled once; calls keep its counters and tagged keys consistent
    Tensor token;                  // Int64 [1]
    Tensor slots;                  // tagged slot maxima of the host-finished argmax
    Tensor normed;                 // Float16 [1, hidden]: the final RMSNorm's output
    WaitStatus status;             // set by the device-token route if its bounded wait gave up
    uint32_t tag{0};               // tag of the last slots call
};

LmHeadW4A16 make_lm_head_w4a16(W4A16QuantizedWeight weight, int64_t vocab);

// Stream-ordered: token and (optional, fp16 [1, vocab]) logits on the device.
// Throws (after re-zeroing the workspace, which synchronises `stream`) if an
// earlier call's wait for the workgroups' keys gave up.
void lm_head_argmax_w4a16(const Tensor& hidden_1xH, LmHeadW4A16& head, Tensor* logits, hipStream_t stream);
// Copies the device token to the host (synchronises `stream`); throws if the
// call that wrote it gave up waiting (token -1).
int64_t lm_head_read_token(LmHeadW4A16& head, hipStream_t stream);

// Stream-ordered, host-finished argmax: the GEMV leaves call-tagged maxima in
// head.slots (no device round trip at the end of the kernel); returns the tag
// to pass to lm_head_read_slots_token.
uint32_t lm_head_argmax_slots_w4a16(const Tensor& hidden_1xH, LmHeadW4A16& head, Tensor* logits, hipStream_t stream);
// Copies the slots to the host (synchronises `stream`) and folds them into the token.
int64_t lm_head_read_slots_token(const LmHeadW4A16& head, uint32_t tag, hipStream_t stream);

// lm_head_greedy semantics: optional final RMSNorm (final_norm may be null),
// then the argmax through the slots; returns the token on the host
// (synchronises `stream`).
int64_t lm_head_greedy_w4a16(const Tensor& last_hidden_1xH, const Tensor* final_norm, double rms_epsilon,
                             LmHeadW4A16& head, hipStream_t stream);

// The W8A8 lm_head (language_model.cpp:434-467) with the reference's
// precision: one activation quantisation with its fp16 scale, the fused int8
// GEMV with the truncated fp16 weight scale, the first-maximum argmax on the
// device -- for an MCV_W8_TILED weight folded into the GEMV (one key per
// 64-column slab, then their reduction), otherwise a separate argmax over the
// logits.  The weight stays owned by the caller.
struct LmHeadW8A8 {
    const W8A8QuantizedWeight* weight{nullptr};   // [hidden, >= vocab]
    int64_t vocab{0};
    Tensor normed;                 // Float16 [1, hidden]
    Tensor xq;                     // Int8 [1, hidden] (weights not in MCV_W8_TILED)
    Tensor xs;                     // Float16 [1]
    Tensor logits;                 // Float16 [1, weight N]: the last call's logits (columns < vocab)
    Tensor keys;                   // Int64 [ceil(vocab / 64)]: per-slab keys (MCV_W8_TILED, hidden > 2048)
    Tensor workspace;              // the one-launch step's (MCV_W8_TILED, hidden <= 2048), zero-filled once
    Tensor token;                  // Int64 [1]
};
LmHeadW8A8 make_lm_head_w8a8(const W8A8QuantizedWeight& weight, int64_t vocab);
int64_t lm_head_greedy_w8a8(const Tensor& last_hidden_1xH, const Tensor* final_norm, double rms_epsilon,
                            LmHeadW8A8& head, hipStream_t stream);

}  // namespace minicpmv
