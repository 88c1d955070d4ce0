// ops.h -- quantized-matmul operators (hot-path subset of the reference's ops.h).
//
// Same names and argument order as src/csrc/include/minicpmv/ops.h:41,95-126
// with aclrtStream -> hipStream_t.  Every operator validates shapes and dtypes
// on the host (std::runtime_error on mismatch, as ops.cpp:1037-1079) and then
// enqueues hand-written gfx950 kernels on `stream` through the C-ABI.  Unlike
// the reference (which synchronises after every op, ops.cpp:374) the calls are
// stream-ordered and asynchronous; Tensor::copy_to_host orders after them.
//
// Generalisations: the M = 1 restriction of matmul_w4a16 / matmul_w8a8_i32 /
// w8a8_quantize / w8a8_dequant (ops.cpp:1049,1110,1148,1182) is lifted to any
// M; scales may be fp16 or fp32.
#pragma once

#include "minicpmv/hip_context.h"
#include "minicpmv/quantized_weight.h"
#include "minicpmv/tensor.h"

#include <hip/hip_runtime_api.h>
#include <vector>

namespace minicpmv {

// out = silu(gate) * up in fp32, RNE to fp16.  gate, up, out: fp16, one shape.
void silu_mul(const Tensor& gate, const Tensor& up, Tensor& out, hipStream_t stream);

// Per-row argmax of fp16 [..., N] into Int64 [rows]; the first maximum wins.
void argmax_last_dim(const Tensor& self, Tensor& out, hipStream_t stream);

// The reference's W4A16 format, M = 1:
//   x fp16 [1, K]; w_int8 int8 [(K/128)*8*tilesPerBlock*128, tile_len] holding
//   (q - z) tile-packed by pack_w4a16_weight; scales fp16 [K/128, N]; out [1, N].
void matmul_w4a16(const Tensor& x, const Tensor& w_int8, const Tensor& scales, Tensor& out, hipStream_t stream);

// x fp16 [M, K] . dequant(w) -> out fp16 [M, N], any M (GEMV for small M,
// LDS-dequant fp16 MFMA GEMM otherwise).  Where the GEMM splits K across
// workgroups it uses a workspace the library keeps per (device, stream) of
// the calling thread: allocated on the first call that needs it (or more of
// it), reused after that.
void matmul_w4a16(const Tensor& x, const W4A16QuantizedWeight& w, Tensor& out, hipStream_t stream);

// The same with a caller-owned workspace (mcv_w4a16_gemm_ws): where the MFMA
// path splits K across workgroups (few rows, long K) its fp32 partial tiles go
// there.  `workspace` (Int8) is reallocated only when a shape needs more than
// it holds; calls that share it must be ordered on one stream.
void matmul_w4a16(const Tensor& x, const W4A16QuantizedWeight& w, Tensor& out, hipStream_t stream, Tensor& workspace);

// Decode MLP front half in one launch: act [M, I] = silu(x . gate) * (x . up),
// gate/up rounded to fp16 first -- bit-identical to two matmul_w4a16 calls and
// silu_mul (the reference's sequence, decoder_layer.cpp:1029-1046).
void mlp_gate_up_silu_w4a16(const Tensor& x, const W4A16QuantizedWeight& gate, const W4A16QuantizedWeight& up,
                            Tensor& act, hipStream_t stream);

// The whole decode MLP block, M = 1: out [1, H] = (silu(x . gate) * (x . up)) . down
// (decoder_layer.cpp:1029-1046), bit-identical to mlp_gate_up_silu_w4a16 +
// matmul_w4a16.  One launch (mcv_w4a16_mlp) where the shape allows, else those
// two launches.  The weights stay owned by the caller and must outlive it.
// The one-launch kernel's waits are bounded; a give-up sets `status`, which
// mlp_w4a16 checks at every call (a plain host read, no synchronisation) and
// check_wait_status at the caller's own synchronisation points: both throw.
struct DecodeMlpW4A16 {
    const W4A16QuantizedWeight* gate{nullptr};   // [H, I]
    const W4A16QuantizedWeight* up{nullptr};     // [H, I]
    const W4A16QuantizedWeight* down{nullptr};   // [I, H]
    Tensor workspace;                            // zero-filled once; one stream at a time
    Tensor act;                                  // fp16 [1, I], for the two-launch path
    WaitStatus status;                           // host-mapped give-up word of the one-launch kernel
    bool one_launch{true};
};
DecodeMlpW4A16 make_decode_mlp_w4a16(const W4A16QuantizedWeight& gate, const W4A16QuantizedWeight& up,
                                     const W4A16QuantizedWeight& down);
void mlp_w4a16(const Tensor& x, DecodeMlpW4A16& mlp, Tensor& out, hipStream_t stream);
// Throws if a wait of an earlier one-launch call gave up (that call's output
// is undefined).  Before throwing it drains `stream` and re-zeroes the
// workspace, so the object works again afterwards.
void check_wait_status(DecodeMlpW4A16& mlp, hipStream_t stream);

// int32 out [M, N] = int8 x [M, K] . int8 w [K, N], exact.
void matmul_w8a8_i32(const Tensor& x, const Tensor& w_int8, Tensor& out, hipStream_t stream);
// The same over a quantized weight object, in whatever layout it holds
// (MCV_W8_TILED: operand-line GEMM / GEMV kernels).
void matmul_w8a8_i32(const Tensor& x, const W8A8QuantizedWeight& w, Tensor& out, hipStream_t stream);

// Per-row symmetric int8 quantisation of fp16 x [M, K]; x_scale is [M]
// (or [1] for M = 1, as the reference) in fp16 or fp32.
void w8a8_quantize(const Tensor& x, Tensor& x_int8, Tensor& x_scale, hipStream_t stream);
// rms_norm followed by w8a8_quantize of the normed row in one launch
// (decoder_layer.cpp:955-966, 1022-1032), bit-identical to the pair; `normed`
// may be null when nothing else reads the fp16 row.
void rms_norm_w8a8_quantize(const Tensor& x, const Tensor& gamma, double epsilon, Tensor* normed, Tensor& x_int8,
                            Tensor& x_scale, hipStream_t stream);

// Up to four W4A16 projections of the same x [M, K] in one launch (q/k/v,
// decoder_layer.cpp:970-972; qkv and z, :1108-1110).  outs[i] is fp16 [M, N_i].
void matmul_w4a16_multi(const Tensor& x, const std::vector<const W4A16QuantizedWeight*>& weights,
                        const std::vector<Tensor*>& outs, hipStream_t stream);

// W8A8 decode MLP front half: act = silu(gate) * up over one quantised x
// (decoder_layer.cpp:1029-1046 + silu_mul), bit-identical to two matmul_w8a8
// calls and silu_mul; one launch for M <= 4 with tiled weights.
void mlp_gate_up_silu_w8a8(const Tensor& x_int8, const Tensor& x_scale, const W8A8QuantizedWeight& gate,
                           const W8A8QuantizedWeight& up, Tensor& act, hipStream_t stream);

// The whole W8A8 decode MLP block, M = 1, from the normed fp16 row:
// w8a8_quantize, mlp_gate_up_silu_w8a8, w8a8_quantize, matmul_w8a8
// (decoder_layer.cpp:1022-1046), bit-identical; one launch (mcv_w8a8_mlp)
// for tiled weights where the grid fits, else those four.  By default every
// epilogue uses the fp16 activation scale and the truncated fp16 weight
// scale, the reference's precision (decoder_layer.cpp:216-237); f32_scales
// selects fp32 scales throughout.  Give-ups are reported as for DecodeMlpW4A16.
struct DecodeMlpW8A8 {
    const W8A8QuantizedWeight* gate{nullptr};    // [H, I]
    const W8A8QuantizedWeight* up{nullptr};      // [H, I]
    const W8A8QuantizedWeight* down{nullptr};    // [I, H]
    Tensor workspace;                            // zero-filled once; one stream at a time
    Tensor xq, xs, act, aq, as;                  // buffers of the four-launch path (scales fp16 or fp32)
    WaitStatus status;                           // host-mapped give-up word of the one-launch kernel
    bool f32_scales{false};
    bool one_launch{true};
};
DecodeMlpW8A8 make_decode_mlp_w8a8(const W8A8QuantizedWeight& gate, const W8A8QuantizedWeight& up,
                                   const W8A8QuantizedWeight& down, bool f32_scales = false);
void mlp_w8a8(const Tensor& x, DecodeMlpW8A8& mlp, Tensor& out, hipStream_t stream);
void check_wait_status(DecodeMlpW8A8& mlp, hipStream_t stream);

// out fp16 [M, N] = RNE((acc * w_scale[n]) * x_scale[m]); scales fp16 or fp32.
void w8a8_dequant(const Tensor& acc, const Tensor& x_scale, const Tensor& w_scale, Tensor& out, hipStream_t stream);

// Fused int8 GEMM + dequant epilogue (the int32 accumulator stays on chip);
// bit-identical to matmul_w8a8_i32 + w8a8_dequant with the same scales.
// Uses w.w_scale_f32 when x_scale is fp32, the fp16 w.w_scale otherwise.
void matmul_w8a8(const Tensor& x_int8, const Tensor& x_scale, const W8A8QuantizedWeight& w, Tensor& out,
                 hipStream_t stream);

// Materialises dequantised weights: w_f16 [K, N] fp16 and/or w_i8 [K, N] int8
// (q - z); either pointer may be null.
void w4a16_dequant(const W4A16QuantizedWeight& w, Tensor* w_f16, Tensor* w_i8, hipStream_t stream);

// Dense fp16 fallback of the decode dispatcher: out [M, N] = a [M, K] . b,
// b given as [N, K] or [K, N] (src/csrc/lib/ops.cpp:159-322 semantics).  A
// plain library GEMM (rocBLAS, fp32 accumulation).
void matmul_b_transposed(const Tensor& a, const Tensor& b, Tensor& out, hipStream_t stream);

// y = fp16(x / sqrt(mean(x^2) + eps) * gamma) per row, fp32 in between.
void rms_norm(const Tensor& x, const Tensor& gamma, Tensor& out, double epsilon, hipStream_t stream);

}  // namespace minicpmv
