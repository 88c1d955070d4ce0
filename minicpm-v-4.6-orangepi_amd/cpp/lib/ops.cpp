// ops.cpp -- host-side validation + launch of the quantized-matmul operators.
//
// Validation mirrors the reference's host wrappers (src/csrc/lib/ops.cpp:
// 437-456, 1030-1210): a mismatch throws std::runtime_error before anything is
// enqueued.  The launches go through the C-ABI (include/mcv_quant.h).
#include "minicpmv/ops.h"

#include "mcv_quant.h"
#include "minicpmv/hip_context.h"

#include <rocblas/rocblas.h>

#include <map>
#include <mutex>
#include <stdexcept>
#include <string>
#include <unordered_map>

namespace minicpmv {
namespace {

void require(bool ok, const std::string& msg) {
    if (!ok) throw std::runtime_error(msg);
}

// The fused W4A16 entry points take slab-layout weights only.
void require_slab(const W4A16QuantizedWeight& w, const char* what) {
    require(w.dense_kn.numel() == 0, std::string(what) +
                                         ": this GPTQ act-order weight is kept dense (its 128-row blocks span more "
                                         "than 16 levels); only matmul_w4a16 takes it");
}

// The workspace of the 4-argument matmul_w4a16: one per (device, stream) of
// this thread, grown on demand and kept, so calls on one stream reuse it in
// stream order and calls on two streams never share one.
Tensor& implicit_gemm_workspace(hipStream_t stream) {
    thread_local std::map<std::pair<int, hipStream_t>, Tensor> per_stream;
    int dev = 0;
    check_hip(hipGetDevice(&dev), "hipGetDevice");
    return per_stream[{dev, stream}];
}

int scale_dtype(const Tensor& t, const char* what) {
    if (t.dtype() == DType::Float32) return MCV_F32;
    if (t.dtype() == DType::Float16) return MCV_F16;
    throw std::runtime_error(std::string(what) + " must be fp16 or fp32");
}

}  // namespace

void silu_mul(const Tensor& gate, const Tensor& up, Tensor& out, hipStream_t stream) {
    require(gate.dtype() == DType::Float16 && up.dtype() == DType::Float16 && out.dtype() == DType::Float16,
            "silu_mul requires fp16 tensors");
    require(gate.shape() == up.shape() && gate.shape() == out.shape(), "silu_mul shape mismatch");
    check_mcv(mcv_silu_mul(gate.data(), up.data(), out.data(), static_cast<int64_t>(gate.numel()), stream), "silu_mul");
}

void argmax_last_dim(const Tensor& self, Tensor& out, hipStream_t stream) {
    require(!self.shape().empty(), "argmax input must have rank >= 1");
    require(self.dtype() == DType::Float16, "argmax input must be fp16");
    require(out.dtype() == DType::Int64, "argmax output must be int64");
    const int64_t n = self.shape().back();
    const int64_t rows = n > 0 ? static_cast<int64_t>(self.numel()) / n : 0;
    require(static_cast<int64_t>(out.numel()) == rows, "argmax output must hold one index per row");
    check_mcv(mcv_argmax_f16(self.data(), rows, n, static_cast<int64_t*>(out.data()), stream), "argmax_last_dim");
}

void matmul_w4a16(const Tensor& x, const Tensor& w_int8, const Tensor& scales, Tensor& out, hipStream_t stream) {
    require(x.dtype() == DType::Float16, "matmul_w4a16 x must be fp16");
    require(w_int8.dtype() == DType::Int8, "matmul_w4a16 w must be int8 (pre-unpacked from GPTQ)");
    require(scales.dtype() == DType::Float16, "matmul_w4a16 scales must be fp16");
    require(out.dtype() == DType::Float16, "matmul_w4a16 out must be fp16");
    require(x.shape().size() == 2 && x.shape()[0] == 1, "matmul_w4a16 x must be [1, K]");
    require(scales.shape().size() == 2, "matmul_w4a16 scales must be 2D");
    require(w_int8.shape().size() == 2, "matmul_w4a16 w must be [packed_rows, tile_len]");
    const int64_t K = x.shape()[1], N = scales.shape()[1];
    require(scales.shape() == std::vector<int64_t>{K / 128, N}, "matmul_w4a16 scales must be [K/128, N]");
    require(out.shape() == std::vector<int64_t>{1, N}, "matmul_w4a16 out must be [1, N]");
    check_mcv(mcv_w4a16_gemv_tiled_i8(x.data(), K, N, w_int8.shape()[1], w_int8.shape()[0],
                                      static_cast<const int8_t*>(w_int8.data()), scales.data(), out.data(), stream),
              "matmul_w4a16");
}

void matmul_w4a16(const Tensor& x, const W4A16QuantizedWeight& w, Tensor& out, hipStream_t stream) {
    matmul_w4a16(x, w, out, stream, implicit_gemm_workspace(stream));
}

void matmul_w4a16(const Tensor& x, const W4A16QuantizedWeight& w, Tensor& out, hipStream_t stream, Tensor& workspace) {
    require(x.dtype() == DType::Float16 && out.dtype() == DType::Float16, "matmul_w4a16 x and out must be fp16");
    require(x.shape().size() == 2 && x.shape()[1] == w.K, "matmul_w4a16 x must be [M, K]");
    require(out.shape() == std::vector<int64_t>{x.shape()[0], w.N}, "matmul_w4a16 out must be [M, N]");
    if (w.dense_kn.numel() > 0) {                // act-order weight kept dense (quantized_weight.h)
        matmul_b_transposed(x, w.dense_kn, out, stream);
        return;
    }
    require(w.w_int8.data() && w.scales.data() && w.zeros.data(), "matmul_w4a16 weight is not loaded");
    const int64_t nb = mcv_w4a16_gemm_workspace_bytes(x.shape()[0], w.K, w.N);
    if (nb > 0 && static_cast<int64_t>(workspace.numel()) < nb) {
        // the split's tile counters must start at zero (calls leave them zero)
        workspace = Tensor({nb}, DType::Int8);
        workspace.zero();
    }
    check_mcv(mcv_w4a16_gemm_ws(x.data(), x.shape()[0], w.K, w.N, w.w_int8.data(), w.scales.data(), w.zeros.data(),
                                w.zero_bias, out.data(), nb > 0 ? workspace.data() : nullptr, nb, stream),
              "matmul_w4a16");
}

void mlp_gate_up_silu_w4a16(const Tensor& x, const W4A16QuantizedWeight& gate, const W4A16QuantizedWeight& up,
                            Tensor& act, hipStream_t stream) {
    require(x.dtype() == DType::Float16 && act.dtype() == DType::Float16, "mlp_gate_up_silu x and act must be fp16");
    require(x.shape().size() == 2 && x.shape()[1] == gate.K, "mlp_gate_up_silu x must be [M, K]");
    require(up.K == gate.K && up.N == gate.N, "mlp_gate_up_silu gate and up must have the same shape");
    require_slab(gate, "mlp_gate_up_silu");
    require_slab(up, "mlp_gate_up_silu");
    require(act.shape() == std::vector<int64_t>{x.shape()[0], gate.N}, "mlp_gate_up_silu act must be [M, N]");
    check_mcv(mcv_w4a16_gate_up_silu(x.data(), x.shape()[0], gate.K, gate.N, gate.w_int8.data(), gate.scales.data(),
                                     gate.zeros.data(), gate.zero_bias, up.w_int8.data(), up.scales.data(),
                                     up.zeros.data(), up.zero_bias, act.data(), stream),
              "mlp_gate_up_silu");
}

DecodeMlpW4A16 make_decode_mlp_w4a16(const W4A16QuantizedWeight& gate, const W4A16QuantizedWeight& up,
                                     const W4A16QuantizedWeight& down) {
    require(up.K == gate.K && up.N == gate.N, "decode MLP gate and up must have the same shape");
    require(down.K == gate.N && down.N == gate.K, "decode MLP down must be [I, H] for gate [H, I]");
    require_slab(gate, "make_decode_mlp_w4a16");
    require_slab(up, "make_decode_mlp_w4a16");
    require_slab(down, "make_decode_mlp_w4a16");
    DecodeMlpW4A16 mlp;
    mlp.gate = &gate;
    mlp.up = &up;
    mlp.down = &down;
    const int64_t ws = mcv_w4a16_mlp_workspace_bytes(gate.K, gate.N);
    mlp.one_launch = ws > 0;
    if (mlp.one_launch) {
        mlp.workspace = Tensor({ws}, DType::UInt8);
        mlp.workspace.zero();
    }
    mlp.act = Tensor({1, gate.N}, DType::Float16);
    mlp.act.allocate();
    return mlp;
}

namespace {

// A give-up leaves the per-workgroup call counters out of step: drain the
// stream, zero the workspace and the status word, then report.
[[noreturn]] void raise_mlp_gave_up(Tensor& workspace, WaitStatus& status, hipStream_t stream, const char* who) {
    check_hip(hipStreamSynchronize(stream), "hipStreamSynchronize");
    workspace.zero();
    status.clear();
    throw std::runtime_error(std::string(who) +
                             ": a wait for another workgroup's words gave up in an earlier call (its output is "
                             "undefined); the workspace was reset");
}

}  // namespace

void check_wait_status(DecodeMlpW4A16& mlp, hipStream_t stream) {
    if (mlp.status.gave_up()) raise_mlp_gave_up(mlp.workspace, mlp.status, stream, "mlp_w4a16");
}

void mlp_w4a16(const Tensor& x, DecodeMlpW4A16& mlp, Tensor& out, hipStream_t stream) {
    const W4A16QuantizedWeight &g = *mlp.gate, &u = *mlp.up, &d = *mlp.down;
    require(x.dtype() == DType::Float16 && x.shape() == std::vector<int64_t>{1, g.K}, "decode MLP x must be fp16 [1, H]");
    require(out.dtype() == DType::Float16 && out.shape() == std::vector<int64_t>{1, g.K},
            "decode MLP out must be fp16 [1, H]");
    if (mlp.one_launch) {
        check_wait_status(mlp, stream);
        const int rc = mcv_w4a16_mlp(x.data(), g.K, g.N, g.w_int8.data(), g.scales.data(), g.zeros.data(), g.zero_bias,
                                     u.w_int8.data(), u.scales.data(), u.zeros.data(), u.zero_bias, d.w_int8.data(),
                                     d.scales.data(), d.zeros.data(), d.zero_bias, out.data(), mlp.workspace.data(),
                                     mlp.status.device_word(), stream);
        if (rc != MCV_ERR_SHAPE) {
            check_mcv(rc, "mlp_w4a16");
            return;
        }
        mlp.one_launch = false;          // this shape or device cannot hold the one-launch grid
    }
    mlp_gate_up_silu_w4a16(x, g, u, mlp.act, stream);
    matmul_w4a16(mlp.act, d, out, stream);
}

void matmul_w8a8_i32(const Tensor& x, const Tensor& w_int8, Tensor& out, hipStream_t stream) {
    require(x.dtype() == DType::Int8, "matmul_w8a8_i32 x must be int8");
    require(w_int8.dtype() == DType::Int8, "matmul_w8a8_i32 w must be int8");
    require(out.dtype() == DType::Int32, "matmul_w8a8_i32 out must be int32");
    require(x.shape().size() == 2, "matmul_w8a8_i32 x must be [M, K]");
    require(w_int8.shape().size() == 2 && w_int8.shape()[0] == x.shape()[1], "matmul_w8a8_i32 w must be [K, N]");
    require(out.shape() == std::vector<int64_t>{x.shape()[0], w_int8.shape()[1]}, "matmul_w8a8_i32 out must be [M, N]");
    check_mcv(mcv_w8a8_gemm_i32(static_cast<const int8_t*>(x.data()), x.shape()[0], x.shape()[1], w_int8.shape()[1],
                                static_cast<const int8_t*>(w_int8.data()), MCV_W8_KN, static_cast<int32_t*>(out.data()),
                                stream),
              "matmul_w8a8_i32");
}

void matmul_w8a8_i32(const Tensor& x, const W8A8QuantizedWeight& w, Tensor& out, hipStream_t stream) {
    require(x.dtype() == DType::Int8 && out.dtype() == DType::Int32, "matmul_w8a8_i32 needs int8 x and int32 out");
    require(x.shape().size() == 2 && x.shape()[1] == w.K, "matmul_w8a8_i32 x must be [M, K]");
    require(out.shape() == std::vector<int64_t>{x.shape()[0], w.N}, "matmul_w8a8_i32 out must be [M, N]");
    require(w.w_int8.data() != nullptr, "matmul_w8a8_i32 weight is not loaded");
    check_mcv(mcv_w8a8_gemm_i32(static_cast<const int8_t*>(x.data()), x.shape()[0], w.K, w.N,
                                static_cast<const int8_t*>(w.w_int8.data()), w.layout, static_cast<int32_t*>(out.data()),
                                stream),
              "matmul_w8a8_i32");
}

void w8a8_quantize(const Tensor& x, Tensor& x_int8, Tensor& x_scale, hipStream_t stream) {
    require(x.dtype() == DType::Float16, "w8a8_quantize x must be fp16");
    require(x_int8.dtype() == DType::Int8, "w8a8_quantize x_int8 must be int8");
    require(x.shape().size() == 2, "w8a8_quantize x must be [M, K]");
    require(x_int8.shape() == x.shape(), "w8a8_quantize x_int8 must match x shape");
    const int64_t M = x.shape()[0], K = x.shape()[1];
    require(static_cast<int64_t>(x_scale.numel()) == M, "w8a8_quantize x_scale must be [M] ([1] for M = 1)");
    const bool f32 = x_scale.dtype() == DType::Float32;
    require(f32 || x_scale.dtype() == DType::Float16, "w8a8_quantize x_scale must be fp16 or fp32");
    check_mcv(mcv_w8a8_quantize_act(x.data(), M, K, static_cast<int8_t*>(x_int8.data()),
                                    f32 ? static_cast<float*>(x_scale.data()) : nullptr, f32 ? nullptr : x_scale.data(),
                                    stream),
              "w8a8_quantize");
}

void rms_norm_w8a8_quantize(const Tensor& x, const Tensor& gamma, double epsilon, Tensor* normed, Tensor& x_int8,
                            Tensor& x_scale, hipStream_t stream) {
    require(x.dtype() == DType::Float16 && gamma.dtype() == DType::Float16, "rms_norm_w8a8_quantize needs fp16 x, gamma");
    require(x.shape().size() == 2, "rms_norm_w8a8_quantize x must be [M, H]");
    const int64_t M = x.shape()[0], H = x.shape()[1];
    require(static_cast<int64_t>(gamma.numel()) == H, "rms_norm_w8a8_quantize gamma must be [H]");
    require(!normed || (normed->dtype() == DType::Float16 && normed->shape() == x.shape()),
            "rms_norm_w8a8_quantize normed must be fp16 [M, H]");
    require(x_int8.dtype() == DType::Int8 && x_int8.shape() == x.shape(), "rms_norm_w8a8_quantize x_int8 must be int8 [M, H]");
    require(static_cast<int64_t>(x_scale.numel()) == M, "rms_norm_w8a8_quantize x_scale must be [M]");
    const bool f32 = x_scale.dtype() == DType::Float32;
    require(f32 || x_scale.dtype() == DType::Float16, "rms_norm_w8a8_quantize x_scale must be fp16 or fp32");
    check_mcv(mcv_rms_norm_w8a8_quantize(x.data(), gamma.data(), M, H, epsilon, normed ? normed->data() : nullptr,
                                         static_cast<int8_t*>(x_int8.data()),
                                         f32 ? static_cast<float*>(x_scale.data()) : nullptr,
                                         f32 ? nullptr : x_scale.data(), stream),
              "rms_norm_w8a8_quantize");
}

DecodeMlpW8A8 make_decode_mlp_w8a8(const W8A8QuantizedWeight& gate, const W8A8QuantizedWeight& up,
                                   const W8A8QuantizedWeight& down, bool f32_scales) {
    require(up.K == gate.K && up.N == gate.N, "decode MLP (W8A8) gate and up must have the same shape");
    require(down.K == gate.N && down.N == gate.K, "decode MLP (W8A8) down must be [I, H] for gate [H, I]");
    for (const W8A8QuantizedWeight* w : {&gate, &up, &down})
        require((f32_scales ? w->w_scale_f32 : w->w_scale).data() != nullptr,
                f32_scales ? "decode MLP (W8A8) needs fp32 weight scales" : "decode MLP (W8A8) needs fp16 weight scales");
    DecodeMlpW8A8 mlp;
    mlp.gate = &gate;
    mlp.up = &up;
    mlp.down = &down;
    mlp.f32_scales = f32_scales;
    const bool tiled = gate.layout == MCV_W8_TILED && up.layout == MCV_W8_TILED && down.layout == MCV_W8_TILED;
    const int64_t ws = tiled ? mcv_w8a8_mlp_workspace_bytes(gate.K, gate.N) : 0;
    mlp.one_launch = ws > 0;
    if (mlp.one_launch) {
        mlp.workspace = Tensor({ws}, DType::UInt8);
        mlp.workspace.zero();
    }
    const DType sd = f32_scales ? DType::Float32 : DType::Float16;
    mlp.xq = Tensor({1, gate.K}, DType::Int8);
    mlp.xs = Tensor({1}, sd);
    mlp.act = Tensor({1, gate.N}, DType::Float16);
    mlp.aq = Tensor({1, gate.N}, DType::Int8);
    mlp.as = Tensor({1}, sd);
    for (Tensor* t : {&mlp.xq, &mlp.xs, &mlp.act, &mlp.aq, &mlp.as}) t->allocate();
    return mlp;
}

void mlp_w8a8(const Tensor& x, DecodeMlpW8A8& mlp, Tensor& out, hipStream_t stream) {
    const W8A8QuantizedWeight &g = *mlp.gate, &u = *mlp.up, &d = *mlp.down;
    require(x.dtype() == DType::Float16 && x.shape() == std::vector<int64_t>{1, g.K},
            "decode MLP (W8A8) x must be fp16 [1, H]");
    require(out.dtype() == DType::Float16 && out.shape() == std::vector<int64_t>{1, g.K},
            "decode MLP (W8A8) out must be fp16 [1, H]");
    if (mlp.one_launch) {
        check_wait_status(mlp, stream);
        auto scales = [&](const W8A8QuantizedWeight& w) { return (mlp.f32_scales ? w.w_scale_f32 : w.w_scale).data(); };
        const int rc = mcv_w8a8_mlp(x.data(), g.K, g.N, static_cast<const int8_t*>(g.w_int8.data()), scales(g),
                                    static_cast<const int8_t*>(u.w_int8.data()), scales(u),
                                    static_cast<const int8_t*>(d.w_int8.data()), scales(d),
                                    mlp.f32_scales ? MCV_F32 : MCV_F16, out.data(), mlp.workspace.data(),
                                    mlp.status.device_word(), stream);
        if (rc != MCV_ERR_SHAPE) {
            check_mcv(rc, "mlp_w8a8");
            return;
        }
        mlp.one_launch = false;          // this shape or device cannot hold the one-launch grid
    }
    w8a8_quantize(x, mlp.xq, mlp.xs, stream);
    mlp_gate_up_silu_w8a8(mlp.xq, mlp.xs, g, u, mlp.act, stream);
    w8a8_quantize(mlp.act, mlp.aq, mlp.as, stream);
    matmul_w8a8(mlp.aq, mlp.as, d, out, stream);
}

void check_wait_status(DecodeMlpW8A8& mlp, hipStream_t stream) {
    if (mlp.status.gave_up()) raise_mlp_gave_up(mlp.workspace, mlp.status, stream, "mlp_w8a8");
}

void w8a8_dequant(const Tensor& acc, const Tensor& x_scale, const Tensor& w_scale, Tensor& out, hipStream_t stream) {
    require(acc.dtype() == DType::Int32 && out.dtype() == DType::Float16, "w8a8_dequant requires int32 acc and fp16 out");
    require(acc.shape().size() == 2, "w8a8_dequant acc must be [M, N]");
    const int64_t M = acc.shape()[0], N = acc.shape()[1];
    require(static_cast<int64_t>(x_scale.numel()) == M, "w8a8_dequant x_scale must be [M]");
    require(w_scale.shape() == std::vector<int64_t>{N}, "w8a8_dequant w_scale must be [N]");
    require(out.shape() == acc.shape(), "w8a8_dequant out must be [M, N]");
    check_mcv(mcv_w8a8_dequant(static_cast<const int32_t*>(acc.data()), x_scale.data(), scale_dtype(x_scale, "x_scale"),
                               w_scale.data(), scale_dtype(w_scale, "w_scale"), M, N, out.data(), stream),
              "w8a8_dequant");
}

void matmul_w8a8(const Tensor& x_int8, const Tensor& x_scale, const W8A8QuantizedWeight& w, Tensor& out,
                 hipStream_t stream) {
    require(x_int8.dtype() == DType::Int8 && out.dtype() == DType::Float16, "matmul_w8a8 needs int8 x and fp16 out");
    require(x_int8.shape().size() == 2 && x_int8.shape()[1] == w.K, "matmul_w8a8 x must be [M, K]");
    const int64_t M = x_int8.shape()[0];
    require(out.shape() == std::vector<int64_t>{M, w.N}, "matmul_w8a8 out must be [M, N]");
    require(static_cast<int64_t>(x_scale.numel()) == M, "matmul_w8a8 x_scale must be [M]");
    const int xs = scale_dtype(x_scale, "x_scale");
    const Tensor& ws = (xs == MCV_F32 && w.w_scale_f32.data() != nullptr) ? w.w_scale_f32 : w.w_scale;
    check_mcv(mcv_w8a8_gemm_f16(static_cast<const int8_t*>(x_int8.data()), x_scale.data(), xs, M, w.K, w.N,
                                static_cast<const int8_t*>(w.w_int8.data()), w.layout, ws.data(),
                                scale_dtype(ws, "w_scale"), out.data(), stream),
              "matmul_w8a8");
}

void matmul_w4a16_multi(const Tensor& x, const std::vector<const W4A16QuantizedWeight*>& weights,
                        const std::vector<Tensor*>& outs, hipStream_t stream) {
    require(x.dtype() == DType::Float16 && x.shape().size() == 2, "matmul_w4a16_multi x must be fp16 [M, K]");
    require(!weights.empty() && weights.size() <= 4 && weights.size() == outs.size(),
            "matmul_w4a16_multi takes 1..4 weights and as many outputs");
    for (const W4A16QuantizedWeight* w : weights) require_slab(*w, "matmul_w4a16_multi");
    const int64_t M = x.shape()[0], K = x.shape()[1];
    std::vector<mcv_w4a16_part> parts(weights.size());
    for (size_t i = 0; i < weights.size(); ++i) {
        const W4A16QuantizedWeight& w = *weights[i];
        Tensor& o = *outs[i];
        require(w.K == K, "matmul_w4a16_multi weight K must match x");
        require(o.dtype() == DType::Float16 && o.shape() == std::vector<int64_t>{M, w.N},
                "matmul_w4a16_multi out must be fp16 [M, N]");
        parts[i] = mcv_w4a16_part{w.w_int8.data(), w.scales.data(), w.zeros.data(), w.zero_bias, w.N, o.data()};
    }
    check_mcv(mcv_w4a16_gemv_multi(x.data(), M, K, parts.data(), static_cast<int>(parts.size()), stream),
              "matmul_w4a16_multi");
}

void mlp_gate_up_silu_w8a8(const Tensor& x_int8, const Tensor& x_scale, const W8A8QuantizedWeight& gate,
                           const W8A8QuantizedWeight& up, Tensor& act, hipStream_t stream) {
    require(x_int8.dtype() == DType::Int8 && act.dtype() == DType::Float16, "mlp_gate_up_silu_w8a8 needs int8 x, fp16 act");
    require(gate.K == up.K && gate.N == up.N, "mlp_gate_up_silu_w8a8 gate and up must have one shape");
    require(x_int8.shape().size() == 2 && x_int8.shape()[1] == gate.K, "mlp_gate_up_silu_w8a8 x must be [M, K]");
    const int64_t M = x_int8.shape()[0];
    require(act.shape() == std::vector<int64_t>{M, gate.N}, "mlp_gate_up_silu_w8a8 act must be [M, N]");
    require(static_cast<int64_t>(x_scale.numel()) == M, "mlp_gate_up_silu_w8a8 x_scale must be [M]");
    const int xs = scale_dtype(x_scale, "x_scale");
    const bool f32 = xs == MCV_F32 && gate.w_scale_f32.data() != nullptr && up.w_scale_f32.data() != nullptr;
    const Tensor& wsg = f32 ? gate.w_scale_f32 : gate.w_scale;
    const Tensor& wsu = f32 ? up.w_scale_f32 : up.w_scale;
    if (M <= 4 && gate.layout == MCV_W8_TILED && up.layout == MCV_W8_TILED) {
        check_mcv(mcv_w8a8_gate_up_silu(static_cast<const int8_t*>(x_int8.data()), x_scale.data(), xs, M, gate.K,
                                        gate.N, static_cast<const int8_t*>(gate.w_int8.data()), wsg.data(),
                                        static_cast<const int8_t*>(up.w_int8.data()), wsu.data(),
                                        scale_dtype(wsg, "w_scale"), act.data(), stream),
                  "mlp_gate_up_silu_w8a8");
        return;
    }
    // prefill sizes or [K, N] weights: the two fused GEMMs and silu_mul
    Tensor g({M, gate.N}, DType::Float16), u({M, gate.N}, DType::Float16);
    g.allocate();
    u.allocate();
    matmul_w8a8(x_int8, x_scale, gate, g, stream);
    matmul_w8a8(x_int8, x_scale, up, u, stream);
    silu_mul(g, u, act, stream);
}

void w4a16_dequant(const W4A16QuantizedWeight& w, Tensor* w_f16, Tensor* w_i8, hipStream_t stream) {
    require_slab(w, "w4a16_dequant");
    const std::vector<int64_t> kn{w.K, w.N};
    if (w_f16) require(w_f16->dtype() == DType::Float16 && w_f16->shape() == kn, "w4a16_dequant f16 out must be [K, N]");
    if (w_i8) require(w_i8->dtype() == DType::Int8 && w_i8->shape() == kn, "w4a16_dequant i8 out must be [K, N]");
    check_mcv(mcv_w4a16_dequant(w.w_int8.data(), w.scales.data(), w.zeros.data(), w.zero_bias, w.K, w.N,
                                w_f16 ? w_f16->data() : nullptr, w_i8 ? static_cast<int8_t*>(w_i8->data()) : nullptr,
                                stream),
              "w4a16_dequant");
}

void rms_norm(const Tensor& x, const Tensor& gamma, Tensor& out, double epsilon, hipStream_t stream) {
    require(x.dtype() == DType::Float16 && gamma.dtype() == DType::Float16 && out.dtype() == DType::Float16,
            "rms_norm requires fp16 tensors");
    require(!x.shape().empty() && out.shape() == x.shape(), "rms_norm out must match x");
    const int64_t H = x.shape().back();
    require(gamma.shape() == std::vector<int64_t>{H}, "rms_norm gamma must be [H]");
    check_mcv(mcv_rms_norm(x.data(), gamma.data(), static_cast<int64_t>(x.numel()) / H, H, epsilon, out.data(), stream),
              "rms_norm");
}

// Row-major out[M, N] = a[M, K] . B.  In rocBLAS's column-major terms that is
// out^T (N x M) = B^T (N x K) . a^T (K x M): B stored [K, N] row-major is a
// column-major N x K matrix (no transpose), B stored [N, K] needs one.
void matmul_b_transposed(const Tensor& a, const Tensor& b, Tensor& out, hipStream_t stream) {
    require(a.shape().size() == 2 && b.shape().size() == 2 && out.shape().size() == 2, "matmul tensors must be 2D");
    require(a.dtype() == DType::Float16 && b.dtype() == DType::Float16 && out.dtype() == DType::Float16,
            "matmul_b_transposed requires fp16 tensors");
    const int64_t M = a.shape()[0], K = a.shape()[1], N = out.shape()[1];
    require(out.shape()[0] == M, "matmul out rows mismatch");
    bool kn;
    if (b.shape() == std::vector<int64_t>{N, K}) kn = false;
    else if (b.shape() == std::vector<int64_t>{K, N}) kn = true;
    else throw std::runtime_error("matmul_b_transposed weight must be [N, K] or [K, N]");
    static std::mutex mu;
    static std::unordered_map<int, rocblas_handle> handles;
    rocblas_handle h;
    {
        std::lock_guard<std::mutex> lock(mu);
        int dev = 0;
        check_hip(hipGetDevice(&dev), "hipGetDevice");
        auto it = handles.find(dev);
        if (it == handles.end()) {
            rocblas_handle nh;
            if (rocblas_create_handle(&nh) != rocblas_status_success) throw std::runtime_error("rocblas_create_handle failed");
            it = handles.emplace(dev, nh).first;
        }
        h = it->second;
        if (rocblas_set_stream(h, stream) != rocblas_status_success) throw std::runtime_error("rocblas_set_stream failed");
        const float alpha = 1.0f, beta = 0.0f;
        const rocblas_status st = rocblas_gemm_ex(
            h, kn ? rocblas_operation_none : rocblas_operation_transpose, rocblas_operation_none,
            static_cast<rocblas_int>(N), static_cast<rocblas_int>(M), static_cast<rocblas_int>(K), &alpha, b.data(),
            rocblas_datatype_f16_r, static_cast<rocblas_int>(kn ? N : K), a.data(), rocblas_datatype_f16_r,
            static_cast<rocblas_int>(K), &beta, out.data(), rocblas_datatype_f16_r, static_cast<rocblas_int>(N),
            out.data(), rocblas_datatype_f16_r, static_cast<rocblas_int>(N), rocblas_datatype_f32_r,
            rocblas_gemm_algo_standard, 0, 0);
        if (st != rocblas_status_success)
            throw std::runtime_error("rocblas_gemm_ex failed with status " + std::to_string(static_cast<int>(st)));
    }
}

}  // namespace minicpmv
