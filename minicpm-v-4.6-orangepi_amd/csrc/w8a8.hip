// w8a8.hip -- W8A8 kernels for gfx950: per-row activation quantiser, int8 MFMA
// GEMM with int32 accumulation and an optional fused fp16 dequant epilogue,
// and the standalone dequant epilogue.
//
// Replaces the NPU operators w8a8_quantize_custom, matmul_w8a8_i32_custom and
// w8a8_dequant_custom (src/csrc/custom_ops/op_kernel/*.cpp) and their host
// wrappers (src/csrc/lib/ops.cpp:1097-1210).
#include <string>

#include "common.h"

namespace mcv {

int launch_w8a8_tiled_gate_up_silu(const int8_t* xq, int64_t M, int64_t K, int64_t N, const int8_t* wg,
                                   const void* wsg, const int8_t* wu, const void* wsu, int ws16, const void* xs,
                                   int xs16, void* act, hipStream_t stream);
std::string w8a8_tiled_name(int64_t M, int64_t K, int64_t N, bool f16);
int launch_w8a8_tiled(const int8_t* xq, int64_t M, int64_t K, int64_t N, const int8_t* w, void* out, bool f16,
                      const void* xs, int xs16, const void* ws, int ws16, hipStream_t stream);
int launch_w8a8_gemv_argmax(const int8_t* xq, int64_t K, int64_t V, const int8_t* w, void* logits, const void* xs,
                            int xs16, const void* ws, int ws16, unsigned long long* keys, hipStream_t stream);
int launch_w8a8_lm_head(const void* x, int64_t K, int64_t V, const int8_t* w, const void* wscale, int ws16, int xs16,
                        void* logits, int64_t* token, void* ws, unsigned* status, hipStream_t stream);
int w8a8_lm_head_spw(int64_t nslab);
int launch_w8a8_gemm_lds_cfg(const int8_t* xq, int64_t M, int64_t K, int64_t N, const int8_t* w, void* out, bool f16,
                             const void* xs, int xs16, const void* ws, int ws16, int bm, int bn, int ns, int wr,
                             hipStream_t stream);

namespace {

// ------------------------------------------------------ activation quant --
// One workgroup per row.  scale = max|x| / 127 (floor 1e-8), inv = 1 / scale,
// q = trunc(clamp(x * inv, -128, 127) +- 0.5): the closed form of
// op_kernel/w8a8_quantize_custom.cpp:25-41 and quantized_weight.cpp:197-202,
// every operation an explicitly rounded IEEE fp32 operation (no contraction).
// Rows of up to 256 * PER elements are held in registers between the two
// passes (PER = 0: strided reloads).
template <int PER>
__global__ __launch_bounds__(256) void w8a8_quant_act_kernel(const uint16_t* __restrict__ x, int K,
                                                             int8_t* __restrict__ xq, float* __restrict__ s32,
                                                             uint16_t* __restrict__ s16) {
    const int row = blockIdx.x;
    const int t = threadIdx.x;
    const uint16_t* xr = x + static_cast<size_t>(row) * K;
    int8_t* qr = xq + static_cast<size_t>(row) * K;
    float m = 0.f;
    float scale;
    if constexpr (PER > 0) {
        uint16_t xv[PER];
#pragma unroll
        for (int j = 0; j < PER; ++j) xv[j] = t + 256 * j < K ? xr[t + 256 * j] : uint16_t(0);
#pragma unroll
        for (int j = 0; j < PER; ++j) {
            const float v = fabsf(h2f(xv[j]));                // padding contributes 0, never above the max
            m = v > m ? v : m;
        }
        scale = act_scale(row_absmax(m));
        const float inv = __fdiv_rn(1.0f, scale);
#pragma unroll
        for (int j = 0; j < PER; ++j)
            if (t + 256 * j < K) qr[t + 256 * j] = act_quant(xv[j], inv);
    } else {
        for (int k = t; k < K; k += blockDim.x) {
            const float v = fabsf(h2f(xr[k]));
            m = v > m ? v : m;
        }
        scale = act_scale(row_absmax(m));
        const float inv = __fdiv_rn(1.0f, scale);
        for (int k = t; k < K; k += blockDim.x) qr[k] = act_quant(xr[k], inv);
    }
    if (t == 0) {
        if (s32) s32[row] = scale;
        if (s16) s16[row] = f2h(scale);
    }
}

// RMSNorm and the activation quantisation in one pass over a row (the decode
// sequence rms_norm -> w8a8_quantize of decoder_layer.cpp:955-966,
// 1022-1032): the normed fp16 row is formed once, optionally stored (the
// other projections of the step still read it), and quantised from the same
// fp16 values -- bit-identical to rms_norm_kernel + w8a8_quant_act_kernel
// (same element order per thread, same reductions).  Rows of up to 256 * PER
// elements stay in registers, x and gamma loaded together up front; longer
// rows take the strided loops (PER = 0).
template <int PER>
__global__ __launch_bounds__(256) void rms_norm_quant_kernel(const uint16_t* __restrict__ x,
                                                             const uint16_t* __restrict__ gamma, int H, float eps,
                                                             uint16_t* __restrict__ normed, int8_t* __restrict__ xq,
                                                             float* __restrict__ s32, uint16_t* __restrict__ s16) {
    const int row = blockIdx.x;
    const int t = threadIdx.x;
    const uint16_t* xr = x + static_cast<size_t>(row) * H;
    uint16_t* nr = normed ? normed + static_cast<size_t>(row) * H : nullptr;
    int8_t* qr = xq + static_cast<size_t>(row) * H;
    float m = 0.f;
    float inv;
    float scale;
    if constexpr (PER > 0) {
        uint16_t xv[PER], gv[PER];
#pragma unroll
        for (int j = 0; j < PER; ++j) {
            const int i = t + 256 * j;
            xv[j] = i < H ? xr[i] : uint16_t(0);
            gv[j] = i < H ? gamma[i] : uint16_t(0);
        }
        float ss = 0.f;
#pragma unroll
        for (int j = 0; j < PER; ++j) {
            if (t + 256 * j < H) {
                const float v = h2f(xv[j]);
                ss = fmaf(v, v, ss);
            }
        }
        const float rstd = block_rstd(ss, H, eps);
#pragma unroll
        for (int j = 0; j < PER; ++j) {
            const int i = t + 256 * j;
            if (i < H) {
                xv[j] = rms_apply(xv[j], rstd, gv[j]);                  // xv now holds the normed row
                if (nr) nr[i] = xv[j];
                const float v = fabsf(h2f(xv[j]));
                m = v > m ? v : m;
            }
        }
        scale = act_scale(row_absmax(m));
        inv = __fdiv_rn(1.0f, scale);
#pragma unroll
        for (int j = 0; j < PER; ++j) {
            const int i = t + 256 * j;
            if (i < H) qr[i] = act_quant(xv[j], inv);
        }
    } else {
        const float rstd = row_rstd(xr, H, eps);
        for (int i = t; i < H; i += blockDim.x) {
            const uint16_t h = rms_apply(xr[i], rstd, gamma[i]);
            if (nr) nr[i] = h;
            const float v = fabsf(h2f(h));
            m = v > m ? v : m;
        }
        scale = act_scale(row_absmax(m));
        inv = __fdiv_rn(1.0f, scale);
        for (int i = t; i < H; i += blockDim.x) qr[i] = act_quant(rms_apply(xr[i], rstd, gamma[i]), inv);
    }
    if (t == 0) {
        if (s32) s32[row] = scale;
        if (s16) s16[row] = f2h(scale);
    }
}

// ------------------------------------------------------------- int8 GEMM --
constexpr int BM = 128, BN = 128, BK = 128;
constexpr int LST = BK + 16;   // bytes per LDS row
constexpr int NT = 256;

// 4x4 byte transpose: rows a, b, c, d (4 bytes each, columns 0..3) -> out[j]
// = (a_j, b_j, c_j, d_j).
__device__ __forceinline__ void transpose4x4(uint32_t a, uint32_t b, uint32_t c, uint32_t d, uint32_t (&o)[4]) {
    const uint32_t ab_lo = __builtin_amdgcn_perm(b, a, 0x05010400u);   // a0 b0 a1 b1
    const uint32_t ab_hi = __builtin_amdgcn_perm(b, a, 0x07030602u);   // a2 b2 a3 b3
    const uint32_t cd_lo = __builtin_amdgcn_perm(d, c, 0x05010400u);   // c0 d0 c1 d1
    const uint32_t cd_hi = __builtin_amdgcn_perm(d, c, 0x07030602u);   // c2 d2 c3 d3
    o[0] = __builtin_amdgcn_perm(cd_lo, ab_lo, 0x05040100u);           // a0 b0 c0 d0
    o[1] = __builtin_amdgcn_perm(cd_lo, ab_lo, 0x07060302u);           // a1 b1 c1 d1
    o[2] = __builtin_amdgcn_perm(cd_hi, ab_hi, 0x05040100u);
    o[3] = __builtin_amdgcn_perm(cd_hi, ab_hi, 0x07060302u);
}

// OUT_F16: fused epilogue fp16 RNE(((float)acc * ws[n]) * xs[m]); otherwise int32.
// W_KN: weight is [K][N] (the reference's layout), else [N][K].
template <bool W_KN, bool OUT_F16>
__global__ __launch_bounds__(NT) void w8a8_gemm_kernel(const int8_t* __restrict__ xq, const int8_t* __restrict__ w,
                                                       int M, int K, int N, void* __restrict__ out,
                                                       const void* __restrict__ xs, int xs16,
                                                       const void* __restrict__ ws, int ws16) {
    __shared__ __attribute__((aligned(16))) int8_t As[BM * LST];
    __shared__ __attribute__((aligned(16))) int8_t Bs[BN * LST];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int m0 = blockIdx.y * BM;
    const int n0 = blockIdx.x * BN;
    const int KT = (K + BK - 1) / BK;

    const int a_row = tid >> 3;            // + 32 p
    const int a_col = (tid & 7) * 16;
    const int b_kq = tid >> 3;             // [K][N]: k rows 4*b_kq .. +3
    const int b_nb = (tid & 7) * 16;       //          columns b_nb .. +15

    uint4 ra[4], rb[4];
    auto load_tile = [&](int kt) {
        const int k0 = kt * BK;
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            const int row = m0 + a_row + 32 * p;
            const int k = k0 + a_col;
            ra[p] = (row < M && k < K) ? *reinterpret_cast<const uint4*>(xq + static_cast<size_t>(row) * K + k)
                                       : make_uint4(0, 0, 0, 0);
        }
        if constexpr (W_KN) {
            const int n = n0 + b_nb;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int k = k0 + 4 * b_kq + r;
                rb[r] = (k < K && n < N) ? *reinterpret_cast<const uint4*>(w + static_cast<size_t>(k) * N + n)
                                         : make_uint4(0, 0, 0, 0);
            }
        } else {
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                const int n = n0 + a_row + 32 * p;
                const int k = k0 + a_col;
                rb[p] = (n < N && k < K) ? *reinterpret_cast<const uint4*>(w + static_cast<size_t>(n) * K + k)
                                         : make_uint4(0, 0, 0, 0);
            }
        }
    };
    auto store_tile = [&]() {
#pragma unroll
        for (int p = 0; p < 4; ++p) *reinterpret_cast<uint4*>(&As[(a_row + 32 * p) * LST + a_col]) = ra[p];
        if constexpr (W_KN) {
            const uint32_t r0[4] = {rb[0].x, rb[0].y, rb[0].z, rb[0].w};
            const uint32_t r1[4] = {rb[1].x, rb[1].y, rb[1].z, rb[1].w};
            const uint32_t r2[4] = {rb[2].x, rb[2].y, rb[2].z, rb[2].w};
            const uint32_t r3[4] = {rb[3].x, rb[3].y, rb[3].z, rb[3].w};
#pragma unroll
            for (int d = 0; d < 4; ++d) {
                uint32_t t[4];
                transpose4x4(r0[d], r1[d], r2[d], r3[d], t);
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    *reinterpret_cast<uint32_t*>(&Bs[(b_nb + 4 * d + j) * LST + 4 * b_kq]) = t[j];
            }
        } else {
#pragma unroll
            for (int p = 0; p < 4; ++p) *reinterpret_cast<uint4*>(&Bs[(a_row + 32 * p) * LST + a_col]) = rb[p];
        }
    };

    const int wm = (wave >> 1) * 64;
    const int wn = (wave & 1) * 64;
    int16_t_v acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;

    load_tile(0);
    for (int kt = 0; kt < KT; ++kt) {
        __syncthreads();
        store_tile();
        __syncthreads();
        if (kt + 1 < KT) load_tile(kt + 1);
#pragma unroll
        for (int ks = 0; ks < BK / 32; ++ks) {
            const int kk = ks * 32 + (lane >> 5) * 16;
            int4_t af[2], bf[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) af[i] = *reinterpret_cast<const int4_t*>(&As[(wm + 32 * i + (lane & 31)) * LST + kk]);
#pragma unroll
            for (int j = 0; j < 2; ++j) bf[j] = *reinterpret_cast<const int4_t*>(&Bs[(wn + 32 * j + (lane & 31)) * LST + kk]);
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
    }

#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int col = n0 + wn + 32 * j + (lane & 31);
            if (col >= N) continue;
            float wsv = 0.f;
            if constexpr (OUT_F16) wsv = ws16 ? h2f(static_cast<const uint16_t*>(ws)[col]) : static_cast<const float*>(ws)[col];
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = m0 + wm + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (row >= M) continue;
                if constexpr (OUT_F16) {
                    const float xsv = xs16 ? h2f(static_cast<const uint16_t*>(xs)[row]) : static_cast<const float*>(xs)[row];
                    const float v = __fmul_rn(__fmul_rn(static_cast<float>(acc[i][j][r]), wsv), xsv);
                    static_cast<uint16_t*>(out)[static_cast<size_t>(row) * N + col] = f2h(v);
                } else {
                    static_cast<int32_t*>(out)[static_cast<size_t>(row) * N + col] = acc[i][j][r];
                }
            }
        }
}

// ------------------------------------------------------- dequant epilogue --
// out = fp16 RNE(((float)acc * ws[n]) * xs[m]): op_kernel/w8a8_dequant_custom.cpp:55-62.
__global__ __launch_bounds__(256) void w8a8_dequant_kernel(const int32_t* __restrict__ acc, const void* __restrict__ xs,
                                                           int xs16, const void* __restrict__ ws, int ws16, int M, int N,
                                                           uint16_t* __restrict__ out) {
    const int n = blockIdx.x * blockDim.x + threadIdx.x;
    const int m = blockIdx.y;
    if (n >= N || m >= M) return;
    const float wsv = ws16 ? h2f(static_cast<const uint16_t*>(ws)[n]) : static_cast<const float*>(ws)[n];
    const float xsv = xs16 ? h2f(static_cast<const uint16_t*>(xs)[m]) : static_cast<const float*>(xs)[m];
    const size_t o = static_cast<size_t>(m) * N + n;
    out[o] = f2h(__fmul_rn(__fmul_rn(static_cast<float>(acc[o]), wsv), xsv));
}

int check_gemm_args(const int8_t* xq, int64_t M, int64_t K, int64_t N, const int8_t* w, int w_layout, const void* out,
                    const char* who) {
    if (!xq || !w || !out) return fail(MCV_ERR_INVALID_ARG, "%s: null pointer", who);
    if (w_layout != MCV_W8_KN && w_layout != MCV_W8_NK && w_layout != MCV_W8_TILED)
        return fail(MCV_ERR_INVALID_ARG, "%s: bad w_layout %d", who, w_layout);
    if (M <= 0 || K <= 0 || N <= 0 || M > (int64_t(1) << 30) || N > (int64_t(1) << 30) || K > (int64_t(1) << 17))
        return fail(MCV_ERR_SHAPE, "%s: bad shape M=%lld K=%lld N=%lld (K <= 131072 keeps int32 exact)", who,
                    (long long)M, (long long)K, (long long)N);
    if (K % 16 != 0) return fail(MCV_ERR_SHAPE, "%s: K must be a multiple of 16 (K=%lld)", who, (long long)K);
    if (w_layout == MCV_W8_KN && N % 16 != 0)
        return fail(MCV_ERR_SHAPE, "%s: [K, N] weights need N %% 16 == 0 (N=%lld)", who, (long long)N);
    if ((reinterpret_cast<uintptr_t>(xq) | reinterpret_cast<uintptr_t>(w)) % 16 != 0)
        return fail(MCV_ERR_INVALID_ARG, "%s: x and w must be 16-byte aligned", who);
    if (ceil_div(M, BM) > 65535) return fail(MCV_ERR_SHAPE, "%s: M too large", who);
    return MCV_OK;
}

template <bool OUT_F16>
int launch_gemm(const int8_t* xq, int64_t M, int64_t K, int64_t N, const int8_t* w, int w_layout, void* out,
                const void* xs, int xs16, const void* ws, int ws16, hipStream_t stream) {
    if (w_layout == MCV_W8_TILED) return launch_w8a8_tiled(xq, M, K, N, w, out, OUT_F16, xs, xs16, ws, ws16, stream);
    dim3 grid(static_cast<unsigned>(ceil_div(N, BN)), static_cast<unsigned>(ceil_div(M, BM)));
    if (w_layout == MCV_W8_KN)
        hipLaunchKernelGGL((w8a8_gemm_kernel<true, OUT_F16>), grid, dim3(NT), 0, stream, xq, w, (int)M, (int)K, (int)N,
                           out, xs, xs16, ws, ws16);
    else
        hipLaunchKernelGGL((w8a8_gemm_kernel<false, OUT_F16>), grid, dim3(NT), 0, stream, xq, w, (int)M, (int)K, (int)N,
                           out, xs, xs16, ws, ws16);
    return check_launch("w8a8_gemm_kernel");
}

bool dtype_ok(int d) { return d == MCV_F32 || d == MCV_F16; }

}  // namespace
}  // namespace mcv

using namespace mcv;

namespace {
thread_local std::string g_w8_kernel_name;
}

extern "C" {

const char* mcv_w8a8_gemm_kernel_name(int64_t M, int64_t K, int64_t N, int w_layout, int out_f16) {
    if (M <= 0 || K <= 0 || N <= 0) {
        g_w8_kernel_name = "none (bad shape)";
    } else if (w_layout == MCV_W8_TILED) {
        g_w8_kernel_name = w8a8_tiled_name(M, K, N, out_f16 != 0);
    } else {
        g_w8_kernel_name = std::string("w8a8_gemm_kernel<") + (w_layout == MCV_W8_KN ? "true" : "false") + ", " +
                           (out_f16 ? "true" : "false") + "> (VALU dot4, " +
                           (w_layout == MCV_W8_KN ? "[K, N]" : "[N, K]") + " weight)";
    }
    return g_w8_kernel_name.c_str();
}

int mcv_w8a8_quantize_act(const void* x, int64_t M, int64_t K, int8_t* xq, float* s32, void* s16, mcv_stream_t stream) {
    if (!x || !xq || (!s32 && !s16)) return fail(MCV_ERR_INVALID_ARG, "w8a8_quantize: null pointer");
    if (M <= 0 || K <= 0 || M > 0x7fffffff || K > 0x7fffffff)
        return fail(MCV_ERR_SHAPE, "w8a8_quantize: bad shape M=%lld K=%lld", (long long)M, (long long)K);
    int rc = require_device();
    if (rc != MCV_OK) return rc;
    auto fn = K <= 1024 ? w8a8_quant_act_kernel<4> : K <= 4096 ? w8a8_quant_act_kernel<16> : w8a8_quant_act_kernel<0>;
    hipLaunchKernelGGL(fn, dim3(static_cast<unsigned>(M)), dim3(256), 0, static_cast<hipStream_t>(stream),
                       static_cast<const uint16_t*>(x), static_cast<int>(K), xq, s32, static_cast<uint16_t*>(s16));
    return check_launch("w8a8_quant_act_kernel");
}

int mcv_rms_norm_w8a8_quantize(const void* x, const void* gamma, int64_t M, int64_t H, double eps, void* normed,
                               int8_t* xq, float* s32, void* s16, mcv_stream_t stream) {
    if (!x || !gamma || !xq || (!s32 && !s16)) return fail(MCV_ERR_INVALID_ARG, "rms_norm_w8a8_quantize: null pointer");
    if (M <= 0 || H <= 0 || M > 0x7fffffff || H > 0x7fffffff || !(eps >= 0.0))
        return fail(MCV_ERR_SHAPE, "rms_norm_w8a8_quantize: bad shape M=%lld H=%lld or eps", (long long)M, (long long)H);
    int rc = require_device();
    if (rc != MCV_OK) return rc;
    auto fn = H <= 1024 ? rms_norm_quant_kernel<4> : H <= 4096 ? rms_norm_quant_kernel<16> : rms_norm_quant_kernel<0>;
    hipLaunchKernelGGL(fn, dim3(static_cast<unsigned>(M)), dim3(256), 0, static_cast<hipStream_t>(stream),
                       static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(gamma), static_cast<int>(H),
                       static_cast<float>(eps), static_cast<uint16_t*>(normed), xq, s32, static_cast<uint16_t*>(s16));
    return check_launch("rms_norm_quant_kernel");
}

int mcv_w8a8_gemm_i32(const int8_t* xq, int64_t M, int64_t K, int64_t N, const int8_t* w, int w_layout, int32_t* acc,
                      mcv_stream_t stream) {
    int rc = check_gemm_args(xq, M, K, N, w, w_layout, acc, "matmul_w8a8_i32");
    if (rc != MCV_OK) return rc;
    if ((rc = require_device()) != MCV_OK) return rc;
    return launch_gemm<false>(xq, M, K, N, w, w_layout, acc, nullptr, 0, nullptr, 0, static_cast<hipStream_t>(stream));
}

int mcv_w8a8_gemm_f16(const int8_t* xq, const void* xs, int xs_dtype, int64_t M, int64_t K, int64_t N, const int8_t* w,
                      int w_layout, const void* ws, int ws_dtype, void* out, mcv_stream_t stream) {
    int rc = check_gemm_args(xq, M, K, N, w, w_layout, out, "matmul_w8a8");
    if (rc != MCV_OK) return rc;
    if (!xs || !ws) return fail(MCV_ERR_INVALID_ARG, "matmul_w8a8: null scale");
    if (!dtype_ok(xs_dtype) || !dtype_ok(ws_dtype)) return fail(MCV_ERR_INVALID_ARG, "matmul_w8a8: bad scale dtype");
    if ((rc = require_device()) != MCV_OK) return rc;
    return launch_gemm<true>(xq, M, K, N, w, w_layout, out, xs, xs_dtype == MCV_F16, ws, ws_dtype == MCV_F16,
                             static_cast<hipStream_t>(stream));
}

int mcv_w8a8_gemm_lds(const int8_t* xq, const void* xs, int xs_dtype, int64_t M, int64_t K, int64_t N, const int8_t* w,
                      const void* ws, int ws_dtype, void* out, int f16_out, int bm, int bn, int stages,
                      int weights_in_registers, mcv_stream_t stream) {
    int rc = check_gemm_args(xq, M, K, N, w, MCV_W8_TILED, out, "mcv_w8a8_gemm_lds");
    if (rc != MCV_OK) return rc;
    if (f16_out && (!xs || !ws)) return fail(MCV_ERR_INVALID_ARG, "mcv_w8a8_gemm_lds: null scale");
    if (f16_out && (!dtype_ok(xs_dtype) || !dtype_ok(ws_dtype)))
        return fail(MCV_ERR_INVALID_ARG, "mcv_w8a8_gemm_lds: bad scale dtype");
    if ((rc = require_device()) != MCV_OK) return rc;
    return launch_w8a8_gemm_lds_cfg(xq, M, K, N, w, out, f16_out != 0, xs, xs_dtype == MCV_F16, ws,
                                    ws_dtype == MCV_F16, bm, bn, stages, weights_in_registers,
                                    static_cast<hipStream_t>(stream));
}

int mcv_w8a8_gate_up_silu(const int8_t* xq, const void* xs, int xs_dtype, int64_t M, int64_t K, int64_t N,
                          const int8_t* w_gate, const void* ws_gate, const int8_t* w_up, const void* ws_up,
                          int ws_dtype, void* act, mcv_stream_t stream) {
    int rc = check_gemm_args(xq, M, K, N, w_gate, MCV_W8_TILED, act, "mcv_w8a8_gate_up_silu");
    if (rc != MCV_OK) return rc;
    if (!w_up || !xs || !ws_gate || !ws_up) return fail(MCV_ERR_INVALID_ARG, "mcv_w8a8_gate_up_silu: null pointer");
    if (reinterpret_cast<uintptr_t>(w_up) % 16 != 0)
        return fail(MCV_ERR_INVALID_ARG, "mcv_w8a8_gate_up_silu: weights must be 16-byte aligned");
    if (M > 4) return fail(MCV_ERR_SHAPE, "mcv_w8a8_gate_up_silu: decode entry point, M must be 1..4 (M=%lld)", (long long)M);
    if (!dtype_ok(xs_dtype) || !dtype_ok(ws_dtype)) return fail(MCV_ERR_INVALID_ARG, "mcv_w8a8_gate_up_silu: bad scale dtype");
    if ((rc = require_device()) != MCV_OK) return rc;
    return launch_w8a8_tiled_gate_up_silu(xq, M, K, N, w_gate, ws_gate, w_up, ws_up, ws_dtype == MCV_F16, xs,
                                          xs_dtype == MCV_F16, act, static_cast<hipStream_t>(stream));
}

int mcv_w8a8_gemv_argmax_partials(const int8_t* xq, const void* xs, int xs_dtype, int64_t K, int64_t N, int64_t V,
                                  const int8_t* w, const void* ws, int ws_dtype, void* logits, void* keys,
                                  mcv_stream_t stream) {
    const char* who = "mcv_w8a8_gemv_argmax_partials";
    int rc = check_gemm_args(xq, 1, K, N, w, MCV_W8_TILED, keys, who);
    if (rc != MCV_OK) return rc;
    if (!xs || !ws) return fail(MCV_ERR_INVALID_ARG, "%s: null scale", who);
    if (!dtype_ok(xs_dtype) || !dtype_ok(ws_dtype)) return fail(MCV_ERR_INVALID_ARG, "%s: bad scale dtype", who);
    if (V <= 0 || V > N) return fail(MCV_ERR_SHAPE, "%s: need 0 < V <= N (V=%lld N=%lld)", who, (long long)V, (long long)N);
    if (reinterpret_cast<uintptr_t>(keys) % 8 != 0) return fail(MCV_ERR_INVALID_ARG, "%s: keys must be 8-byte aligned", who);
    if ((rc = require_device()) != MCV_OK) return rc;
    return launch_w8a8_gemv_argmax(xq, K, V, w, logits, xs, xs_dtype == MCV_F16, ws, ws_dtype == MCV_F16,
                                   static_cast<unsigned long long*>(keys), static_cast<hipStream_t>(stream));
}

int64_t mcv_w8a8_lm_head_slabs_per_workgroup(int64_t V) {
    if (V <= 0 || V >= (int64_t(1) << 24)) return 0;
    return w8a8_lm_head_spw(ceil_div(V, kSlab));
}

int mcv_w8a8_lm_head_argmax(const void* x, int64_t K, int64_t N, int64_t V, const int8_t* w, const void* w_scale,
                            int w_scale_dtype, int x_scale_dtype, void* logits, int64_t* token, void* workspace,
                            uint32_t* status, mcv_stream_t stream) {
    const char* who = "mcv_w8a8_lm_head_argmax";
    if (!x || !w || !w_scale || !token || !workspace) return fail(MCV_ERR_INVALID_ARG, "%s: null pointer", who);
    if (!dtype_ok(w_scale_dtype) || !dtype_ok(x_scale_dtype))
        return fail(MCV_ERR_INVALID_ARG, "%s: bad scale dtype", who);
    if (K <= 0 || K > 2048 || K % 16 != 0 || N <= 0 || N > (int64_t(1) << 30))
        return fail(MCV_ERR_SHAPE, "%s: need K a multiple of 16 up to 2048 (K=%lld N=%lld)", who, (long long)K,
                    (long long)N);
    if (V <= 0 || V > N || V >= (int64_t(1) << 24))
        return fail(MCV_ERR_SHAPE, "%s: need 0 < V <= N and V < 2^24 (V=%lld N=%lld)", who, (long long)V, (long long)N);
    if (reinterpret_cast<uintptr_t>(workspace) % 128 != 0)
        return fail(MCV_ERR_INVALID_ARG, "%s: workspace must be 128-byte aligned", who);
    if (reinterpret_cast<uintptr_t>(x) % 2 != 0) return fail(MCV_ERR_INVALID_ARG, "%s: x must be 2-byte aligned", who);
    int rc = require_device();
    if (rc != MCV_OK) return rc;
    return launch_w8a8_lm_head(x, K, V, w, w_scale, w_scale_dtype == MCV_F16, x_scale_dtype == MCV_F16, logits, token,
                               workspace, status, static_cast<hipStream_t>(stream));
}

int mcv_w8a8_dequant(const int32_t* acc, const void* xs, int xs_dtype, const void* ws, int ws_dtype, int64_t M, int64_t N,
                     void* out, mcv_stream_t stream) {
    if (!acc || !xs || !ws || !out) return fail(MCV_ERR_INVALID_ARG, "w8a8_dequant: null pointer");
    if (!dtype_ok(xs_dtype) || !dtype_ok(ws_dtype)) return fail(MCV_ERR_INVALID_ARG, "w8a8_dequant: bad scale dtype");
    if (M <= 0 || N <= 0 || M > 65535 || N > 0x7fffffff)
        return fail(MCV_ERR_SHAPE, "w8a8_dequant: bad shape M=%lld N=%lld", (long long)M, (long long)N);
    int rc = require_device();
    if (rc != MCV_OK) return rc;
    hipLaunchKernelGGL(w8a8_dequant_kernel, dim3(static_cast<unsigned>(ceil_div(N, 256)), static_cast<unsigned>(M)), dim3(256),
                       0, static_cast<hipStream_t>(stream), acc, xs, xs_dtype == MCV_F16, ws, ws_dtype == MCV_F16,
                       static_cast<int>(M), static_cast<int>(N), static_cast<uint16_t*>(out));
    return check_launch("w8a8_dequant_kernel");
}

}  // extern "C"
