// elementwise.hip -- silu*mul and the greedy argmax for gfx950.
#include "common.h"

namespace mcv {
namespace {

// out = silu_mul_f16(g, u) elementwise (common.h).
__global__ __launch_bounds__(256) void silu_mul_kernel(const uint16_t* __restrict__ g, const uint16_t* __restrict__ u,
                                                       uint16_t* __restrict__ out, int64_t n) {
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x)
        out[i] = silu_mul_f16(g[i], u[i]);
}

// One workgroup per row: 64-bit keys (value, then lowest index) reduced with
// wave shuffles and LDS.
__global__ __launch_bounds__(256) void argmax_kernel(const uint16_t* __restrict__ x, int64_t N, int64_t* __restrict__ idx) {
    const uint16_t* xr = x + static_cast<size_t>(blockIdx.x) * N;
    unsigned long long best = 0ull;
    for (int64_t i = threadIdx.x; i < N; i += blockDim.x) {
        const unsigned long long k = argmax_key64(argmax_key16(xr[i]), static_cast<uint32_t>(i));
        best = k > best ? k : best;
    }
    best = wave_max_u64(best);
    __shared__ unsigned long long wbest[4];
    if ((threadIdx.x & 63) == 0) wbest[threadIdx.x >> 6] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < static_cast<int>(blockDim.x >> 6); ++w) best = wbest[w] > best ? wbest[w] : best;
        best = wbest[0] > best ? wbest[0] : best;
        idx[blockIdx.x] = argmax_index(best);
    }
}

// One workgroup per row: y = fp16((x * rstd) * gamma), rstd = 1 / sqrt(mean(x^2)
// + eps), every step an IEEE fp32 operation (row_rstd, rms_apply).
__global__ __launch_bounds__(256) void rms_norm_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ gamma,
                                                       int H, float eps, uint16_t* __restrict__ out) {
    const uint16_t* xr = x + static_cast<size_t>(blockIdx.x) * H;
    const float rstd = row_rstd(xr, H, eps);
    uint16_t* orow = out + static_cast<size_t>(blockIdx.x) * H;
    for (int i = threadIdx.x; i < H; i += blockDim.x) orow[i] = rms_apply(xr[i], rstd, gamma[i]);
}

}  // namespace
}  // namespace mcv

using namespace mcv;

extern "C" {

int mcv_silu_mul(const void* gate, const void* up, void* out, int64_t n, mcv_stream_t stream) {
    if (!gate || !up || !out) return fail(MCV_ERR_INVALID_ARG, "silu_mul: null pointer");
    if (n <= 0) return fail(MCV_ERR_SHAPE, "silu_mul: n must be positive (n=%lld)", (long long)n);
    int rc = require_device();
    if (rc != MCV_OK) return rc;
    const int64_t blocks = ceil_div(n, 256) < 4096 ? ceil_div(n, 256) : 4096;
    hipLaunchKernelGGL(silu_mul_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, static_cast<hipStream_t>(stream),
                       static_cast<const uint16_t*>(gate), static_cast<const uint16_t*>(up), static_cast<uint16_t*>(out), n);
    return check_launch("silu_mul_kernel");
}

int mcv_argmax_f16(const void* x, int64_t M, int64_t N, int64_t* idx, mcv_stream_t stream) {
    if (!x || !idx) return fail(MCV_ERR_INVALID_ARG, "argmax: null pointer");
    if (M <= 0 || N <= 0 || M > 0x7fffffff || N > 0xffffffffll)
        return fail(MCV_ERR_SHAPE, "argmax: bad shape M=%lld N=%lld", (long long)M, (long long)N);
    int rc = require_device();
    if (rc != MCV_OK) return rc;
    hipLaunchKernelGGL(argmax_kernel, dim3(static_cast<unsigned>(M)), dim3(256), 0, static_cast<hipStream_t>(stream),
                       static_cast<const uint16_t*>(x), N, idx);
    return check_launch("argmax_kernel");
}

}  // extern "C"

extern "C" int mcv_rms_norm(const void* x, const void* gamma, int64_t M, int64_t H, double eps, void* out,
                            mcv_stream_t stream) {
    if (!x || !gamma || !out) return fail(MCV_ERR_INVALID_ARG, "rms_norm: null pointer");
    if (M <= 0 || H <= 0 || M > 0x7fffffff || H > 0x7fffffff || !(eps >= 0.0))
        return fail(MCV_ERR_SHAPE, "rms_norm: bad shape M=%lld H=%lld or eps", (long long)M, (long long)H);
    int rc = require_device();
    if (rc != MCV_OK) return rc;
    hipLaunchKernelGGL(rms_norm_kernel, dim3(static_cast<unsigned>(M)), dim3(256), 0, static_cast<hipStream_t>(stream),
                       static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(gamma), static_cast<int>(H),
                       static_cast<float>(eps), static_cast<uint16_t*>(out));
    return check_launch("rms_norm_kernel");
}
