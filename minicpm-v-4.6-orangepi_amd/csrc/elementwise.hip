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

// One workgroup of 1024 threads per row.  The row is read in 16-byte loads
// (eight values), four in flight per lane, after a head of at most seven
// values up to the first 16-byte boundary; each lane keeps the best 16-bit
// key it saw and the first index holding it (a lane visits its elements in
// increasing index order, so only a strictly larger key replaces), and the
// lanes' 64-bit keys (value, then lowest index) meet through wave shuffles
// and LDS.  A single workgroup of 256 threads with one 2-byte load at a time
// took 209 us over the 248094 logits of the lm_head shape (MI355X).
constexpr int kArgThreads = 1024;
__global__ __launch_bounds__(kArgThreads) void argmax_kernel(const uint16_t* __restrict__ x, int64_t N,
                                                             int64_t* __restrict__ idx) {
    const uint16_t* xr = x + static_cast<size_t>(blockIdx.x) * N;
    const int tid = threadIdx.x;
    uint32_t bk = 0, bi = 0;                     // best 16-bit key (0: none yet) and its index
    auto visit = [&](uint32_t h, uint32_t i) {
        const uint32_t k = argmax_key16(static_cast<uint16_t>(h));
        const bool take = k > bk;
        bk = take ? k : bk;
        bi = take ? i : bi;
    };
    const int64_t head64 = static_cast<int64_t>((16u - (reinterpret_cast<uintptr_t>(xr) & 15u)) & 15u) / 2;
    const int64_t head = head64 < N ? head64 : N;
    if (tid < head) visit(xr[tid], static_cast<uint32_t>(tid));
    const uint4* __restrict__ v = reinterpret_cast<const uint4*>(xr + head);
    const int64_t nv = (N - head) / 8;
    constexpr int U = 4;
    for (int64_t j0 = tid; j0 < nv; j0 += int64_t(kArgThreads) * U) {
        uint4 q[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t j = j0 + int64_t(u) * kArgThreads;
            q[u] = j < nv ? v[j] : make_uint4(0u, 0u, 0u, 0u);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t j = j0 + int64_t(u) * kArgThreads;
            if (j >= nv) break;
            const uint32_t base = static_cast<uint32_t>(head + 8 * j);
            const uint32_t w[4] = {q[u].x, q[u].y, q[u].z, q[u].w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                visit(w[e] & 0xffffu, base + 2 * e);
                visit(w[e] >> 16, base + 2 * e + 1);
            }
        }
    }
    for (int64_t i = head + 8 * nv + tid; i < N; i += kArgThreads) visit(xr[i], static_cast<uint32_t>(i));
    unsigned long long best = wave_max_u64(bk ? argmax_key64(bk, bi) : 0ull);
    __shared__ unsigned long long wbest[kArgThreads / 64];
    if ((tid & 63) == 0) wbest[tid >> 6] = best;
    __syncthreads();
    if (tid < 64) {
        best = wave_max_u64(tid < kArgThreads / 64 ? wbest[tid] : 0ull);
        if (tid == 0) idx[blockIdx.x] = argmax_index(best);
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
    hipLaunchKernelGGL(argmax_kernel, dim3(static_cast<unsigned>(M)), dim3(kArgThreads), 0, static_cast<hipStream_t>(stream),
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
