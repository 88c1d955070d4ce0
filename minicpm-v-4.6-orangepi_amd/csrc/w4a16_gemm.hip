// w4a16_gemm.hip -- W4A16 prefill GEMM (M > 1) on fp16 MFMA, gfx950.
//
// out[M][N] = x[M][K] . W[K][N], W in the slab-64 int4 layout.  Each 128x128
// output tile walks K in steps of 64.  Per step the workgroup copies the x tile
// to LDS and dequantises the int4 tile straight from its packed 16-byte lane
// chunks into LDS as fp16 (q - z) * s -- the same correctly rounded values
// mcv_w4a16_dequant materialises -- stored n-major so both MFMA operands are
// read as 16-byte k-runs.  Four waves each own a 64x64 sub-tile computed with
// v_mfma_f32_32x32x16_f16 (fp32 accumulation).  The next step's global loads
// are issued before the current step's MFMAs so HBM latency hides behind them.
//
// The reference has no M > 1 quantised path: its prefill runs dense fp16
// aclnnMm through matmul_b_transposed (src/csrc/lib/decoder_layer.cpp:459-462,
// 656-659, 857-860; src/csrc/lib/ops.cpp:159-322).
#include "common.h"

namespace mcv {

int launch_w4a16_gemv(const void* x, int64_t M, int64_t K, int64_t N, const void* qw, const void* scales,
                      const void* zeros, int zero_bias, void* out, hipStream_t stream);

namespace {

constexpr int BM = 128, BN = 128, BK = 64;
constexpr int LDS_STRIDE = BK + 8;   // halves per LDS row: 144 B keeps 16-lane b128 reads conflict-free
constexpr int NTHREADS = 256;

__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t smask, uint32_t vmagic) {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "s"(smask), "v"(vmagic));
    return r;
}

struct TileRegs {
    uint4 a[4];      // 4 x 16 B of the x tile
    uint4 b;         // one 16-byte packed chunk: 32 k of one column
    uint32_t z;      // effective zero of that column/group
    uint32_t s;      // its fp16 scale
};

__global__ __launch_bounds__(NTHREADS) void w4a16_gemm_kernel(const uint16_t* __restrict__ x,
                                                              const uint4* __restrict__ qw,
                                                              const uint16_t* __restrict__ scales,
                                                              const uint32_t* __restrict__ zeros, uint32_t zero_bias,
                                                              uint16_t* __restrict__ out, int M, int K, int N,
                                                              int nslab) {
    __shared__ __attribute__((aligned(16))) uint16_t As[BM * LDS_STRIDE];
    __shared__ __attribute__((aligned(16))) uint16_t Bs[BN * LDS_STRIDE];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int m0 = blockIdx.y * BM;
    const int n0 = blockIdx.x * BN;
    const int C = K / kChunkK;
    const int Npad = nslab * kSlab;
    const int KT = K / BK;

    // A copy assignment: 4 passes of (row = tid/8 + 32p, 16-byte column tid%8).
    const int a_row = tid >> 3;
    const int a_col = (tid & 7) * 8;
    // B dequant assignment: column nl = (tid/128)*64 + lane, chunk (tid/64)%2 of the step.
    const int b_slab_local = tid >> 7;
    const int b_chunk = (tid >> 6) & 1;
    const int b_nl = b_slab_local * 64 + lane;
    const int b_slab = blockIdx.x * 2 + b_slab_local;
    const bool b_valid = b_slab < nslab;
    const int b_n = b_slab * kSlab + lane;

    auto load_tile = [&](int kt, TileRegs& r) {
        const int k0 = kt * BK;
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            const int row = m0 + a_row + 32 * p;
            if (row < M) r.a[p] = *reinterpret_cast<const uint4*>(x + static_cast<size_t>(row) * K + k0 + a_col);
            else r.a[p] = make_uint4(0, 0, 0, 0);
        }
        if (b_valid) {
            const int c = k0 / kChunkK + b_chunk;
            const int g = k0 / kGroup;
            r.b = qw[(static_cast<size_t>(b_slab) * C + c) * kSlab + lane];
            r.s = scales[static_cast<size_t>(g) * Npad + b_n];
            r.z = ((zeros[static_cast<size_t>(g) * (Npad >> 3) + (b_n >> 3)] >> ((b_n & 7) * 4)) & 15u) + zero_bias;
        } else {
            r.b = make_uint4(0, 0, 0, 0);
            r.s = 0;
            r.z = 0;
        }
    };

    uint32_t vmagic;
    asm("v_mov_b32 %0, 0x64006400" : "=v"(vmagic));
    const uint32_t mlo = __builtin_amdgcn_readfirstlane(0x000F000Fu);

    auto store_tile = [&](const TileRegs& r) {
#pragma unroll
        for (int p = 0; p < 4; ++p)
            *reinterpret_cast<uint4*>(&As[(a_row + 32 * p) * LDS_STRIDE + a_col]) = r.a[p];
        const half2_t zz = as_h2((0x6400u + r.z) * 0x10001u);   // half2(1024 + z)
        const half2_t ss = as_h2(r.s * 0x10001u);
        const uint32_t words[4] = {r.b.x, r.b.y, r.b.z, r.b.w};
        uint16_t* dst = &Bs[b_nl * LDS_STRIDE + b_chunk * kChunkK];
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const uint32_t q = words[w];
            uint4 o;
            // (1024 + q) - (1024 + z) is exact; one RNE multiply by s.
            o.x = as_u32((as_h2(and_or(q, mlo, vmagic)) - zz) * ss);          // k+0, k+1
            o.y = as_u32((as_h2(and_or(q >> 4, mlo, vmagic)) - zz) * ss);     // k+2, k+3
            o.z = as_u32((as_h2(and_or(q >> 8, mlo, vmagic)) - zz) * ss);     // k+4, k+5
            o.w = as_u32((as_h2(and_or(q >> 12, mlo, vmagic)) - zz) * ss);    // k+6, k+7
            *reinterpret_cast<uint4*>(dst + w * 8) = o;
        }
    };

    const int wm = (wave >> 1) * 64;   // wave sub-tile origin inside the block tile
    const int wn = (wave & 1) * 64;
    float16_t acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    TileRegs regs;
    load_tile(0, regs);
    for (int kt = 0; kt < KT; ++kt) {
        __syncthreads();
        store_tile(regs);
        __syncthreads();
        if (kt + 1 < KT) load_tile(kt + 1, regs);
#pragma unroll
        for (int ks = 0; ks < BK / 16; ++ks) {
            const int kk = ks * 16 + (lane >> 5) * 8;
            half8_t af[2], bf[2];
#pragma unroll
            for (int i = 0; i < 2; ++i)
                af[i] = *reinterpret_cast<const half8_t*>(&As[(wm + 32 * i + (lane & 31)) * LDS_STRIDE + kk]);
#pragma unroll
            for (int j = 0; j < 2; ++j)
                bf[j] = *reinterpret_cast<const half8_t*>(&Bs[(wn + 32 * j + (lane & 31)) * LDS_STRIDE + kk]);
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
    }

    // 32x32 accumulator layout: register r of lane l holds
    // row 8*(r/4) + 4*(l/32) + r%4, column l%32.
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int col = n0 + wn + 32 * j + (lane & 31);
            if (col >= N) continue;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = m0 + wm + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (row < M) out[static_cast<size_t>(row) * N + col] = f2h(acc[i][j][r]);
            }
        }
}

}  // namespace

int launch_w4a16_gemm_mfma(const void* x, int64_t M, int64_t K, int64_t N, const void* qw, const void* scales,
                           const void* zeros, int zero_bias, void* out, hipStream_t stream) {
    if (!x || !out || !qw || !scales || !zeros) return fail(MCV_ERR_INVALID_ARG, "mcv_w4a16_gemm_mfma: null pointer");
    if (zero_bias != 0 && zero_bias != 1) return fail(MCV_ERR_INVALID_ARG, "mcv_w4a16_gemm_mfma: zero_bias must be 0 or 1");
    if (K <= 0 || K % kGroup != 0 || K > (int64_t(1) << 24))
        return fail(MCV_ERR_SHAPE, "mcv_w4a16_gemm_mfma: K must be a positive multiple of 128 (K=%lld)", (long long)K);
    if (N <= 0 || N > (int64_t(1) << 30) || M <= 0 || M > (int64_t(1) << 30))
        return fail(MCV_ERR_SHAPE, "mcv_w4a16_gemm_mfma: bad M/N (M=%lld N=%lld)", (long long)M, (long long)N);
    if (ceil_div(M, BM) > 65535) return fail(MCV_ERR_SHAPE, "mcv_w4a16_gemm_mfma: M too large");
    if (reinterpret_cast<uintptr_t>(x) % 16 != 0) return fail(MCV_ERR_INVALID_ARG, "mcv_w4a16_gemm_mfma: x must be 16-byte aligned");
    int rc = require_device();
    if (rc != MCV_OK) return rc;
    const int64_t nslab = ceil_div(N, kSlab);
    hipLaunchKernelGGL(w4a16_gemm_kernel, dim3(static_cast<unsigned>(ceil_div(N, BN)), static_cast<unsigned>(ceil_div(M, BM))),
                       dim3(NTHREADS), 0, stream, static_cast<const uint16_t*>(x), static_cast<const uint4*>(qw),
                       static_cast<const uint16_t*>(scales), static_cast<const uint32_t*>(zeros),
                       static_cast<uint32_t>(zero_bias), static_cast<uint16_t*>(out), static_cast<int>(M),
                       static_cast<int>(K), static_cast<int>(N), static_cast<int>(nslab));
    return check_launch("w4a16_gemm_kernel");
}

}  // namespace mcv

using namespace mcv;

extern "C" {

int mcv_w4a16_gemm_mfma(const void* x, int64_t M, int64_t K, int64_t N, const void* qw, const void* scales,
                        const void* zeros, int zero_bias, void* out, mcv_stream_t stream) {
    return launch_w4a16_gemm_mfma(x, M, K, N, qw, scales, zeros, zero_bias, out, static_cast<hipStream_t>(stream));
}

// Decode-sized M streams the weights once per row through the GEMV; from
// 8 rows on the MFMA tile reuses each dequantised tile across 128 rows.
int mcv_w4a16_gemm(const void* x, int64_t M, int64_t K, int64_t N, const void* qw, const void* scales,
                   const void* zeros, int zero_bias, void* out, mcv_stream_t stream) {
    if (M >= 1 && M < 8)
        return launch_w4a16_gemv(x, M, K, N, qw, scales, zeros, zero_bias, out, static_cast<hipStream_t>(stream));
    return launch_w4a16_gemm_mfma(x, M, K, N, qw, scales, zeros, zero_bias, out, static_cast<hipStream_t>(stream));
}

}  // extern "C"
