"""Pins the oracle's W4A16 formula (tests/test_matmul_w4a16.cpp:217-227), its
dequantised fp16 values, and the build-defined int4 quantiser.

Checks: a float64 numpy product of the dequantised matrix; exact integer
cases whose every partial sum is representable (so any dropped term, swapped
group index or transposed operand shows as an exact mismatch); numpy's RNE
of the exact (q - z) * s; quantiser invariants.
"""
import numpy as np

from helpers import f16_normal, rel_l2


def _expand(scales_u16, K):
    return np.repeat(scales_u16.view(np.float16).astype(np.float64), 128, axis=0)[:K]


def test_matmul_vs_float64(oracle):
    rng = np.random.default_rng(4)
    M, K, N = 3, 512, 96
    x = f16_normal(rng, (M, K), 1.0)
    w8 = rng.integers(-15, 16, (K, N)).astype(np.int8)
    s = f16_normal(rng, (K // 128, N), 0.01)
    got = oracle.w4a16_matmul(x, w8, s)
    ref = x.view(np.float16).astype(np.float64) @ (w8.astype(np.float64) * _expand(s, K))
    assert rel_l2(got, ref) < 1e-6
    assert np.max(np.abs(got - ref)) < 1e-4


def test_matmul_exact_integer_groups(oracle):
    # x small integers, per-group scales 2^g: every partial sum is an exact
    # fp32 integer times a power of two, so the result is exact.
    rng = np.random.default_rng(5)
    M, K, N = 2, 512, 40
    x = rng.integers(-3, 4, (M, K)).astype(np.float16).view(np.uint16)
    w8 = rng.integers(-15, 16, (K, N)).astype(np.int8)
    g = np.arange(K // 128)
    s = np.repeat((2.0 ** g)[:, None], N, axis=1).astype(np.float16).view(np.uint16)
    s[:, 7] = np.float16(0.5).view(np.uint16)       # one column with its own scale
    got = oracle.w4a16_matmul(x, w8, s)
    xi = x.view(np.float16).astype(np.int64)
    want = np.zeros((M, N), np.float64)
    for gi in range(K // 128):
        part = xi[:, gi * 128:(gi + 1) * 128] @ w8[gi * 128:(gi + 1) * 128].astype(np.int64)
        want += part * s[gi].view(np.float16).astype(np.float64)
    assert np.array_equal(got.astype(np.float64), want)


def test_matmul_threads_bit_identical(oracle):
    rng = np.random.default_rng(6)
    x = f16_normal(rng, (1, 1024), 1.0)
    w8 = rng.integers(-15, 16, (1024, 1000)).astype(np.int8)
    s = f16_normal(rng, (8, 1000), 0.01)
    a = oracle.w4a16_matmul(x, w8, s, nthreads=1)
    b = oracle.w4a16_matmul(x, w8, s, nthreads=8)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_dequant_f16_is_rne_of_exact_product(oracle):
    rng = np.random.default_rng(7)
    K, N = 256, 64
    w8 = rng.integers(-16, 16, (K, N)).astype(np.int8)
    s = np.concatenate([f16_normal(rng, (1, N), 0.01),
                        rng.integers(1, 0x400, (1, N)).astype(np.uint16)])   # second group: subnormal scales
    got = oracle.w4a16_dequant_f16(w8, s)
    want = (w8.astype(np.float64) * _expand(s, K)).astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


def test_quantizer_invariants(oracle):
    rng = np.random.default_rng(8)
    K, N = 256, 64
    w = f16_normal(rng, (K, N), 0.02)
    w[:128, 3] = 0                                     # constant group -> floor on the range
    w[128:, 5] = np.float16(0.01).view(np.uint16)      # all-positive group -> z clamps to 0
    qweight, qzeros, scales = oracle.quantize_int4_awq(w)
    # unpack through the (separately pinned) AWQ unpacker
    w8 = oracle.unpack_awq(qweight, qzeros)
    zero_only = np.zeros_like(qweight)
    q = oracle.unpack_awq(qweight, np.zeros_like(qzeros))    # raw q (zero 0)
    assert q.min() >= 0 and q.max() <= 15
    z = q.astype(np.int64) - w8.astype(np.int64)             # per-element zero
    zg = z.reshape(2, 128, N)
    assert (zg == zg[:, :1, :]).all() and z.min() >= 0 and z.max() <= 15
    s = scales.view(np.float16).astype(np.float64)
    wf = w.view(np.float16).astype(np.float64)
    sk = np.repeat(s, 128, axis=0)
    recon = w8.astype(np.float64) * sk
    lo = wf.reshape(2, 128, N).min(axis=1)
    hi = wf.reshape(2, 128, N).max(axis=1)
    # every value within half a step of its reconstruction unless clamped
    err = np.abs(recon - wf)
    assert (err <= sk * 0.5 + 1e-9).mean() > 0.99
    # the scale is fp16 RNE of (hi - lo) / 15 (with the 1e-5 floor)
    rng_ = np.maximum((hi - lo).astype(np.float32), np.float32(1e-5))
    assert np.array_equal(scales, (rng_ / np.float32(15)).astype(np.float16).view(np.uint16))
    assert z[0, 5 + 0] >= 0 and zg[1, 0, 5] == 0
    del zero_only
