"""Pins the oracle's W8A8 pieces: quantize_i8 (quantized_weight.cpp:197-202),
the per-channel weight quantiser (:231-268), the per-row activation
quantiser (op_kernel/w8a8_quantize_custom.cpp:25-41), the exact int32 GEMM
(tests/test_matmul_w8a8_i32.cpp:40-49) and the dequant epilogue
(op_kernel/w8a8_dequant_custom.cpp:55-62, tests/test_w8a8_dequant.cpp)."""
import numpy as np
import pytest

from helpers import f16_normal


@pytest.mark.parametrize("v,inv,want", [
    (2.5, 1.0, 3), (-2.5, 1.0, -3), (0.5, 1.0, 1), (-0.5, 1.0, -1), (0.4, 1.0, 0), (-0.4, 1.0, 0),
    (127.4, 1.0, 127), (127.6, 1.0, 127), (1000.0, 1.0, 127), (-128.4, 1.0, -128), (-1000.0, 1.0, -128),
    (np.float32(0.49999997), 1.0, 1),     # v + 0.5 rounds up to 1.0 in fp32 before the truncation
    (3.0, 0.5, 2), (-3.0, 0.5, -2),       # 1.5 -> 2 (away from zero)
])
def test_quantize_i8_known_answers(oracle, v, inv, want):
    assert oracle.quantize_i8(float(v), float(inv)) == want


def test_quantize_i8_error_bound(oracle):
    rng = np.random.default_rng(9)
    for v in rng.uniform(-127, 127, 2000):
        q = oracle.quantize_i8(float(v), 1.0)
        assert abs(q - np.float32(v)) <= 0.5 + 1e-6


def test_weight_quantizer(oracle):
    rng = np.random.default_rng(10)
    K, N = 256, 48
    w = f16_normal(rng, (K, N), 0.02)
    w[:, 4] = 0                                   # all-zero column
    q, s32, s16 = oracle.w8a8_quantize_weight(w)
    wf = w.view(np.float16).astype(np.float32)
    amax = np.abs(wf).max(axis=0)
    want = np.maximum(amax / np.float32(127), np.float32(1e-8))
    assert np.array_equal(s32.view(np.uint32), want.astype(np.float32).view(np.uint32))
    assert np.array_equal(s16, oracle.f2h_trunc(s32))
    nz = amax > 0
    assert (np.abs(q[:, nz]).max(axis=0) == 127).all()
    assert (q[:, 4] == 0).all() and s32[4] == np.float32(1e-8)
    err = np.abs(q.astype(np.float64) * s32.astype(np.float64) - wf.astype(np.float64))
    assert (err <= 0.5 * s32.astype(np.float64) * (1 + 1e-5) + 1e-12).all()


def test_act_quantizer_per_row(oracle):
    rng = np.random.default_rng(11)
    x = f16_normal(rng, (5, 1024), 1.0)
    x[3] = 0
    q, s32, s16 = oracle.w8a8_quantize_act(x)
    xf = x.view(np.float16).astype(np.float32)
    want = np.maximum(np.abs(xf).max(axis=1) / np.float32(127), np.float32(1e-8))
    assert np.array_equal(s32.view(np.uint32), want.view(np.uint32))
    assert np.array_equal(s16, s32.astype(np.float16).view(np.uint16))      # RNE
    for m in range(5):
        inv = np.float32(1) / s32[m]
        for k in range(0, 1024, 97):
            assert q[m, k] == oracle.quantize_i8(float(xf[m, k]), float(inv))
    assert (q[3] == 0).all()
    assert (np.abs(q[[0, 1, 2, 4]]).max(axis=1) == 127).all()


def test_gemm_i32_exact(oracle):
    rng = np.random.default_rng(12)
    x = rng.integers(-128, 128, (7, 640)).astype(np.int8)
    w = rng.integers(-128, 128, (640, 200)).astype(np.int8)
    got = oracle.gemm_i32(x, w)
    assert np.array_equal(got, (x.astype(np.int64) @ w.astype(np.int64)).astype(np.int32))


def test_dequant_reference_vectors(oracle):
    # tests/test_w8a8_dequant.cpp:42-46 (deterministic), its f2h truncates
    N = 3584
    acc = (np.arange(N) - 1024).astype(np.int32)[None, :]
    ws16 = oracle.f2h_trunc((np.float32(0.01) + (np.arange(N) % 7).astype(np.float32) * np.float32(0.001)))
    xs16 = oracle.f2h_trunc(np.array([0.02], np.float32))
    ws = oracle.h2f(ws16)
    xs = oracle.h2f(xs16)
    got = oracle.w8a8_dequant(acc, xs, ws)
    ref = acc[0].astype(np.float32) * xs[0] * ws            # the test's reference (:58)
    assert np.max(np.abs(got.view(np.float16).astype(np.float32) - ref)) < 0.02   # its bound (:63)
    # exact: (acc * ws) * xs in fp32, then RNE
    exact = ((acc[0].astype(np.float32) * ws) * xs[0]).astype(np.float16).view(np.uint16)
    assert np.array_equal(got[0], exact)


def test_dequant_order_matters(oracle):
    # the epilogue multiplies by the channel scale first (w8a8_dequant_custom.cpp:58-59);
    # on random data the other order differs somewhere, so the exact check above discriminates
    rng = np.random.default_rng(13)
    acc = rng.integers(-2**20, 2**20, (4, 4096)).astype(np.int32)
    ws = rng.uniform(1e-4, 1e-2, 4096).astype(np.float32)
    xs = rng.uniform(1e-3, 1e-1, 4).astype(np.float32)
    got = oracle.w8a8_dequant(acc, xs, ws)
    a = ((acc.astype(np.float32) * ws[None, :]) * xs[:, None]).astype(np.float16).view(np.uint16)
    b = ((acc.astype(np.float32) * xs[:, None]) * ws[None, :]).astype(np.float16).view(np.uint16)
    assert np.array_equal(got, a)
    assert not np.array_equal(a, b)
