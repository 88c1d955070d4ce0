"""Pins the oracle's AutoAWQ / GPTQ unpackers (quantized_weight.cpp:75-160).

Known answers from hand-built words, and a vectorised numpy restatement
written from the packing description (shift-and-mask plus the column order
{0,2,4,6,1,3,5,7}) rather than from the loop.
"""
import numpy as np
import pytest

ORDER = np.array([0, 2, 4, 6, 1, 3, 5, 7])


def test_awq_known_answer(oracle):
    K, N = 128, 16
    qweight = np.full((K, N // 8), 0x76543210, np.uint32).view(np.int32)
    qzeros = np.zeros((1, N // 8), np.int32)
    w8 = oracle.unpack_awq(qweight, qzeros)
    # slot s holds value s and lands in column order[s]
    assert w8[0, :8].tolist() == [0, 4, 1, 5, 2, 6, 3, 7]
    assert (w8 == w8[0]).all()
    qzeros[:] = np.int32(0x11111111)
    assert (oracle.unpack_awq(qweight, qzeros) == w8 - 1).all()


def test_awq_vs_vectorised(oracle):
    rng = np.random.default_rng(2)
    K, N = 256, 64
    qweight = rng.integers(0, 2**32, (K, N // 8), dtype=np.uint64).astype(np.uint32).view(np.int32)
    qzeros = rng.integers(0, 2**32, (K // 128, N // 8), dtype=np.uint64).astype(np.uint32).view(np.int32)
    shifts = 4 * np.arange(8, dtype=np.uint32)
    q = (qweight.view(np.uint32)[:, :, None] >> shifts) & 15          # [K, N/8, slot]
    z = (qzeros.view(np.uint32)[:, :, None] >> shifts) & 15
    zk = np.repeat(z, 128, axis=0)
    want = np.empty((K, N), np.int64)
    cols = (np.arange(N // 8)[:, None] * 8 + ORDER[None, :])           # [N/8, slot] -> column
    want[:, cols] = q.astype(np.int64) - zk.astype(np.int64)
    assert np.array_equal(oracle.unpack_awq(qweight, qzeros), want.astype(np.int8))


def test_gptq_known_answer(oracle):
    K, N = 128, 8
    qweight = np.full((K // 8, N), 0x76543210, np.uint32).view(np.int32)
    qzeros = np.full((1, N // 8), 0x76543210, np.uint32).view(np.int32)   # column n has stored zero n
    g_idx = np.zeros(K, np.int32)
    w8 = oracle.unpack_gptq(qweight, qzeros, g_idx, 1)
    # row k = 8*k0 + i holds nibble i; zero = stored + 1
    for k in range(K):
        assert w8[k].tolist() == [(k % 8) - (n + 1) for n in range(N)]


def test_gptq_vs_vectorised_and_act_order(oracle):
    rng = np.random.default_rng(3)
    K, N, G = 256, 16, 2
    qweight = rng.integers(0, 2**32, (K // 8, N), dtype=np.uint64).astype(np.uint32).view(np.int32)
    qzeros = rng.integers(0, 2**32, (G, N // 8), dtype=np.uint64).astype(np.uint32).view(np.int32)
    for g_idx in (np.arange(K) // 128, rng.permutation(np.arange(K) // 128)):
        g_idx = g_idx.astype(np.int32)
        shifts = 4 * np.arange(8, dtype=np.uint32)
        q = ((qweight.view(np.uint32)[:, None, :] >> shifts[None, :, None]) & 15).reshape(K, N)
        zall = ((qzeros.view(np.uint32)[:, :, None] >> shifts) & 15).reshape(G, N) + 1
        want = q.astype(np.int64) - zall[g_idx].astype(np.int64)
        assert np.array_equal(oracle.unpack_gptq(qweight, qzeros, g_idx, G), want.astype(np.int8))


def test_gptq_bad_g_idx_is_an_error(oracle):
    K, N = 128, 8
    g_idx = np.zeros(K, np.int32)
    g_idx[5] = 3
    rc = oracle.unpack_gptq(np.zeros((K // 8, N), np.int32), np.zeros((1, 1), np.int32), g_idx, 1)
    assert rc == 2


def test_awq_rejects_bad_shape(oracle):
    import ctypes
    q = np.zeros((100, 1), np.int32)
    out = np.zeros((100, 8), np.int8)
    assert oracle.L.or_unpack_awq(q.ctypes.data, q.ctypes.data, 100, 8, out.ctypes.data) != 0
