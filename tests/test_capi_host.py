"""CPU tests of the C-ABI library: it loads, exports every entry point that
include/*.h declares, and its host-side functions (packers, quantisers,
validation) agree with the pinned oracle.  No kernel is launched here."""
import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

from helpers import ROOT, f16_normal, synth_w4a16, too_wide_gptq


def _declared_functions():
    names = []
    for h in sorted((ROOT / "include").glob("*.h")):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names += re.findall(r"^\s*(?:const\s+)?[a-z_0-9]+\s*\*?\s*(mcv_[a-z0-9_]+)\s*\(", text, flags=re.M)
    return sorted(set(names))


def test_library_exports_every_declared_symbol(mcv):
    names = _declared_functions()
    assert len(names) >= 20
    L = mcv.lib()
    for n in names:
        assert hasattr(L, n), n
    assert set(names) == set(mcv._SIGS), set(names) ^ set(mcv._SIGS)
    assert b"gfx950" in L.mcv_version()


def test_packed_sizes(mcv):
    assert mcv.packed_sizes(1024, 248094) == (3877 * 64 * 512, 8 * 3877 * 64 * 2, 8 * 3877 * 64 // 2)
    assert mcv.packed_sizes(1000, 64) == (0, 0, 0)


def test_layout_known_answer(mcv):
    # one nibble set at (k, n): its byte position must follow the documented formula
    K, N = 256, 136
    for (k, n, v) in [(0, 0, 1), (1, 0, 2), (2, 0, 3), (7, 5, 9), (37, 70, 15), (255, 135, 6)]:
        q = np.zeros((K, N), np.uint8)
        q[k, n] = v
        order = [0, 2, 4, 6, 1, 3, 5, 7]
        qweight = np.zeros((K, N // 8), np.uint32)
        for j in range(N // 8):
            for s in range(8):
                qweight[:, j] |= q[:, 8 * j + order[s]].astype(np.uint32) << (4 * s)
        qw, sc, zr = mcv.pack_awq(qweight.view(np.int32), np.zeros((K // 128, N // 8), np.int32),
                                  np.zeros((K // 128, N), np.uint16))
        words = qw.view(np.uint32)
        slab, lane, c, w = n // 64, n % 64, k // 32, (k % 32) // 8
        slot = [0, 4, 1, 5, 2, 6, 3, 7][k % 8]
        idx = ((slab * (K // 32) + c) * 64 + lane) * 4 + w
        assert words[idx] == v << (4 * slot)
        assert np.count_nonzero(words) == 1


def test_awq_pack_roundtrip_vs_oracle(mcv, oracle):
    rng = np.random.default_rng(20)
    for K, N in [(128, 8), (256, 64), (384, 200), (1024, 520)]:
        _, qweight, qzeros, scales = synth_w4a16(rng, K, N)
        qw, sc, zr = mcv.pack_awq(qweight, qzeros, scales)
        q, zeff, s = mcv.unpack(qw, sc, zr, 0, K, N)
        w8 = q.astype(np.int16) - np.repeat(zeff, 128, axis=0).astype(np.int16)
        assert np.array_equal(w8.astype(np.int8), oracle.unpack_awq(qweight, qzeros))
        assert np.array_equal(s, scales)
        npad = -(-N // 64) * 64
        assert (sc.reshape(K // 128, npad)[:, N:] == 0).all()


def test_gptq_pack_roundtrip_vs_oracle(mcv, oracle):
    rng = np.random.default_rng(21)
    K, N, G = 384, 72, 3
    qweight = rng.integers(0, 2**32, (K // 8, N), dtype=np.uint64).astype(np.uint32).view(np.int32)
    qzeros = rng.integers(0, 2**32, (G, N // 8), dtype=np.uint64).astype(np.uint32).view(np.int32)
    scales = f16_normal(rng, (G, N), 0.01)
    g_idx = (np.arange(K) // 128).astype(np.int32)
    qw, sc, zr = mcv.pack_gptq(qweight, qzeros, g_idx, scales)
    q, zeff, s = mcv.unpack(qw, sc, zr, 1, K, N)
    w8 = q.astype(np.int16) - np.repeat(zeff, 128, axis=0).astype(np.int16)
    assert np.array_equal(w8.astype(np.int8), oracle.unpack_gptq(qweight, qzeros, g_idx, G))
    assert zeff.min() >= 1 and zeff.max() <= 16
    # g_idx omitted is the same as trivial g_idx
    qw2, _, _ = mcv.pack_gptq(qweight, qzeros, None, scales)
    assert np.array_equal(qw, qw2)


def _gptq_words(rng, K, N, G, qmax, zlo, zhi):
    """GPTQ v1 tensors with nibbles in [0, qmax] and stored zeros in [zlo, zhi]."""
    qn = rng.integers(0, qmax + 1, (K, N)).astype(np.uint32)
    qweight = np.zeros((K // 8, N), np.uint32)
    for i in range(8):
        qweight |= qn[i::8] << (4 * i)
    zn = rng.integers(zlo, zhi + 1, (G, N)).astype(np.uint32)
    qzeros = np.zeros((G, N // 8), np.uint32)
    for s in range(8):
        qzeros |= zn[:, s::8] << (4 * s)
    return qweight.view(np.int32), qzeros.view(np.int32)


def _slab_w8(mcv, qw, sc, zr, K, N):
    q, zeff, s = mcv.unpack(qw, sc, zr, 1, K, N)
    return (q.astype(np.int16) - np.repeat(zeff, 128, axis=0).astype(np.int16)).astype(np.int8), s


def test_gptq_act_order_symmetric(mcv, oracle):
    # sym=True checkpoints store zero 7 everywhere: act-order changes no value,
    # and the packed nibbles equal those of the trivial g_idx
    rng = np.random.default_rng(24)
    K, N, G = 512, 72, 4
    qweight, qzeros = _gptq_words(rng, K, N, G, 15, 7, 7)
    scales = f16_normal(rng, (G, N), 0.01)
    g_idx = rng.permutation(np.arange(K) // 128).astype(np.int32)
    qw, sc, zr = mcv.pack_gptq(qweight, qzeros, g_idx, scales)
    w8, s = _slab_w8(mcv, qw, sc, zr, K, N)
    assert np.array_equal(w8, oracle.unpack_gptq(qweight, qzeros, g_idx, G))
    assert np.array_equal(s, scales)          # scales stay with group k / 128, as in the reference
    qw2, _, zr2 = mcv.pack_gptq(qweight, qzeros, None, scales)
    assert np.array_equal(qw, qw2) and np.array_equal(zr, zr2)


def test_gptq_act_order_rebased(mcv, oracle):
    # zeros that differ between the groups a 128-row block draws from: every
    # (block, column) is re-based on one common zero, the int8 values exact
    rng = np.random.default_rng(25)
    K, N, G = 1024, 136, 8
    qweight, qzeros = _gptq_words(rng, K, N, G, 12, 5, 8)       # w8 = q - zero in [-9, 6]: 16 levels
    scales = f16_normal(rng, (G, N), 0.01)
    for g_idx in (rng.permutation(np.arange(K) // 128), np.arange(K) % G, (np.arange(K) * 7 // K) % G):
        g_idx = g_idx.astype(np.int32)
        qw, sc, zr = mcv.pack_gptq(qweight, qzeros, g_idx, scales)
        w8, s = _slab_w8(mcv, qw, sc, zr, K, N)
        assert np.array_equal(w8, oracle.unpack_gptq(qweight, qzeros, g_idx, G))
        assert np.array_equal(s, scales)


def test_gptq_act_order_too_wide_dense(mcv, oracle):
    # blocks whose values span more than 16 levels: the slab packer refuses
    # them (MCV_ERR_UNSUPPORTED), and the dense fp16 weight the loaders then
    # use is RNE((q - zero[g_idx[k]]) * scale[k/128]) bit for bit
    rng = np.random.default_rng(26)
    K, N = 512, 72
    qweight, qzeros, g_idx = too_wide_gptq(rng, K, N)
    scales = f16_normal(rng, (K // 128, N), 0.01)
    with pytest.raises(mcv.McvError, match="levels") as e:
        mcv.pack_gptq(qweight, qzeros, g_idx, scales)
    assert e.value.status == mcv.MCV_ERR_UNSUPPORTED
    w8 = oracle.unpack_gptq(qweight, qzeros, g_idx, K // 128)
    assert w8.min() < -8 and w8.max() > 8                    # more than 16 levels in use
    want = (w8.astype(np.float32) * np.repeat(oracle.h2f(scales), 128, axis=0)).astype(np.float16).view(np.uint16)
    assert np.array_equal(mcv.dequant_gptq(qweight, qzeros, g_idx, scales), want)
    # without g_idx (or a trivial one) the same function gives the in-order values
    w8t = oracle.unpack_gptq(qweight, qzeros, (np.arange(K) // 128).astype(np.int32), K // 128)
    want_t = (w8t.astype(np.float32) * np.repeat(oracle.h2f(scales), 128, axis=0)).astype(np.float16).view(np.uint16)
    assert np.array_equal(mcv.dequant_gptq(qweight, qzeros, None, scales), want_t)


def test_gptq_g_idx_out_of_range(mcv):
    K, N = 256, 8
    g_idx = (np.arange(K) // 128).astype(np.int32)
    g_idx[7] = 2
    with pytest.raises(mcv.McvError, match="out of range"):
        mcv.pack_gptq(np.zeros((K // 8, N), np.int32), np.zeros((2, 1), np.int32), g_idx,
                      np.zeros((2, N), np.uint16))


def test_product_quantizer_matches_oracle(mcv, oracle):
    rng = np.random.default_rng(22)
    for K, N in [(128, 8), (256, 136), (1024, 1000)]:
        w = f16_normal(rng, (K, N), 0.02)
        w[:, 1] = 0
        for nt in (1, 4):
            a = mcv.quantize_int4(w, nthreads=nt)
            b = oracle.quantize_int4_awq(w)
            for x, y in zip(a, b):
                assert np.array_equal(x.view(np.uint8), y.view(np.uint8))


def test_w8a8_host_quantizer_matches_oracle(mcv, oracle):
    rng = np.random.default_rng(23)
    w = f16_normal(rng, (320, 96), 0.02)
    w[:, 7] = 0
    q_o, s32_o, s16_o = oracle.w8a8_quantize_weight(w)
    q, s32, s16 = mcv.quantize_w8a8_weight_host(w, mcv.W8_KN)
    assert np.array_equal(q, q_o) and np.array_equal(s32.view(np.uint32), s32_o.view(np.uint32))
    assert np.array_equal(s16, s16_o)
    qt, _, _ = mcv.quantize_w8a8_weight_host(w, mcv.W8_NK)
    assert np.array_equal(qt, q_o.T)
    qtile, _, _ = mcv.quantize_w8a8_weight_host(w, mcv.W8_TILED)
    assert np.array_equal(qtile, mcv.pack_w8a8_tiled(q_o))


def test_quantisers_non_finite(mcv, oracle):
    """Inf and NaN weights.  W8A8: max|w| skips NaN (the reference's std::max
    keeps the running value), an inf makes the scale inf and its inverse 0,
    so the channel quantises to 0, and a NaN product quantises to 0 (what the
    reference's undefined float-to-int8 cast gives on aarch64 and x86-64).
    Int4: a group holding an inf has scale inf and zero point 0 and every
    nibble 0 (inf / inf = NaN -> 0).  Product and oracle agree bit for bit."""
    rng = np.random.default_rng(31)
    K, N = 256, 64
    w = f16_normal(rng, (K, N), 0.02)
    inf, ninf, nan = np.uint16(0x7C00), np.uint16(0xFC00), np.uint16(0x7E00)
    w[5, 3], w[130, 9], w[7, 11], w[0, 12] = inf, ninf, nan, nan
    q_o, s32_o, s16_o = oracle.w8a8_quantize_weight(w)
    for layout in (mcv.W8_KN, mcv.W8_TILED):
        q, s32, s16 = mcv.quantize_w8a8_weight_host(w, layout)
        assert np.array_equal(q, q_o if layout == mcv.W8_KN else mcv.pack_w8a8_tiled(q_o))
        assert np.array_equal(s32.view(np.uint32), s32_o.view(np.uint32)) and np.array_equal(s16, s16_o)
    assert np.all(q_o[:, 3] == 0) and np.all(q_o[:, 9] == 0)
    assert np.isinf(s32_o[3]) and s16_o[3] == 0x7C00
    finite = w[:, 11].copy()
    finite[7] = 0
    want = oracle.w8a8_quantize_weight(np.ascontiguousarray(np.stack([finite] * 8, 1)))
    assert q_o[7, 11] == 0 and np.array_equal(q_o[:, 11], want[0][:, 0]) and s32_o[11] == want[1][0]
    # bf16 values beyond the fp16 range load as inf (weights.cpp:25-33)
    bf = np.full((N, K), 0x3C00, np.uint16)                      # 2^-7
    bf[2, 17] = 0x4780                                          # 65536.0 -> fp16 inf
    qb, sb, _ = mcv.quantize_w8a8_weight_nk_host(bf, mcv.SRC_BF16, mcv.W8_KN)
    assert np.all(qb[:, 2] == 0) and np.isinf(sb[2]) and np.all(qb[:, 3] == 127)
    a = mcv.quantize_int4(w)
    b = oracle.quantize_int4_awq(w)
    for x, y in zip(a, b):
        assert np.array_equal(x.view(np.uint8), y.view(np.uint8))
    qweight, qzeros, scales = a
    shifts = 4 * np.arange(8, dtype=np.uint32)
    order = [0, 2, 4, 6, 1, 3, 5, 7]                            # AutoAWQ column order in a word
    q_kn = np.zeros((K, N), np.uint32)
    q_kn.reshape(K, N // 8, 8)[:, :, order] = (qweight.view(np.uint32)[:, :, None] >> shifts) & 15
    z_gn = np.zeros((K // 128, N), np.uint32)
    z_gn.reshape(K // 128, N // 8, 8)[:, :, order] = (qzeros.view(np.uint32)[:, :, None] >> shifts) & 15
    for g, n in [(0, 3), (1, 9)]:                               # the groups holding +inf / -inf
        assert scales[g, n] == 0x7C00 and z_gn[g, n] == 0
        assert np.all(q_kn[g * 128:(g + 1) * 128, n] == 0)
    assert q_kn[7, 11] == 0 and q_kn[0, 12] == 0                 # the NaN elements
    assert np.all(np.isfinite(scales[:, 11].view(np.float16)))


def _tiled_reference(q_kn):
    """MCV_W8_TILED restated from its definition in include/mcv_quant.h: pad
    to 64 columns / 128 k, then [slab][k-block of 32][half of 32 columns]
    [lane = column%32 + 32 * (k%32 >= 16)][k%16]."""
    K, N = q_kn.shape
    Np, Kp = -(-N // 64) * 64, -(-K // 128) * 128
    p = np.zeros((Kp, Np), np.int8)
    p[:K, :N] = q_kn
    # k = 32 kb + 16 kh + b ; n = 64 s + 32 j + c
    t = p.reshape(Kp // 32, 2, 16, Np // 64, 2, 32)          # kb, kh, b, s, j, c
    t = t.transpose(3, 0, 4, 1, 5, 2)                         # s, kb, j, kh, c, b
    return np.ascontiguousarray(t).reshape(-1)


@pytest.mark.parametrize("K,N", [(128, 64), (1024, 3584), (16, 80), (1040, 208), (256, 1)])
def test_w8a8_tiled_layout(mcv, K, N):
    rng = np.random.default_rng(K + N)
    q = rng.integers(-128, 128, (K, N)).astype(np.int8)
    tiled = mcv.pack_w8a8_tiled(q)
    assert tiled.nbytes == mcv.w8a8_tiled_bytes(K, N) == (-(-N // 64) * 64) * (-(-K // 128) * 128)
    assert np.array_equal(tiled, _tiled_reference(q))
    # a hand-placed known answer: w[k=17][n=70] sits in slab 1, k-block 0,
    # half 0, lane 6 + 32, byte 1
    q2 = np.zeros((128, 128), np.int8)
    q2[17, 70] = 5
    t2 = mcv.pack_w8a8_tiled(q2)
    off = ((((1 * 4 + 0) * 2 + 0) * 64) + 38) * 16 + 1
    assert t2[off] == 5 and np.count_nonzero(t2) == 1


def test_validation_errors_without_device(mcv):
    L = mcv.lib()
    # null pointers and bad shapes are rejected on the host before any HIP call
    assert L.mcv_w4a16_gemm(None, 1, 1024, 64, None, None, None, 0, None, None) == 1
    assert b"null" in L.mcv_last_error()
    fake = ctypes.c_void_p(0x1000)
    assert L.mcv_w4a16_gemv(fake, 1, 1000, 64, fake, fake, fake, 0, fake, None) == 2
    assert b"multiple of 128" in L.mcv_last_error()
    assert L.mcv_w4a16_gemv(fake, 1, 1024, 64, fake, fake, fake, 2, fake, None) == 1
    assert L.mcv_w8a8_gemm_i32(fake, 1, 1000, 64, fake, 0, fake, None) == 2        # K % 16
    assert L.mcv_w8a8_gemm_i32(fake, 1, 1024, 72, fake, 0, fake, None) == 2        # [K,N] needs N % 16
    assert L.mcv_w4a16_gemv_tiled_i8(fake, 1024, 3584, 450, 0, fake, fake, fake, None) == 2
    assert b"tile_len" in L.mcv_last_error()
    assert L.mcv_silu_mul(fake, fake, fake, 0, None) == 2
    # the fused and multi-part entry points validate on the host too
    assert L.mcv_w4a16_gemv_multi(fake, 1, 1024, fake, 0, None) == 1
    assert b"parts" in L.mcv_last_error()
    assert L.mcv_w4a16_gemv_multi(fake, 1, 1024, None, 2, None) == 1
    parts = (mcv._W4Part * 2)(mcv._W4Part(0x1000, 0x1000, 0x1000, 0, 64, 0x1000),
                              mcv._W4Part(0x1000, 0x1000, 0x1000, 0, 64, None))
    assert L.mcv_w4a16_gemv_multi(fake, 1, 1024, ctypes.cast(parts, ctypes.c_void_p), 2, None) == 1
    assert b"null out" in L.mcv_last_error()
    assert L.mcv_w4a16_gemv_multi(fake, 1, 1000, ctypes.cast(parts, ctypes.c_void_p), 1, None) == 2
    assert L.mcv_w8a8_gate_up_silu(fake, fake, 0, 5, 1024, 64, fake, fake, fake, fake, 0, fake, None) == 2
    assert b"M must be 1..4" in L.mcv_last_error()
    assert L.mcv_w8a8_gate_up_silu(fake, fake, 0, 1, 1024, 64, fake, fake, None, fake, 0, fake, None) == 1
    assert L.mcv_rms_norm_w8a8_quantize(fake, fake, 1, 1024, 1e-6, None, None, None, None, None) == 1
    assert L.mcv_rms_norm_w8a8_quantize(fake, fake, 0, 1024, 1e-6, None, fake, fake, None, None) == 2
    assert L.mcv_w4a16_gate_up_silu(fake, 1, 1024, 64, fake, fake, fake, 0, fake, fake, fake, 2, fake, None) == 1
    # the one-launch decode MLP: workspace size, shapes, pointers, alignment
    assert L.mcv_w4a16_mlp_workspace_bytes(1024, 3584) == 4 * (64 + 1024) + 3584 * 4 + 16 * 16 * 64 * 8
    assert L.mcv_w4a16_mlp_workspace_bytes(0, 3584) == 0
    w3 = (fake, fake, fake, 0)
    assert L.mcv_w4a16_mlp(fake, 1024, 3584, *w3, *w3, *w3, fake, None, None, None) == 1
    assert b"workspace" in L.mcv_last_error()
    assert L.mcv_w4a16_mlp(fake, 1000, 3584, *w3, *w3, *w3, fake, fake, None, None) == 2
    assert L.mcv_w4a16_mlp(fake, 1024, 6144, *w3, *w3, *w3, fake, fake, None, None) == 2   # 48 groups over 16 slots
    assert b"two groups" in L.mcv_last_error()
    assert L.mcv_w4a16_mlp(fake, 1024, 3584, *w3, *w3, fake, fake, None, 0, fake, fake, None, None) == 1
    assert L.mcv_w4a16_mlp(fake, 1024, 3584, *w3, *w3, fake, fake, fake, 2, fake, fake, None, None) == 1
    assert L.mcv_w4a16_mlp(fake, 1024, 3584, *w3, *w3, *w3, fake, ctypes.c_void_p(0x1080), None, None) == 1
    # the one-launch W8A8 MLP block (scale dtype 1 = the reference's fp16 scales, 0 = fp32)
    assert L.mcv_w8a8_mlp_workspace_bytes(1024, 3584) > 3584 * 4
    assert L.mcv_w8a8_mlp_workspace_bytes(8192 + 128, 3584) == 0
    w2 = (fake, fake)
    assert L.mcv_w8a8_mlp(fake, 1024, 3584, *w2, *w2, *w2, 1, fake, None, None, None) == 1
    assert L.mcv_w8a8_mlp(fake, 1000, 3584, *w2, *w2, *w2, 1, fake, fake, None, None) == 2
    assert L.mcv_w8a8_mlp(fake, 1024, 3584, *w2, *w2, fake, None, 0, fake, fake, None, None) == 1
    assert L.mcv_w8a8_mlp(fake, 1024, 3584, *w2, *w2, *w2, 7, fake, fake, None, None) == 1
    assert b"scale_dtype" in L.mcv_last_error()
    assert L.mcv_w8a8_mlp(fake, 1024, 3584, *w2, *w2, ctypes.c_void_p(0x1008), fake, 1, fake, fake, None, None) == 1
    assert b"16-byte" in L.mcv_last_error()
    assert b"aligned" in L.mcv_last_error()


def test_device_entry_fails_loudly_without_gpu(mcv):
    from helpers import gpu_available
    if gpu_available():
        pytest.skip("a GPU is present")
    L = mcv.lib()
    fake = ctypes.c_void_p(0x1000)
    rc = L.mcv_w4a16_gemm(fake, 1, 1024, 64, fake, fake, fake, 0, fake, None)
    assert rc == 5, L.mcv_last_error()


def test_lm_head_slots_token_known_answer(mcv):
    """Host fold of the tagged slot maxima: only this call's tag counts, the
    larger fp16 key wins, ties go to the smaller column, no candidate -> 0."""
    L = mcv.lib()
    stride = 16
    slots = np.zeros(64 * stride, np.uint64)

    def key(tag, h16, n):
        k16 = (h16 | 0x8000) if not (h16 & 0x8000) else (~h16 & 0xFFFF)
        return np.uint64((tag << 40) | (k16 << 24) | (0xFFFFFF - n))

    slots[3 * stride] = key(5, 0x3C00, 100)          # 1.0 at column 100
    slots[7 * stride] = key(5, 0x3C00, 50)           # 1.0 at column 50: tie, smaller index wins
    slots[9 * stride] = key(4, 0x4000, 7)            # 2.0, but an older call's tag
    slots[11 * stride] = key(5, 0xBC00, 3)           # -1.0
    assert L.mcv_lm_head_slots_token(slots.ctypes.data, 5) == 50
    assert L.mcv_lm_head_slots_token(slots.ctypes.data, 4) == 7
    assert L.mcv_lm_head_slots_token(slots.ctypes.data, 6) == 0      # no slot carries tag 6
    empty = np.zeros(64 * stride, np.uint64)
    empty[0] = np.uint64(9 << 40)                                    # present, but no candidate
    assert L.mcv_lm_head_slots_token(empty.ctypes.data, 9) == 0
    assert L.mcv_lm_head_slots_bytes() == 64 * stride * 8
    fake = ctypes.c_void_p(0x1000)
    assert L.mcv_w4a16_lm_head_argmax_slots(fake, 1024, 1024, 1024, fake, fake, fake, 0, None, fake, 0, None) == 1
    assert b"tag" in L.mcv_last_error()
    big = 1 << 24
    assert L.mcv_w4a16_lm_head_argmax_slots(fake, 128, big, big, fake, fake, fake, 0, None, fake, 1, None) == 2


def test_w4a16_gemm_workspace_query(mcv):
    """Workspace of the K split across workgroups: none where the GEMV (few
    rows) or an unsplit tile grid (it covers most of the chip) takes the
    shape, or for an invalid K; otherwise the 4 KiB counter region plus S fp32
    partial tiles of 32 x 64 per tile, S the most ways that keep the grid
    within 256 workgroups and leave at least 7 groups per workgroup on average
    (S need not divide K/128); the kernel label names the same
    configuration."""
    L = mcv.lib()
    q = L.mcv_w4a16_gemm_workspace_bytes
    part = 32 * 64 * 4
    for (M, K, N), S in [((128, 3584, 1024), 4), ((64, 3584, 1024), 4), ((96, 3584, 2048), 2),
                         ((128, 2048, 2048), 2), ((128, 4096, 1024), 4), ((128, 2688, 1024), 3),
                         ((128, 2048, 1024), 2), ((64, 8192, 1024), 8)]:
        tiles = -(-M // 32) * -(-N // 64)
        assert q(M, K, N) == 4096 + tiles * S * part, (M, K, N)
        assert f"K split {S} ways".encode() in L.mcv_w4a16_gemm_kernel_name(M, K, N, 1)
        assert b"K split 1 ways" in L.mcv_w4a16_gemm_kernel_name(M, K, N, 0)      # no workspace: unsplit
    for shape in [(4, 1024, 1024), (32, 1024, 1024), (2048, 1024, 3584), (2048, 3584, 1024), (128, 1024, 3584), (512, 3584, 1024),
                  (128, 1024, 1024), (512, 1024, 3584), (128, 1000, 1024), (0, 1024, 1024), (128, 0, 1024)]:
        assert q(*shape) == 0, shape
    assert b"w4a16_gemv_kernel" in L.mcv_w4a16_gemm_kernel_name(4, 1024, 1024, 1)
    assert b"<128, 8, 3, 1, 1, 0>" in L.mcv_w4a16_gemm_kernel_name(2048, 1024, 3584, 1)
    # even group counts of at least 8 (64-row tiles) or 14 (32-row tiles) take two k-parts
    assert b"<64, 4, 3, 2, 2, 1>" in L.mcv_w4a16_gemm_kernel_name(2048, 3584, 1024, 1)
    assert b"<32, 2, 3, 2, 2, 1> (K split 1 ways, 256 workgroups" in L.mcv_w4a16_gemm_kernel_name(512, 3584, 1024, 1)
    assert b"<32, 2, 3, 2, 2, 1> (K split 4 ways, 256 workgroups" in L.mcv_w4a16_gemm_kernel_name(128, 3584, 1024, 1)
    assert b"<64, 4, 3, 2, 2, 1>" in L.mcv_w4a16_gemm_kernel_name(512, 1024, 3584, 1)
    assert b"<32, 2, 3, 2, 2, 1> (K split 1 ways, 224 workgroups" in L.mcv_w4a16_gemm_kernel_name(128, 1024, 3584, 1)


def test_w4a16_gemm_dispatch_builds(mcv):
    """Every configuration the GEMM dispatch picks, with and without a
    workspace, over a grid of shapes, is one the library built (the label
    says NOT BUILT otherwise, and the launch would fail)."""
    L = mcv.lib()
    seen = set()
    for K in (128, 256, 384, 1024, 1152, 2048, 2688, 3584, 4096, 8192):
        for N in (8, 64, 200, 1000, 1024, 2048, 3584, 6144, 18944):
            for M in (8, 16, 33, 48, 64, 96, 128, 192, 256, 384, 512, 768, 1024, 1536, 2048, 4096, 8192):
                for ws in (0, 1):
                    name = L.mcv_w4a16_gemm_kernel_name(M, K, N, ws).decode()
                    assert "NOT BUILT" not in name, (M, K, N, ws, name)
                    seen.add(name.split(" (")[0])
    assert any("<64, 2, 3, 2, 2, 1>" in s for s in seen) and any("<32, 2, 3, 2, 2, 1>" in s for s in seen), seen


def test_lm_head_grid_choice(mcv):
    """Slabs per workgroup by vocabulary: 16 on the full vocabulary (243
    workgroups), fewer on a GPU's share of a column split, one slab per
    workgroup once that grid fits two workgroups per CU; the workspace holds
    a 128-byte header and one key word per slab, so a workspace serves every
    V up to the one it was sized for."""
    L = mcv.lib()
    spw = L.mcv_lm_head_slabs_per_workgroup
    cases = {248094: 16, 124047: 8, 100000: 4, 62024: 4, 40000: 2, 31012: 1, 8320: 1, 4097: 1, 1: 1}
    for V, want in cases.items():
        assert spw(V) == want, V
        assert mcv.lm_head_slabs_per_workgroup(V) == want
        nslab = -(-V // 64)
        assert -(-nslab // want) >= min(nslab, 240) or want == 1
        assert L.mcv_lm_head_workspace_bytes(V) == 128 + 8 * nslab
        assert L.mcv_lm_head_workspace_bytes(V) <= L.mcv_lm_head_workspace_bytes(248094)
    assert spw(0) == 0 and spw(1 << 24) == 0


def test_w8a8_lm_head_grid_choice(mcv):
    """The one-launch W8A8 lm_head: 4 slabs per workgroup while that still
    gives >= 512 workgroups (970 on the full vocabulary), then 2, then 1; its
    keys fit the same workspace (one key word per slab)."""
    L = mcv.lib()
    spw = L.mcv_w8a8_lm_head_slabs_per_workgroup
    cases = {248094: 4, 150000: 4, 130817: 4, 130816: 2, 100000: 2, 65409: 2, 65408: 1, 31012: 1, 1: 1}
    for V, want in cases.items():
        assert spw(V) == want, V
        assert mcv.w8a8_lm_head_slabs_per_workgroup(V) == want
        nslab = -(-V // 64)
        assert want == 1 or -(-nslab // want) >= 512
        assert -(-nslab // want) <= nslab                    # one key word per workgroup fits
    assert spw(0) == 0 and spw(1 << 24) == 0


@pytest.mark.parametrize("K,N", [(1024, 3584), (200, 72), (2048, 1000)])
def test_w8a8_checkpoint_quantiser(mcv, oracle, K, N):
    """[N, K] checkpoint bits -> int8 + scales in one host pass, bit-identical
    to the reference's load (bf16 -> fp16 truncating), host transpose and
    per-channel quantiser, for fp16 and bf16 sources and every layout."""
    rng = np.random.default_rng(K + N)
    w_nk = f16_normal(rng, (N, K), 0.02)
    w_nk[3, :] = 0                                      # all-zero channel -> scale floor
    q_o, s_o, s16_o = oracle.w8a8_quantize_weight(np.ascontiguousarray(w_nk.T))
    for layout in (mcv.W8_KN, mcv.W8_NK, mcv.W8_TILED):
        q, s32, s16 = mcv.quantize_w8a8_weight_nk_host(w_nk, mcv.SRC_F16, layout)
        want = {mcv.W8_KN: q_o, mcv.W8_NK: np.ascontiguousarray(q_o.T), mcv.W8_TILED: mcv.pack_w8a8_tiled(q_o)}[layout]
        assert np.array_equal(q, want), layout
        assert np.array_equal(s32.view(np.uint32), s_o.view(np.uint32))
        assert np.array_equal(s16, s16_o)
    # bf16 source: random bf16 patterns around N(0, 0.02), plus out-of-range ones
    f = (rng.standard_normal((N, K)).astype(np.float32) * np.float32(0.02))
    bf = (f.view(np.uint32) >> 16).astype(np.uint16)
    bf[0, :4] = [0x0001, 0x8001, 0x3880, 0x387F]        # bf16 subnormal / f16-subnormal range -> signed zero
    q, s32, s16 = mcv.quantize_w8a8_weight_nk_host(bf, mcv.SRC_BF16, mcv.W8_TILED)
    as16 = np.ascontiguousarray(oracle.bf16_to_f16_trunc(bf).T)
    q_o, s_o, s16_o = oracle.w8a8_quantize_weight(as16)
    assert np.array_equal(q, mcv.pack_w8a8_tiled(q_o))
    assert np.array_equal(s32.view(np.uint32), s_o.view(np.uint32))
    assert np.array_equal(s16, s16_o)
    # pre-quantised int8 [N, K] (safetensors I8) -> tiled
    q_nk = rng.integers(-128, 128, (N, K)).astype(np.int8)
    assert np.array_equal(mcv.pack_w8a8_tiled_nk(q_nk), mcv.pack_w8a8_tiled(np.ascontiguousarray(q_nk.T)))


@pytest.mark.parametrize("V,H,N", [(1000, 256, 1024), (61, 128, 64), (4097, 384, 4160)])
def test_embedding_quantisers(mcv, oracle, V, H, N):
    """The tied embedding [V, H] as the lm_head's [H, N] projection, columns
    from V on zero: the int4 quantiser equals mcv_w4a16_quantize_host on the
    transposed, zero-padded matrix, and the int8 one the oracle's per-channel
    quantiser on it (the reference's padded chunks, language_model.cpp:
    238-270), bit for bit, from fp16 and from bf16 bits."""
    rng = np.random.default_rng(V + H)
    emb = f16_normal(rng, (V, H), 0.02)
    pad = np.zeros((H, N), np.uint16)
    pad[:, :V] = emb.T
    got = mcv.quantize_int4_embedding(emb, N)
    want = mcv.quantize_int4(pad)
    for g, w in zip(got, want):
        assert np.array_equal(g, w)
    q, s32, s16 = mcv.quantize_w8a8_embedding(emb, N, mcv.SRC_F16, mcv.W8_TILED)
    q_o, s_o, s16_o = oracle.w8a8_quantize_weight(pad)
    assert np.array_equal(q, mcv.pack_w8a8_tiled(q_o))
    assert np.array_equal(s32.view(np.uint32), s_o.view(np.uint32))
    assert np.array_equal(s16, s16_o)
    assert np.all(s32[V:] == np.float32(1e-8))                 # zero columns: the scale floor
    # bf16 bits: converted as the reference loads bf16 (truncating to fp16)
    f = rng.standard_normal((V, H)).astype(np.float32) * np.float32(0.02)
    bf = (f.view(np.uint32) >> 16).astype(np.uint16)
    as16 = oracle.bf16_to_f16_trunc(bf)
    pad16 = np.zeros((H, N), np.uint16)
    pad16[:, :V] = as16.T
    for g, w in zip(mcv.quantize_int4_embedding(bf, N, mcv.SRC_BF16), mcv.quantize_int4(pad16)):
        assert np.array_equal(g, w)
    q, s32, _ = mcv.quantize_w8a8_embedding(bf, N, mcv.SRC_BF16, mcv.W8_KN)
    q_o, s_o, _ = oracle.w8a8_quantize_weight(pad16)
    assert np.array_equal(q, q_o) and np.array_equal(s32.view(np.uint32), s_o.view(np.uint32))
