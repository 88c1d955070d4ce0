"""GPU parity of the W4A16 kernels against the CPU oracle.

Bar: dequantised values bit-exact; fp16 outputs
within max_abs <= 2e-2 and rel-L2 <= 1e-3 of the reference CPU formula
(tests/test_matmul_w4a16.cpp:217-227) on the same seeded inputs; the lm_head
argmax bit-exact.  Full-size shapes that the oracle cannot finish quickly are
checked against an fp64 product of the oracle-exact dequantised weights.
"""
import numpy as np
import pytest

from helpers import f16_normal, rel_l2, synth_w4a16, too_wide_gptq

pytestmark = pytest.mark.gpu

MAX_ABS = 2e-2
REL_L2 = 1e-3


def _dev_weight(mcv, qweight, qzeros, scales):
    return mcv.W4A16QuantizedWeight.from_awq(qweight, qzeros, scales)


def _torch():
    import torch
    return torch


def _to_dev(a_u16):
    torch = _torch()
    return torch.from_numpy(np.ascontiguousarray(a_u16).view(np.int16)).cuda().view(torch.float16)


def _host_f32(t):
    return t.float().cpu().numpy()


def _case(seed, M, K, N):
    rng = np.random.default_rng(seed)
    n8 = -(-N // 8) * 8
    _, qweight, qzeros, scales = synth_w4a16(rng, K, n8)
    x = f16_normal(rng, (M, K), 1.0)
    return x, qweight, qzeros, scales, n8


def _check(got, ref, what):
    d = np.abs(got - ref)
    assert d.max() <= MAX_ABS, f"{what}: max_abs {d.max()}"
    r = rel_l2(got, ref)
    assert r <= REL_L2, f"{what}: rel_l2 {r}"
    return d.max(), r


@pytest.mark.parametrize("M,K,N", [
    (1, 1024, 1024),      # the K = N = 1024 benchmark GEMV
    (1, 1024, 3584),      # gate / up
    (1, 3584, 1024),      # down
    (1, 1024, 6144), (1, 1024, 2048), (1, 2048, 1024), (1, 1024, 4096), (1, 1024, 512), (1, 1024, 16),
    (1, 128, 8), (1, 256, 200), (1, 384, 72),       # ragged N, single-group K
    (2, 1024, 1024), (3, 512, 136), (7, 1024, 520),
], ids=lambda v: str(v))
def test_gemv_vs_oracle(mcv, oracle, cuda, M, K, N):
    x, qweight, qzeros, scales, n8 = _case(1000 + M * 7 + K + N, M, K, N)
    w = _dev_weight(mcv, qweight, qzeros, scales)
    out = mcv.matmul_w4a16_gemv(_to_dev(x), w)
    _torch().cuda.synchronize()
    ref = oracle.w4a16_matmul(x, oracle.unpack_awq(qweight, qzeros), scales)
    _check(_host_f32(out), ref, f"gemv M={M} K={K} N={N}")


def test_gemv_1024_tight(mcv, oracle, cuda):
    # the fp32-accumulating kernel is far inside the bar; a dropped group or
    # misplaced nibble would be O(1) off
    x, qweight, qzeros, scales, _ = _case(1, 1, 1024, 1024)
    w = _dev_weight(mcv, qweight, qzeros, scales)
    got = _host_f32(mcv.matmul_w4a16(_to_dev(x), w))
    ref = oracle.w4a16_matmul(x, oracle.unpack_awq(qweight, qzeros), scales)
    assert np.abs(got - ref).max() < 2e-3
    # fp16 output is the RNE of a value within a few fp32 ulps of the oracle's
    ref16 = ref.astype(np.float16).astype(np.float32)
    assert (got == ref16).mean() > 0.98


def test_dequant_bit_exact(mcv, oracle, cuda):
    rng = np.random.default_rng(2)
    for K, N in [(256, 72), (1024, 3584)]:
        _, qweight, qzeros, scales = synth_w4a16(rng, K, N)
        w = _dev_weight(mcv, qweight, qzeros, scales)
        wf, w8 = mcv.w4a16_dequant(w, f16=True, i8=True)
        _torch().cuda.synchronize()
        w8_ref = oracle.unpack_awq(qweight, qzeros)
        assert np.array_equal(w8.cpu().numpy(), w8_ref)
        assert np.array_equal(wf.cpu().view(_torch().int16).numpy().view(np.uint16),
                              oracle.w4a16_dequant_f16(w8_ref, scales))


@pytest.mark.parametrize("M,K,N", [
    # the dispatch's unsplit configurations: 32 x 128 tiles (few rows), ragged
    # M and N, one stage (fewer stages than buffers)
    (8, 1024, 3584), (128, 1024, 3584), (130, 1024, 1000), (128, 3584, 1024), (256, 256, 264),
    # 128 x 256 tiles (eight waves), ragged M and N (57 slabs: the last tile's
    # fourth slab past the end), one k stage
    (2050, 128, 3592),
    # 64 x 128 tiles, ragged M and N
    (1100, 256, 3000), (1700, 512, 1000),
], ids=lambda v: str(v))
def test_gemm_mfma_vs_oracle(mcv, oracle, cuda, M, K, N):
    x, qweight, qzeros, scales, _ = _case(3000 + M + K + N, M, K, N)
    w = _dev_weight(mcv, qweight, qzeros, scales)
    out = mcv.matmul_w4a16_mfma(_to_dev(x), w)
    _torch().cuda.synchronize()
    ref = oracle.w4a16_matmul(x, oracle.unpack_awq(qweight, qzeros), scales)
    _check(_host_f32(out), ref, f"mfma M={M} K={K} N={N}")


@pytest.mark.parametrize("M,K,N", [(512, 1024, 3584), (512, 3584, 1024), (1024, 1024, 3584), (2048, 1024, 3584),
                                   (2048, 3584, 1024)], ids=lambda v: str(v))
def test_gemm_mfma_full_size(mcv, oracle, cuda, M, K, N):
    # prefill benchmark sizes: fp64 product of the oracle-exact dequantised weights
    torch = _torch()
    x, qweight, qzeros, scales, _ = _case(4000 + M + K, M, K, N)
    w = _dev_weight(mcv, qweight, qzeros, scales)
    out = mcv.matmul_w4a16(_to_dev(x), w)
    w8 = oracle.unpack_awq(qweight, qzeros)
    wexact = torch.from_numpy(w8.astype(np.float64) * np.repeat(scales.view(np.float16).astype(np.float64), 128, 0)).cuda()
    xd = _to_dev(x).double()
    ref = (xd @ wexact).cpu().numpy()
    _check(_host_f32(out), ref, f"mfma full M={M} K={K} N={N}")


# K split across workgroups (mcv_w4a16_gemm_ws, the Python mirror's route):
# few rows and a long K leave the tile grid far below the CU count; the
# partial tiles are added inside the launch by the last workgroup of each
# tile.  K=3584 four ways at M=128, M=64 and M=96 N=2048, two at M=200,
# ragged rows and an odd N (the element-store epilogue).
@pytest.mark.parametrize("M,K,N", [(128, 3584, 1024), (64, 3584, 1024), (200, 3584, 1024), (97, 3584, 1001),
                                   (96, 3584, 2048)], ids=lambda v: str(v))
def test_gemm_split_k_vs_oracle(mcv, oracle, cuda, M, K, N):
    torch = _torch()
    x, qweight, qzeros, scales, _ = _case(6000 + M + K + N, M, K, N)
    w = _dev_weight(mcv, qweight, qzeros, scales)
    nb = int(mcv.lib().mcv_w4a16_gemm_workspace_bytes(M, w.K, w.N))           # (N padded to 8 columns)
    assert nb > 0
    xd = _to_dev(x)
    out = mcv.matmul_w4a16(xd, w)
    again = mcv.matmul_w4a16(xd, w)
    ref = oracle.w4a16_matmul(x, oracle.unpack_awq(qweight, qzeros), scales)
    _check(_host_f32(out), ref, f"split-K M={M} K={K} N={N}")
    # the partials are added in split order: the same bits on every call
    assert torch.equal(out.view(torch.int16), again.view(torch.int16))
    # a workspace one byte short runs unsplit: the MFMA kernel's own bits
    short = torch.empty(nb, dtype=torch.uint8, device="cuda")
    got = torch.empty_like(out)
    q, sc, z = w.ptrs()
    stream = torch.cuda.current_stream().cuda_stream
    assert mcv.lib().mcv_w4a16_gemm_ws(xd.data_ptr(), M, w.K, w.N, q, sc, z, w.zero_bias, got.data_ptr(),
                                       short.data_ptr(), nb - 1, stream) == 0
    assert torch.equal(got.view(torch.int16), mcv.matmul_w4a16_mfma(xd, w).view(torch.int16))
    # so does a large enough workspace that is not 16-byte aligned
    got.zero_()
    big = torch.empty(nb + 16, dtype=torch.uint8, device="cuda")
    assert mcv.lib().mcv_w4a16_gemm_ws(xd.data_ptr(), M, w.K, w.N, q, sc, z, w.zero_bias, got.data_ptr(),
                                       big.data_ptr() + 4, nb, stream) == 0
    assert torch.equal(got.view(torch.int16), mcv.matmul_w4a16_mfma(xd, w).view(torch.int16))


def test_gemm_split_k_graph_replays(mcv, cuda):
    """The split path under HIP graph capture (the capture stream's own
    zero-filled workspace, made by the call before the capture; no memset in
    the graph): every replay, with eager work and host synchronisation
    between them, gives the eager call's bits -- the tile counters are back at
    zero after every call."""
    torch = _torch()
    M, K, N = 128, 3584, 1024
    x, qweight, qzeros, scales, _ = _case(77, M, K, N)
    w = _dev_weight(mcv, qweight, qzeros, scales)
    assert int(mcv.lib().mcv_w4a16_gemm_workspace_bytes(M, w.K, w.N)) > 0
    xd = _to_dev(x)
    want = mcv.matmul_w4a16(xd, w)
    out = torch.empty_like(want)
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        mcv.matmul_w4a16(xd, w, out)                       # warm the pool on the capture stream
        with torch.cuda.graph(g, stream=s):
            mcv.matmul_w4a16(xd, w, out)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    for i in range(4):
        out.zero_()
        mcv.matmul_w4a16(_to_dev(x[: M // 2]), w)          # eager work between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), want.view(torch.int16)), f"replay {i}"


# Every built configuration of the half-slab GEMM (mcv_w4a16_gemm_sk), the
# dispatch's and the rest, against the oracle on ragged shapes, all through
# ONE zero-filled workspace (calls of different shapes and splits must leave
# its counters zero for each other), each split twice for identical bits.
SK_CONFIGS = [(128, 8, 3, 1, 1, 0), (128, 4, 3, 1, 1, 0), (64, 8, 3, 1, 1, 0), (64, 4, 3, 1, 1, 0), (32, 4, 3, 1, 1, 0),
              (64, 4, 3, 2, 1, 0), (32, 4, 3, 2, 1, 0), (64, 4, 3, 2, 2, 0), (32, 4, 3, 2, 2, 0), (128, 8, 4, 1, 1, 1),
              (64, 4, 3, 1, 1, 1), (64, 4, 3, 2, 2, 1), (64, 4, 4, 2, 2, 1), (32, 4, 3, 1, 1, 1), (32, 4, 3, 2, 1, 1),
              (32, 4, 3, 2, 2, 1), (32, 2, 3, 1, 1, 1), (32, 2, 3, 2, 2, 1), (64, 2, 3, 2, 2, 1), (32, 2, 4, 2, 2, 1),
              (128, 2, 3, 1, 1, 1), (128, 2, 2, 2, 2, 1), (64, 2, 3, 1, 1, 1)]


@pytest.mark.parametrize("M,K,N", [(200, 1024, 1000), (70, 2048, 520)], ids=lambda v: str(v))
def test_gemm_every_configuration(mcv, oracle, cuda, M, K, N):
    torch = _torch()
    L = mcv.lib()
    x, qweight, qzeros, scales, _ = _case(8000 + M + K + N, M, K, N)
    w = _dev_weight(mcv, qweight, qzeros, scales)
    xd = _to_dev(x)
    ref = oracle.w4a16_matmul(x, oracle.unpack_awq(qweight, qzeros), scales)
    ws = torch.zeros(32 << 20, dtype=torch.uint8, device="cuda")
    q, sc, z = w.ptrs()
    stream = torch.cuda.current_stream().cuda_stream
    G = K // 128
    for tm, nwv, ns, kg, kw, wr in SK_CONFIGS:
        for S in [s for s in (1, 2, 3, 4, 8, 16) if G % kg == 0 and s <= G // kg]:
            assert L.mcv_w4a16_gemm_sk_workspace_bytes(M, w.N, tm, nwv, S) <= ws.numel()
            outs = []
            for _ in range(2 if S > 1 else 1):
                out = torch.full((M, N), 7.0, dtype=torch.float16, device="cuda")
                rc = L.mcv_w4a16_gemm_sk(xd.data_ptr(), M, w.K, w.N, q, sc, z, w.zero_bias, out.data_ptr(), tm, nwv,
                                         ns, kg, kw, wr, (S + tm + nwv) % 4, S, ws.data_ptr(), ws.numel(), stream)
                assert rc == 0, L.mcv_last_error()
                outs.append(out)
            torch.cuda.synchronize()
            _check(_host_f32(outs[0]), ref, f"sk tm={tm} waves={nwv} ns={ns} kg={kg} kw={kw} wr={wr} S={S} M={M} K={K} N={N}")
            if S > 1:
                assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16)), (tm, nwv, ns, kg, kw, wr, S)
    # the counters are zero after every call
    assert int(ws[:4096].count_nonzero().item()) == 0
    # an unbuilt configuration, more splits than groups, more splits than
    # stages, two k-parts with one group per stage, a missing workspace, a bad
    # tile order: clear errors
    assert L.mcv_w4a16_gemm_sk(xd.data_ptr(), M, w.K, w.N, q, sc, z, 0, xd.data_ptr(), 96, 4, 3, 1, 1, 0, 0, 1, None, 0,
                               stream) == 1
    assert L.mcv_w4a16_gemm_sk(xd.data_ptr(), M, w.K, w.N, q, sc, z, 0, xd.data_ptr(), 32, 4, 3, 1, 1, 0, 0, G + 1,
                               ws.data_ptr(), ws.numel(), stream) == 1
    assert L.mcv_w4a16_gemm_sk(xd.data_ptr(), M, w.K, w.N, q, sc, z, 0, xd.data_ptr(), 32, 4, 3, 2, 1, 0, 0, G,
                               ws.data_ptr(), ws.numel(), stream) == 1
    assert L.mcv_w4a16_gemm_sk(xd.data_ptr(), M, w.K, w.N, q, sc, z, 0, xd.data_ptr(), 32, 4, 3, 1, 2, 0, 0, 1,
                               ws.data_ptr(), ws.numel(), stream) == 1
    assert L.mcv_w4a16_gemm_sk(xd.data_ptr(), M, w.K, w.N, q, sc, z, 0, xd.data_ptr(), 32, 4, 3, 1, 1, 0, 0, 2, None, 0,
                               stream) == 1
    assert L.mcv_w4a16_gemm_sk(xd.data_ptr(), M, w.K, w.N, q, sc, z, 0, xd.data_ptr(), 32, 4, 3, 1, 1, 0, 4, 1, None, 0,
                               stream) == 1


def test_gemv_and_mfma_agree(mcv, cuda):
    x, qweight, qzeros, scales, _ = _case(5, 8, 1024, 520)
    w = _dev_weight(mcv, qweight, qzeros, scales)
    xd = _to_dev(x)
    a = _host_f32(mcv.matmul_w4a16_gemv(xd, w))
    b = _host_f32(mcv.matmul_w4a16_mfma(xd, w))
    assert np.abs(a - b).max() < 5e-3


def test_gptq_zero_bias(mcv, oracle, cuda):
    rng = np.random.default_rng(6)
    K, N, G = 1024, 520, 8
    qweight = rng.integers(0, 2**32, (K // 8, N), dtype=np.uint64).astype(np.uint32).view(np.int32)
    # stored zeros 6..9 keep (q - zero) in the usual range
    zn = rng.integers(6, 10, (G, N))
    qzeros = np.zeros((G, N // 8), np.uint32)
    for s in range(8):
        qzeros |= zn[:, s::8].astype(np.uint32) << (4 * s)
    qzeros = qzeros.view(np.int32)
    scales = f16_normal(rng, (G, N), 0.002)
    g_idx = (np.arange(K) // 128).astype(np.int32)
    w = mcv.W4A16QuantizedWeight.from_gptq(qweight, qzeros, g_idx, scales)
    assert w.zero_bias == 1
    w8 = oracle.unpack_gptq(qweight, qzeros, g_idx, G)
    for M in (1, 64):
        x = f16_normal(rng, (M, K), 1.0)
        out = _host_f32(mcv.matmul_w4a16(_to_dev(x), w))
        _check(out, oracle.w4a16_matmul(x, w8, scales), f"gptq M={M}")
    _, w8_dev = mcv.w4a16_dequant(w, f16=False, i8=True)
    assert np.array_equal(w8_dev.cpu().numpy(), w8)


def test_gptq_act_order(mcv, oracle, cuda):
    # act-order g_idx: row k's zero from group g_idx[k], the scale of group
    # k / 128 (quantized_weight.cpp:98-117); zeros that differ between the
    # groups a block draws from are re-based onto one zero per block
    rng = np.random.default_rng(7)
    K, N, G = 1024, 520, 8
    qn = rng.integers(0, 13, (K, N)).astype(np.uint32)
    qweight = np.zeros((K // 8, N), np.uint32)
    for i in range(8):
        qweight |= qn[i::8] << (4 * i)
    zn = rng.integers(5, 9, (G, N)).astype(np.uint32)
    qzeros = np.zeros((G, N // 8), np.uint32)
    for s in range(8):
        qzeros |= zn[:, s::8] << (4 * s)
    qweight, qzeros = qweight.view(np.int32), qzeros.view(np.int32)
    scales = f16_normal(rng, (G, N), 0.002)
    g_idx = rng.permutation(np.arange(K) // 128).astype(np.int32)
    w = mcv.W4A16QuantizedWeight.from_gptq(qweight, qzeros, g_idx, scales)
    w8 = oracle.unpack_gptq(qweight, qzeros, g_idx, G)
    _, w8_dev = mcv.w4a16_dequant(w, f16=False, i8=True)
    assert np.array_equal(w8_dev.cpu().numpy(), w8)
    for M in (1, 64):
        x = f16_normal(rng, (M, K), 1.0)
        out = _host_f32(mcv.matmul_w4a16(_to_dev(x), w))
        _check(out, oracle.w4a16_matmul(x, w8, scales), f"gptq act-order M={M}")


def test_gptq_act_order_too_wide_dense(mcv, oracle, cuda):
    # act-order blocks spanning more than 16 levels: the weight is kept as
    # its exact dense fp16 values and matmul_w4a16 runs the vendor's fp16
    # GEMM over it, within the GEMMs' tolerance of the oracle's product; the
    # fused entry points refuse it
    rng = np.random.default_rng(27)
    K, N = 1024, 520
    qweight, qzeros, g_idx = too_wide_gptq(rng, K, N)
    scales = f16_normal(rng, (K // 128, N), 0.002)
    w = mcv.W4A16QuantizedWeight.from_gptq(qweight, qzeros, g_idx, scales)
    assert w.dense is not None and w.qweight is None
    w8 = oracle.unpack_gptq(qweight, qzeros, g_idx, K // 128)
    for M in (1, 64):
        x = f16_normal(rng, (M, K), 1.0)
        out = _host_f32(mcv.matmul_w4a16(_to_dev(x), w))
        _check(out, oracle.w4a16_matmul(x, w8, scales), f"gptq act-order dense M={M}")
    with pytest.raises(mcv.McvError, match="kept dense"):
        mcv.matmul_w4a16_gemv(_to_dev(f16_normal(rng, (1, K), 1.0)), w)


def _reference_tile_pack(w8, K, N):
    """The reference's pack_w4a16_weight + choose_w4a16_tile_len
    (src/csrc/lib/quantized_weight.cpp:41-73), restated to build its input format."""
    block_len = (N + 7) // 8
    tiles = (block_len + 447) // 448
    tile_len = max(16, ((block_len + tiles - 1) // tiles + 15) // 16 * 16)
    tpb = (block_len + tile_len - 1) // tile_len
    G = K // 128
    packed = np.zeros((G, 8, tpb, 128, tile_len), np.int8)
    for b in range(8):
        start = b * block_len
        valid = max(0, min(block_len, N - start))
        for t in range(tpb):
            ts = t * tile_len
            tv = max(0, min(tile_len, valid - ts))
            if tv:
                packed[:, b, t, :, :tv] = w8[:, start + ts:start + ts + tv].reshape(G, 128, tv)
    return packed.reshape(-1, tile_len), tile_len


# tile_len 448, 128, 384 (two tiles per block), 16 and 64 (bands of 16 or 64
# rows per wave-load, wider than a group), and the lm_head's width (70 tiles
# per block, the last one part padding).
@pytest.mark.parametrize("K,N", [(1024, 3584), (1024, 1024), (256, 6144), (256, 128), (384, 512), (128, 248064)])
def test_reference_int8_tile_format(mcv, oracle, cuda, K, N):
    torch = _torch()
    rng = np.random.default_rng(7)
    _, qweight, qzeros, scales = synth_w4a16(rng, K, N)
    w8 = oracle.unpack_awq(qweight, qzeros)
    packed, tile_len = _reference_tile_pack(w8, K, N)
    x = f16_normal(rng, (1, K), 1.0)
    out = torch.empty((1, N), dtype=torch.float16, device="cuda")
    mcv.matmul_w4a16_tiled(_to_dev(x), torch.from_numpy(packed).cuda(), _to_dev(scales), out)
    _check(_host_f32(out), oracle.w4a16_matmul(x, w8, scales), f"tiled K={K} N={N}")


def test_lm_head_full_vocab(mcv, oracle, cuda):
    """The model's lm_head shape: K=1024, V=248094 (weight padded to 248096 for AutoAWQ packing)."""
    torch = _torch()
    K, V = 1024, 248094
    rng = np.random.default_rng(3)
    _, qweight, qzeros, scales = synth_w4a16(rng, K, 248096)
    x = f16_normal(rng, (1, K), 1.0)
    w = _dev_weight(mcv, qweight, qzeros, scales)
    head = mcv.LmHeadW4A16(w, V)
    logits = torch.empty(V, dtype=torch.float16, device="cuda")
    tok = head(_to_dev(x), logits)                      # host-finished slots route
    got16 = logits.cpu().view(torch.int16).numpy().view(np.uint16)
    ref = oracle.w4a16_matmul(x, oracle.unpack_awq(qweight, qzeros), scales)[0, :V]
    _check(got16.view(np.float16).astype(np.float32), ref, "lm_head logits")
    # argmax bit-exact: against the oracle's scan of the kernel's own logits ...
    assert tok == oracle.argmax_f16(got16)
    # ... and against the oracle's logits (this seed has a clear top-1)
    top2 = np.sort(ref)[-2:]
    assert top2[1] - top2[0] > 1e-2
    assert tok == int(np.argmax(ref))
    # the device-token route: same token, same logits, no wait gave up
    lt = torch.empty(V, dtype=torch.float16, device="cuda")
    assert int(head.launch(_to_dev(x), lt).item()) == tok
    assert torch.equal(lt.view(torch.int16), logits.view(torch.int16))
    assert int(head.workspace[:4].view(torch.int32).item()) == 0
    # repeated calls (slots and workspace reused) give the same answer
    assert head(_to_dev(x)) == tok
    assert head(_to_dev(x), logits) == tok


@pytest.mark.parametrize("V", [1, 63, 64, 65, 1000])
def test_lm_head_small_and_ties(mcv, oracle, cuda, V):
    torch = _torch()
    K = 256
    rng = np.random.default_rng(V)
    w_f16 = f16_normal(rng, (K, 1024), 0.02)
    # duplicate columns -> exactly tied logits: the first index must win
    w_f16[:, V // 2] = w_f16[:, V - 1]
    qweight, qzeros, scales = mcv.quantize_int4(w_f16)
    w = _dev_weight(mcv, qweight, qzeros, scales)
    head = mcv.LmHeadW4A16(w, V)
    x = f16_normal(rng, (1, K), 1.0)
    logits = torch.empty(V, dtype=torch.float16, device="cuda")
    tok = head(_to_dev(x), logits)
    got16 = logits.cpu().view(torch.int16).numpy().view(np.uint16)
    assert tok == oracle.argmax_f16(got16)
    assert int(head.launch(_to_dev(x)).item()) == tok
    full = _host_f32(mcv.matmul_w4a16(_to_dev(x), w))[0, :V]
    assert np.array_equal(full.astype(np.float16).view(np.uint16), got16)


# K = 2048 takes the generic path (two groups per wave); V = 1000 leaves the
# last workgroup with a partial run of slabs; zero_bias = 1 is GPTQ's zero + 1.
@pytest.mark.parametrize("K,V,zb", [(1024, 1000, 0), (2048, 1000, 0), (2048, 5000, 1), (128, 777, 1)])
def test_lm_head_shapes(mcv, oracle, cuda, K, V, zb):
    torch = _torch()
    rng = np.random.default_rng(K + V + zb)
    NW = -(-V // 8) * 8
    _, qweight, qzeros, scales = synth_w4a16(rng, K, NW)
    x = f16_normal(rng, (1, K), 1.0)
    w = _dev_weight(mcv, qweight, qzeros, scales)
    if zb:
        w = mcv.W4A16QuantizedWeight(w.qweight, w.scales, w.zeros, K, NW, 1)
    head = mcv.LmHeadW4A16(w, V)
    logits = torch.empty(V, dtype=torch.float16, device="cuda")
    tok = head(_to_dev(x), logits)
    got16 = logits.cpu().view(torch.int16).numpy().view(np.uint16)
    w8 = oracle.unpack_awq(qweight, qzeros) - np.int8(zb)
    _check(got16.view(np.float16).astype(np.float32), oracle.w4a16_matmul(x, w8, scales)[0, :V], "lm_head")
    assert tok == oracle.argmax_f16(got16)
    assert int(head.launch(_to_dev(x)).item()) == tok


# K = 1024 takes the lm_head's one-group-per-wave path.  Slabs per
# workgroup follow V: 4097 and 8320 one (65, 130 workgroups), 40000 two
# (313), 100000 four (391), 124047 eight (243); three calls in a row per shape.
@pytest.mark.parametrize("K,V", [(K, V) for K in (512, 1024) for V in (4097, 8320, 100000)]
                         + [(1024, 40000), (1024, 124047)])
def test_lm_head_routes_agree(mcv, oracle, cuda, V, K):
    """The call-tagged key words read by the grid's last workgroup,
    the host-finished tagged slots and the two-kernel keys + reduction give
    the same token and logits, call after call with no wait giving up."""
    torch = _torch()
    NW = -(-V // 8) * 8
    rng = np.random.default_rng(V + 11 + K)
    w_f16 = f16_normal(rng, (K, NW), 0.02)
    qweight, qzeros, scales = mcv.quantize_int4(w_f16)
    w = _dev_weight(mcv, qweight, qzeros, scales)
    head = mcv.LmHeadW4A16(w, V)
    for trial in range(3):
        x = _to_dev(f16_normal(rng, (1, K), 1.0 + trial))
        la = torch.empty(V, dtype=torch.float16, device="cuda")
        lb = torch.empty(V, dtype=torch.float16, device="cuda")
        lc = torch.empty(V, dtype=torch.float16, device="cuda")
        tree = int(head.launch(x, la).item())
        assert int(head.workspace[:4].view(torch.int32).item()) == 0
        head.launch_partials(x, lb)
        two = int(head.reduce_partials().item())
        slots = head(x, lc)
        assert tree == two == slots
        assert torch.equal(la.view(torch.int16), lb.view(torch.int16))
        assert torch.equal(la.view(torch.int16), lc.view(torch.int16))
        assert tree == oracle.argmax_f16(la.cpu().view(torch.int16).numpy().view(np.uint16))


def test_lm_head_slot_tag_wrap(mcv, oracle, cuda):
    """Tags grow call by call; at the wrap the slots are zero-filled again and
    an older call's larger tag cannot leak into the next token."""
    torch = _torch()
    K, V = 256, 3000
    rng = np.random.default_rng(42)
    qweight, qzeros, scales = mcv.quantize_int4(f16_normal(rng, (K, V), 0.02))
    head = mcv.LmHeadW4A16(_dev_weight(mcv, qweight, qzeros, scales), V)
    xa, xb = (_to_dev(f16_normal(rng, (1, K), 1.0)) for _ in range(2))
    ta, tb = int(head.launch(xa).item()), int(head.launch(xb).item())
    assert ta != tb
    head.tag = head.TAG_MAX - 1
    assert head(xa) == ta and head.tag == head.TAG_MAX
    assert head(xb) == tb and head.tag == 1
    assert head(xa) == ta and head.tag == 2


@pytest.mark.parametrize("M,K,N", [(1, 1024, 3584), (2, 1024, 3584), (1, 2048, 6144), (3, 1024, 520), (1, 128, 64)],
                         ids=lambda v: str(v))
def test_gate_up_silu_fused(mcv, oracle, cuda, M, K, N):
    """One launch == gate GEMV, up GEMV, silu_mul (bit-identical), and within
    tolerance of the oracle's gate/up formula + silu*mul."""
    torch = _torch()
    rng = np.random.default_rng(900 + M + K + N)
    _, qg, zg, sg = synth_w4a16(rng, K, N)
    _, qu, zu, su = synth_w4a16(rng, K, N)
    x = f16_normal(rng, (M, K), 1.0)
    wg, wu = _dev_weight(mcv, qg, zg, sg), _dev_weight(mcv, qu, zu, su)
    xd = _to_dev(x)
    fused = mcv.mlp_gate_up_silu_w4a16(xd, wg, wu)
    g = mcv.matmul_w4a16_gemv(xd, wg)
    u = mcv.matmul_w4a16_gemv(xd, wu)
    three = mcv.silu_mul(g, u)
    torch.cuda.synchronize()
    assert torch.equal(fused.view(torch.int16), three.view(torch.int16))
    g_o = oracle.w4a16_matmul(x, oracle.unpack_awq(qg, zg), sg)
    u_o = oracle.w4a16_matmul(x, oracle.unpack_awq(qu, zu), su)
    a_o = oracle.silu_mul(oracle.f2h_rne(g_o), oracle.f2h_rne(u_o))
    _check(_host_f32(fused), a_o.view(np.float16).astype(np.float32), f"gate_up_silu M={M} K={K} N={N}")


# The decode step's shared-input projections: linear attention qkv + z,
# full attention q / k / v, a GPTQ-style part (zero_bias 1), ragged N, M = 2.
@pytest.mark.parametrize("M,K,Ns", [(1, 1024, (6144, 2048)), (1, 1024, (4096, 512, 512)), (2, 1024, (3584, 3584)),
                                    (1, 256, (200, 72, 1000, 8)), (3, 1024, (520,))], ids=lambda v: str(v))
def test_gemv_multi(mcv, oracle, cuda, M, K, Ns):
    torch = _torch()
    rng = np.random.default_rng(M + K + sum(Ns))
    x = f16_normal(rng, (M, K), 1.0)
    xd = _to_dev(x)
    ws, refs = [], []
    for i, N in enumerate(Ns):
        _, qw, qz, sc = synth_w4a16(rng, K, N)
        w = _dev_weight(mcv, qw, qz, sc)
        zb = 1 if i == 1 else 0
        if zb:
            w = mcv.W4A16QuantizedWeight(w.qweight, w.scales, w.zeros, K, N, 1)
        ws.append(w)
        refs.append(oracle.w4a16_matmul(x, oracle.unpack_awq(qw, qz) - np.int8(zb), sc))
    outs = mcv.matmul_w4a16_multi(xd, ws)
    torch.cuda.synchronize()
    for w, o, ref in zip(ws, outs, refs):
        single = mcv.matmul_w4a16_gemv(xd, w)
        assert torch.equal(o.view(torch.int16), single.view(torch.int16))
        _check(_host_f32(o), ref, f"multi N={w.N}")


@pytest.mark.gpu
def test_lm_head_bound_launchers(mcv, oracle, cuda):
    """bind() resolves the arguments once; its launchers give the tokens and
    logits of launch() / launch_slots() over the same buffers, tags keep
    growing, and a bad route or buffer is refused up front."""
    torch = _torch()
    K, V = 1024, 9000
    rng = np.random.default_rng(7)
    qweight, qzeros, scales = mcv.quantize_int4(f16_normal(rng, (K, V), 0.02))
    head = mcv.LmHeadW4A16(_dev_weight(mcv, qweight, qzeros, scales), V)
    x = _to_dev(f16_normal(rng, (1, K), 1.0))
    la = torch.empty(V, dtype=torch.float16, device="cuda")
    lb = torch.empty(V, dtype=torch.float16, device="cuda")
    want = int(head.launch(x, la).item())
    tree = head.bind(x, lb)
    for _ in range(3):
        lb.fill_(0)
        assert int(tree().item()) == want
        assert torch.equal(la.view(torch.int16), lb.view(torch.int16))
    assert int(head.workspace[:4].view(torch.int32).item()) == 0
    slots = head.bind(x, lb, route="slots")
    t0 = head.tag
    for i in range(3):
        tag = slots()
        assert tag == t0 + i + 1
        assert head.read_slots_token(tag) == want
    assert want == oracle.argmax_f16(la.cpu().view(torch.int16).numpy().view(np.uint16))
    with pytest.raises(mcv.McvError):
        head.bind(x, lb, route="both")
    with pytest.raises(mcv.McvError):
        head.bind(x, torch.empty(V - 1, dtype=torch.float16, device="cuda"))


def test_lm_head_slots_on_side_stream(mcv, oracle, cuda):
    """Slot launches on a non-current stream, including the zero-fill at the
    tag wrap: read_slots_token waits for that stream before it copies."""
    torch = _torch()
    K, V = 512, 5000
    rng = np.random.default_rng(17)
    qweight, qzeros, scales = mcv.quantize_int4(f16_normal(rng, (K, V), 0.02))
    head = mcv.LmHeadW4A16(_dev_weight(mcv, qweight, qzeros, scales), V)
    xs = [_to_dev(f16_normal(rng, (1, K), 1.0)) for _ in range(2)]
    want = [int(head.launch(x).item()) for x in xs]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    head.tag = head.TAG_MAX - 2
    for i in range(4):                                # crosses the wrap at the third call
        tag = head.launch_slots(xs[i % 2], stream=side)
        assert head.read_slots_token(tag) == want[i % 2]
    bound = head.bind(xs[1], stream=side, route="slots")
    assert head.read_slots_token(bound()) == want[1]
