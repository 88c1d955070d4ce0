"""GPU parity of the W8A8 kernels: activation quantiser, int8 MFMA GEMM
(int32 accumulators bit-exact), dequant epilogue and the fused path (bit-exact
against the oracle's epilogue).  Benchmark shapes: M in {1, 256, 1024}, K=1024, N=3584."""
import numpy as np
import pytest

from helpers import f16_normal, rel_l2

pytestmark = pytest.mark.gpu


def _torch():
    import torch
    return torch


def _f16_dev(a_u16):
    torch = _torch()
    return torch.from_numpy(np.ascontiguousarray(a_u16).view(np.int16)).cuda().view(torch.float16)


def _u16(t):
    torch = _torch()
    return t.contiguous().cpu().view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("M,K", [(1, 1024), (256, 1024), (1024, 1024), (3, 3584), (2, 1040), (1, 16), (2, 5000), (1, 4096)])
def test_quantize_act_bit_exact(mcv, oracle, cuda, M, K):
    torch = _torch()
    rng = np.random.default_rng(M * 10 + K)
    x = f16_normal(rng, (M, K), 1.0)
    if M > 2:
        x[1] = 0                                 # all-zero row -> scale floor
        x[2, :7] = np.float16(0.5).view(np.uint16)
    s16 = torch.empty(M, dtype=torch.float16, device="cuda")
    xq, s32, _ = mcv.w8a8_quantize(_f16_dev(x), x_scale_f16=s16)
    q_o, s32_o, s16_o = oracle.w8a8_quantize_act(x)
    assert np.array_equal(xq.cpu().numpy(), q_o)
    assert np.array_equal(s32.cpu().numpy().view(np.uint32), s32_o.view(np.uint32))
    assert np.array_equal(_u16(s16), s16_o)


def test_quantize_act_ties(mcv, oracle, cuda):
    # values whose x * inv lands on k + 0.5 exactly: max|x| = 127 -> scale 1, inv 1
    x = np.array([[127.0, 2.5, -2.5, 0.5, -0.5, 126.5, -127.0, 3.5]], np.float16).view(np.uint16)
    xq, _, _ = mcv.w8a8_quantize(_f16_dev(x))
    assert xq.cpu().numpy().tolist() == oracle.w8a8_quantize_act(x)[0].tolist()
    assert xq.cpu().numpy().tolist() == [[127, 3, -3, 1, -1, 127, -127, 4]]


def _int8_case(rng, M, K, N):
    x = rng.integers(-128, 128, (M, K)).astype(np.int8)
    w = rng.integers(-128, 128, (K, N)).astype(np.int8)
    return x, w


def _dev_weight(mcv, w, layout):
    """int8 [K, N] -> device tensor in `layout` (kn / nk / tiled)."""
    torch = _torch()
    if layout == "kn":
        return torch.from_numpy(w).cuda(), mcv.W8_KN
    if layout == "nk":
        return torch.from_numpy(np.ascontiguousarray(w.T)).cuda(), mcv.W8_NK
    return torch.from_numpy(mcv.pack_w8a8_tiled(w)).cuda(), mcv.W8_TILED


@pytest.mark.parametrize("M,K,N", [(1, 1024, 3584), (256, 1024, 3584), (5, 1040, 208), (130, 256, 144)],
                         ids=lambda v: str(v))
@pytest.mark.parametrize("layout", ["kn", "nk", "tiled"])
def test_gemm_i32_bit_exact(mcv, oracle, cuda, M, K, N, layout):
    torch = _torch()
    rng = np.random.default_rng(M + K + N)
    x, w = _int8_case(rng, M, K, N)
    wdev, wl = _dev_weight(mcv, w, layout)
    acc = mcv.matmul_w8a8_i32(torch.from_numpy(x).cuda(), wdev, layout=wl, N=N)
    assert np.array_equal(acc.cpu().numpy(), oracle.gemm_i32(x, w))


# The tiled path's GEMV (M <= 4; M <= 2 past K = 2048) and every GEMM tile shape, ragged K and N
# (K padded to 128 with zero weights, N to 64), extreme values.
@pytest.mark.parametrize("M,K,N", [(2, 1024, 3584), (3, 208, 80), (4, 2048, 1000), (6, 1024, 3584),
                                   (64, 16, 64), (100, 1040, 3584), (1024, 1024, 3584), (300, 3584, 1024),
                                   (2, 3584, 1024), (4, 3584, 1024)],
                         ids=lambda v: str(v))
def test_tiled_gemm_i32_bit_exact(mcv, oracle, cuda, M, K, N):
    torch = _torch()
    rng = np.random.default_rng(7 * M + K + N)
    x, w = _int8_case(rng, M, K, N)
    x[0, :] = -128
    w[:, 0] = -128
    wdev, _ = _dev_weight(mcv, w, "tiled")
    acc = mcv.matmul_w8a8_i32(torch.from_numpy(x).cuda(), wdev, layout=mcv.W8_TILED, N=N)
    if M * K * N <= 300 * 1024 * 1024:
        assert np.array_equal(acc.cpu().numpy(), oracle.gemm_i32(x, w))
    else:
        ref = (torch.from_numpy(x).cuda().double() @ torch.from_numpy(w).cuda().double()).to(torch.int64)
        assert torch.equal(acc.to(torch.int64), ref)
    assert int(acc[0, 0]) == K * 128 * 128


def test_gemm_i32_full_size_exact(mcv, cuda):
    # M=1024, K=1024, N=3584 with extreme values: the fp64 product is exact at this size
    torch = _torch()
    rng = np.random.default_rng(55)
    M, K, N = 1024, 1024, 3584
    x, w = _int8_case(rng, M, K, N)
    x[0, :] = -128
    w[:, 0] = -128                               # |acc| = 2^24 at (0, 0)
    xd, wd = torch.from_numpy(x).cuda(), torch.from_numpy(w).cuda()
    ref = (xd.double() @ wd.double()).to(torch.int64)
    for layout in ("kn", "tiled"):
        wdev, wl = _dev_weight(mcv, w, layout)
        acc = mcv.matmul_w8a8_i32(xd, wdev, layout=wl, N=N)
        assert torch.equal(acc.to(torch.int64), ref), layout
        assert int(acc[0, 0]) == 1 << 24


def test_dequant_reference_vectors(mcv, oracle, cuda):
    torch = _torch()
    N = 3584
    acc = (np.arange(N) - 1024).astype(np.int32)[None, :]
    ws16 = oracle.f2h_trunc(np.float32(0.01) + (np.arange(N) % 7).astype(np.float32) * np.float32(0.001))
    xs16 = oracle.f2h_trunc(np.array([0.02], np.float32))
    out = mcv.w8a8_dequant(torch.from_numpy(acc).cuda(), _f16_dev(xs16), _f16_dev(ws16))
    want = oracle.w8a8_dequant(acc, oracle.h2f(xs16), oracle.h2f(ws16))
    assert np.array_equal(_u16(out), want)


@pytest.mark.parametrize("M", [1, 256, 1024])
def test_w8a8_end_to_end(mcv, oracle, cuda, M):
    """fp16 x -> per-token int8 + fp32 scale; fp16 W -> per-channel int8 + fp32
    scale; fused GEMM + epilogue.  Every stage bit-exact against the oracle."""
    torch = _torch()
    K, N = 1024, 3584
    rng = np.random.default_rng(500 + M)
    x = f16_normal(rng, (M, K), 1.0)
    wf = f16_normal(rng, (K, N), 0.02)
    wq = mcv.quantize_dense_weight_w8a8(_f16_dev(wf))
    xq, xs, _ = mcv.w8a8_quantize(_f16_dev(x))
    out = mcv.matmul_w8a8(xq, xs, wq)                    # fp32 scales
    q_o, s_o, _ = oracle.w8a8_quantize_act(x)
    wq_o, ws_o, ws16_o = oracle.w8a8_quantize_weight(wf)
    assert wq.layout == mcv.W8_TILED
    assert np.array_equal(wq.w_int8.cpu().numpy(), mcv.pack_w8a8_tiled(wq_o))
    rows = np.arange(M) if M <= 256 else np.arange(0, M, 8)
    acc_o = oracle.gemm_i32(q_o[rows], wq_o)
    want = oracle.w8a8_dequant(acc_o, s_o[rows], ws_o)
    got = _u16(out)[rows]
    bad = np.argwhere(got != want)
    assert bad.size == 0, f"{len(bad)} mismatches, first at {bad[:3].tolist()}: {got[tuple(bad[0])]:#06x} vs {want[tuple(bad[0])]:#06x}"
    # fused == two-kernel path, with the reference's fp16 scales too
    acc = mcv.matmul_w8a8_i32(xq, wq)
    assert torch.equal(mcv.w8a8_dequant(acc, xs, wq.w_scale_f32), out)
    xs16 = xs.half()
    assert torch.equal(mcv.matmul_w8a8(xq, xs16, wq, use_f32_scale=False),
                       mcv.w8a8_dequant(acc, xs16, wq.w_scale))


# The M > 4 GEMM's fused epilogue on ragged shapes: a last tile past M and N,
# K padded with zero weights, N % 4 != 0 (scales loaded one per column, not
# four at once), with fp32 and with the reference's fp16 scales.
@pytest.mark.parametrize("M,K,N", [(257, 1040, 1000), (70, 256, 1003), (1030, 384, 3590)], ids=lambda v: str(v))
def test_w8a8_gemm_fused_ragged(mcv, oracle, cuda, M, K, N):
    rng = np.random.default_rng(900 + M + N)
    x = f16_normal(rng, (M, K), 1.0)
    wf = f16_normal(rng, (K, N), 0.02)
    wq = mcv.quantize_dense_weight_w8a8(_f16_dev(wf))
    wq_np = mcv.quantize_dense_weight_w8a8(wf)            # a host array in: the same weight on the GPU
    assert wq_np.w_int8.is_cuda and _torch().equal(wq_np.w_int8, wq.w_int8)
    xq, xs, _ = mcv.w8a8_quantize(_f16_dev(x))
    xs16 = xs.half()
    q_o, s_o, s16_o = oracle.w8a8_quantize_act(x)
    assert np.array_equal(_u16(xs16), s16_o)
    wq_o, ws_o, ws16_o = oracle.w8a8_quantize_weight(wf)
    acc_o = oracle.gemm_i32(q_o, wq_o)
    got = _u16(mcv.matmul_w8a8(xq, xs, wq))
    assert np.array_equal(got, oracle.w8a8_dequant(acc_o, s_o, ws_o))
    got16 = _u16(mcv.matmul_w8a8(xq, xs16, wq, use_f32_scale=False))
    assert np.array_equal(got16, oracle.w8a8_dequant(acc_o, oracle.h2f(s16_o), oracle.h2f(ws16_o)))


# Every built tile configuration of the M > 4 GEMM through mcv_w8a8_gemm_lds
# (the dispatch runs one per shape): int32 accumulators bit-exact against the
# oracle's product, the fused epilogue bit-exact with fp32 and with fp16
# scales, on ragged shapes (a last tile past M and N, K padded with zero
# weights, N % 4 != 0); then unbuilt configurations fail cleanly.
W8_LDS_CONFIGS = [(128, 128, 3, 0), (128, 128, 4, 0), (64, 128, 4, 0), (128, 64, 4, 0), (64, 64, 4, 0),
                  (64, 64, 3, 0), (128, 128, 3, 1), (128, 128, 4, 1), (64, 128, 4, 1)]


@pytest.mark.parametrize("M,K,N", [(257, 1040, 1000), (70, 384, 1003)], ids=lambda v: str(v))
def test_w8a8_gemm_every_configuration(mcv, oracle, cuda, M, K, N):
    torch = _torch()
    L = mcv.lib()
    rng = np.random.default_rng(1300 + M + N)
    x = f16_normal(rng, (M, K), 1.0)
    wf = f16_normal(rng, (K, N), 0.02)
    wq = mcv.quantize_dense_weight_w8a8(_f16_dev(wf))
    xq, xs, _ = mcv.w8a8_quantize(_f16_dev(x))
    xs16 = xs.half()
    q_o, s_o, s16_o = oracle.w8a8_quantize_act(x)
    wq_o, ws_o, ws16_o = oracle.w8a8_quantize_weight(wf)
    acc_o = oracle.gemm_i32(q_o, wq_o)
    want32 = oracle.w8a8_dequant(acc_o, s_o, ws_o)
    want16 = oracle.w8a8_dequant(acc_o, oracle.h2f(s16_o), oracle.h2f(ws16_o))
    stream = torch.cuda.current_stream().cuda_stream
    for bm, bn, ns, wr in W8_LDS_CONFIGS:
        tag = f"{bm}x{bn} ns={ns} wr={wr} M={M} K={K} N={N}"
        acc = torch.full((M, N), 7, dtype=torch.int32, device="cuda")
        rc = L.mcv_w8a8_gemm_lds(xq.data_ptr(), None, 0, M, K, N, wq.w_int8.data_ptr(), None, 0, acc.data_ptr(), 0,
                                 bm, bn, ns, wr, stream)
        assert rc == 0, (tag, L.mcv_last_error())
        out = torch.full((M, N), 7.0, dtype=torch.float16, device="cuda")
        rc = L.mcv_w8a8_gemm_lds(xq.data_ptr(), xs.data_ptr(), mcv.MCV_F32, M, K, N, wq.w_int8.data_ptr(),
                                 wq.w_scale_f32.data_ptr(), mcv.MCV_F32, out.data_ptr(), 1, bm, bn, ns, wr, stream)
        assert rc == 0, (tag, L.mcv_last_error())
        out16 = torch.full((M, N), 7.0, dtype=torch.float16, device="cuda")
        rc = L.mcv_w8a8_gemm_lds(xq.data_ptr(), xs16.data_ptr(), mcv.MCV_F16, M, K, N, wq.w_int8.data_ptr(),
                                 wq.w_scale.data_ptr(), mcv.MCV_F16, out16.data_ptr(), 1, bm, bn, ns, wr, stream)
        assert rc == 0, (tag, L.mcv_last_error())
        torch.cuda.synchronize()
        assert np.array_equal(acc.cpu().numpy(), acc_o), tag
        assert np.array_equal(_u16(out), want32), tag
        assert np.array_equal(_u16(out16), want16), tag
    for bm, bn, ns, wr in [(96, 128, 3, 0), (64, 64, 4, 1), (128, 128, 2, 0)]:
        assert L.mcv_w8a8_gemm_lds(xq.data_ptr(), None, 0, M, K, N, wq.w_int8.data_ptr(), None, 0,
                                   xq.data_ptr(), 0, bm, bn, ns, wr, stream) == 1, (bm, bn, ns, wr)


def test_nk_layout_fused(mcv, cuda):
    torch = _torch()
    rng = np.random.default_rng(77)
    K, N, M = 1024, 3584, 64
    wf = f16_normal(rng, (K, N), 0.02)
    a = mcv.quantize_dense_weight_w8a8(_f16_dev(wf), layout=mcv.W8_KN)
    b = mcv.quantize_dense_weight_w8a8(_f16_dev(wf), layout=mcv.W8_NK)
    c = mcv.quantize_dense_weight_w8a8(_f16_dev(wf), layout=mcv.W8_TILED)
    xq, xs, _ = mcv.w8a8_quantize(_f16_dev(f16_normal(rng, (M, K), 1.0)))
    ref = mcv.matmul_w8a8(xq, xs, a)
    assert torch.equal(ref, mcv.matmul_w8a8(xq, xs, b))
    assert torch.equal(ref, mcv.matmul_w8a8(xq, xs, c))
    # fp16 scales and the M <= 4 GEMV through the same epilogue
    xs16 = xs.half()
    assert torch.equal(mcv.matmul_w8a8(xq, xs16, a, use_f32_scale=False), mcv.matmul_w8a8(xq, xs16, c, use_f32_scale=False))
    assert torch.equal(mcv.matmul_w8a8(xq[:3], xs[:3], a), mcv.matmul_w8a8(xq[:3], xs[:3], c))


# Every projection of one decode step (K, N): qkv, z, out, gate/up, down of the
# linear-attention layers and q, k/v, o of the full-attention layers.
@pytest.mark.parametrize("K,N", [(1024, 6144), (1024, 2048), (2048, 1024), (1024, 3584), (3584, 1024),
                                 (1024, 4096), (1024, 512), (1024, 16)], ids=lambda v: str(v))
def test_decode_shapes_fused(mcv, oracle, cuda, K, N):
    torch = _torch()
    rng = np.random.default_rng(K * 3 + N)
    x = f16_normal(rng, (1, K), 1.0)
    wf = f16_normal(rng, (K, N), 0.02)
    wq = mcv.quantize_dense_weight_w8a8(_f16_dev(wf))
    xq, xs, _ = mcv.w8a8_quantize(_f16_dev(x))
    out = mcv.matmul_w8a8(xq, xs, wq)
    acc = mcv.matmul_w8a8_i32(xq, wq)
    q_o, s_o, _ = oracle.w8a8_quantize_act(x)
    wq_o, ws_o, _ = oracle.w8a8_quantize_weight(wf)
    acc_o = oracle.gemm_i32(q_o, wq_o)
    assert np.array_equal(acc.cpu().numpy(), acc_o)
    assert np.array_equal(_u16(out), oracle.w8a8_dequant(acc_o, s_o, ws_o))


@pytest.mark.parametrize("M,K,N", [(1, 1024, 3584), (2, 1024, 3584), (4, 2048, 6144), (3, 384, 208), (1, 128, 64)],
                         ids=lambda v: str(v))
def test_gate_up_silu_fused(mcv, oracle, cuda, M, K, N):
    """One launch == gate and up fused GEMVs + silu_mul, bit for bit, with fp32
    and with fp16 scales; and the oracle's composition of the same stages."""
    torch = _torch()
    rng = np.random.default_rng(M * 31 + K + N)
    wg = mcv.quantize_dense_weight_w8a8(_f16_dev(f16_normal(rng, (K, N), 0.02)))
    wu = mcv.quantize_dense_weight_w8a8(_f16_dev(f16_normal(rng, (K, N), 0.02)))
    x = f16_normal(rng, (M, K), 1.0)
    s16 = torch.empty(M, dtype=torch.float16, device="cuda")
    xq, xs, _ = mcv.w8a8_quantize(_f16_dev(x), x_scale_f16=s16)
    for f32 in (True, False):
        xsc = xs if f32 else s16
        fused = mcv.mlp_gate_up_silu_w8a8(xq, xsc, wg, wu, use_f32_scale=f32)
        three = mcv.silu_mul(mcv.matmul_w8a8(xq, xsc, wg, use_f32_scale=f32),
                             mcv.matmul_w8a8(xq, xsc, wu, use_f32_scale=f32))
        assert torch.equal(fused.view(torch.int16), three.view(torch.int16)), f32
    # oracle: int32 products, reference epilogue, silu*mul
    q_o = xq.cpu().numpy()
    s_o = xs.cpu().numpy()
    g_o = oracle.w8a8_dequant(oracle.gemm_i32(q_o, _tiled_to_kn(mcv, wg)), s_o, wg.w_scale_f32.cpu().numpy())
    u_o = oracle.w8a8_dequant(oracle.gemm_i32(q_o, _tiled_to_kn(mcv, wu)), s_o, wu.w_scale_f32.cpu().numpy())
    want = oracle.silu_mul(g_o, u_o)
    got = _u16(mcv.mlp_gate_up_silu_w8a8(xq, xs, wg, wu))
    gv, wv = got.view(np.float16).astype(np.float64), want.view(np.float16).astype(np.float64)
    ulp = np.abs(np.spacing(want.view(np.float16))).astype(np.float64)
    assert (np.abs(gv - wv) <= ulp).all()                 # exp may differ by an fp32 ulp between libms
    assert (got == want).mean() > 0.99


def _tiled_to_kn(mcv, w):
    """int8 [K, N] of a tiled weight, read back through the documented layout formula."""
    t = w.w_int8.cpu().numpy()
    K, N = w.K, w.N
    kb = -(-K // 128) * 4
    k = np.arange(K)[:, None]
    n = np.arange(N)[None, :]
    l = n % 32 + 32 * ((k % 32) // 16)
    off = ((((n // 64) * kb + k // 32) * 2 + (n % 64) // 32) * 64 + l) * 16 + k % 16
    return t[off]


def _oracle_w8a8_proj(oracle, mcv, x_u16, w, f32):
    """The reference's W8A8 projection of one row by the oracle: per-tensor
    quantisation, exact int32 products, dequant with the activation and weight
    scales -- fp16 (the reference's stored forms, decoder_layer.cpp:216-237)
    or fp32."""
    q_o, s_o, s16_o = oracle.w8a8_quantize_act(x_u16)
    ws = w.w_scale_f32.cpu().numpy() if f32 else oracle.h2f(_u16(w.w_scale))
    xs = s_o if f32 else oracle.h2f(s16_o)
    return oracle.w8a8_dequant(oracle.gemm_i32(q_o, _tiled_to_kn(mcv, w)), xs, ws)


@pytest.mark.parametrize("H,I", [(1024, 3584), (3584, 1024), (256, 384), (2048, 6144)], ids=lambda v: str(v))
def test_decode_mlp_reference_precision_vs_oracle(mcv, oracle, cuda, H, I):
    """DecodeMlpW8A8's default (reference) precision, one launch, bit-exact
    against the oracle's composition of the reference's steps: quantise the
    row (fp16 scale), gate and up through gemm_i32 + dequant with the fp16
    x_scale and the truncated fp16 w_scale, silu_mul, the same for down.  exp
    inside silu is the one step host and device libms may round differently,
    so that step uses the device's silu_mul (within one fp16 ulp of the
    oracle's, checked here too)."""
    torch = _torch()
    rng = np.random.default_rng(H * 7 + I)
    wg = mcv.quantize_dense_weight_w8a8(_f16_dev(f16_normal(rng, (H, I), 0.02)))
    wu = mcv.quantize_dense_weight_w8a8(_f16_dev(f16_normal(rng, (H, I), 0.02)))
    wd = mcv.quantize_dense_weight_w8a8(_f16_dev(f16_normal(rng, (I, H), 0.02)))
    mlp = mcv.DecodeMlpW8A8(wg, wu, wd)                  # precision="reference"
    out = torch.empty((1, H), dtype=torch.float16, device="cuda")
    for trial in range(2):
        x = f16_normal(rng, (1, H), 1.0 + trial)
        mlp(_f16_dev(x), out)
        assert mlp.one_launch
        g_o = _oracle_w8a8_proj(oracle, mcv, x, wg, False)
        u_o = _oracle_w8a8_proj(oracle, mcv, x, wu, False)
        act = _u16(mcv.silu_mul(_f16_dev(g_o), _f16_dev(u_o)))
        act_o = oracle.silu_mul(g_o, u_o)
        assert (np.abs(act.astype(np.int32) - act_o.astype(np.int32)) <= 1).all()
        want = _oracle_w8a8_proj(oracle, mcv, act.reshape(1, I), wd, False)
        got = _u16(out)
        bad = np.flatnonzero(got != want)
        assert bad.size == 0, f"trial {trial}: {bad.size} mismatches, first at {bad[:4].tolist()}"
    assert not mlp.wait_gave_up()
    # the same block through the separate operators, reference precision
    want4 = torch.empty_like(out)
    mlp._four_launches(_f16_dev(x), want4, None)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), want4.view(torch.int16))


@pytest.mark.parametrize("H,I", [(1024, 3584), (3584, 1024), (256, 384), (128, 128), (2048, 6144)],
                         ids=lambda v: str(v))
def test_decode_mlp_block_one_launch(mcv, oracle, cuda, H, I):
    """The whole W8A8 MLP block in one launch with fp32 scales == quantise x,
    gate+up+silu*mul, quantise act, down GEMV, bit for bit, call after call;
    and the oracle's composition of the same stages."""
    torch = _torch()
    rng = np.random.default_rng(H * 5 + I)
    wg = mcv.quantize_dense_weight_w8a8(_f16_dev(f16_normal(rng, (H, I), 0.02)))
    wu = mcv.quantize_dense_weight_w8a8(_f16_dev(f16_normal(rng, (H, I), 0.02)))
    wd = mcv.quantize_dense_weight_w8a8(_f16_dev(f16_normal(rng, (I, H), 0.02)))
    mlp = mcv.DecodeMlpW8A8(wg, wu, wd, precision="f32")
    out = torch.empty((1, H), dtype=torch.float16, device="cuda")
    want = torch.empty_like(out)
    for trial in range(3):
        x = f16_normal(rng, (1, H), 1.0 + trial)
        xd = _f16_dev(x)
        mlp(xd, out)
        assert mlp.one_launch
        mlp._four_launches(xd, want, None)
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), want.view(torch.int16)), f"trial {trial}"
    assert not mlp.wait_gave_up()
    # oracle: quantise, int32 products, reference epilogues, silu*mul, quantise, down
    q_o, s_o, _ = oracle.w8a8_quantize_act(x)
    g_o = oracle.w8a8_dequant(oracle.gemm_i32(q_o, _tiled_to_kn(mcv, wg)), s_o, wg.w_scale_f32.cpu().numpy())
    u_o = oracle.w8a8_dequant(oracle.gemm_i32(q_o, _tiled_to_kn(mcv, wu)), s_o, wu.w_scale_f32.cpu().numpy())
    a_o = oracle.silu_mul(g_o, u_o)
    aq_o, as_o, _ = oracle.w8a8_quantize_act(a_o.reshape(1, I))
    y_o = oracle.w8a8_dequant(oracle.gemm_i32(aq_o, _tiled_to_kn(mcv, wd)), as_o, wd.w_scale_f32.cpu().numpy())
    got = _u16(out).view(np.float16).astype(np.float32)
    ref = y_o.view(np.float16).astype(np.float32)
    # silu's exp may differ by an fp32 ulp between libms, which can move an act
    # value by one fp16 ulp and so a quantised act by one step
    assert np.abs(got - ref).max() <= 2e-2 and rel_l2(got, ref) <= 1e-3
    assert (_u16(out) == y_o).mean() > 0.9


def test_decode_mlp_block_falls_back(mcv, oracle, cuda):
    """H = 8320 does not fit the one-launch kernel's LDS x row: the object
    runs the four launches and returns their result."""
    torch = _torch()
    rng = np.random.default_rng(77)
    H, I = 8320, 128
    wg = mcv.quantize_dense_weight_w8a8(_f16_dev(f16_normal(rng, (H, I), 0.02)))
    wu = mcv.quantize_dense_weight_w8a8(_f16_dev(f16_normal(rng, (H, I), 0.02)))
    wd = mcv.quantize_dense_weight_w8a8(_f16_dev(f16_normal(rng, (I, H), 0.02)))
    mlp = mcv.DecodeMlpW8A8(wg, wu, wd, precision="f32")
    assert not mlp.one_launch
    xd = _f16_dev(f16_normal(rng, (1, H), 1.0))
    out = mlp(xd)
    xq, xs, _ = mcv.w8a8_quantize(xd)
    aq, asc, _ = mcv.w8a8_quantize(mcv.mlp_gate_up_silu_w8a8(xq, xs, wg, wu))
    want = mcv.matmul_w8a8(aq, asc, wd)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), want.view(torch.int16))


# The W8A8 lm_head step in one launch (mcv_w8a8_lm_head_argmax): the
# activation quantisation, the GEMV and the argmax exchange inside one kernel,
# bit-identical to w8a8_quantize + the argmax GEMV + the key reduction, call
# after call through one workspace, with the fp16 (reference) and fp32 scales;
# a forced give-up writes token -1 and the give-up words, and the next call
# needs no reset.
# The vocabularies take every grid the launcher picks (1, 2 and 4 slabs per
# workgroup) and K every k-block count per wave (1, 2 and 4).
@pytest.mark.parametrize("K,N,V", [(1024, 20000, 19997), (256, 4096, 4096), (1040, 5000, 4999),
                                   (512, 40000, 39990), (2048, 100032, 100000), (1024, 150016, 150000),
                                   (1024, 248096, 248094)], ids=lambda v: str(v))
def test_lm_head_w8a8_one_launch(mcv, oracle, cuda, K, N, V):
    assert mcv.w8a8_lm_head_slabs_per_workgroup(V) == {39990: 1, 100000: 2, 150000: 4, 248094: 4}.get(V, 1)
    torch = _torch()
    rng = np.random.default_rng(K * 3 + V)
    x = f16_normal(rng, (1, K), 1.0)
    wq = mcv.quantize_dense_weight_w8a8(f16_normal(rng, (K, N), 0.02))
    xd = _f16_dev(x)
    xq, xs, _ = mcv.w8a8_quantize(xd)
    ws = torch.zeros(mcv.lm_head_workspace_bytes(V), dtype=torch.uint8, device="cuda")
    for use32 in (False, True):
        want_logits = torch.empty(V, dtype=torch.float16, device="cuda")
        want = int(mcv.lm_head_argmax_w8a8(xq, xs if use32 else xs.half(), wq, V, want_logits,
                                           use_f32_scale=use32).item())
        for call in range(3):                    # the generation word advances call after call
            logits = torch.full((V,), 7.0, dtype=torch.float16, device="cuda")
            tok = int(mcv.lm_head_argmax_w8a8_fused(xd, wq, V, ws, logits, use_f32_scale=use32).item())
            assert tok == want, (use32, call)
            assert torch.equal(logits.view(torch.int16), want_logits.view(torch.int16)), (use32, call)
        assert int(mcv.lm_head_argmax_w8a8_fused(xd, wq, V, ws, use_f32_scale=use32).item()) == want
        if not use32:
            assert want == oracle.argmax_f16(_u16(want_logits))
    assert int(ws[:4].view(torch.int32).item()) == 0
    if V == 4096:
        status = torch.zeros(1, dtype=torch.int32, device="cuda")
        mcv.lib().mcv_testing_lm_head_skew_poll(1)
        try:
            tok = int(mcv.lm_head_argmax_w8a8_fused(xd, wq, V, ws, status=status).item())
        finally:
            mcv.lib().mcv_testing_lm_head_skew_poll(0)
        assert tok == -1 and int(status.item()) == 1 and int(ws[:4].view(torch.int32).item()) != 0
        assert int(mcv.lm_head_argmax_w8a8_fused(xd, wq, V, ws).item()) == want


# The W8A8 lm_head with the argmax folded into the GEMV: logits bit-identical
# to matmul_w8a8, the token the first maximum of them, with ragged V (keys for
# 313 slabs), a tie at the maximum, and the model's vocabulary (3877 slabs).
@pytest.mark.parametrize("K,N,V", [(1024, 20000, 19997), (256, 4096, 4096), (1024, 248096, 248094)],
                         ids=lambda v: str(v))
def test_lm_head_w8a8_fused_argmax(mcv, oracle, cuda, K, N, V):
    torch = _torch()
    rng = np.random.default_rng(K + V)
    x = f16_normal(rng, (1, K), 1.0)
    wf = f16_normal(rng, (K, N), 0.02)
    xq, xs, _ = mcv.w8a8_quantize(_f16_dev(x))
    xs16 = xs.half()
    if V == 4096:
        # an exact tie at the maximum: column 50 becomes a copy of the winner
        wq = mcv.quantize_dense_weight_w8a8(wf)
        top = int(mcv.lm_head_argmax_w8a8(xq, xs16, wq, V).item())
        if top != 50:
            wf[:, 50] = wf[:, top]
    wq = mcv.quantize_dense_weight_w8a8(wf)
    logits = torch.empty(V, dtype=torch.float16, device="cuda")
    tok = int(mcv.lm_head_argmax_w8a8(xq, xs16, wq, V, logits).item())
    full = mcv.matmul_w8a8(xq, xs16, wq, use_f32_scale=False)
    assert torch.equal(logits.view(torch.int16), full[0, :V].view(torch.int16))
    got = _u16(logits)
    assert tok == oracle.argmax_f16(got)
    if V == 4096:
        assert tok == 50
    if K * N <= 1024 * 20000:
        q_o, _, s16_o = oracle.w8a8_quantize_act(x)
        wq_o, _, ws16_o = oracle.w8a8_quantize_weight(wf)
        want = oracle.w8a8_dequant(oracle.gemm_i32(q_o, wq_o), oracle.h2f(s16_o), oracle.h2f(ws16_o))
        assert np.array_equal(got, want[0, :V])
    # without logits: the same token; fp32 scales: the token of their logits
    assert int(mcv.lm_head_argmax_w8a8(xq, xs16, wq, V).item()) == tok
    l32 = torch.empty(V, dtype=torch.float16, device="cuda")
    t32 = int(mcv.lm_head_argmax_w8a8(xq, xs, wq, V, l32, use_f32_scale=True).item())
    assert torch.equal(l32.view(torch.int16), mcv.matmul_w8a8(xq, xs, wq)[0, :V].view(torch.int16))
    assert t32 == oracle.argmax_f16(_u16(l32))


@pytest.mark.gpu
def test_lm_head_w8a8_one_launch_graph_replays(mcv, cuda):
    """The one-launch W8A8 lm_head captured into a HIP graph: the kernel reads
    the workspace's generation word afresh on every replay, so replays with
    eager calls through the same workspace between them (the same head, and a
    smaller vocabulary on another grid) all give the eager token and logits."""
    torch = _torch()
    K, N, V = 1024, 100032, 100000
    rng = np.random.default_rng(4242)
    x = f16_normal(rng, (1, K), 1.0)
    wq = mcv.quantize_dense_weight_w8a8(f16_normal(rng, (K, N), 0.02))
    xd = _f16_dev(x)
    ws = torch.zeros(mcv.lm_head_workspace_bytes(V), dtype=torch.uint8, device="cuda")
    want_logits = torch.empty(V, dtype=torch.float16, device="cuda")
    want = int(mcv.lm_head_argmax_w8a8_fused(xd, wq, V, ws, want_logits).item())
    Vs = V // 3                                          # another grid: 1 slab per workgroup instead of 2
    assert mcv.w8a8_lm_head_slabs_per_workgroup(Vs) != mcv.w8a8_lm_head_slabs_per_workgroup(V)
    want_s = int(np.argmax(want_logits[:Vs].float().cpu().numpy()))
    logits = torch.empty_like(want_logits)
    tok = torch.empty(1, dtype=torch.int64, device="cuda")
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        mcv.lm_head_argmax_w8a8_fused(xd, wq, V, ws, logits, tok)
        with torch.cuda.graph(g, stream=s):
            mcv.lm_head_argmax_w8a8_fused(xd, wq, V, ws, logits, tok)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    for i in range(4):
        logits.zero_()
        tok.fill_(-2)
        assert int(mcv.lm_head_argmax_w8a8_fused(xd, wq, V, ws).item()) == want, f"eager {i}"
        assert int(mcv.lm_head_argmax_w8a8_fused(xd, wq, Vs, ws).item()) == want_s, f"eager small {i}"
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert int(tok.item()) == want, f"replay {i}"
        assert torch.equal(logits.view(torch.int16), want_logits.view(torch.int16)), f"replay {i}"
    assert int(ws[:4].view(torch.int32).item()) == 0         # no wait gave up
