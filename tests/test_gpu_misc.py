"""GPU parity of silu*mul and the greedy argmax against the oracle."""
import numpy as np
import pytest

from helpers import f16_normal

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


@pytest.mark.parametrize("n", [1, 3584, 100003])
def test_silu_mul(mcv, oracle, cuda, n):
    rng = np.random.default_rng(n)
    g = f16_normal(rng, n, 3.0)
    u = f16_normal(rng, n, 2.0)
    got = _u16(mcv.silu_mul(_f16_dev(g), _f16_dev(u)))
    want = oracle.silu_mul(g, u)
    gv = got.view(np.float16).astype(np.float64)
    wv = want.view(np.float16).astype(np.float64)
    ulp = np.abs(np.spacing(want.view(np.float16))).astype(np.float64)
    # exp differs by at most an fp32 ulp between libms: at most 1 fp16 ulp apart
    assert (np.abs(gv - wv) <= ulp).all()
    assert (got == want).mean() > 0.99


def test_argmax_rows(mcv, oracle, cuda):
    torch = _torch()
    rng = np.random.default_rng(9)
    M, N = 6, 248094
    x = f16_normal(rng, (M, N), 1.0)
    x[1, 5000] = x[1, 7000] = 0x7000                 # tie: first index wins
    x[2, :] = 0xFC00                                 # all -inf -> 0
    x[3, 100] = 0x7E00                               # NaN never wins
    x[4, :] = 0x0001                                 # subnormals compare as zero: first wins
    x[4, 9] = 0x8000
    x[5, 12345] = 0x7C00                             # +inf wins
    got = mcv.argmax_last_dim(_f16_dev(x)).cpu().numpy()
    want = [oracle.argmax_f16(x[m]) for m in range(M)]
    assert got.tolist() == want
    assert want[1] == 5000 and want[2] == 0 and want[4] == 0 and want[5] == 12345


# Odd row lengths put every row start at another 2-byte offset from a 16-byte
# boundary (the kernel's head of single loads before the vector loads); a tie
# between a head element and one in the vector part or the tail.
@pytest.mark.parametrize("M,N", [(3, 7), (9, 1001), (2, 1), (4, 65537)])
def test_argmax_ragged_rows(mcv, oracle, cuda, M, N):
    rng = np.random.default_rng(M * 31 + N)
    x = f16_normal(rng, (M, N), 1.0)
    if N > 600:
        x[1, 3] = x[1, 500] = x[1, N - 1] = 0x7000
    got = mcv.argmax_last_dim(_f16_dev(x)).cpu().numpy()
    assert got.tolist() == [oracle.argmax_f16(x[m]) for m in range(M)]
    if N > 600:
        assert got[1] == 3


@pytest.mark.parametrize("M,H", [(1, 1024), (3, 2048), (64, 1024), (2, 100)])
def test_rms_norm_vs_oracle(mcv, oracle, cuda, M, H):
    rng = np.random.default_rng(M * 7 + H)
    x = f16_normal(rng, (M, H), 2.0)
    g = f16_normal(rng, H, 1.0)
    got = _u16(mcv.rms_norm(_f16_dev(x), _f16_dev(g), 1e-6))
    want = oracle.rms_norm(x, g, 1e-6)
    gv = got.view(np.float16).astype(np.float64)
    wv = want.view(np.float16).astype(np.float64)
    ulp = np.abs(np.spacing(want.view(np.float16))).astype(np.float64)
    assert (np.abs(gv - wv) <= ulp).all()
    assert (got == want).mean() > 0.98


@pytest.mark.parametrize("M,H", [(1, 1024), (1, 2048), (4, 3584), (64, 1024), (3, 100), (2, 5000), (1, 4096), (1, 1025)])
def test_rms_norm_w8a8_quantize_fused(mcv, oracle, cuda, M, H):
    """One launch == rms_norm then w8a8_quantize (every output bit-identical),
    and the int8 row and scales are the oracle's quantisation of that normed row."""
    torch = _torch()
    rng = np.random.default_rng(M + H)
    x = f16_normal(rng, (M, H), 1.5)
    if M > 2:
        x[1] = 0                                            # zero row: normed 0, scale floor 1e-8
        x[2, 0] = np.float16(300.0).view(np.uint16)         # one dominant element
    g = f16_normal(rng, H, 1.0)
    xd, gd = _f16_dev(x), _f16_dev(g)
    s16 = torch.empty(M, dtype=torch.float16, device="cuda")
    normed, xq, xs, _ = mcv.rms_norm_w8a8_quantize(xd, gd, 1e-6, x_scale_f16=s16)
    ref_n = mcv.rms_norm(xd, gd, 1e-6)
    r16 = torch.empty(M, dtype=torch.float16, device="cuda")
    ref_q, ref_s, _ = mcv.w8a8_quantize(ref_n, x_scale_f16=r16)
    assert torch.equal(normed.view(torch.int16), ref_n.view(torch.int16))
    assert torch.equal(xq, ref_q)
    assert torch.equal(xs.view(torch.int32), ref_s.view(torch.int32))
    assert torch.equal(s16.view(torch.int16), r16.view(torch.int16))
    q_o, s_o, s16_o = oracle.w8a8_quantize_act(_u16(normed))
    assert np.array_equal(xq.cpu().numpy(), q_o)
    assert np.array_equal(xs.cpu().numpy().view(np.uint32), s_o.view(np.uint32))
    assert np.array_equal(_u16(s16), s16_o)
    # without the fp16 row
    none, xq2, xs2, _ = mcv.rms_norm_w8a8_quantize(xd, gd, 1e-6, want_normed=False)
    assert none is None and torch.equal(xq2, xq) and torch.equal(xs2, xs)
