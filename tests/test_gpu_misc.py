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
