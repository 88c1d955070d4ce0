"""Pins the oracle's silu*mul (op_kernel/silu_mul_custom.cpp:59-75) and greedy
argmax (language_model.cpp:444-479), including the reference's lm_head
pipeline test patterns (tests/test_lm_head_pipeline.cpp:51-63,95-107)."""
import numpy as np

from helpers import f16_normal


def test_silu_mul_within_one_ulp(oracle):
    rng = np.random.default_rng(14)
    g = f16_normal(rng, 50000, 3.0)
    u = f16_normal(rng, 50000, 2.0)
    got = oracle.silu_mul(g, u).view(np.float16).astype(np.float64)
    gf = g.view(np.float16).astype(np.float64)
    uf = u.view(np.float16).astype(np.float64)
    ref = (gf / (1 + np.exp(-gf)) * uf).astype(np.float16)
    ulp = np.abs(np.spacing(ref.astype(np.float16))).astype(np.float64)
    assert (np.abs(got - ref.astype(np.float64)) <= ulp).all()
    assert (got == ref.astype(np.float64)).mean() > 0.99


def _ftz(h):
    v = h.view(np.float16).astype(np.float32)
    sub = (h & 0x7C00) == 0
    return np.where(sub, np.float32(0), v)


def test_argmax_first_max_and_specials(oracle):
    rng = np.random.default_rng(15)
    for trial in range(50):
        n = int(rng.integers(1, 3000))
        h = f16_normal(rng, n, 1.0)
        if trial % 5 == 1:
            h[rng.integers(0, n, 5)] = h.max() if h.max() < 0x7C00 else h[0]  # ties
        if trial % 5 == 2:
            h[rng.integers(0, n, 3)] = 0x7E00                                # NaNs
        v = _ftz(h)
        vv = np.where(np.isnan(v), -np.inf, v)
        want = int(np.argmax(vv)) if np.isfinite(vv).any() or (vv == np.inf).any() else 0
        if not (vv > -np.inf).any():
            want = 0
        assert oracle.argmax_f16(h) == want


def test_argmax_edge_rows(oracle):
    assert oracle.argmax_f16(np.full(10, 0xFC00, np.uint16)) == 0          # all -inf
    assert oracle.argmax_f16(np.full(10, 0x7E00, np.uint16)) == 0          # all NaN
    h = np.array([0x8001, 0x0001, 0x0000, 0x8000], np.uint16)               # subnormals == 0: first wins
    assert oracle.argmax_f16(h) == 0
    h = np.array([0xBC00, 0x0001, 0x3C00, 0x3C00], np.uint16)
    assert oracle.argmax_f16(h) == 2
    assert oracle.argmax_f16(np.array([0xFC00, 0x7C00, 0x7C00], np.uint16)) == 1


def test_reference_lm_head_pipeline_patterns(oracle):
    # hidden[i] = ((i*13+7)%31/31 - 0.5)*0.25, weight[i] = ((i*17+3)%29/29 - 0.5)*0.5,
    # both through the test's truncating f2h; logits by the test's fp32 loop; strict '>'.
    N, H, V = 4, 64, 128
    i = np.arange(N * H)
    hid = oracle.f2h_trunc((((i * 13 + 7) % 31).astype(np.float32) / np.float32(31) - np.float32(0.5)) * np.float32(0.25))
    j = np.arange(H * V)
    wt = oracle.f2h_trunc((((j * 17 + 3) % 29).astype(np.float32) / np.float32(29) - np.float32(0.5)) * np.float32(0.5))
    hf = oracle.h2f(hid).reshape(N, H)
    wf = oracle.h2f(wt).reshape(H, V)
    tokens = []
    for n in range(N):
        acc = np.zeros(V, np.float32)
        for h in range(H):
            acc = (acc + hf[n, h] * wf[h]).astype(np.float32)
        best, bv = -1, -np.inf
        for v in range(V):
            if acc[v] > bv:
                bv, best = acc[v], v
        tokens.append(best)
        # the oracle's argmax over the fp16 logits agrees when the maximum is unique in fp16
        logits16 = acc.astype(np.float16).view(np.uint16)
        if (logits16 == logits16[best]).sum() == 1:
            assert oracle.argmax_f16(logits16) == best
    ref64 = [int(np.argmax(hf[n].astype(np.float64) @ wf.astype(np.float64))) for n in range(N)]
    assert tokens == ref64


def test_rms_norm_vs_float64(oracle):
    rng = np.random.default_rng(16)
    x = f16_normal(rng, (4, 1024), 1.0)
    x[2] = 0
    g = f16_normal(rng, 1024, 0.5)
    got = oracle.rms_norm(x, g, 1e-6).view(np.float16).astype(np.float64)
    xf = x.view(np.float16).astype(np.float64)
    ref = (xf / np.sqrt((xf ** 2).mean(axis=1, keepdims=True) + 1e-6) * g.view(np.float16).astype(np.float64)).astype(np.float16)
    ulp = np.abs(np.spacing(ref)).astype(np.float64)
    assert (np.abs(got - ref.astype(np.float64)) <= ulp + 1e-12).all()
    assert (got[2] == 0).all()
