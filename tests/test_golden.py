"""The committed golden fixtures (tests/golden/*.npz, written by
tests/golden/make_golden.py) are reproduced exactly by the oracle, by the
product's host code, and -- on a GPU -- by the kernels."""
from pathlib import Path

import numpy as np
import pytest

GOLD = Path(__file__).resolve().parent / "golden"


def load(name):
    return dict(np.load(GOLD / name, allow_pickle=False))


def test_oracle_reproduces_fixtures(oracle):
    d = load("w8a8_dequant_reference.npz")
    assert np.array_equal(oracle.w8a8_dequant(d["acc"], oracle.h2f(d["xs16"]), oracle.h2f(d["ws16"])), d["out16"])
    ref = d["acc"][0].astype(np.float32) * oracle.h2f(d["xs16"])[0] * oracle.h2f(d["ws16"])
    assert np.max(np.abs(d["out16"][0].view(np.float16).astype(np.float32) - ref)) < 0.02   # the reference's bound
    w = load("w4a16_small.npz")
    q, z, s = oracle.quantize_int4_awq(w["w16"])
    assert np.array_equal(q, w["qweight"]) and np.array_equal(z, w["qzeros"]) and np.array_equal(s, w["scales16"])
    assert np.array_equal(oracle.unpack_awq(q, z), w["w8"])
    assert np.array_equal(oracle.w4a16_matmul(w["x16"], w["w8"], w["scales16"]).view(np.uint32), w["out32"].view(np.uint32))
    assert np.array_equal(oracle.w4a16_dequant_f16(w["w8"], w["scales16"]), w["dequant16"])
    e = load("w8a8_small.npz")
    q, s32, s16 = oracle.w8a8_quantize_weight(e["w16"])
    assert np.array_equal(q, e["wq"]) and np.array_equal(s32, e["ws32"]) and np.array_equal(s16, e["ws16"])
    xq, xs32, xs16 = oracle.w8a8_quantize_act(e["x16"])
    assert np.array_equal(xq, e["xq"]) and np.array_equal(xs32, e["xs32"]) and np.array_equal(xs16, e["xs16"])
    assert np.array_equal(oracle.gemm_i32(xq, q), e["acc"])
    lm = load("lm_head_pipeline_reference.npz")
    hf = oracle.h2f(lm["hidden16"]).astype(np.float64)
    wf = oracle.h2f(lm["weight16"]).astype(np.float64)
    assert [int(np.argmax(hf[n] @ wf)) for n in range(4)] == lm["tokens"].tolist()


def test_product_host_code_reproduces_fixtures(mcv):
    w = load("w4a16_small.npz")
    for a, b in zip(mcv.quantize_int4(w["w16"]), (w["qweight"], w["qzeros"], w["scales16"])):
        assert np.array_equal(a.view(np.uint8), b.view(np.uint8))
    K, N = w["w16"].shape
    q, zeff, s = mcv.unpack(*mcv.pack_awq(w["qweight"], w["qzeros"], w["scales16"]), 0, K, N)
    assert np.array_equal(q.astype(np.int16) - np.repeat(zeff, 128, 0).astype(np.int16), w["w8"])
    e = load("w8a8_small.npz")
    q, s32, s16 = mcv.quantize_w8a8_weight_host(e["w16"])
    assert np.array_equal(q, e["wq"]) and np.array_equal(s32, e["ws32"]) and np.array_equal(s16, e["ws16"])


@pytest.mark.gpu
def test_kernels_reproduce_fixtures(mcv, cuda):
    import torch

    def f16(a):
        return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).cuda().view(torch.float16)

    def u16(t):
        return t.contiguous().cpu().view(torch.int16).numpy().view(np.uint16)

    w = load("w4a16_small.npz")
    wq = mcv.W4A16QuantizedWeight.from_awq(w["qweight"], w["qzeros"], w["scales16"])
    wf, w8 = mcv.w4a16_dequant(wq, f16=True, i8=True)
    assert np.array_equal(u16(wf), w["dequant16"]) and np.array_equal(w8.cpu().numpy(), w["w8"])
    for fn in (mcv.matmul_w4a16_gemv, mcv.matmul_w4a16_mfma):
        out = u16(fn(f16(w["x16"]), wq)).view(np.float16).astype(np.float32)
        assert np.abs(out - w["out32"]).max() <= 2e-2
    e = load("w8a8_small.npz")
    xq, xs, _ = mcv.w8a8_quantize(f16(e["x16"]))
    assert np.array_equal(xq.cpu().numpy(), e["xq"]) and np.array_equal(xs.cpu().numpy(), e["xs32"])
    acc = mcv.matmul_w8a8_i32(xq, torch.from_numpy(e["wq"]).cuda())
    assert np.array_equal(acc.cpu().numpy(), e["acc"])
    d = load("w8a8_dequant_reference.npz")
    out = mcv.w8a8_dequant(torch.from_numpy(d["acc"]).cuda(), f16(d["xs16"]), f16(d["ws16"]))
    assert np.array_equal(u16(out), d["out16"])


@pytest.mark.gpu
def test_lm_head_pipeline_fixture_on_gpu(mcv, cuda):
    """The reference's deterministic lm_head pipeline (tests/test_lm_head_pipeline.cpp:
    51-120: four rows whose maximum logit is shared by four columns each) through
    this build's argmax kernel: the logits on the device (fp32 products of the
    fp16 operands, rounded to fp16 -- equal columns give equal logits), then
    mcv_argmax_f16, whose first-maximum rule must return the fixture's tokens."""
    import torch
    lm = load("lm_head_pipeline_reference.npz")
    h = torch.from_numpy(lm["hidden16"].view(np.int16)).cuda().view(torch.float16)
    w = torch.from_numpy(lm["weight16"].view(np.int16)).cuda().view(torch.float16)
    logits = (h.float() @ w.float()).half()
    tok = mcv.argmax_last_dim(logits)
    assert tok.cpu().tolist() == lm["tokens"].tolist()
