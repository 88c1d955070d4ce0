"""The one-launch W4A16 decode MLP block (mcv_w4a16_mlp) against the
two-launch sequence it replaces (gate+up+silu*mul, then the down GEMV:
bit-identical) and against the oracle's formula (fp16 tolerance).  Shapes: the
model's H=1024, I=3584; H > I; ragged slab counts; a GPTQ-style zero bias."""
import numpy as np
import pytest

from helpers import f16_normal, rel_l2, synth_w4a16

pytestmark = pytest.mark.gpu

MAX_ABS, REL_L2 = 2e-2, 1e-3


def _torch():
    import torch
    return torch


def _to_dev(a_u16):
    torch = _torch()
    return torch.from_numpy(np.ascontiguousarray(a_u16).view(np.int16)).cuda().view(torch.float16)


def _weights(mcv, oracle, rng, K, N, zero_bias=0):
    _, qw, qz, sc = synth_w4a16(rng, K, N)
    w = mcv.W4A16QuantizedWeight.from_awq(qw, qz, sc)
    if zero_bias:
        w = mcv.W4A16QuantizedWeight(w.qweight, w.scales, w.zeros, K, N, 1)
    return w, (oracle.unpack_awq(qw, qz) - np.int8(zero_bias), sc)


@pytest.mark.parametrize("H,I,zb_down", [(1024, 3584, 0), (3584, 1024, 0), (256, 384, 1), (128, 128, 0),
                                         (1536, 4096, 0), (1024, 2048, 1)], ids=lambda v: str(v))
def test_decode_mlp_matches_two_launches_and_oracle(mcv, oracle, cuda, H, I, zb_down):
    torch = _torch()
    rng = np.random.default_rng(H * 7 + I)
    wg, rg = _weights(mcv, oracle, rng, H, I)
    wu, ru = _weights(mcv, oracle, rng, H, I)
    wd, rd = _weights(mcv, oracle, rng, I, H, zb_down)
    mlp = mcv.DecodeMlpW4A16(wg, wu, wd)
    out = torch.empty((1, H), dtype=torch.float16, device="cuda")
    for trial in range(3):                       # the call counters advance call after call
        assert mlp.one_launch
        x = f16_normal(rng, (1, H), 1.0 + trial)
        xd = _to_dev(x)
        out.fill_(0)
        mlp(xd, out)
        act = mcv.mlp_gate_up_silu_w4a16(xd, wg, wu)
        two = mcv.matmul_w4a16(act, wd)
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), two.view(torch.int16)), f"trial {trial}"
        a_o = oracle.silu_mul(oracle.f2h_rne(oracle.w4a16_matmul(x, *rg)), oracle.f2h_rne(oracle.w4a16_matmul(x, *ru)))
        ref = oracle.w4a16_matmul(a_o.reshape(1, I), *rd)
        got = out.float().cpu().numpy()
        assert np.abs(got - ref).max() <= MAX_ABS and rel_l2(got, ref) <= REL_L2
    assert not mlp.act_wait_gave_up()


def test_decode_mlp_bound_and_back_to_back(mcv, oracle, cuda):
    """Many calls queued back to back (each one waits for its own call tag,
    never an older one) give the same rows as one-by-one calls."""
    torch = _torch()
    H, I = 1024, 3584
    rng = np.random.default_rng(5)
    wg, _ = _weights(mcv, oracle, rng, H, I)
    wu, _ = _weights(mcv, oracle, rng, H, I)
    wd, _ = _weights(mcv, oracle, rng, I, H)
    mlp = mcv.DecodeMlpW4A16(wg, wu, wd)
    xs = [_to_dev(f16_normal(rng, (1, H), 1.0)) for _ in range(4)]
    want = [mlp(x).clone() for x in xs]
    outs = [torch.empty((1, H), dtype=torch.float16, device="cuda") for _ in xs]
    launches = [mlp.bind(x, o) for x, o in zip(xs, outs)]
    for _ in range(20):
        for f in launches:
            f()
    torch.cuda.synchronize()
    for o, w in zip(outs, want):
        assert torch.equal(o.view(torch.int16), w.view(torch.int16))
    assert not mlp.act_wait_gave_up()


def test_decode_mlp_graph_replay(mcv, oracle, cuda):
    """Captured in a HIP graph and replayed several times, with eager work
    and synchronisations in between, every replay equals the eager result."""
    torch = _torch()
    H, I = 1024, 3584
    rng = np.random.default_rng(6)
    wg, _ = _weights(mcv, oracle, rng, H, I)
    wu, _ = _weights(mcv, oracle, rng, H, I)
    wd, _ = _weights(mcv, oracle, rng, I, H)
    mlp = mcv.DecodeMlpW4A16(wg, wu, wd)
    x = _to_dev(f16_normal(rng, (1, H), 1.0))
    want = mlp(x).clone()
    out = torch.empty((1, H), dtype=torch.float16, device="cuda")
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            mlp(x, out, stream=s)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    for _ in range(4):
        out.fill_(0)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), want.view(torch.int16))
        mlp(x)                                   # eager call between replays
        torch.cuda.synchronize()
    assert not mlp.act_wait_gave_up()


def test_decode_mlp_rejects_bad_shapes(mcv, oracle, cuda):
    torch = _torch()
    rng = np.random.default_rng(8)
    wg, _ = _weights(mcv, oracle, rng, 256, 384)
    wu, _ = _weights(mcv, oracle, rng, 256, 384)
    wd, _ = _weights(mcv, oracle, rng, 384, 256)
    with pytest.raises(mcv.McvError):
        mcv.DecodeMlpW4A16(wg, wu, wg)           # down must be [I, H]



def test_decode_mlp_falls_back_to_two_launches(mcv, oracle, cuda):
    """I = 6144 puts three down-projection groups on a wave slot: the
    one-launch kernel refuses it and the object runs the two launches."""
    torch = _torch()
    rng = np.random.default_rng(9)
    H, I = 256, 6144
    wg, rg = _weights(mcv, oracle, rng, H, I)
    wu, ru = _weights(mcv, oracle, rng, H, I)
    wd, rd = _weights(mcv, oracle, rng, I, H)
    mlp = mcv.DecodeMlpW4A16(wg, wu, wd)
    x = f16_normal(rng, (1, H), 1.0)
    xd = _to_dev(x)
    out = mlp(xd)
    assert not mlp.one_launch
    two = mcv.matmul_w4a16(mcv.mlp_gate_up_silu_w4a16(xd, wg, wu), wd)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), two.view(torch.int16))
    a_o = oracle.silu_mul(oracle.f2h_rne(oracle.w4a16_matmul(x, *rg)), oracle.f2h_rne(oracle.w4a16_matmul(x, *ru)))
    ref = oracle.w4a16_matmul(a_o.reshape(1, I), *rd)
    got = out.float().cpu().numpy()
    assert np.abs(got - ref).max() <= MAX_ABS and rel_l2(got, ref) <= REL_L2
    mlp = mcv.DecodeMlpW4A16(wg, wu, wd)
    with pytest.raises(mcv.McvError):
        mlp(torch.zeros((1, 128), dtype=torch.float16, device="cuda"))
    with pytest.raises(mcv.McvError):
        mlp(torch.zeros((1, 256), dtype=torch.float16, device="cuda"),
            torch.empty((1, 128), dtype=torch.float16, device="cuda"))
