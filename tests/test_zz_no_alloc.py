"""The no-allocation lm_head entry point (mcv_w4a16_lm_head_argmax_noalloc)
through the C-ABI, against the workspace entry point it mirrors
(mcv_w4a16_lm_head_argmax): identical tokens and logits on two calls in a
row, the second with a smaller problem (smaller V, K and N), then the first
shape again."""
import ctypes

import numpy as np
import pytest

from helpers import f16_normal

pytestmark = pytest.mark.gpu


def _case(mcv, rng, K, N):
    import torch
    w = f16_normal(rng, (K, N), 0.02)
    qweight, qzeros, scales = mcv.quantize_int4(w)
    wq = mcv.W4A16QuantizedWeight.from_awq(qweight, qzeros, scales, device="cuda:0")
    x = torch.from_numpy(f16_normal(rng, (1, K), 1.0).view(np.int16)).cuda().view(torch.float16)
    return wq, x


def _workspace_route(mcv, wq, x, V):
    import torch
    L = mcv.lib()
    ws = torch.zeros(L.mcv_lm_head_workspace_bytes(V), dtype=torch.uint8, device="cuda")
    tok = torch.zeros(1, dtype=torch.int64, device="cuda")
    lg = torch.empty(V, dtype=torch.float16, device="cuda")
    q, s, z = wq.ptrs()
    rc = L.mcv_w4a16_lm_head_argmax(x.data_ptr(), wq.K, wq.N, V, q, s, z, wq.zero_bias, lg.data_ptr(), tok.data_ptr(),
                                    ws.data_ptr(), None, torch.cuda.current_stream().cuda_stream)
    assert rc == 0, L.mcv_last_error()
    torch.cuda.synchronize()
    return int(tok.item()), lg.cpu()


def _noalloc_route(mcv, wq, x, V):
    import torch
    L = mcv.lib()
    tok = torch.full((1,), -7, dtype=torch.int64, device="cuda")
    lg = torch.empty(V, dtype=torch.float16, device="cuda")
    q, s, z = wq.ptrs()
    rc = L.mcv_w4a16_lm_head_argmax_noalloc(x.data_ptr(), wq.K, wq.N, V, q, s, z, wq.zero_bias, lg.data_ptr(),
                                            tok.data_ptr(), None, torch.cuda.current_stream().cuda_stream)
    assert rc == 0, L.mcv_last_error()
    torch.cuda.synchronize()
    return int(tok.item()), lg.cpu()


def test_noalloc_lm_head_matches_workspace_route(mcv, cuda):
    import torch
    rng = np.random.default_rng(2024)
    L = mcv.lib()
    assert L.mcv_lm_head_noalloc_max_vocab() == 1 << 20
    big = (1024, 40000, 39999)          # K, N, V: 625 slabs, 40 workgroups
    small = (256, 4096, 3001)           # the second call: smaller in every dimension
    cases = {shape: _case(mcv, rng, shape[0], shape[1]) for shape in (big, small)}
    for shape in (big, small, big, big):
        wq, x = cases[shape]
        V = shape[2]
        want_tok, want_lg = _workspace_route(mcv, wq, x, V)
        got_tok, got_lg = _noalloc_route(mcv, wq, x, V)
        assert got_tok == want_tok, (shape, got_tok, want_tok)
        assert torch.equal(got_lg.view(torch.int16), want_lg.view(torch.int16)), shape
    # beyond the scratch: a clear error, nothing launched
    fake = ctypes.c_void_p(0x1000)
    rc = L.mcv_w4a16_lm_head_argmax_noalloc(fake, 128, (1 << 20) + 64, (1 << 20) + 1, fake, fake, fake, 0, None,
                                            fake, None, None)
    assert rc == 2 and b"scratch" in L.mcv_last_error()


def test_noalloc_lm_head_graph_replays_interleaved(mcv, cuda):
    """A captured noalloc call replays correctly between eager noalloc calls at
    another V: the array's generation word and fixed-offset keys live in
    device memory, so no host-side decision is baked into the graph."""
    import torch
    rng = np.random.default_rng(77)
    L = mcv.lib()
    big, small = (1024, 40000, 39999), (256, 4096, 3001)
    cases = {shape: _case(mcv, rng, shape[0], shape[1]) for shape in (big, small)}
    want = {shape: _workspace_route(mcv, *cases[shape], shape[2]) for shape in (big, small)}
    wq, x = cases[big]
    V = big[2]
    q, s, z = wq.ptrs()
    tok = torch.full((1,), -7, dtype=torch.int64, device="cuda")
    lg = torch.empty(V, dtype=torch.float16, device="cuda")
    _noalloc_route(mcv, wq, x, V)                       # an eager call before the capture
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(g, stream=side):
            rc = L.mcv_w4a16_lm_head_argmax_noalloc(x.data_ptr(), wq.K, wq.N, V, q, s, z, wq.zero_bias,
                                                    lg.data_ptr(), tok.data_ptr(), None, side.cuda_stream)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    assert rc == 0, L.mcv_last_error()
    for rep in range(4):
        got_small = _noalloc_route(mcv, *cases[small], small[2])      # eager, another V
        assert got_small[0] == want[small][0], (rep, got_small[0], want[small][0])
        tok.fill_(-7)
        lg.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert int(tok.item()) == want[big][0], (rep, int(tok.item()), want[big][0])
        assert torch.equal(lg.cpu().view(torch.int16), want[big][1].view(torch.int16)), rep
