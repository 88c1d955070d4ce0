"""Writes the committed golden fixtures (small .npz files) in tests/golden/.

The reference commits no fixtures: every one of its tests draws inputs at run
time.  These are therefore (a) the reference's deterministic test inputs with
the outputs its closed forms define (tests/test_w8a8_dequant.cpp:42-46,
tests/test_lm_head_pipeline.cpp:51-63), computed by the pinned oracle, and
(b) seeded build-defined vectors through the oracle, frozen so later changes
to the oracle or the product show up as a diff.  Run from the repository root:

    python tests/golden/make_golden.py
"""
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent))
from helpers import f16_normal, load_oracle  # noqa: E402


def main():
    o = load_oracle()
    # (a) reference deterministic vectors
    N = 3584
    acc = (np.arange(N) - 1024).astype(np.int32)[None, :]
    ws16 = o.f2h_trunc(np.float32(0.01) + (np.arange(N) % 7).astype(np.float32) * np.float32(0.001))
    xs16 = o.f2h_trunc(np.array([0.02], np.float32))
    out = o.w8a8_dequant(acc, o.h2f(xs16), o.h2f(ws16))
    np.savez_compressed(HERE / "w8a8_dequant_reference.npz", acc=acc, ws16=ws16, xs16=xs16, out16=out)

    Nr, H, V = 4, 64, 128
    i = np.arange(Nr * H)
    hid = o.f2h_trunc((((i * 13 + 7) % 31).astype(np.float32) / np.float32(31) - np.float32(0.5)) * np.float32(0.25))
    j = np.arange(H * V)
    wt = o.f2h_trunc((((j * 17 + 3) % 29).astype(np.float32) / np.float32(29) - np.float32(0.5)) * np.float32(0.5))
    hf, wf = o.h2f(hid).reshape(Nr, H), o.h2f(wt).reshape(H, V)
    tokens = []
    for n in range(Nr):
        a = np.zeros(V, np.float32)
        for h in range(H):
            a = (a + hf[n, h] * wf[h]).astype(np.float32)
        tokens.append(int(np.argmax(a)))
    np.savez_compressed(HERE / "lm_head_pipeline_reference.npz", hidden16=hid.reshape(Nr, H),
                        weight16=wt.reshape(H, V), tokens=np.array(tokens, np.int64))

    # (b) seeded build-defined vectors
    rng = np.random.default_rng(20261201)
    K, Nw, M = 256, 72, 2
    w = f16_normal(rng, (K, Nw), 0.02)
    qweight, qzeros, scales = o.quantize_int4_awq(w)
    w8 = o.unpack_awq(qweight, qzeros)
    x = f16_normal(rng, (M, K), 1.0)
    np.savez_compressed(HERE / "w4a16_small.npz", w16=w, x16=x, qweight=qweight, qzeros=qzeros, scales16=scales,
                        w8=w8, dequant16=o.w4a16_dequant_f16(w8, scales), out32=o.w4a16_matmul(x, w8, scales))

    Kq, Nq, Mq = 256, 64, 4
    wq16 = f16_normal(rng, (Kq, Nq), 0.02)
    xq16 = f16_normal(rng, (Mq, Kq), 1.0)
    q, s32, s16 = o.w8a8_quantize_weight(wq16)
    xq, xs32, xs16b = o.w8a8_quantize_act(xq16)
    acc2 = o.gemm_i32(xq, q)
    np.savez_compressed(HERE / "w8a8_small.npz", w16=wq16, x16=xq16, wq=q, ws32=s32, ws16=s16, xq=xq, xs32=xs32,
                        xs16=xs16b, acc=acc2, out16=o.w8a8_dequant(acc2, xs32, s32))
    print("wrote", sorted(p.name for p in HERE.glob("*.npz")))


if __name__ == "__main__":
    main()
