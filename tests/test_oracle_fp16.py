"""Pins the oracle's fp16 conversions.

or_h2f / or_f2h_rne are checked against numpy's IEEE binary16 conversions
exhaustively; or_f2h_trunc (the reference's truncating encode,
quantized_weight.cpp:186-195) against a brute-force characterisation: the
largest-magnitude fp16 not above |f|, zero below the smallest normal,
infinity from 65536 up.  or_h2f_ftz (language_model.cpp:444-459) flushes
subnormals.
"""
import numpy as np

ALL = np.arange(65536, dtype=np.uint32).astype(np.uint16)


def test_h2f_exhaustive(oracle):
    got = oracle.h2f(ALL)
    ref = ALL.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_h2f_ftz_flushes_subnormals_only(oracle):
    for h in [0x0001, 0x03FF, 0x8001, 0x83FF, 0x0000, 0x8000]:
        v = oracle.L.or_h2f_ftz(h)
        assert v == 0.0 and (np.signbit(np.float32(v)) == bool(h & 0x8000))
    for h in [0x0400, 0x3C00, 0xFBFF, 0x7C00, 0xFC00, 0x1234]:
        assert oracle.L.or_h2f_ftz(h) == oracle.L.or_h2f(h)


def test_f2h_rne_matches_numpy(oracle):
    rng = np.random.default_rng(0)
    f = np.concatenate([
        rng.standard_normal(200000).astype(np.float32) * 10,
        (rng.standard_normal(100000) * 1e-5).astype(np.float32),            # subnormal fp16 range
        (rng.standard_normal(50000) * 3e4).astype(np.float32),             # near overflow
        np.array([65504, 65519.99, 65520, 1e9, -1e9, 0.0, -0.0, np.inf, -np.inf, 2.0**-25, 2.0**-24,
                  3 * 2.0**-26, 2.0**-26], np.float32),
    ])
    got = oracle.f2h_rne(f)
    with np.errstate(over="ignore"):                     # the overflow cases are deliberate
        ref = f.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, ref)


def test_f2h_rne_ties_to_even(oracle):
    # exact midpoints between consecutive fp16 values (all are fp32-representable)
    h = np.arange(0x0000, 0x7BFF, dtype=np.uint32).astype(np.uint16)
    lo = h.view(np.float16).astype(np.float64)
    hi = (h + 1).view(np.float16).astype(np.float64)
    mid = ((lo + hi) / 2).astype(np.float32)
    got = oracle.f2h_rne(mid)
    expect = np.where(h % 2 == 0, h, h + 1).astype(np.uint16)
    assert np.array_equal(got, expect)


def test_f2h_rne_roundtrip_exhaustive(oracle):
    f = ALL.view(np.float16).astype(np.float32)
    ok = ~np.isnan(f)
    assert np.array_equal(oracle.f2h_rne(f[ok]), ALL[ok])


def test_f2h_trunc_is_largest_not_above(oracle):
    rng = np.random.default_rng(1)
    f = np.concatenate([rng.standard_normal(100000) * 100, rng.standard_normal(50000) * 1e-3,
                        rng.uniform(6e4, 7e4, 1000) * rng.choice([-1, 1], 1000)]).astype(np.float32)
    t = oracle.f2h_trunc(f)
    tv = t.view(np.float16).astype(np.float64)
    af = np.abs(f.astype(np.float64))
    sign_ok = (np.signbit(tv) == np.signbit(f))
    assert sign_ok.all()
    tiny = af < 2.0 ** -14
    big = af >= 65536.0
    mid = ~tiny & ~big
    assert (tv[tiny] == 0).all()
    assert np.isinf(tv[big]).all()
    # largest fp16 magnitude <= |f|: |t| <= |f| < next fp16 above |t|
    at = np.abs(tv[mid])
    with np.errstate(over="ignore"):                     # 65504 steps to inf
        nxt = np.nextafter(np.abs(t[mid].view(np.float16)), np.float16(np.inf)).astype(np.float64)
    assert (at <= af[mid]).all() and (af[mid] < nxt).all()


def test_f2h_trunc_nan_becomes_inf(oracle):
    # exponent field 255 maps to >= 31: the reference encodes NaN as infinity
    assert oracle.L.or_f2h_trunc(float("nan")) in (0x7C00, 0xFC00)


def test_bf16_to_f16_trunc_exhaustive(oracle):
    """All 65536 bf16 patterns: where the value is an fp16 normal the
    conversion is exact (bf16's 7 mantissa bits fit in fp16's 10); below the
    fp16 normal range it is signed zero (no subnormals), above it and for NaN
    signed infinity (language_model loads, src/csrc/lib/weights.cpp:25-33)."""
    bf = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = oracle.bf16_to_f16_trunc(bf)
    val = (bf.astype(np.uint32) << 16).view(np.float32)
    sign = (bf & 0x8000).astype(np.uint16)
    a = np.abs(val)
    normal = (a >= np.float32(2.0 ** -14)) & (a < np.float32(65536.0))
    assert np.array_equal(got[normal], val[normal].astype(np.float16).view(np.uint16))
    assert np.array_equal(got[normal].view(np.float16).astype(np.float32), val[normal])   # exact
    low = a < np.float32(2.0 ** -14)
    assert np.array_equal(got[low], sign[low])
    high = ~normal & ~low                                         # >= 65536, inf, NaN
    assert np.array_equal(got[high], sign[high] | np.uint16(0x7C00))
    # known answers
    assert oracle.bf16_to_f16_trunc(np.array([0x3F80, 0xC020, 0x4780, 0x7FC0, 0x3880, 0x387F], np.uint16)).tolist() == \
        [0x3C00, 0xC100, 0x7C00, 0x7C00, 0x0400, 0x0000]
