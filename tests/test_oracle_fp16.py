"""CPU: the oracle's fp16 conversions against numpy's (IEEE binary16, round
to nearest even, subnormals kept) — exhaustive for fp16 -> fp32, and for
fp32 -> fp16 every tie point, its neighbours and a large random sample."""
import numpy as np

import oracle as O


def _c_h2f_all():
    # vectorise through the dequantiser: Q8_0 blocks with q = 1 give d exactly
    h = np.arange(65536, dtype=np.uint16)
    b = np.zeros((65536, 34), np.uint8)
    b[:, 0:2] = h.view(np.uint8).reshape(-1, 2)
    b[:, 2] = 1
    return O.c_dequant(O.Q8_0, b).reshape(-1, 32)[:, 0]


def test_h2f_exhaustive():
    got = _c_h2f_all()
    ref = np.arange(65536, dtype=np.uint16).view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))
    assert np.all(np.isnan(got[nan]))
    # spot values through the scalar entry point
    assert O.c_h2f(0x0001) == 2.0 ** -24 and O.c_h2f(0x7BFF) == 65504.0 and O.c_h2f(0x8400) == -(2.0 ** -14)


def _f2h_many(x):
    return np.array([O.c_f2h(float(v)) for v in x], np.uint16)


def test_f2h_ties_and_neighbours():
    h = np.arange(0, 0x7C00, dtype=np.uint16)          # every finite non-negative half
    lo = h[:-1].view(np.float16).astype(np.float64)
    hi = h[1:].view(np.float16).astype(np.float64)
    mid = ((lo + hi) / 2).astype(np.float32)             # exact tie points (all representable in fp32)
    sample = np.concatenate([mid, np.nextafter(mid, np.float32(0)), np.nextafter(mid, np.float32(1e9))])
    sample = sample[::7]                                   # bounded CPU time, still every tie class
    for s in (sample, -sample):
        assert np.array_equal(_f2h_many(s), s.astype(np.float16).view(np.uint16))


def test_f2h_random_and_specials():
    rng = np.random.default_rng(5)
    x = np.concatenate([
        rng.normal(0, 1, 20000), rng.normal(0, 1e-5, 20000), rng.normal(0, 3e4, 5000),
        [0.0, -0.0, 65504.0, 65519.99, 65520.0, 1e9, -1e9, 2.0 ** -25, 2.0 ** -25 * 1.0000001,
         2.0 ** -24, 1.5 * 2.0 ** -24, 2.5 * 2.0 ** -24, np.inf, -np.inf]]).astype(np.float32)
    with np.errstate(over="ignore"):
        assert np.array_equal(_f2h_many(x), x.astype(np.float16).view(np.uint16))
    assert O.c_f2h(float("nan")) & 0x7C00 == 0x7C00 and O.c_f2h(float("nan")) & 0x3FF
