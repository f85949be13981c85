"""CPU: pins the oracle's Q8_1 quantizer (ggml quantize_row_q8_1_ref rule,
which the reference's kernels/dequant_q8_1.glsl decodes but never produces).

Invariants that do not restate the code: |q| <= 127; the largest |x| of a
block maps to |q| = 127; |x - d*q| <= d/2 (+1 ulp); dequantising with the
oracle's Q8_1 decoder gives fp16(d)*q; s is fp16 of the fp32 product
float(sum q) * d (two roundings, as ggml's FP32_TO_FP16(sum*d) writes it).
"""
import numpy as np

import oracle as O

# A block of the benchmark's C5 activations (seed 1050, block 10086) where
# rounding sum*d once, straight to fp16, gives 0xC823 but the reference's
# fp32-then-fp16 rounding gives 0xC824 (a compiler fold of the two
# conversions into one mixed-precision FMA produced the former on the GPU).
DOUBLE_ROUNDING_BLOCK = np.array([
    1.033948540687561, -0.4651213586330414, 0.35263121128082275, 0.10091086477041245,
    -0.18085873126983643, 0.22475922107696533, 1.4879918098449707, -0.7829322218894958,
    -0.3093419671058655, 0.46353450417518616, -0.6165685653686523, -0.6127054691314697,
    -1.806795358657837, -0.37307751178741455, 0.3104515075683594, -0.161019429564476,
    0.007352560758590698, -0.5750263929367065, -0.6947004795074463, -0.459099143743515,
    0.6835755109786987, -2.3053128719329834, 0.954106867313385, -1.7606369256973267,
    -0.35235634446144104, -2.0800135135650635, -0.5899048447608948, -1.409772515296936,
    -0.46246564388275146, 0.83463054895401, 1.8862159252166748, -0.6178545951843262], np.float32)


def _fields(qb):
    qb = qb.reshape(-1, 36)
    d = qb[:, 0:2].copy().view(np.float16).reshape(-1)
    s = qb[:, 2:4].copy().view(np.float16).reshape(-1)
    q = qb[:, 4:].view(np.int8).astype(np.int64)
    return d, s, q


def _inputs():
    rng = np.random.default_rng(11)
    x = [rng.normal(0, 1, 32 * 500), rng.normal(0, 1e-6, 32 * 50), rng.normal(0, 3e4, 32 * 50),
         np.zeros(32), np.arange(32) - 15.5, DOUBLE_ROUNDING_BLOCK]
    return np.concatenate(x).astype(np.float32)


def test_c_equals_numpy_twin():
    x = _inputs()
    assert np.array_equal(O.c_quantize_q8_1(x), O.np_quantize_q8_1(x))


def test_invariants():
    x = _inputs().reshape(-1, 32)
    d, s, q = _fields(O.c_quantize_q8_1(x))
    amax = np.abs(x).max(1).astype(np.float64)
    d32 = (amax.astype(np.float32) / np.float32(127)).astype(np.float64)
    assert np.all(np.abs(q) <= 127)
    nz = amax > 0
    top = np.abs(x).argmax(1)
    assert np.all(np.abs(q[np.arange(len(q)), top])[nz] == 127)
    assert np.all(q[~nz] == 0) and np.all(d[~nz] == 0)
    err = np.abs(x.astype(np.float64) - d32[:, None] * q)
    assert np.all(err[nz] <= d32[nz, None] * (0.5 + 1e-6))
    assert np.array_equal(d, d32.astype(np.float32).astype(np.float16))   # fp16(d), d = amax/127 in fp32
    # decoding with the oracle's Q8_1 decoder gives fp16(d) * q exactly
    y = O.c_dequant(O.Q8_1, O.c_quantize_q8_1(x.reshape(-1))).reshape(-1, 32)
    assert np.array_equal(y.astype(np.float64), d.astype(np.float64)[:, None] * q)


def test_s_is_double_rounded():
    x = DOUBLE_ROUNDING_BLOCK
    d, s, q = _fields(O.c_quantize_q8_1(x))
    d32 = np.float32(np.abs(x).max()) / np.float32(127)
    prod32 = np.float32(q.sum()) * d32                         # fp32 product, then fp16
    assert s[0].view(np.uint16) == np.float16(prod32).view(np.uint16) == 0xC824
    single = np.float16(float(q.sum()) * float(d32))           # one rounding of the exact product
    assert single.view(np.uint16) == 0xC823                    # so the test tells the two rules apart


def test_round_half_away_from_zero():
    # amax = 127 -> d = 1, id = 1: x*id = x exactly, so ties show the rounding rule
    x = np.zeros(32, np.float32)
    x[0] = 127.0
    x[1:9] = [0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 3.49999976, -126.5]
    _, _, q = _fields(O.c_quantize_q8_1(x))
    assert q[0, :9].tolist() == [127, 1, 2, 3, -1, -2, -3, 3, -127]
