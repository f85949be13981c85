"""CPU: pins the oracle's integer products and activation epilogue."""
import math

import numpy as np

import oracle as O
from test_oracle_dequant import enc_q6_k


def test_gemm_i8_nt_matches_int64_matmul():
    rng = np.random.default_rng(21)
    A = rng.integers(-128, 128, (37, 300)).astype(np.int8)
    B = rng.integers(-128, 128, (23, 300)).astype(np.int8)
    assert np.array_equal(O.c_gemm_i8_nt(A, B), A.astype(np.int64) @ B.astype(np.int64).T)
    # extreme magnitudes: K * 127^2 at the configuration's K stays exact
    A = np.full((2, 5120), 127, np.int8)
    assert O.c_gemm_i8_nt(A, A)[0, 0] == 5120 * 127 * 127


def test_q6k_q8_1_partials_from_encoded_fields():
    """Partials against sums formed directly from the generator's integer
    fields (6-bit codes, scales, q8), encoded with ggml's Q6_K writer."""
    rng = np.random.default_rng(22)
    N, K, M = 3, 512, 2
    nsb = K // 256
    L = rng.integers(0, 64, (N, nsb, 256))
    sc = rng.integers(-128, 128, (N, nsb, 16)).astype(np.int8)
    w = np.zeros((N, nsb, 210), np.uint8)
    for n in range(N):
        for s in range(nsb):
            ql, qh = enc_q6_k(L[n, s])
            w[n, s, :128], w[n, s, 128:192] = ql, qh
            w[n, s, 192:208] = sc[n, s].view(np.uint8)
            w[n, s, 208:210] = np.array([1.0], np.float16).view(np.uint8)
    x = rng.normal(0, 1, (M, K)).astype(np.float32)
    xq = O.c_quantize_q8_1(x).reshape(M, K // 32, 36)
    q8 = xq[:, :, 4:].view(np.int8).astype(np.int64).reshape(M, K)
    wv = (sc.astype(np.int64).repeat(16, axis=2) * (L - 32)).reshape(N, K)
    expect = (q8[:, None, :] * wv[None, :, :]).reshape(M, N, K // 32, 32).sum(-1)
    P = O.c_q6k_q8_1_partials(w.reshape(N, -1), xq.reshape(M, -1), M, N, K)
    assert np.array_equal(P.astype(np.int64), expect)


def test_activation_epilogue():
    for v in (-6.0, -1.3, -0.2, 0.0, 0.4, 2.0, 9.0):
        assert O.c_act(0, v) == np.float32(v)
        assert O.c_act(2, v) == max(np.float32(v), 0)
        assert abs(O.c_act(1, v) - v / (1 + math.exp(-v))) <= 1e-6 * max(1, abs(v))
        # A&S 7.1.26 erf is within 1.5e-7 of erf: GELU within ~1e-6 of the exact form
        assert abs(O.c_act(3, v) - 0.5 * v * (1 + math.erf(v / math.sqrt(2)))) <= 2e-6 * max(1, abs(v))
        assert abs(float(O.np_act(3, np.array([v], np.float32))[0]) - O.c_act(3, v)) <= 1e-6 * max(1, abs(v))
