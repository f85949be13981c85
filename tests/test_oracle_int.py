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


def test_act_i8_quantiser_known_answers():
    """kernels/linear_int8.glsl:63-70 worked by hand: q = clamp(round(x /
    act_scale), -127, 127), halves to even, in float32."""
    x = np.array([0.0, 1.0, -1.0, 2.5, 3.5, -2.5, -0.5, 0.49, 126.6, 200.0, -300.0, 65504.0], np.float16)
    assert O.np_quantize_act_i8(x, 1.0).tolist() == [0, 1, -1, 2, 4, -2, 0, 0, 127, 127, -127, 127]
    # act_scale 0.25: x / 0.25 exact (a power of two), 0.125 -> 0.5 -> 0, 0.375 -> 1.5 -> 2
    y = np.array([0.125, 0.375, -0.375, 1.0, 31.75, 32.0], np.float16)
    assert O.np_quantize_act_i8(y, 0.25).tolist() == [0, 2, -2, 4, 127, 127]


def test_act_i8_quantiser_identity_and_row_rule():
    """With act_scale = 1, integer-valued fp16 activations in [-127, 127] pass
    through unchanged (the reference's only act_scale); with each row's own
    max|x|/127 it is the per-row quantiser (tools/quantise.py:35-41)."""
    rng = np.random.default_rng(11)
    a = rng.integers(-127, 128, (7, 300)).astype(np.float16)
    assert np.array_equal(O.np_quantize_act_i8(a, 1.0), a.astype(np.int8))
    x = (rng.normal(0, 2, (5, 256))).astype(np.float16)
    q_rows, s_rows = O.np_quantize_rows_i8(x.astype(np.float32))
    for m in range(5):
        assert np.array_equal(O.np_quantize_act_i8(x[m], float(s_rows[m])), q_rows[m])


def test_ref_linear_int8_fp16a_exact_core():
    """The reference contract's int32 core equals the int64 product of the
    quantised operands; with act_scale 1 and integer A it is A . W^T."""
    rng = np.random.default_rng(12)
    A = rng.integers(-127, 128, (9, 160)).astype(np.float16)
    W = rng.integers(-127, 128, (11, 160)).astype(np.int8)
    acc, y = O.ref_linear_int8_fp16a(A, W, 1.0, None)
    assert np.array_equal(acc, A.astype(np.int64) @ W.astype(np.int64).T)
    assert np.array_equal(y, acc.astype(np.float32))
    ws = np.abs(rng.normal(0, 0.01, 11)).astype(np.float32)
    acc2, y2 = O.ref_linear_int8_fp16a(A * np.float16(0.5), W, 0.5, ws)
    assert np.array_equal(acc2, acc)  # (A/2) / 0.5 = A exactly
    assert np.allclose(y2, acc * ws[None, :] * 0.5, rtol=1e-6)


def test_q8_0_q8_1_partials_known_answers_and_sums():
    """Block dots of Q8_0 x Q8_1 codes: a hand-worked pair of blocks, and on
    random blocks the sum over blocks equals the int8 GEMM of the codes
    (vkfo_gemm_i8_nt) while each block equals its own slice's product."""
    w = np.zeros((1, 34), np.uint8)
    x = np.zeros((1, 36), np.uint8)
    qw = np.arange(-16, 16, dtype=np.int8)
    qx = np.full(32, 3, np.int8)
    qx[0] = -127
    w[0, 2:] = qw.view(np.uint8)
    x[0, 4:] = qx.view(np.uint8)
    # sum(3 * q) over q = -16..15 is -48, with q = -16 at index 0 weighted -127 instead of 3: -48 - 3*(-16) + (-127)*(-16)
    assert O.np_q8_0_q8_1_partials(w, x, 1, 1, 32)[0, 0, 0] == -48 + 48 + 2032
    M, N, K = 5, 7, 160
    w = O.gen_weight(O.Q8_0, N, K, 21)
    xq = O.np_quantize_q8_1(np.random.default_rng(22).normal(0, 1, (M, K)).astype(np.float32)).reshape(M, -1)
    P = O.np_q8_0_q8_1_partials(w, xq, M, N, K)
    codes_w = w.reshape(N, K // 32, 34)[:, :, 2:].reshape(N, K).view(np.int8)
    codes_x = xq.reshape(M, K // 32, 36)[:, :, 4:].reshape(M, K).view(np.int8)
    assert np.array_equal(P.astype(np.int64).sum(axis=2), O.c_gemm_i8_nt(codes_x, codes_w).astype(np.int64))
    for kb in range(K // 32):
        sl = slice(32 * kb, 32 * kb + 32)
        assert np.array_equal(P[:, :, kb], O.c_gemm_i8_nt(np.ascontiguousarray(codes_x[:, sl]),
                                                           np.ascontiguousarray(codes_w[:, sl])))
