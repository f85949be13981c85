"""GPU parity: decode GEMV / small GEMM (M <= 16) over ggml weights
(vkflame_dispatch_gemm_q through the C ABI) against the float64 product of
the oracle's exact dequantised operands; Q6_K x Q8_1 integer partials
bit-exact."""
import numpy as np
import pytest

import oracle as O
from _util import TOL_F32, bits_equal, first_mismatch, rel_err, seed_for, to_dev

pytestmark = pytest.mark.gpu

WTYPES = [O.Q4_0, O.Q4_1, O.Q8_0, O.Q5_0, O.Q4_K, O.Q5_K, O.Q6_K]


def _x(kind, M, K, seed):
    rng = np.random.default_rng(seed)
    x = rng.normal(0, 1, (M, K)).astype(np.float32)
    if kind == "f16":
        return x.astype(np.float16), x.astype(np.float16).astype(np.float64)
    if kind == "f32":
        return x, x.astype(np.float64)
    q = O.np_quantize_q8_1(x).reshape(M, -1)
    return q, O.np_dequant(O.Q8_1, q).reshape(M, K).astype(np.float64)


@pytest.mark.parametrize("qt", WTYPES, ids=[O.QNAMES[q] for q in WTYPES])
@pytest.mark.parametrize("kind", ["f16", "f32", "q8_1"])
@pytest.mark.parametrize("M", [1, 3, 16])
def test_gemv_small(dev, qt, kind, M):
    import torch
    from vkflame_amd import ops
    N, K = 77, 2048 + (256 if O.BLOCK_ELEMS[qt] == 256 else 32)   # ragged N, K not a multiple of 64 chunks
    w = O.gen_weight(qt, N, K, seed_for(2, qt))
    xa, x64 = _x(kind, M, K, seed_for(2, 10 + M))
    y = ops.gemm_q(to_dev(w, dev), qt, to_dev(xa, dev), N, K)
    torch.cuda.synchronize()
    ref = O.ref_gemv(x64, O.np_dequant(qt, w).reshape(N, K))
    assert rel_err(y.cpu().numpy(), ref) <= TOL_F32


def test_gemv_accumulates_into_strided_output(dev):
    """ldy > N: output rows land at their stride, padding untouched."""
    import torch
    from vkflame_amd import ops
    N, K, M = 64, 512, 4
    w = O.gen_weight(O.Q4_K, N, K, seed_for(2, 50))
    xa, x64 = _x("f16", M, K, seed_for(2, 51))
    ybig = torch.full((M, N + 8), 7.0, device=dev)
    ops.gemm_q(to_dev(w, dev), O.Q4_K, to_dev(xa, dev), N, K, out=ybig[:, :N])
    torch.cuda.synchronize()
    yb = ybig.cpu().numpy()
    assert np.all(yb[:, N:] == 7.0)
    assert rel_err(yb[:, :N], O.ref_gemv(x64, O.np_dequant(O.Q4_K, w).reshape(N, K))) <= TOL_F32


def _rows_check(y, x64, w, qt, K, rows):
    wd = O.np_dequant(qt, w[rows]).reshape(len(rows), K)
    return rel_err(y[:, rows], O.ref_gemv(x64, wd))


def test_config1_q8_0_gemv(dev):
    import torch
    from vkflame_amd import ops
    N = K = 4096
    w = O.gen_weight(O.Q8_0, N, K, seed_for(1))
    xa, x64 = _x("f32", 1, K, seed_for(1, 1))
    y = ops.gemm_q(to_dev(w, dev), O.Q8_0, to_dev(xa, dev), N, K)
    torch.cuda.synchronize()
    assert rel_err(y.cpu().numpy(), O.ref_gemv(x64, O.np_dequant(O.Q8_0, w).reshape(N, K))) <= TOL_F32


@pytest.mark.parametrize("qt", [O.Q4_0, O.Q4_1], ids=["q4_0", "q4_1"])
@pytest.mark.parametrize("M", [1, 4, 16])
def test_config2_q4_gemv(dev, qt, M):
    import torch
    from vkflame_amd import ops
    N, K = 11008, 4096
    w = O.gen_weight(qt, N, K, seed_for(2, qt))
    xa, x64 = _x("f16", M, K, seed_for(2, M))
    y = ops.gemm_q(to_dev(w, dev), qt, to_dev(xa, dev), N, K).cpu().numpy()
    rows = np.random.default_rng(0).choice(N, 1024, replace=False)
    rows = np.concatenate([[0, N - 1], rows])
    assert _rows_check(y, x64, w, qt, K, rows) <= TOL_F32


@pytest.mark.parametrize("shape", [(13824, 5120), (5120, 13824)], ids=["13824x5120", "5120x13824"])
@pytest.mark.parametrize("M", [1, 8])
def test_config3_q4_k_gemv(dev, shape, M):
    from vkflame_amd import ops
    N, K = shape
    w = O.gen_weight(O.Q4_K, N, K, seed_for(3, 0 if N == 13824 else 1))
    xa, x64 = _x("f16", M, K, seed_for(3, M))
    y = ops.gemm_q(to_dev(w, dev), O.Q4_K, to_dev(xa, dev), N, K).cpu().numpy()
    rows = np.concatenate([[0, N - 1], np.random.default_rng(1).choice(N, 1024, replace=False)])
    assert _rows_check(y, x64, w, O.Q4_K, K, rows) <= TOL_F32


def test_q6_k_q8_1_partials_bit_exact(dev):
    import torch
    from vkflame_amd import ops
    N, K, M = 40, 1024, 5
    w = O.gen_weight(O.Q6_K, N, K, seed_for(5, 3))
    xq, _ = _x("q8_1", M, K, seed_for(5, 4))
    P = ops.q6k_q81_partials(to_dev(w, dev), to_dev(xq, dev), M, N, K)
    torch.cuda.synchronize()
    ref = O.c_q6k_q8_1_partials(w, xq, M, N, K)
    assert bits_equal(P.cpu().numpy(), ref), first_mismatch(P.cpu().numpy(), ref)


def test_q6_k_q8_1_partials_config5_k(dev):
    """At C5's K = 5120: 20 super-blocks and 160 Q8_1 blocks per row, 48
    generated weight rows against 4 activation rows."""
    import torch
    from vkflame_amd import ops
    N, K, M = 48, 5120, 4
    w = O.gen_weight(O.Q6_K, N, K, seed_for(5, 8))
    xq, _ = _x("q8_1", M, K, seed_for(5, 9))
    P = ops.q6k_q81_partials(to_dev(w, dev), to_dev(xq, dev), M, N, K)
    torch.cuda.synchronize()
    ref = O.c_q6k_q8_1_partials(w, xq, M, N, K)
    assert bits_equal(P.cpu().numpy(), ref), first_mismatch(P.cpu().numpy(), ref)


def test_q6_k_q8_1_partials_extreme_scales(dev):
    """Scales across the whole int8 range (|sc*(q-32)| up to 4096)."""
    import torch
    from vkflame_amd import ops
    N, K, M = 24, 512, 18   # M > 16 exercises the host's 16-row split
    rng = np.random.default_rng(seed_for(5, 5))
    w = O.gen_weight(O.Q6_K, N, K, seed_for(5, 6)).reshape(-1, 210)
    w[:, 192:208] = rng.integers(-128, 128, (w.shape[0], 16)).astype(np.int8).view(np.uint8)
    w = w.reshape(N, -1)
    xq, _ = _x("q8_1", M, K, seed_for(5, 7))
    P = ops.q6k_q81_partials(to_dev(w, dev), to_dev(xq, dev), M, N, K)
    torch.cuda.synchronize()
    assert bits_equal(P.cpu().numpy(), O.c_q6k_q8_1_partials(w, xq, M, N, K))


def test_config5_q6_k_q8_1_gemv(dev):
    """C5 at M=1: fp32 activations quantised on the GPU, vocab projection."""
    import torch
    from vkflame_amd import ops
    N, K = 152064, 5120
    w = O.gen_weight(O.Q6_K, N, K, seed_for(5))
    x = np.random.default_rng(seed_for(5, 1)).normal(0, 1, (1, K)).astype(np.float32)
    xq = ops.quantize_q8_1(to_dev(x, dev))
    y = ops.gemm_q(to_dev(w, dev), O.Q6_K, xq, N, K).cpu().numpy()
    torch.cuda.synchronize()
    xq_ref = O.np_quantize_q8_1(x).reshape(1, -1)
    assert bits_equal(xq.cpu().numpy(), xq_ref)
    x64 = O.np_dequant(O.Q8_1, xq_ref).reshape(1, K).astype(np.float64)
    rows = np.concatenate([[0, N - 1], np.random.default_rng(2).choice(N, 2048, replace=False)])
    assert _rows_check(y, x64, w, O.Q6_K, K, rows) <= TOL_F32


DOT_TYPES = [O.Q4_0, O.Q4_1, O.Q8_0, O.Q4_K, O.Q5_K]


def _per_row_err(y, x64, w, qt, N, K):
    ref = O.ref_gemv(x64, O.np_dequant(qt, w).reshape(N, K))
    return max(rel_err(y[m], ref[m]) for m in range(y.shape[0]))


@pytest.mark.parametrize("qt", DOT_TYPES, ids=[O.QNAMES[q] for q in DOT_TYPES])
@pytest.mark.parametrize("kind", ["f16", "f32"])
@pytest.mark.parametrize("M", [1, 2, 4])
@pytest.mark.parametrize("N", [77, 3001])
def test_gemv_dot_path(dev, qt, kind, M, N):
    """The integer dot-product GEMV (K % 64 == 0, M <= 4): every format,
    activation kind and row-segment width the host picks for small and
    large N, checked per activation row.  (fp16 activations at M = 2, 4 of
    the Q4 formats take the matrix-core GEMV instead, checked the same way.)"""
    from vkflame_amd import ops
    K = 1536
    w = O.gen_weight(qt, N, K, seed_for(2, 20 + qt))
    xa, x64 = _x(kind, M, K, seed_for(2, 30 + M))
    y = ops.gemm_q(to_dev(w, dev), qt, to_dev(xa, dev), N, K).cpu().numpy()
    assert _per_row_err(y, x64, w, qt, N, K) <= TOL_F32


@pytest.mark.parametrize("qt", DOT_TYPES, ids=[O.QNAMES[q] for q in DOT_TYPES])
def test_gemv_dot_dynamic_range(dev, qt):
    """Activations whose 32-element groups span 12 decades, an all-zero row
    and a row with a single non-zero: each group gets its own exponent."""
    from vkflame_amd import ops
    N, K, M = 300, 2048, 4
    rng = np.random.default_rng(seed_for(2, 40 + qt))
    x = rng.normal(0, 1, (M, K)).astype(np.float32)
    x[0] *= np.repeat(10.0 ** rng.uniform(-6, 6, K // 32), 32).astype(np.float32)
    x[1] = 0.0
    x[2] = 0.0
    x[2, 777] = -3.5
    w = O.gen_weight(qt, N, K, seed_for(2, 50 + qt))
    y = ops.gemm_q(to_dev(w, dev), qt, to_dev(x, dev), N, K).cpu().numpy()
    x64 = x.astype(np.float64)
    ref = O.ref_gemv(x64, O.np_dequant(qt, w).reshape(N, K))
    assert np.all(y[1] == 0.0)
    for m in (0, 2, 3):
        assert rel_err(y[m], ref[m]) <= TOL_F32, m


@pytest.mark.parametrize("qt", DOT_TYPES, ids=[O.QNAMES[q] for q in DOT_TYPES])
@pytest.mark.parametrize("N", [77, 3001, 13824])
@pytest.mark.parametrize("K", [1536, 5120, 16384])
def test_gemv_dot_q8_1_m1(dev, qt, N, K):
    """Q8_1 activations at M = 1 on the dot GEMV: each 8-element item staged
    from its block as fp32 d*q (exact), then into the kernel's integer image
    like fp32 activations; K = 16384 is the longest row the LDS image holds."""
    from vkflame_amd import ops
    w = O.gen_weight(qt, N, K, seed_for(2, 130 + qt))
    xa, x64 = _x("q8_1", 1, K, seed_for(2, 131))
    y = ops.gemm_q(to_dev(w, dev), qt, to_dev(xa, dev), N, K).cpu().numpy()
    assert _per_row_err(y, x64, w, qt, N, K) <= TOL_F32


@pytest.mark.parametrize("qt", DOT_TYPES, ids=[O.QNAMES[q] for q in DOT_TYPES])
def test_gemv_dot_q8_1_m1_range(dev, qt):
    """Q8_1 blocks whose scales span 12 decades (neighbouring blocks of one
    64-element chunk share its exponent), d*q past fp16's range, all-zero
    blocks and a row of a single non-zero code."""
    from vkflame_amd import ops
    N, K = 300, 4096
    rng = np.random.default_rng(seed_for(2, 140 + qt))
    w = O.gen_weight(qt, N, K, seed_for(2, 141 + qt))
    for case in range(3):
        x = rng.normal(0, 1, (1, K)).astype(np.float32)
        if case == 0:
            x[0] *= np.repeat(10.0 ** rng.uniform(-6, 6, K // 32), 32).astype(np.float32)
        elif case == 1:
            x[0] *= 1e5
            x[0, 64:256] = 0.0
        else:
            x[0] = 0.0
            x[0, 1001] = 7.25
        xa = O.np_quantize_q8_1(x).reshape(1, -1)
        x64 = O.np_dequant(O.Q8_1, xa).reshape(1, K).astype(np.float64)
        y = ops.gemm_q(to_dev(w, dev), qt, to_dev(xa, dev), N, K).cpu().numpy()
        ref = O.ref_gemv(x64, O.np_dequant(qt, w).reshape(N, K))
        assert rel_err(y[0], ref[0]) <= TOL_F32, case


@pytest.mark.parametrize("N", [1, 77, 3001, 20011])
@pytest.mark.parametrize("K", [2048, 4608, 5120, 6144])
def test_gemv_q6k_q81_dot(dev, N, K):
    """The Q6_K x Q8_1 integer GEMV at M = 1 (4-byte aligned rows, chunks at
    alternating 2- and 4-byte offsets), including scales over the whole int8
    range.  N and K cover every row-segment width the host picks (8..64 lanes)
    and row tails that end 0, 4, 8 or 12 bytes into a 16-byte piece."""
    from vkflame_amd import ops
    w = O.gen_weight(O.Q6_K, N, K, seed_for(5, 10 + N % 7)).reshape(-1, 210)
    rng = np.random.default_rng(seed_for(5, 11))
    w[::3, 192:208] = rng.integers(-128, 128, (w[::3].shape[0], 16)).astype(np.int8).view(np.uint8)
    w = w.reshape(N, -1)
    xq, x64 = _x("q8_1", 1, K, seed_for(5, 12))
    y = ops.gemm_q(to_dev(w, dev), O.Q6_K, to_dev(xq, dev), N, K).cpu().numpy()
    ref = O.ref_gemv(x64, O.np_dequant(O.Q6_K, w).reshape(N, K))
    assert rel_err(y, ref) <= TOL_F32


MFMA_TYPES = [O.Q4_K, O.Q5_K, O.Q4_0, O.Q4_1, O.Q8_0, O.Q5_0]


@pytest.mark.parametrize("qt", MFMA_TYPES, ids=[O.QNAMES[q] for q in MFMA_TYPES])
@pytest.mark.parametrize("M", [2, 5, 8, 9, 16])
@pytest.mark.parametrize("N", [77, 3001])
@pytest.mark.parametrize("K", [2304, 13824])
def test_gemv_mfma(dev, qt, M, N, K):
    """Q4_K, Q5_K, Q4_0, Q4_1, Q8_0, Q5_0 x fp16 at 2 <= M <= 16 on the matrix cores: 8- and
    16-row activation images, every K-split width the host picks, and
    K = 13824, which runs as several K-slice launches accumulating into y
    (Q5_K, Q8_0, Q5_0) or, for Q4_K, Q4_0 and Q4_1, as K slices side by side
    in one launch with a workspace for their partials."""
    from vkflame_amd import ops
    w = O.gen_weight(qt, N, K, seed_for(2, 60 + M + 20 * qt))
    xa, x64 = _x("f16", M, K, seed_for(2, 70 + M))
    y = ops.gemm_q(to_dev(w, dev), qt, to_dev(xa, dev), N, K).cpu().numpy()
    assert _per_row_err(y, x64, w, qt, N, K) <= TOL_F32


@pytest.mark.parametrize("qt,K", [(O.Q4_0, 2304), (O.Q4_0, 4096), (O.Q4_1, 4096), (O.Q4_K, 2304), (O.Q4_K, 5120)],
                         ids=["q4_0-2304", "q4_0-4096", "q4_1-4096", "q4_k-2304", "q4_k-5120"])
@pytest.mark.parametrize("M", [3, 16])
def test_gemv_mfma_many_rounds(dev, qt, K, M):
    """The register-activation kernel on more 16-row tiles than two rounds of
    one workgroup per CU (the next round's weights requested while a round's
    partial tiles are added) with a ragged last tile; K = 2304 leaves some
    waves without groups."""
    import torch
    from vkflame_amd import ops
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    N = 16 * cus * 2 + 40
    w = O.gen_weight(qt, N, K, seed_for(2, 90 + M + 20 * qt))
    xa, x64 = _x("f16", M, K, seed_for(2, 95 + M))
    y = ops.gemm_q(to_dev(w, dev), qt, to_dev(xa, dev), N, K).cpu().numpy()
    assert _per_row_err(y, x64, w, qt, N, K) <= TOL_F32


KS_CASES = [(q, k, m) for q, k in [(O.Q4_K, 256 * 34), (O.Q4_K, 13824), (O.Q4_K, 256 * 160), (O.Q4_0, 256 * 36),
                                    (O.Q4_0, 11008), (O.Q4_1, 11008), (O.Q4_1, 256 * 128)] for m in (2, 7, 16)]
KS_CASES += [(O.Q8_0, 13824, 9), (O.Q8_0, 13824, 16), (O.Q8_0, 256 * 192, 16)]


@pytest.mark.parametrize("qt,K,M", KS_CASES, ids=[f"{O.QNAMES[q]}-{k}-m{m}" for q, k, m in KS_CASES])
@pytest.mark.parametrize("N", [77, "rounds"])
def test_gemv_mfma_k_slices(dev, qt, K, M, N):
    """Long K on the register-activation kernel as K slices side by side in
    one launch (2 to 8 slices: K/256 = 34 and 36 groups, 13824, 11008, and
    the longest K the route takes, 8 slices of 20, 16 or 24 groups; Q8_0 at
    M > 8 only), each workgroup on one slice, the partials added in slice
    order by a second launch: against the float64 product per activation
    row, against the no-workspace route (K-slice launches one after another)
    within the same tolerance, and bit for bit between two calls.  N =
    "rounds" gives every workgroup more than one 16-row tile and a ragged
    last tile."""
    import torch
    from vkflame_amd import ops
    from vkflame_amd import _lib as L
    if N == "rounds":
        cus = torch.cuda.get_device_properties(0).multi_processor_count
        N = 16 * cus + 40 if K <= 13824 else 600
    S = L.lib().vkflame_gemm_q_workspace_bytes(qt, L.DTYPE_FP16, M, N, K) // (M * N * 4)
    assert 2 <= S <= 8, S
    print(f"k slices: {O.QNAMES[qt]} {N}x{K} M={M} S={S}", flush=True)
    w = O.gen_weight(qt, N, K, seed_for(2, 110 + M + 20 * qt))
    xa, x64 = _x("f16", M, K, seed_for(2, 115 + M))
    wd, xd = to_dev(w, dev), to_dev(xa, dev)
    y = ops.gemm_q(wd, qt, xd, N, K)
    y2 = ops.gemm_q(wd, qt, xd, N, K)
    y_seq = ops.gemm_q(wd, qt, xd, N, K, workspace=False)
    torch.cuda.synchronize()
    a, b = y.cpu().numpy(), y2.cpu().numpy()
    assert bits_equal(a, b), first_mismatch(a, b)
    assert _per_row_err(a, x64, w, qt, N, K) <= TOL_F32
    assert _per_row_err(y_seq.cpu().numpy(), x64, w, qt, N, K) <= TOL_F32
    assert max(rel_err(a[m], y_seq.cpu().numpy()[m]) for m in range(M)) <= TOL_F32


@pytest.mark.parametrize("N", [1, 9, 16, 17])
def test_gemv_mfma_k_slices_few_rows(dev, N):
    """K slices with a single (ragged) 16-row tile or two: one workgroup per
    slice, the rows past N of the tile clamped to the last row."""
    from vkflame_amd import ops
    K, M = 13824, 6
    w = O.gen_weight(O.Q4_K, N, K, seed_for(2, 150 + N))
    xa, x64 = _x("f16", M, K, seed_for(2, 151))
    y = ops.gemm_q(to_dev(w, dev), O.Q4_K, to_dev(xa, dev), N, K).cpu().numpy()
    assert _per_row_err(y, x64, w, O.Q4_K, N, K) <= TOL_F32


def test_gemv_mfma_k_slices_strided_output(dev):
    """The slice sum writes y at its row stride and leaves the padding."""
    import torch
    from vkflame_amd import ops
    N, K, M = 300, 13824, 5
    w = O.gen_weight(O.Q4_K, N, K, seed_for(2, 140))
    xa, x64 = _x("f16", M, K, seed_for(2, 141))
    ybig = torch.full((M, N + 24), 7.0, device=dev)
    ops.gemm_q(to_dev(w, dev), O.Q4_K, to_dev(xa, dev), N, K, out=ybig[:, :N])
    torch.cuda.synchronize()
    yb = ybig.cpu().numpy()
    assert np.all(yb[:, N:] == 7.0)
    assert _per_row_err(yb[:, :N], x64, w, O.Q4_K, N, K) <= TOL_F32


@pytest.mark.parametrize("M", [2, 5, 8, 9, 16])
@pytest.mark.parametrize("N", [77, 3001])
@pytest.mark.parametrize("K", [2560, 13824])
def test_gemv_mfma_q6_k(dev, M, N, K):
    """Q6_K x fp16 at 2 <= M <= 16 on the matrix cores: 210-byte super-blocks
    at alternating 2-byte alignment (every odd one), K = 13824 as two K-slice
    launches of 27 super-blocks (the second slice starting 2 bytes into a
    dword).  The operand sc*(q-32) is rounded to fp16 above 2048."""
    from vkflame_amd import ops
    w = O.gen_weight(O.Q6_K, N, K, seed_for(2, 90 + M))
    xa, x64 = _x("f16", M, K, seed_for(2, 95 + M))
    y = ops.gemm_q(to_dev(w, dev), O.Q6_K, to_dev(xa, dev), N, K).cpu().numpy()
    assert _per_row_err(y, x64, w, O.Q6_K, N, K) <= TOL_F32


MFMA_ALL = [O.Q4_K, O.Q5_K, O.Q4_0, O.Q4_1, O.Q8_0, O.Q6_K, O.Q5_0]


@pytest.mark.parametrize("kind", ["f16", "f32", "q8_1"])
@pytest.mark.parametrize("N", [77, 3001, 20011])
@pytest.mark.parametrize("K", [2304, 13824])
def test_gemv_mfma_q5_0_m1(dev, kind, N, K):
    """Q5_0 at M = 1: the generic GEMV below two 16-row tiles per CU, the
    matrix-core GEMV above (N = 20011), whose staged rows past the first
    repeat it and are not written."""
    from vkflame_amd import ops
    w = O.gen_weight(O.Q5_0, N, K, seed_for(2, 150))
    xa, x64 = _x(kind, 1, K, seed_for(2, 151))
    y = ops.gemm_q(to_dev(w, dev), O.Q5_0, to_dev(xa, dev), N, K).cpu().numpy()
    assert _per_row_err(y, x64, w, O.Q5_0, N, K) <= TOL_F32


@pytest.mark.parametrize("qt", MFMA_ALL, ids=[O.QNAMES[q] for q in MFMA_ALL])
@pytest.mark.parametrize("kind", ["f32", "q8_1"])
@pytest.mark.parametrize("M", [2, 9])
@pytest.mark.parametrize("K", [2560, 13824])
def test_gemv_mfma_activation_kinds(dev, qt, kind, M, K):
    """fp32 and Q8_1 activations on the matrix-core GEMV: each 16-byte piece
    of the fp16 LDS image converted from its source (Q8_1 as fp16(d*q)),
    K = 13824 as K-slice launches whose activation pointers advance by the
    slice's bytes in the source format."""
    from vkflame_amd import ops
    N = 3001
    w = O.gen_weight(qt, N, K, seed_for(2, 100 + qt))
    xa, x64 = _x(kind, M, K, seed_for(2, 110 + M))
    y = ops.gemm_q(to_dev(w, dev), qt, to_dev(xa, dev), N, K).cpu().numpy()
    assert _per_row_err(y, x64, w, qt, N, K) <= TOL_F32


@pytest.mark.parametrize("kind", ["f32", "q8_1"])
def test_gemv_mfma_activation_range(dev, kind):
    """Rows far outside fp16's range (up to ~4e6, Q8_1 d*q past 65504), a row
    of tiny values (~1e-30), an all-zero row: the per-row power-of-two
    scaling of the fp16 LDS image keeps every row within the tolerance."""
    from vkflame_amd import ops
    N, K, M = 300, 4096, 6
    rng = np.random.default_rng(seed_for(2, 120))
    x = rng.normal(0, 1, (M, K)).astype(np.float32)
    x[0] *= 1e6
    x[1] *= 1e-30
    x[2] = 0.0
    x[3, ::7] *= 3e4
    if kind == "q8_1":
        xa = O.np_quantize_q8_1(x).reshape(M, -1)
        x64 = O.np_dequant(O.Q8_1, xa).reshape(M, K).astype(np.float64)
    else:
        xa, x64 = x, x.astype(np.float64)
    for qt in (O.Q4_K, O.Q6_K):
        w = O.gen_weight(qt, N, K, seed_for(2, 121 + qt))
        y = ops.gemm_q(to_dev(w, dev), qt, to_dev(xa, dev), N, K).cpu().numpy()
        ref = O.ref_gemv(x64, O.np_dequant(qt, w).reshape(N, K))
        assert np.all(y[2] == 0.0)
        for m in (0, 1, 3, 4, 5):
            assert rel_err(y[m], ref[m]) <= TOL_F32, (O.QNAMES[qt], m)


def test_gemv_mfma_q6_k_extreme_scales(dev):
    """Every scale at -128 or 127 and codes at 0 / 63: operands of magnitude
    up to 4096, the fp16 rounding at its largest."""
    from vkflame_amd import ops
    N, K, M = 300, 4096, 8
    w = O.gen_weight(O.Q6_K, N, K, seed_for(2, 97)).reshape(N, K // 256, 210).copy()
    rng = np.random.default_rng(seed_for(2, 98))
    w[:, :, 192:208] = rng.choice(np.array([0x80, 0x7F], dtype=np.uint8), size=(N, K // 256, 16))
    w[:, :, 0:192] = rng.choice(np.array([0x00, 0xFF], dtype=np.uint8), size=(N, K // 256, 192))
    w = w.reshape(N, -1)
    xa, x64 = _x("f16", M, K, seed_for(2, 99))
    y = ops.gemm_q(to_dev(w, dev), O.Q6_K, to_dev(xa, dev), N, K).cpu().numpy()
    assert _per_row_err(y, x64, w, O.Q6_K, N, K) <= TOL_F32


@pytest.mark.parametrize("qt", [O.Q4_0, O.Q4_1, O.Q4_K, O.Q5_K, O.Q8_0], ids=["q4_0", "q4_1", "q4_k", "q5_k", "q8_0"])
@pytest.mark.parametrize("kind", ["f16", "f32", "q8_1"])
@pytest.mark.parametrize("NK", [(77, 1600), (77, 1664), (77, 1728), (3001, 4096), (100003, 2624)],
                         ids=["77x1600", "77x1664", "77x1728", "3001x4096", "100003x2624"])
def test_gemv_dot_lds_tails(dev, qt, kind, NK):
    """M = 1 through LDS: row regions that end 4, 8 or 12 bytes into a
    16-byte piece (Q4_0 / Q4_1 / Q8_0 rows of 25..27 chunks; on the large N
    in the middle of a multi-iteration row walk), checked on a spread of
    rows.  Q8_0 runs on the twelve-wave variant (fp16 / fp32 activations;
    Q8_1 ones take the register-loading kernel)."""
    from vkflame_amd import ops
    N, K = NK
    if qt in (O.Q4_K, O.Q5_K) and K % 256:
        pytest.skip("K-quant rows are whole 256-element super-blocks")
    w = O.gen_weight(qt, N, K, seed_for(2, 80 + qt))
    xa, x64 = _x(kind, 1, K, seed_for(2, 81))
    y = ops.gemm_q(to_dev(w, dev), qt, to_dev(xa, dev), N, K).cpu().numpy()
    rows = np.unique(np.concatenate([np.arange(0, N, max(1, N // 150)), [N - 1]]))
    assert _rows_check(y, x64, w, qt, K, rows) <= TOL_F32


def test_stream_read_hook(dev):
    """The read-bandwidth hook reads a buffer (ragged last pass included) and
    leaves the sink alone unless the folded data hits its constant."""
    import torch
    from vkflame_amd import ops
    sink = torch.full((1,), 7, dtype=torch.int32, device=dev)
    for nbytes in (16, 4096 + 16, 39813120):
        buf = torch.arange(nbytes // 4, dtype=torch.int32, device=dev)
        ops.stream_read(buf, sink)
    torch.cuda.synchronize()
    assert int(sink.item()) == 7


@pytest.mark.parametrize("qt", [O.Q4_K, O.Q5_K], ids=["q4_k", "q5_k"])
@pytest.mark.parametrize("M", [1, 3])
def test_gemv_dot_largest_codes(dev, qt, M):
    """Every code at its maximum (15 / 31), every 6-bit scale and min 63 and
    activations that quantise to the largest integers: the dot GEMV's integer
    products reach their bound (|sc * P| < 2^31 for Q5_K) without overflow."""
    from vkflame_amd import ops
    N, K = 300, 4096
    w = O.gen_weight(qt, N, K, seed_for(2, 90 + qt)).reshape(-1, O.BLOCK_BYTES[qt])
    w[:, 4:16] = 0xFF                      # scales / mins: all 63
    w[:, 16:] = 0xFF                       # (Q5_K qh and) qs: every code at its maximum
    w = w.reshape(N, -1)
    x = np.ones((M, K), np.float32)
    x[:, 1::2] = -1.0 if M == 1 else 1.0
    xa = x.astype(np.float16)
    y = ops.gemm_q(to_dev(w, dev), qt, to_dev(xa, dev), N, K).cpu().numpy()
    ref = O.ref_gemv(x.astype(np.float64), O.np_dequant(qt, w.reshape(-1)).reshape(N, K))
    assert rel_err(y, ref) <= TOL_F32


@pytest.mark.parametrize("kind", ["f16", "f32"])
@pytest.mark.parametrize("N", [1, 77, 3001, 20011])
@pytest.mark.parametrize("K", [2048, 4608, 5120, 16384])
def test_gemv_q6k_float_activations(dev, kind, N, K):
    """Q6_K x fp16 / fp32 activations at M = 1: the Q6_K integer GEMV with the
    activations split into two int8 rows per 32-element block (x ~ dh*qh +
    dl*ql, error <= max|x|/(4*127*127) per block), checked against the
    float64 product of the exact fp16 / fp32 activations; rows whose tails end
    0, 4, 8 or 12 bytes into a 16-byte piece, every row-segment width, scales
    over the whole int8 range."""
    from vkflame_amd import ops
    w = O.gen_weight(O.Q6_K, N, K, seed_for(5, 20 + N % 7)).reshape(-1, 210)
    rng = np.random.default_rng(seed_for(5, 21))
    w[::3, 192:208] = rng.integers(-128, 128, (w[::3].shape[0], 16)).astype(np.int8).view(np.uint8)
    w = w.reshape(N, -1)
    xa, x64 = _x(kind, 1, K, seed_for(5, 22))
    y = ops.gemm_q(to_dev(w, dev), O.Q6_K, to_dev(xa, dev), N, K).cpu().numpy()
    rows = np.unique(np.concatenate([np.arange(0, N, max(1, N // 150)), [N - 1]]))
    assert _rows_check(y, x64, w, O.Q6_K, K, rows) <= TOL_F32
