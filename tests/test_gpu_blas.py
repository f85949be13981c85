"""GPU parity of the hipBLAS / hipBLASLt entry points exported by
libvkflame_amd.so (column-major BLAS semantics with op, ld, alpha, beta,
epilogue, bias and scale vectors honoured)."""
import ctypes

import numpy as np
import pytest

import oracle as O
from _util import TOL_F16, TOL_F32, rel_err, seed_for, to_dev
import blas_abi as B

pytestmark = pytest.mark.gpu


def _cm(a):
    """numpy column-major view helper: returns the Fortran-ordered copy."""
    return np.asfortranarray(a)


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr())


@pytest.fixture(scope="module")
def L(dev):
    return B.blas()


@pytest.fixture
def handle(L):
    import torch
    h = ctypes.c_void_p()
    assert L.hipblasCreate(ctypes.byref(h)) == 0
    assert L.hipblasSetStream(h, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)) == 0
    yield h
    L.hipblasDestroy(h)


@pytest.mark.parametrize("opA,opB", [(B.OP_T, B.OP_N), (B.OP_N, B.OP_N), (B.OP_N, B.OP_T), (B.OP_T, B.OP_T)])
@pytest.mark.parametrize("ctype", [B.R_32F, B.R_16F])
def test_gemm_ex_fp16(dev, L, handle, opA, opB, ctype):
    import torch
    m, n, k = 150, 90, 200
    rng = np.random.default_rng(seed_for(4, 80) + opA + 3 * opB + ctype)
    opa = rng.normal(0, 1, (m, k)).astype(np.float16)   # op(A)
    opb = rng.normal(0, 1, (k, n)).astype(np.float16)   # op(B)
    A = opa if opA == B.OP_N else opa.T                  # stored matrix, column-major
    Bm = opb if opB == B.OP_N else opb.T
    lda, ldb, ldc = A.shape[0] + 3, Bm.shape[0] + 5, m + 2
    Ad = np.zeros((A.shape[1], lda), np.float16); Ad[:, :A.shape[0]] = A.T      # column j at Ad[j]
    Bd = np.zeros((Bm.shape[1], ldb), np.float16); Bd[:, :Bm.shape[0]] = Bm.T
    cdt = np.float32 if ctype == B.R_32F else np.float16
    C0 = rng.normal(0, 1, (n, ldc)).astype(cdt)
    tA, tB, tC = to_dev(Ad, dev), to_dev(Bd, dev), to_dev(C0, dev)
    if ctype == B.R_32F:
        al, be, comp = ctypes.c_float(0.75), ctypes.c_float(-0.5), B.COMPUTE_32F
    else:
        al = ctypes.c_uint16(int(np.float16(0.75).view(np.uint16)))
        be = ctypes.c_uint16(int(np.float16(-0.5).view(np.uint16)))
        comp = B.COMPUTE_16F
    st = L.hipblasGemmEx(handle, opA, opB, m, n, k, ctypes.byref(al), _ptr(tA), B.R_16F, lda, _ptr(tB), B.R_16F,
                         ldb, ctypes.byref(be), _ptr(tC), ctype, ldc, comp, B.GEMM_DEFAULT)
    assert st == B.ST_SUCCESS
    torch.cuda.synchronize()
    got = tC.cpu().numpy()
    ref = 0.75 * (opa.astype(np.float64) @ opb.astype(np.float64)) - 0.5 * C0[:, :m].T.astype(np.float64)
    assert rel_err(got[:, :m].T, ref) <= (TOL_F32 if ctype == B.R_32F else TOL_F16)
    assert np.array_equal(got[:, m:], C0[:, m:])      # ld padding untouched


@pytest.mark.parametrize("m,n,k", [(256, 96, 128), (136, 40, 96), (200, 33, 64)])
def test_gemm_strided_batched_fp16_nn_aligned(dev, L, handle, m, n, k):
    """Both ops N with aligned leading dimensions (torch.mm's call): B
    column-major k x n is the K-contiguous operand and A column-major m x k
    the [K, M] one, read back through ds_read_b64_tr_b16; n <= 64 takes the
    skinny kernel.  Three batches with strides of whole 16-byte pieces, fp32
    C with alpha and beta."""
    import torch
    nb = 3
    rng = np.random.default_rng(seed_for(4, 85) + m + n + k)
    A = rng.normal(0, 1, (nb, k, m)).astype(np.float16)    # column j of A (m x k, lda = m) at A[b, j]
    Bm = rng.normal(0, 1, (nb, n, k)).astype(np.float16)   # column j of B (k x n, ldb = k) at Bm[b, j]
    C0 = rng.normal(0, 1, (nb, n, m)).astype(np.float32)   # column j of C (m x n, ldc = m) at C0[b, j]
    tA, tB, tC = to_dev(A, dev), to_dev(Bm, dev), to_dev(C0, dev)
    al, be = ctypes.c_float(0.75), ctypes.c_float(-0.5)
    st = L.hipblasGemmStridedBatchedEx(handle, B.OP_N, B.OP_N, m, n, k, ctypes.byref(al), _ptr(tA), B.R_16F, m,
                                       m * k, _ptr(tB), B.R_16F, k, n * k, ctypes.byref(be), _ptr(tC), B.R_32F, m,
                                       n * m, nb, B.COMPUTE_32F, B.GEMM_DEFAULT)
    assert st == B.ST_SUCCESS
    torch.cuda.synchronize()
    got = tC.cpu().numpy()
    for b in range(nb):
        opa = A[b].T.astype(np.float64)                      # m x k
        opb = Bm[b].T.astype(np.float64)                     # k x n
        ref = 0.75 * (opa @ opb) - 0.5 * C0[b].T.astype(np.float64)
        assert rel_err(got[b].T, ref) <= TOL_F32


def test_gemm_ex_int8_int32(dev, L, handle):
    import torch
    m, n, k = 257, 129, 320
    rng = np.random.default_rng(seed_for(4, 90))
    A = rng.integers(-127, 128, (m, k)).astype(np.int8)   # op(A) = A^T stored k x m (opA = T)
    Bm = rng.integers(-127, 128, (k, n)).astype(np.int8)
    tA = to_dev(np.ascontiguousarray(A), dev)              # column-major k x m == row-major m x k
    tB = to_dev(np.ascontiguousarray(Bm.T), dev)           # column-major k x n
    C = torch.zeros((n, m), dtype=torch.int32, device=dev)
    al, be = ctypes.c_int32(1), ctypes.c_int32(0)
    st = L.hipblasGemmEx(handle, B.OP_T, B.OP_N, m, n, k, ctypes.byref(al), _ptr(tA), B.R_8I, k, _ptr(tB),
                         B.R_8I, k, ctypes.byref(be), _ptr(C), B.R_32I, m, B.COMPUTE_32I, B.GEMM_DEFAULT)
    assert st == B.ST_SUCCESS
    torch.cuda.synchronize()
    ref = (A.astype(np.int64) @ Bm.astype(np.int64))
    assert np.array_equal(C.cpu().numpy().T.astype(np.int64), ref)


@pytest.mark.parametrize("m,n,k", [(64, 48, 96), (256, 200, 512)])
def test_gemm_strided_batched_int8(dev, L, handle, m, n, k):
    """int8 batch strides in int8 elements (the reference uses 4 bytes,
    shim/hipblas_shim.cpp:332-334).  256 x 200 x 512: three batches of a
    grid that fits the CUs with whole K pairs, the narrow-tile kernel."""
    import torch
    nb = 3
    rng = np.random.default_rng(seed_for(4, 91) + m)
    A = rng.integers(-127, 128, (nb, m, k)).astype(np.int8)
    Bm = rng.integers(-127, 128, (nb, n, k)).astype(np.int8)
    tA, tB = to_dev(A, dev), to_dev(Bm, dev)
    C = torch.zeros((nb, n, m), dtype=torch.int32, device=dev)
    al, be = ctypes.c_int32(2), ctypes.c_int32(0)
    st = L.hipblasGemmStridedBatchedEx(handle, B.OP_T, B.OP_N, m, n, k, ctypes.byref(al), _ptr(tA), B.R_8I, k,
                                       m * k, _ptr(tB), B.R_8I, k, n * k, ctypes.byref(be), _ptr(C), B.R_32I, m,
                                       n * m, nb, B.COMPUTE_32I, B.GEMM_DEFAULT)
    assert st == B.ST_SUCCESS
    torch.cuda.synchronize()
    for b in range(nb):
        ref = 2 * (A[b].astype(np.int64) @ Bm[b].astype(np.int64).T)
        assert np.array_equal(C[b].cpu().numpy().T.astype(np.int64), ref)


def test_gemm_strided_batched_int8_256_tiles(dev, L, handle):
    """Sixteen batches of 1024 x 1024 x 128 int8: 16 x 16 256x256 tiles, at
    least one per CU, so the batched grid runs on the 256 x 256 kernel;
    exact int32 with integer alpha."""
    import torch
    m = n = 1024
    k, nb = 128, 16
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    assert nb * (m // 256) * (n // 256) >= cus
    rng = np.random.default_rng(seed_for(4, 92))
    A = rng.integers(-127, 128, (nb, m, k)).astype(np.int8)
    Bm = rng.integers(-127, 128, (nb, n, k)).astype(np.int8)
    tA, tB = to_dev(A, dev), to_dev(Bm, dev)
    C = torch.zeros((nb, n, m), dtype=torch.int32, device=dev)
    al, be = ctypes.c_int32(-3), ctypes.c_int32(0)
    st = L.hipblasGemmStridedBatchedEx(handle, B.OP_T, B.OP_N, m, n, k, ctypes.byref(al), _ptr(tA), B.R_8I, k,
                                       m * k, _ptr(tB), B.R_8I, k, n * k, ctypes.byref(be), _ptr(C), B.R_32I, m,
                                       n * m, nb, B.COMPUTE_32I, B.GEMM_DEFAULT)
    assert st == B.ST_SUCCESS
    torch.cuda.synchronize()
    got = C.cpu().numpy()
    for b in range(nb):
        ref = -3 * (A[b].astype(np.float64) @ Bm[b].astype(np.float64).T)  # exact: |sum| < 2^53
        assert np.array_equal(got[b].T.astype(np.float64), ref), b


def _lt_matmul(L, dev, A_t, adesc, B_t, bdesc, D_t, ddesc, desc, alpha=1.0, beta=0.0, C_t=None):
    import torch
    h = ctypes.c_void_p()
    assert L.hipblasLtCreate(ctypes.byref(h)) == 0
    pref = ctypes.c_void_p()
    assert L.hipblasLtMatmulPreferenceCreate(ctypes.byref(pref)) == 0
    res = (B.HeuristicResult * 1)()
    cnt = ctypes.c_int()
    assert L.hipblasLtMatmulAlgoGetHeuristic(h, desc, adesc, bdesc, ddesc, ddesc, pref, 1, res,
                                             ctypes.byref(cnt)) == 0 and cnt.value == 1
    al, be = ctypes.c_float(alpha), ctypes.c_float(beta)
    Cp = _ptr(C_t) if C_t is not None else _ptr(D_t)
    st = L.hipblasLtMatmul(h, desc, ctypes.byref(al), _ptr(A_t), adesc, _ptr(B_t), bdesc, ctypes.byref(be), Cp,
                           ddesc, _ptr(D_t), ddesc, ctypes.byref(res[0]), None, 0,
                           ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    L.hipblasLtMatmulPreferenceDestroy(pref)
    L.hipblasLtDestroy(h)
    return st


@pytest.mark.parametrize("epi,act", [(B.EPI_BIAS, 0), (B.EPI_GELU_BIAS, 3), (B.EPI_RELU_BIAS, 2),
                                     (B.EPI_SWISH_BIAS, 1)])
def test_lt_int8_linear_scales_bias(dev, L, epi, act):
    """The C4 contract through hipblasLtMatmul, column-major as PyTorch calls
    it: D^T[out, tok] = W[out,K] x X[tok,K]^T, a_scale per output channel
    (rows of op(A)), b_scale per token (columns of op(B)), bias per row of D."""
    import torch
    M, N, K = 96, 200, 512        # tokens, out features, in features
    inp = O.gen_int8_linear(M, N, K, seed_for(4, 100 + epi % 97))
    W, X = to_dev(inp.W, dev), to_dev(inp.A, dev)
    ws, as_ = to_dev(inp.w_scale, dev), to_dev(inp.a_scale, dev)
    bias = to_dev(inp.bias, dev)
    D = torch.empty((M, N), dtype=torch.float16, device=dev)   # column-major N x M
    adesc = B.layout(L, B.R_8I, K, N, K)   # W stored col-major K x N, opA = T -> N x K
    bdesc = B.layout(L, B.R_8I, K, M, K)   # X stored col-major K x M, opB = N
    ddesc = B.layout(L, B.R_16F, N, M, N)
    desc = ctypes.c_void_p()
    assert L.hipblasLtMatmulDescCreate(ctypes.byref(desc), B.COMPUTE_32I, B.R_32F) == 0
    assert B.set_desc(L, desc, B.DESC_TRANSA, B.OP_T) == 0
    assert B.set_desc(L, desc, B.DESC_TRANSB, B.OP_N) == 0
    assert B.set_desc(L, desc, B.DESC_EPILOGUE, ctypes.c_uint32(epi)) == 0
    assert B.set_desc(L, desc, B.DESC_BIAS_POINTER, ctypes.c_void_p(bias.data_ptr())) == 0
    assert B.set_desc(L, desc, B.DESC_A_SCALE_POINTER, ctypes.c_void_p(ws.data_ptr())) == 0
    assert B.set_desc(L, desc, B.DESC_B_SCALE_POINTER, ctypes.c_void_p(as_.data_ptr())) == 0
    assert B.set_desc(L, desc, B.DESC_A_SCALE_MODE, B.SCALE_OUTER_VEC_32F) == 0
    assert B.set_desc(L, desc, B.DESC_B_SCALE_MODE, B.SCALE_OUTER_VEC_32F) == 0
    st = _lt_matmul(L, dev, W, adesc, X, bdesc, D, ddesc, desc)
    assert st == B.ST_SUCCESS
    _, yref, _ = O.ref_linear_int8(inp, act=act)
    assert rel_err(D.cpu().numpy().astype(np.float32), yref) <= TOL_F16
    for h in (adesc, bdesc, ddesc):
        L.hipblasLtMatrixLayoutDestroy(h)
    L.hipblasLtMatmulDescDestroy(desc)


def test_lt_fp16_row_major(dev, L):
    """Row-major layouts (HIPBLASLT_MATRIX_LAYOUT_ORDER = ROW): D[m,n] =
    alpha A[m,k] B[n,k]^T + beta C, bias per row of D, fp32 out."""
    import torch
    m, n, k = 130, 70, 96
    rng = np.random.default_rng(seed_for(4, 120))
    A = rng.normal(0, 1, (m, k)).astype(np.float16)
    Bm = rng.normal(0, 1, (n, k)).astype(np.float16)
    C = rng.normal(0, 1, (m, n)).astype(np.float32)
    bias = rng.normal(0, 1, m).astype(np.float32)
    tA, tB, tC, tb = to_dev(A, dev), to_dev(Bm, dev), to_dev(C, dev), to_dev(bias, dev)
    D = torch.empty((m, n), dtype=torch.float32, device=dev)
    adesc = B.layout(L, B.R_16F, m, k, k, B.ORDER_ROW)
    bdesc = B.layout(L, B.R_16F, n, k, k, B.ORDER_ROW)
    ddesc = B.layout(L, B.R_32F, m, n, n, B.ORDER_ROW)
    desc = ctypes.c_void_p()
    assert L.hipblasLtMatmulDescCreate(ctypes.byref(desc), B.COMPUTE_32F, B.R_32F) == 0
    assert B.set_desc(L, desc, B.DESC_TRANSB, B.OP_T) == 0
    assert B.set_desc(L, desc, B.DESC_EPILOGUE, ctypes.c_uint32(B.EPI_BIAS)) == 0
    assert B.set_desc(L, desc, B.DESC_BIAS_POINTER, ctypes.c_void_p(tb.data_ptr())) == 0
    st = _lt_matmul(L, dev, tA, adesc, tB, bdesc, D, ddesc, desc, alpha=2.0, beta=0.5, C_t=tC)
    assert st == B.ST_SUCCESS
    ref = 2.0 * (A.astype(np.float64) @ Bm.astype(np.float64).T) + 0.5 * C + bias[:, None]
    assert rel_err(D.cpu().numpy(), ref) <= TOL_F32


def test_launch_table_executes_dequant(dev):
    """A ggml-style dequantize_block_q4_K launch decoded by the name table and
    run by vkflame_execute_launch."""
    import torch
    from vkflame_amd import lib
    from vkflame_amd._lib import resolve_launch, LAUNCH_DEQUANT
    nb = 300
    w = O.gen_blocks(O.Q4_K, nb, np.random.default_rng(seed_for(0, 99)))
    src = to_dev(w, dev)
    dst = torch.empty(nb * 256, dtype=torch.float16, device=dev)
    name = "_Z21dequantize_block_q4_KI6__halfEvPKvPT_"
    plan = resolve_launch(name, (nb, 1, 1), (32, 1, 1), [ctypes.c_void_p(src.data_ptr()),
                                                         ctypes.c_void_p(dst.data_ptr())])
    assert plan.kind == LAUNCH_DEQUANT and plan.n_blocks == nb and plan.out_dtype == 1
    assert lib().vkflame_execute_launch(ctypes.byref(plan),
                                        ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)) == 0
    torch.cuda.synchronize()
    ref = O.c_dequant(O.Q4_K, w, out_f16=True)
    assert np.array_equal(dst.cpu().numpy().view(np.uint16), ref.view(np.uint16))


def _colmajor_dev(M, ld, dev, dtype):
    """Upload the column-major matrix M (rows x cols) with leading dimension
    ld: column j at offset j*ld."""
    buf = np.zeros((M.shape[1], ld), dtype)
    buf[:, :M.shape[0]] = M.T
    return to_dev(buf, dev)


@pytest.mark.parametrize("opA,opB", [(B.OP_T, B.OP_N), (B.OP_N, B.OP_N), (B.OP_N, B.OP_T), (B.OP_T, B.OP_T)])
def test_sgemm(dev, L, handle, opA, opB):
    """hipblasSgemm on the fp32 matrix cores: every op combination, padded ld,
    alpha and beta (shim/hipblas_shim.cpp:84-113 ignores ld, alpha, beta)."""
    import torch
    m, n, k = 133, 77, 300
    rng = np.random.default_rng(seed_for(4, 140) + opA + 3 * opB)
    opa = rng.normal(0, 1, (m, k)).astype(np.float32)
    opb = rng.normal(0, 1, (k, n)).astype(np.float32)
    A = opa if opA == B.OP_N else opa.T
    Bm = opb if opB == B.OP_N else opb.T
    lda, ldb, ldc = A.shape[0] + 1, Bm.shape[0] + 4, m + 3
    C0 = rng.normal(0, 1, (m, n)).astype(np.float32)
    tA, tB = _colmajor_dev(A, lda, dev, np.float32), _colmajor_dev(Bm, ldb, dev, np.float32)
    tC = _colmajor_dev(C0, ldc, dev, np.float32)
    al, be = ctypes.c_float(1.25), ctypes.c_float(-0.75)
    assert L.hipblasSgemm(handle, opA, opB, m, n, k, ctypes.byref(al), _ptr(tA), lda, _ptr(tB), ldb,
                          ctypes.byref(be), _ptr(tC), ldc) == B.ST_SUCCESS
    torch.cuda.synchronize()
    got = tC.cpu().numpy()
    ref = 1.25 * (opa.astype(np.float64) @ opb.astype(np.float64)) - 0.75 * C0.astype(np.float64)
    assert rel_err(got[:, :m].T, ref) <= 1e-5
    assert np.all(got[:, m:] == 0)                    # ld padding untouched


def test_gemm_ex_fp32_and_linear_fp32(dev, L, handle):
    """fp32 through hipblasGemmEx (32F, compute 32F) and
    vkflame_dispatch_linear(VKF_DTYPE_FP32), row-major, C and beta."""
    import torch
    from vkflame_amd import ops
    from vkflame_amd._lib import DTYPE_FP32
    m, n, k = 256, 384, 512
    rng = np.random.default_rng(seed_for(4, 141))
    a = rng.normal(0, 1, (m, k)).astype(np.float32)
    b = rng.normal(0, 1, (n, k)).astype(np.float32)
    c = rng.normal(0, 1, (m, n)).astype(np.float32)
    D = ops.linear(to_dev(a, dev), to_dev(b, dev), m, n, k, DTYPE_FP32, transB=1, C=to_dev(c, dev), alpha=0.5,
                   beta=2.0)
    torch.cuda.synchronize()
    ref = 0.5 * (a.astype(np.float64) @ b.astype(np.float64).T) + 2.0 * c
    assert rel_err(D.cpu().numpy(), ref) <= 1e-5
    # column-major C^T[n, m] = b . a^T: opA = T on b stored [n,k] row-major = col-major k x n
    Ct = torch.zeros((m, n), dtype=torch.float32, device=dev)
    one, zero = ctypes.c_float(1.0), ctypes.c_float(0.0)
    assert L.hipblasGemmEx(handle, B.OP_T, B.OP_N, n, m, k, ctypes.byref(one), _ptr(to_dev(b, dev)), B.R_32F, k,
                           _ptr(to_dev(a, dev)), B.R_32F, k, ctypes.byref(zero), _ptr(Ct), B.R_32F, n,
                           B.COMPUTE_32F, B.GEMM_DEFAULT) == B.ST_SUCCESS
    torch.cuda.synchronize()
    assert rel_err(Ct.cpu().numpy(), a.astype(np.float64) @ b.astype(np.float64).T) <= 1e-5


def test_sgemm_strided_and_batched_one_launch(dev, L, handle):
    """Strided and pointer-array batches (the arrays of device pointers live
    in device memory, as hipBLAS defines them) run as one launch each and
    match per-matrix products."""
    import torch
    m, n, k, nb = 96, 64, 160, 5
    rng = np.random.default_rng(seed_for(4, 142))
    A = rng.normal(0, 1, (nb, k, m)).astype(np.float32)   # column-major m x k (opA = N): column j = A[b, j]
    Bm = rng.normal(0, 1, (nb, n, k)).astype(np.float32)  # column-major k x n
    tA, tB = to_dev(A, dev), to_dev(Bm, dev)
    C = torch.zeros((nb, n, m), dtype=torch.float32, device=dev)
    al, be = ctypes.c_float(1.0), ctypes.c_float(0.0)
    assert L.hipblasSgemmStridedBatched(handle, B.OP_N, B.OP_N, m, n, k, ctypes.byref(al), _ptr(tA), m, k * m,
                                        _ptr(tB), k, n * k, ctypes.byref(be), _ptr(C), m, n * m, nb) == B.ST_SUCCESS
    C2 = torch.zeros_like(C)
    pa = torch.tensor([tA[b].data_ptr() for b in range(nb)], dtype=torch.int64, device=dev)
    pb = torch.tensor([tB[b].data_ptr() for b in range(nb)], dtype=torch.int64, device=dev)
    pc = torch.tensor([C2[b].data_ptr() for b in range(nb)], dtype=torch.int64, device=dev)
    assert L.hipblasSgemmBatched(handle, B.OP_N, B.OP_N, m, n, k, ctypes.byref(al), _ptr(pa), m, _ptr(pb), k,
                                 ctypes.byref(be), _ptr(pc), m, nb) == B.ST_SUCCESS
    torch.cuda.synchronize()
    for b in range(nb):
        ref = A[b].T.astype(np.float64) @ Bm[b].T.astype(np.float64)   # (m x k) @ (k x n)
        assert rel_err(C[b].cpu().numpy().T, ref) <= 1e-5
        assert rel_err(C2[b].cpu().numpy().T, ref) <= 1e-5


def test_hgemm_batched_device_pointer_arrays(dev, L, handle):
    import torch
    m, n, k, nb = 128, 128, 256, 3
    rng = np.random.default_rng(seed_for(4, 143))
    A = rng.normal(0, 1, (nb, m, k)).astype(np.float16)   # opA = T: stored col-major k x m = row-major m x k
    Bm = rng.normal(0, 1, (nb, n, k)).astype(np.float16)  # opB = N: col-major k x n
    tA, tB = to_dev(A, dev), to_dev(Bm, dev)
    C = torch.zeros((nb, n, m), dtype=torch.float16, device=dev)
    pa = torch.tensor([tA[b].data_ptr() for b in range(nb)], dtype=torch.int64, device=dev)
    pb = torch.tensor([tB[b].data_ptr() for b in range(nb)], dtype=torch.int64, device=dev)
    pc = torch.tensor([C[b].data_ptr() for b in range(nb)], dtype=torch.int64, device=dev)
    one = ctypes.c_uint16(int(np.float16(1.0).view(np.uint16)))
    zero = ctypes.c_uint16(0)
    assert L.hipblasHgemmBatched(handle, B.OP_T, B.OP_N, m, n, k, ctypes.byref(one), _ptr(pa), k, _ptr(pb), k,
                                 ctypes.byref(zero), _ptr(pc), m, nb) == B.ST_SUCCESS
    torch.cuda.synchronize()
    for b in range(nb):
        ref = A[b].astype(np.float64) @ Bm[b].astype(np.float64).T
        assert rel_err(C[b].cpu().numpy().T.astype(np.float32), ref) <= TOL_F16


def test_gemm_ex_bf16_forwarded_to_rocm(dev, L, handle):
    """A type pair this library does not run (bf16) is forwarded to ROCm's
    hipblasGemmEx with the same (ROCm-created) handle and succeeds."""
    import torch
    m, n, k = 64, 48, 128
    a = torch.randn(m, k, device=dev).to(torch.bfloat16)   # opA = T: col-major k x m (lda = k) = row-major m x k
    b = torch.randn(n, k, device=dev).to(torch.bfloat16)   # opB = N: col-major k x n (ldb = k) = row-major n x k
    c = torch.zeros(n, m, device=dev, dtype=torch.bfloat16)  # col-major m x n (ldc = m)
    one, zero = ctypes.c_float(1.0), ctypes.c_float(0.0)
    assert L.hipblasGemmEx(handle, B.OP_T, B.OP_N, m, n, k, ctypes.byref(one), _ptr(a), B.R_16BF, k, _ptr(b),
                           B.R_16BF, k, ctypes.byref(zero), _ptr(c), B.R_16BF, m, B.COMPUTE_32F, B.GEMM_DEFAULT) == B.ST_SUCCESS
    torch.cuda.synchronize()
    ref = a.float().cpu().numpy().astype(np.float64) @ b.float().cpu().numpy().T.astype(np.float64)
    assert rel_err(c.float().cpu().numpy().T, ref) <= TOL_F16


def test_handle_works_with_rocm_functions(dev, L, handle):
    """The handle hipblasCreate returns is ROCm's own: a hipBLAS function this
    library does not export (hipblasSscal) runs on it."""
    import torch
    V = B.vendor_hipblas()
    x = torch.arange(100, dtype=torch.float32, device=dev)
    a = ctypes.c_float(3.0)
    assert V.hipblasSscal(handle, 100, ctypes.byref(a), _ptr(x), 1) == B.ST_SUCCESS
    torch.cuda.synchronize()
    assert np.array_equal(x.cpu().numpy(), 3.0 * np.arange(100, dtype=np.float32))


def test_lt_forwarded_and_rocm_objects(dev, L):
    """hipBLASLt: a bf16 matmul (not run here) is forwarded to ROCm's
    hipblasLtMatmul on ROCm-created objects, and a function this library does
    not export (hipblasLtMatmulPreferenceGetAttribute) works on its
    preference object."""
    import torch
    V = B.vendor_hipblaslt()
    pref = ctypes.c_void_p()
    assert L.hipblasLtMatmulPreferenceCreate(ctypes.byref(pref)) == 0
    ws = ctypes.c_uint64(1 << 20)
    assert L.hipblasLtMatmulPreferenceSetAttribute(pref, B.PREF_MAX_WORKSPACE, ctypes.byref(ws), 8) == 0
    got = ctypes.c_uint64(0)
    n_w = ctypes.c_size_t(0)
    assert V.hipblasLtMatmulPreferenceGetAttribute(pref, B.PREF_MAX_WORKSPACE, ctypes.byref(got), 8,
                                                   ctypes.byref(n_w)) == 0 and got.value == 1 << 20
    L.hipblasLtMatmulPreferenceDestroy(pref)
    m, n, k = 64, 32, 96
    a = torch.randn(m, k, device=dev).to(torch.bfloat16)   # opA = T: col-major k x m = row-major m x k
    b = torch.randn(n, k, device=dev).to(torch.bfloat16)   # col-major k x n = row-major n x k
    d = torch.zeros(n, m, device=dev, dtype=torch.bfloat16)
    adesc = B.layout(L, B.R_16BF, k, m, k)
    bdesc = B.layout(L, B.R_16BF, k, n, k)
    ddesc = B.layout(L, B.R_16BF, m, n, m)
    desc = ctypes.c_void_p()
    assert L.hipblasLtMatmulDescCreate(ctypes.byref(desc), B.COMPUTE_32F, B.R_32F) == 0
    assert B.set_desc(L, desc, B.DESC_TRANSA, B.OP_T) == 0
    st = _lt_matmul(L, dev, a, adesc, b, bdesc, d, ddesc, desc)
    assert st == B.ST_SUCCESS
    ref = a.float().cpu().numpy().astype(np.float64) @ b.float().cpu().numpy().T.astype(np.float64)
    assert rel_err(d.float().cpu().numpy().T, ref) <= TOL_F16
    for h in (adesc, bdesc, ddesc):
        L.hipblasLtMatrixLayoutDestroy(h)
    L.hipblasLtMatmulDescDestroy(desc)


def test_lt_batched_one_launch_and_int32_alpha(dev, L):
    """A strided batch of int8 -> int32 products with an integer alpha of 3
    (scale type 32F), one launch for the batch, exact."""
    import torch
    m, n, k, nb = 128, 96, 256, 4
    rng = np.random.default_rng(seed_for(4, 144))
    A = rng.integers(-127, 128, (nb, m, k)).astype(np.int8)   # opA = T: col-major k x m
    Bm = rng.integers(-127, 128, (nb, n, k)).astype(np.int8)  # col-major k x n
    tA, tB = to_dev(A, dev), to_dev(Bm, dev)
    D = torch.zeros((nb, n, m), dtype=torch.int32, device=dev)
    adesc = B.layout(L, B.R_8I, k, m, k)
    bdesc = B.layout(L, B.R_8I, k, n, k)
    ddesc = B.layout(L, B.R_32I, m, n, m)
    for h, stride in ((adesc, m * k), (bdesc, n * k), (ddesc, n * m)):
        cnt, st_ = ctypes.c_int32(nb), ctypes.c_int64(stride)
        assert L.hipblasLtMatrixLayoutSetAttribute(h, B.LAYOUT_BATCH_COUNT, ctypes.byref(cnt), 4) == 0
        assert L.hipblasLtMatrixLayoutSetAttribute(h, B.LAYOUT_STRIDE, ctypes.byref(st_), 8) == 0
    desc = ctypes.c_void_p()
    assert L.hipblasLtMatmulDescCreate(ctypes.byref(desc), B.COMPUTE_32I, B.R_32F) == 0
    assert B.set_desc(L, desc, B.DESC_TRANSA, B.OP_T) == 0
    st = _lt_matmul(L, dev, tA, adesc, tB, bdesc, D, ddesc, desc, alpha=3.0)
    assert st == B.ST_SUCCESS
    for b in range(nb):
        ref = 3 * (A[b].astype(np.int64) @ Bm[b].astype(np.int64).T)
        assert np.array_equal(D[b].cpu().numpy().T.astype(np.int64), ref)
    for h in (adesc, bdesc, ddesc):
        L.hipblasLtMatrixLayoutDestroy(h)
    L.hipblasLtMatmulDescDestroy(desc)
