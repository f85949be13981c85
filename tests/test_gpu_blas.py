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
                         ldb, ctypes.byref(be), _ptr(tC), ctype, ldc, comp, 0)
    assert st == B.ST_SUCCESS
    torch.cuda.synchronize()
    got = tC.cpu().numpy()
    ref = 0.75 * (opa.astype(np.float64) @ opb.astype(np.float64)) - 0.5 * C0[:, :m].T.astype(np.float64)
    assert rel_err(got[:, :m].T, ref) <= (TOL_F32 if ctype == B.R_32F else TOL_F16)
    assert np.array_equal(got[:, m:], C0[:, m:])      # ld padding untouched


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
                         B.R_8I, k, ctypes.byref(be), _ptr(C), B.R_32I, m, B.COMPUTE_32I, 0)
    assert st == B.ST_SUCCESS
    torch.cuda.synchronize()
    ref = (A.astype(np.int64) @ Bm.astype(np.int64))
    assert np.array_equal(C.cpu().numpy().T.astype(np.int64), ref)


def test_gemm_strided_batched_int8(dev, L, handle):
    """int8 batch strides in int8 elements (the reference uses 4 bytes,
    shim/hipblas_shim.cpp:332-334)."""
    import torch
    m, n, k, nb = 64, 48, 96, 3
    rng = np.random.default_rng(seed_for(4, 91))
    A = rng.integers(-127, 128, (nb, m, k)).astype(np.int8)
    Bm = rng.integers(-127, 128, (nb, n, k)).astype(np.int8)
    tA, tB = to_dev(A, dev), to_dev(Bm, dev)
    C = torch.zeros((nb, n, m), dtype=torch.int32, device=dev)
    al, be = ctypes.c_int32(2), ctypes.c_int32(0)
    st = L.hipblasGemmStridedBatchedEx(handle, B.OP_T, B.OP_N, m, n, k, ctypes.byref(al), _ptr(tA), B.R_8I, k,
                                       m * k, _ptr(tB), B.R_8I, k, n * k, ctypes.byref(be), _ptr(C), B.R_32I, m,
                                       n * m, nb, B.COMPUTE_32I, 0)
    assert st == B.ST_SUCCESS
    torch.cuda.synchronize()
    for b in range(nb):
        ref = 2 * (A[b].astype(np.int64) @ Bm[b].astype(np.int64).T)
        assert np.array_equal(C[b].cpu().numpy().T.astype(np.int64), ref)


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
