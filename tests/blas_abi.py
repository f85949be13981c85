"""ctypes declarations of the hipBLAS / hipBLASLt entry points exported by
libvkflame_amd.so, with the ROCm 7.2 enum values (hipblas-common.h,
library_types.h, hipblaslt.h)."""
import ctypes

from vkflame_amd import lib

P, I, U64, I64, SZ = ctypes.c_void_p, ctypes.c_int, ctypes.c_uint64, ctypes.c_int64, ctypes.c_size_t

OP_N, OP_T, OP_C = 111, 112, 113
GEMM_DEFAULT = 160  # HIPBLAS_GEMM_DEFAULT
R_32F, R_16F, R_8I, R_32I, R_16BF = 0, 2, 3, 10, 14
COMPUTE_16F, COMPUTE_32F, COMPUTE_32I = 0, 2, 9
ST_SUCCESS, ST_NOT_INIT, ST_INVALID_VALUE, ST_NOT_SUPPORTED, ST_HANDLE_NULL = 0, 1, 3, 7, 9

# hipblasLt
LAYOUT_BATCH_COUNT, LAYOUT_STRIDE, LAYOUT_TYPE, LAYOUT_ORDER, LAYOUT_ROWS, LAYOUT_COLS, LAYOUT_LD = 0, 1, 2, 3, 4, 5, 6
ORDER_COL, ORDER_ROW = 0, 1
DESC_TRANSA, DESC_TRANSB, DESC_EPILOGUE, DESC_BIAS_POINTER, DESC_BIAS_DATA_TYPE = 0, 1, 2, 3, 4
DESC_A_SCALE_POINTER, DESC_B_SCALE_POINTER, DESC_A_SCALE_MODE, DESC_B_SCALE_MODE = 5, 6, 31, 32
EPI_DEFAULT, EPI_RELU, EPI_BIAS, EPI_RELU_BIAS, EPI_GELU, EPI_GELU_BIAS = 1, 2, 4, 6, 32, 36
EPI_SWISH, EPI_SWISH_BIAS = 65536, 65540
SCALE_SCALAR_32F, SCALE_OUTER_VEC_32F = 0, 3
PREF_MAX_WORKSPACE = 1


class HeuristicResult(ctypes.Structure):
    _fields_ = [("algo_data", ctypes.c_uint8 * 16), ("algo_max_ws", SZ), ("workspaceSize", SZ),
                ("state", I), ("wavesCount", ctypes.c_float), ("reserved", I * 4)]


def blas():
    L = lib()
    L.hipblasCreate.argtypes = [ctypes.POINTER(P)]
    L.hipblasDestroy.argtypes = [P]
    L.hipblasSetStream.argtypes = [P, P]
    L.hipblasGetStream.argtypes = [P, ctypes.POINTER(P)]
    L.hipblasGemmEx.argtypes = [P, I, I, I, I, I, P, P, I, I, P, I, I, P, P, I, I, I, I]
    L.hipblasGemmStridedBatchedEx.argtypes = [P, I, I, I, I, I, P, P, I, I, I64, P, I, I, I64, P, P, I, I, I64,
                                              I, I, I]
    L.hipblasHgemm.argtypes = [P, I, I, I, I, I, P, P, I, P, I, P, P, I]
    L.hipblasHgemmBatched.argtypes = [P, I, I, I, I, I, P, P, I, P, I, P, P, I, I]
    L.hipblasSgemm.argtypes = [P, I, I, I, I, I, P, P, I, P, I, P, P, I]
    L.hipblasSgemmBatched.argtypes = [P, I, I, I, I, I, P, P, I, P, I, P, P, I, I]
    L.hipblasSgemmStridedBatched.argtypes = [P, I, I, I, I, I, P, P, I, I64, P, I, I64, P, P, I, I64, I]
    L.hipblasGemmBatchedEx.argtypes = [P, I, I, I, I, I, P, P, I, I, P, I, I, P, P, I, I, I, I, I]
    L.hipblasLtCreate.argtypes = [ctypes.POINTER(P)]
    L.hipblasLtDestroy.argtypes = [P]
    L.hipblasLtMatrixLayoutCreate.argtypes = [ctypes.POINTER(P), I, U64, U64, I64]
    L.hipblasLtMatrixLayoutDestroy.argtypes = [P]
    L.hipblasLtMatrixLayoutSetAttribute.argtypes = [P, I, P, SZ]
    L.hipblasLtMatrixLayoutGetAttribute.argtypes = [P, I, P, SZ, ctypes.POINTER(SZ)]
    L.hipblasLtMatmulDescCreate.argtypes = [ctypes.POINTER(P), I, I]
    L.hipblasLtMatmulDescDestroy.argtypes = [P]
    L.hipblasLtMatmulDescSetAttribute.argtypes = [P, I, P, SZ]
    L.hipblasLtMatmulDescGetAttribute.argtypes = [P, I, P, SZ, ctypes.POINTER(SZ)]
    L.hipblasLtMatmulPreferenceCreate.argtypes = [ctypes.POINTER(P)]
    L.hipblasLtMatmulPreferenceDestroy.argtypes = [P]
    L.hipblasLtMatmulPreferenceSetAttribute.argtypes = [P, I, P, SZ]
    L.hipblasLtMatmulAlgoGetHeuristic.argtypes = [P, P, P, P, P, P, P, I, ctypes.POINTER(HeuristicResult),
                                                  ctypes.POINTER(I)]
    L.hipblasLtMatmul.argtypes = [P, P, P, P, P, P, P, P, P, P, P, P, P, P, SZ, P]
    return L


def set_desc(L, desc, attr, value):
    if isinstance(value, ctypes._SimpleCData):
        v = value
    else:
        v = ctypes.c_int32(value)
    return L.hipblasLtMatmulDescSetAttribute(desc, attr, ctypes.byref(v), ctypes.sizeof(v))


def layout(L, dtype, rows, cols, ld, order=ORDER_COL):
    h = P()
    assert L.hipblasLtMatrixLayoutCreate(ctypes.byref(h), dtype, rows, cols, ld) == 0
    if order != ORDER_COL:
        o = ctypes.c_int32(order)
        assert L.hipblasLtMatrixLayoutSetAttribute(h, LAYOUT_ORDER, ctypes.byref(o), 4) == 0
    return h


def vendor_hipblas():
    """ROCm's own hipBLAS (for calls this library does not export)."""
    V = ctypes.CDLL("libhipblas.so")
    V.hipblasSscal.argtypes = [P, I, P, P, I]
    return V


def vendor_hipblaslt():
    V = ctypes.CDLL("libhipblaslt.so")
    V.hipblasLtMatmulPreferenceGetAttribute.argtypes = [P, I, P, SZ, ctypes.POINTER(SZ)]
    return V
