// vkf_hipblas.cpp — hipBLAS GEMM entry points over the gfx950 MFMA kernels.
//
// Same names and signatures as ROCm 7.2's hipblas.h (included, so the compiler
// checks every signature), exported from libvkflame_amd.so.  Replaces
// shim/hipblas_shim.cpp:47-349.  The reference converts column-major to
// row-major by swapping A<->B and m<->n and then drops op, ld, alpha, beta and
// the stream (shim/hipblas_shim.cpp:84-290, runtime/dispatch.cpp:262-267);
// here every argument is honoured:
//   C = alpha * op(A) * op(B) + beta * C   (column-major, op in {N, T, C})
// Mapping onto the kernel core D[r, c] = sum_k X[r,k] Y[c,k]: r = column j of
// C, c = row i of C, X = op(B)^T, Y = op(A); opB = N and opA = T make both
// operands K-contiguous (the layout ggml and PyTorch use), the other
// combinations read through the transposed-operand loaders.
// Type pairs: (16F,16F -> 16F | 32F, compute 16F/32F) and (8I,8I -> 32I,
// compute 32I).  Pointer mode: host scalars only.
#include <hipblas/hipblas.h>

#include <cstdint>
#include <new>

#include "vkf_runtime.h"

namespace {

struct Handle {
    hipStream_t stream = nullptr;
    hipblasPointerMode_t mode = HIPBLAS_POINTER_MODE_HOST;
};

inline float half_to_float(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 0x1fu, m = h & 0x3ffu, bits;
    if (e == 0) {
        float v = (float)m * 5.9604644775390625e-08f;
        return sign ? -v : v;
    }
    bits = e == 31 ? (sign | 0x7f800000u | (m << 13)) : (sign | ((e + 112u) << 23) | (m << 13));
    float f;
    __builtin_memcpy(&f, &bits, 4);
    return f;
}

inline bool valid_op(hipblasOperation_t o) { return o == HIPBLAS_OP_N || o == HIPBLAS_OP_T || o == HIPBLAS_OP_C; }

hipblasStatus_t to_status(hipError_t e) {
    if (e == hipSuccess) return HIPBLAS_STATUS_SUCCESS;
    if (e == hipErrorInvalidValue) return HIPBLAS_STATUS_INVALID_VALUE;
    if (e == hipErrorNotSupported) return HIPBLAS_STATUS_NOT_SUPPORTED;
    return HIPBLAS_STATUS_EXECUTION_FAILED;
}

// One column-major GEMM.  esz_*: element bytes (for ld checks only).
hipblasStatus_t gemm_one(Handle *h, hipblasOperation_t ta, hipblasOperation_t tb, int m, int n, int k,
                         const void *alpha, const void *A, hipDataType at, int lda, const void *B, hipDataType bt,
                         int ldb, const void *beta, void *C, hipDataType ct, int ldc, hipblasComputeType_t comp) {
    if (!h) return HIPBLAS_STATUS_NOT_INITIALIZED;
    if (!valid_op(ta) || !valid_op(tb)) return HIPBLAS_STATUS_INVALID_ENUM;
    if (m < 0 || n < 0 || k < 0) return HIPBLAS_STATUS_INVALID_VALUE;
    const bool a_n = ta == HIPBLAS_OP_N, b_n = tb == HIPBLAS_OP_N;
    if (lda < (a_n ? (m > 1 ? m : 1) : (k > 1 ? k : 1)) || ldb < (b_n ? (k > 1 ? k : 1) : (n > 1 ? n : 1)) ||
        ldc < (m > 1 ? m : 1))
        return HIPBLAS_STATUS_INVALID_VALUE;
    if (m == 0 || n == 0) return HIPBLAS_STATUS_SUCCESS;
    if (!alpha || !beta) return HIPBLAS_STATUS_INVALID_VALUE;
    if (h->mode != HIPBLAS_POINTER_MODE_HOST) return HIPBLAS_STATUS_NOT_SUPPORTED;

    VkfGemmArgs g{};
    g.X = B;
    g.Y = A;
    g.D = C;
    g.Cin = C;
    g.R = (uint32_t)n;
    g.Cn = (uint32_t)m;
    g.K = (uint32_t)k;
    g.ldx = (uint64_t)ldb;
    g.ldy = (uint64_t)lda;
    g.ldd = (uint64_t)ldc;
    g.ldc = (uint64_t)ldc;
    g.flags = (b_n ? 0u : VKF_GF_X_TRANS) | (a_n ? VKF_GF_Y_TRANS : 0u);

    VkfKernelId kid;
    if (at == HIP_R_16F && bt == HIP_R_16F && (ct == HIP_R_16F || ct == HIP_R_32F)) {
        if (comp == HIPBLAS_COMPUTE_16F || comp == HIPBLAS_COMPUTE_16F_PEDANTIC) {
            if (ct != HIP_R_16F) return HIPBLAS_STATUS_NOT_SUPPORTED;
            g.alpha = half_to_float(*(const uint16_t *)alpha);
            g.beta = half_to_float(*(const uint16_t *)beta);
        } else if (comp == HIPBLAS_COMPUTE_32F || comp == HIPBLAS_COMPUTE_32F_PEDANTIC) {
            g.alpha = *(const float *)alpha;
            g.beta = *(const float *)beta;
        } else {
            return HIPBLAS_STATUS_NOT_SUPPORTED;
        }
        if (ct == HIP_R_32F) g.flags |= VKF_GF_D_F32 | VKF_GF_CIN_F32;
        kid = VKF_K_GEMM_F16;
    } else if (at == HIP_R_8I && bt == HIP_R_8I && ct == HIP_R_32I &&
               (comp == HIPBLAS_COMPUTE_32I || comp == HIPBLAS_COMPUTE_32I_PEDANTIC)) {
        g.alpha = (float)*(const int32_t *)alpha;
        g.beta = (float)*(const int32_t *)beta;
        g.flags |= VKF_GF_D_I32;
        kid = VKF_K_GEMM_I8;
    } else {
        return HIPBLAS_STATUS_NOT_SUPPORTED;
    }
    if (!A || !B || !C) return HIPBLAS_STATUS_INVALID_VALUE;
    if (vkf::debug_enabled())
        vkf::debug_log("hipblasGemmEx m=%d n=%d k=%d opA=%d opB=%d a=%d c=%d", m, n, k, (int)ta, (int)tb, (int)at,
                       (int)ct);
    return to_status(vkf::launch_gemm(kid, g, h->stream));
}

size_t dtype_bytes(hipDataType t) {
    switch (t) {
    case HIP_R_16F: return 2;
    case HIP_R_32F: return 4;
    case HIP_R_8I: return 1;
    case HIP_R_32I: return 4;
    default: return 0;
    }
}

}  // namespace

extern "C" {

hipblasStatus_t hipblasCreate(hipblasHandle_t *handle) {
    if (!handle) return HIPBLAS_STATUS_HANDLE_IS_NULLPTR;
    Handle *h = new (std::nothrow) Handle();
    if (!h) return HIPBLAS_STATUS_ALLOC_FAILED;
    *handle = h;
    return HIPBLAS_STATUS_SUCCESS;
}

hipblasStatus_t hipblasDestroy(hipblasHandle_t handle) {
    if (!handle) return HIPBLAS_STATUS_HANDLE_IS_NULLPTR;
    delete static_cast<Handle *>(handle);
    return HIPBLAS_STATUS_SUCCESS;
}

hipblasStatus_t hipblasSetStream(hipblasHandle_t handle, hipStream_t stream) {
    if (!handle) return HIPBLAS_STATUS_HANDLE_IS_NULLPTR;
    static_cast<Handle *>(handle)->stream = stream;
    return HIPBLAS_STATUS_SUCCESS;
}

hipblasStatus_t hipblasGetStream(hipblasHandle_t handle, hipStream_t *stream) {
    if (!handle) return HIPBLAS_STATUS_HANDLE_IS_NULLPTR;
    if (!stream) return HIPBLAS_STATUS_INVALID_VALUE;
    *stream = static_cast<Handle *>(handle)->stream;
    return HIPBLAS_STATUS_SUCCESS;
}

hipblasStatus_t hipblasSetPointerMode(hipblasHandle_t handle, hipblasPointerMode_t mode) {
    if (!handle) return HIPBLAS_STATUS_HANDLE_IS_NULLPTR;
    if (mode != HIPBLAS_POINTER_MODE_HOST && mode != HIPBLAS_POINTER_MODE_DEVICE) return HIPBLAS_STATUS_INVALID_ENUM;
    static_cast<Handle *>(handle)->mode = mode;
    return HIPBLAS_STATUS_SUCCESS;
}

hipblasStatus_t hipblasGetPointerMode(hipblasHandle_t handle, hipblasPointerMode_t *mode) {
    if (!handle) return HIPBLAS_STATUS_HANDLE_IS_NULLPTR;
    if (!mode) return HIPBLAS_STATUS_INVALID_VALUE;
    *mode = static_cast<Handle *>(handle)->mode;
    return HIPBLAS_STATUS_SUCCESS;
}

// shim/hipblas_shim.cpp:251-290
hipblasStatus_t hipblasGemmEx(hipblasHandle_t handle, hipblasOperation_t transA, hipblasOperation_t transB, int m,
                              int n, int k, const void *alpha, const void *A, hipDataType aType, int lda,
                              const void *B, hipDataType bType, int ldb, const void *beta, void *C, hipDataType cType,
                              int ldc, hipblasComputeType_t computeType, hipblasGemmAlgo_t algo) {
    (void)algo;
    return gemm_one(static_cast<Handle *>(handle), transA, transB, m, n, k, alpha, A, aType, lda, B, bType, ldb,
                    beta, C, cType, ldc, computeType);
}

// shim/hipblas_shim.cpp:293-314 (one launch per batch entry, as there)
hipblasStatus_t hipblasGemmBatchedEx(hipblasHandle_t handle, hipblasOperation_t transA, hipblasOperation_t transB,
                                     int m, int n, int k, const void *alpha, const void *A[], hipDataType aType,
                                     int lda, const void *B[], hipDataType bType, int ldb, const void *beta,
                                     void *C[], hipDataType cType, int ldc, int batchCount,
                                     hipblasComputeType_t computeType, hipblasGemmAlgo_t algo) {
    (void)algo;
    if (batchCount < 0) return HIPBLAS_STATUS_INVALID_VALUE;
    if (batchCount > 0 && (!A || !B || !C)) return HIPBLAS_STATUS_INVALID_VALUE;
    for (int b = 0; b < batchCount; b++) {
        hipblasStatus_t s = gemm_one(static_cast<Handle *>(handle), transA, transB, m, n, k, alpha, A[b], aType,
                                     lda, B[b], bType, ldb, beta, C[b], cType, ldc, computeType);
        if (s != HIPBLAS_STATUS_SUCCESS) return s;
    }
    return HIPBLAS_STATUS_SUCCESS;
}

// shim/hipblas_shim.cpp:317-349; element sizes follow the data types (the
// reference strides int8 with 4-byte elements, 332-334).
hipblasStatus_t hipblasGemmStridedBatchedEx(hipblasHandle_t handle, hipblasOperation_t transA,
                                            hipblasOperation_t transB, int m, int n, int k, const void *alpha,
                                            const void *A, hipDataType aType, int lda, hipblasStride strideA,
                                            const void *B, hipDataType bType, int ldb, hipblasStride strideB,
                                            const void *beta, void *C, hipDataType cType, int ldc,
                                            hipblasStride strideC, int batchCount, hipblasComputeType_t computeType,
                                            hipblasGemmAlgo_t algo) {
    (void)algo;
    if (batchCount < 0) return HIPBLAS_STATUS_INVALID_VALUE;
    size_t ea = dtype_bytes(aType), eb = dtype_bytes(bType), ec = dtype_bytes(cType);
    if (!ea || !eb || !ec) return HIPBLAS_STATUS_NOT_SUPPORTED;
    for (int b = 0; b < batchCount; b++) {
        hipblasStatus_t s = gemm_one(static_cast<Handle *>(handle), transA, transB, m, n, k, alpha,
                                     (const char *)A + (int64_t)b * strideA * ea, aType, lda,
                                     (const char *)B + (int64_t)b * strideB * eb, bType, ldb, beta,
                                     (char *)C + (int64_t)b * strideC * ec, cType, ldc, computeType);
        if (s != HIPBLAS_STATUS_SUCCESS) return s;
    }
    return HIPBLAS_STATUS_SUCCESS;
}

// shim/hipblas_shim.cpp:116-142 (fp16 in/out, fp16 scalars)
hipblasStatus_t hipblasHgemm(hipblasHandle_t handle, hipblasOperation_t transA, hipblasOperation_t transB, int m,
                             int n, int k, const hipblasHalf *alpha, const hipblasHalf *AP, int lda,
                             const hipblasHalf *BP, int ldb, const hipblasHalf *beta, hipblasHalf *CP, int ldc) {
    return gemm_one(static_cast<Handle *>(handle), transA, transB, m, n, k, alpha, AP, HIP_R_16F, lda, BP,
                    HIP_R_16F, ldb, beta, CP, HIP_R_16F, ldc, HIPBLAS_COMPUTE_16F);
}

// shim/hipblas_shim.cpp:168-188
hipblasStatus_t hipblasHgemmBatched(hipblasHandle_t handle, hipblasOperation_t transA, hipblasOperation_t transB,
                                    int m, int n, int k, const hipblasHalf *alpha, const hipblasHalf *const AP[],
                                    int lda, const hipblasHalf *const BP[], int ldb, const hipblasHalf *beta,
                                    hipblasHalf *const CP[], int ldc, int batchCount) {
    if (batchCount < 0) return HIPBLAS_STATUS_INVALID_VALUE;
    for (int b = 0; b < batchCount; b++) {
        hipblasStatus_t s = hipblasHgemm(handle, transA, transB, m, n, k, alpha, AP[b], lda, BP[b], ldb, beta,
                                         CP[b], ldc);
        if (s != HIPBLAS_STATUS_SUCCESS) return s;
    }
    return HIPBLAS_STATUS_SUCCESS;
}

// shim/hipblas_shim.cpp:219-245
hipblasStatus_t hipblasHgemmStridedBatched(hipblasHandle_t handle, hipblasOperation_t transA,
                                           hipblasOperation_t transB, int m, int n, int k, const hipblasHalf *alpha,
                                           const hipblasHalf *AP, int lda, long long strideA, const hipblasHalf *BP,
                                           int ldb, long long strideB, const hipblasHalf *beta, hipblasHalf *CP,
                                           int ldc, long long strideC, int batchCount) {
    if (batchCount < 0) return HIPBLAS_STATUS_INVALID_VALUE;
    for (int b = 0; b < batchCount; b++) {
        hipblasStatus_t s = hipblasHgemm(handle, transA, transB, m, n, k, alpha, AP + b * strideA, lda,
                                         BP + b * strideB, ldb, beta, CP + b * strideC, ldc);
        if (s != HIPBLAS_STATUS_SUCCESS) return s;
    }
    return HIPBLAS_STATUS_SUCCESS;
}

}  // extern "C"
