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
// Type pairs run here: (16F,16F -> 16F | 32F, compute 16F/32F), (32F,32F ->
// 32F, compute 32F; the Sgemm family) and (8I,8I -> 32I, compute 32I), with
// host-pointer scalars.
//
// Handles: with ROCm's hipBLAS present and a GPU visible, hipblasCreate
// returns ROCm's own handle (created by ROCm's hipblasCreate), so the
// functions this library does not export work on it unchanged, and the calls
// it does not run itself (other types, device-pointer scalars) are forwarded
// to ROCm's function of the same name.  Without ROCm's hipBLAS the handle is
// the library's own and such calls return HIPBLAS_STATUS_NOT_SUPPORTED.
#include <hipblas/hipblas.h>

#include <cstdint>
#include <mutex>
#include <new>
#include <unordered_map>

#include "vkf_runtime.h"

namespace {

// A handle of the library's own (no vendor hipBLAS).
struct Own {
    hipStream_t stream = nullptr;
    hipblasPointerMode_t mode = HIPBLAS_POINTER_MODE_HOST;
};

std::mutex g_mu;
std::unordered_map<void *, Own> g_own;

bool own_handle(hipblasHandle_t h) {
    std::lock_guard<std::mutex> lk(g_mu);
    return g_own.count(h) != 0;
}

template <class F>
F vendor(const char *name) {
    return reinterpret_cast<F>(vkf::vendor_symbol("libhipblas.so", name));
}

// The handle's stream and pointer mode (the library's own state, or asked
// of ROCm for a ROCm handle).
hipblasStatus_t handle_state(hipblasHandle_t h, hipStream_t *s, hipblasPointerMode_t *m) {
    if (!h) return HIPBLAS_STATUS_NOT_INITIALIZED;
    {
        std::lock_guard<std::mutex> lk(g_mu);
        auto it = g_own.find(h);
        if (it != g_own.end()) {
            *s = it->second.stream;
            *m = it->second.mode;
            return HIPBLAS_STATUS_SUCCESS;
        }
    }
    auto gs = vendor<hipblasStatus_t (*)(hipblasHandle_t, hipStream_t *)>("hipblasGetStream");
    auto gm = vendor<hipblasStatus_t (*)(hipblasHandle_t, hipblasPointerMode_t *)>("hipblasGetPointerMode");
    if (!gs || !gm) return HIPBLAS_STATUS_NOT_INITIALIZED;
    hipblasStatus_t st = gs(h, s);
    return st != HIPBLAS_STATUS_SUCCESS ? st : gm(h, m);
}

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

// Whether this library's kernels take the type combination.
bool ours(hipDataType at, hipDataType bt, hipDataType ct, hipblasComputeType_t comp) {
    if (at == HIP_R_16F && bt == HIP_R_16F) {
        if (comp == HIPBLAS_COMPUTE_16F || comp == HIPBLAS_COMPUTE_16F_PEDANTIC) return ct == HIP_R_16F;
        return (comp == HIPBLAS_COMPUTE_32F || comp == HIPBLAS_COMPUTE_32F_PEDANTIC) &&
               (ct == HIP_R_16F || ct == HIP_R_32F);
    }
    if (at == HIP_R_32F && bt == HIP_R_32F && ct == HIP_R_32F)
        return comp == HIPBLAS_COMPUTE_32F || comp == HIPBLAS_COMPUTE_32F_PEDANTIC;
    return at == HIP_R_8I && bt == HIP_R_8I && ct == HIP_R_32I &&
           (comp == HIPBLAS_COMPUTE_32I || comp == HIPBLAS_COMPUTE_32I_PEDANTIC);
}

// One column-major GEMM on this library's kernels, set up but not launched:
// HIPBLAS_STATUS_NOT_SUPPORTED for what they do not take; *empty when there
// is nothing to compute.  Matrix pointers are the caller's to check.
struct Prepared {
    VkfGemmArgs g;
    VkfKernelId kid;
    hipStream_t stream;
    bool empty;
};

hipblasStatus_t prepare(hipblasHandle_t h, hipblasOperation_t ta, hipblasOperation_t tb, int m, int n, int k,
                        const void *alpha, const void *A, hipDataType at, int lda, const void *B, hipDataType bt,
                        int ldb, const void *beta, void *C, hipDataType ct, int ldc, hipblasComputeType_t comp,
                        Prepared *p) {
    hipblasPointerMode_t mode;
    hipblasStatus_t st = handle_state(h, &p->stream, &mode);
    if (st != HIPBLAS_STATUS_SUCCESS) return st;
    if (!valid_op(ta) || !valid_op(tb)) return HIPBLAS_STATUS_INVALID_ENUM;
    if (m < 0 || n < 0 || k < 0) return HIPBLAS_STATUS_INVALID_VALUE;
    const bool a_n = ta == HIPBLAS_OP_N, b_n = tb == HIPBLAS_OP_N;
    if (lda < (a_n ? (m > 1 ? m : 1) : (k > 1 ? k : 1)) || ldb < (b_n ? (k > 1 ? k : 1) : (n > 1 ? n : 1)) ||
        ldc < (m > 1 ? m : 1))
        return HIPBLAS_STATUS_INVALID_VALUE;
    if (!ours(at, bt, ct, comp) || mode != HIPBLAS_POINTER_MODE_HOST) return HIPBLAS_STATUS_NOT_SUPPORTED;
    p->empty = m == 0 || n == 0;
    if (p->empty) return HIPBLAS_STATUS_SUCCESS;
    if (!alpha || !beta) return HIPBLAS_STATUS_INVALID_VALUE;

    VkfGemmArgs &g = p->g;
    g = VkfGemmArgs{};
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
    if (at == HIP_R_16F) {
        if (comp == HIPBLAS_COMPUTE_16F || comp == HIPBLAS_COMPUTE_16F_PEDANTIC) {
            g.alpha = half_to_float(*(const uint16_t *)alpha);
            g.beta = half_to_float(*(const uint16_t *)beta);
        } else {
            g.alpha = *(const float *)alpha;
            g.beta = *(const float *)beta;
        }
        if (ct == HIP_R_32F) g.flags |= VKF_GF_D_F32 | VKF_GF_CIN_F32;
        p->kid = VKF_K_GEMM_F16;
    } else if (at == HIP_R_32F) {
        g.alpha = *(const float *)alpha;
        g.beta = *(const float *)beta;
        g.flags |= VKF_GF_D_F32 | VKF_GF_CIN_F32;
        p->kid = VKF_K_GEMM_F32;
    } else {
        vkf_gemm_set_int_scalars(g, *(const int32_t *)alpha, *(const int32_t *)beta);
        g.flags |= VKF_GF_D_I32;
        p->kid = VKF_K_GEMM_I8;
    }
    if (vkf::debug_enabled())
        vkf::debug_log("hipblas gemm m=%d n=%d k=%d opA=%d opB=%d a=%d c=%d", m, n, k, (int)ta, (int)tb, (int)at,
                       (int)ct);
    return HIPBLAS_STATUS_SUCCESS;
}

hipblasStatus_t gemm_one(hipblasHandle_t h, hipblasOperation_t ta, hipblasOperation_t tb, int m, int n, int k,
                         const void *alpha, const void *A, hipDataType at, int lda, const void *B, hipDataType bt,
                         int ldb, const void *beta, void *C, hipDataType ct, int ldc, hipblasComputeType_t comp) {
    Prepared p;
    const hipblasStatus_t st = prepare(h, ta, tb, m, n, k, alpha, A, at, lda, B, bt, ldb, beta, C, ct, ldc, comp, &p);
    if (st != HIPBLAS_STATUS_SUCCESS || p.empty) return st;
    if (!A || !B || !C) return HIPBLAS_STATUS_INVALID_VALUE;
    return to_status(vkf::launch_gemm(p.kid, p.g, p.stream));
}

// The batch dimension rides on grid z, at most this many matrices per launch.
constexpr int kMaxBatchPerLaunch = 65535;

size_t dtype_bytes(hipDataType t) {
    switch (t) {
    case HIP_R_16F: return 2;
    case HIP_R_32F: return 4;
    case HIP_R_8I: return 1;
    case HIP_R_32I: return 4;
    default: return 0;
    }
}

// The library runs the call (status other than NOT_SUPPORTED), or, for a ROCm
// handle, ROCm's function of the same name runs it with the same arguments.
#define VKF_OR_VENDOR(status_expr, name, FnType, ...)                              \
    do {                                                                           \
        const hipblasStatus_t s_ = (status_expr);                                  \
        if (s_ != HIPBLAS_STATUS_NOT_SUPPORTED || own_handle(handle)) return s_;   \
        auto f_ = vendor<FnType>(name);                                            \
        if (!f_) return s_;                                                        \
        if (vkf::debug_enabled()) vkf::debug_log("%s -> ROCm hipBLAS", name);      \
        return f_(__VA_ARGS__);                                                    \
    } while (0)

}  // namespace

extern "C" {

hipblasStatus_t hipblasCreate(hipblasHandle_t *handle) {
    if (!handle) return HIPBLAS_STATUS_HANDLE_IS_NULLPTR;
    if (auto f = vendor<hipblasStatus_t (*)(hipblasHandle_t *)>("hipblasCreate")) {
        if (f(handle) == HIPBLAS_STATUS_SUCCESS) return HIPBLAS_STATUS_SUCCESS;
    }
    void *h = new (std::nothrow) char[1];
    if (!h) return HIPBLAS_STATUS_ALLOC_FAILED;
    std::lock_guard<std::mutex> lk(g_mu);
    g_own.emplace(h, Own{});
    *handle = h;
    return HIPBLAS_STATUS_SUCCESS;
}

hipblasStatus_t hipblasDestroy(hipblasHandle_t handle) {
    if (!handle) return HIPBLAS_STATUS_HANDLE_IS_NULLPTR;
    {
        std::lock_guard<std::mutex> lk(g_mu);
        if (g_own.erase(handle)) {
            delete[] static_cast<char *>(handle);
            return HIPBLAS_STATUS_SUCCESS;
        }
    }
    auto f = vendor<hipblasStatus_t (*)(hipblasHandle_t)>("hipblasDestroy");
    return f ? f(handle) : HIPBLAS_STATUS_NOT_INITIALIZED;
}

hipblasStatus_t hipblasSetStream(hipblasHandle_t handle, hipStream_t stream) {
    if (!handle) return HIPBLAS_STATUS_HANDLE_IS_NULLPTR;
    {
        std::lock_guard<std::mutex> lk(g_mu);
        auto it = g_own.find(handle);
        if (it != g_own.end()) {
            it->second.stream = stream;
            return HIPBLAS_STATUS_SUCCESS;
        }
    }
    auto f = vendor<hipblasStatus_t (*)(hipblasHandle_t, hipStream_t)>("hipblasSetStream");
    return f ? f(handle, stream) : HIPBLAS_STATUS_NOT_INITIALIZED;
}

hipblasStatus_t hipblasGetStream(hipblasHandle_t handle, hipStream_t *stream) {
    if (!handle) return HIPBLAS_STATUS_HANDLE_IS_NULLPTR;
    if (!stream) return HIPBLAS_STATUS_INVALID_VALUE;
    hipblasPointerMode_t m;
    return handle_state(handle, stream, &m);
}

hipblasStatus_t hipblasSetPointerMode(hipblasHandle_t handle, hipblasPointerMode_t mode) {
    if (!handle) return HIPBLAS_STATUS_HANDLE_IS_NULLPTR;
    if (mode != HIPBLAS_POINTER_MODE_HOST && mode != HIPBLAS_POINTER_MODE_DEVICE) return HIPBLAS_STATUS_INVALID_ENUM;
    {
        std::lock_guard<std::mutex> lk(g_mu);
        auto it = g_own.find(handle);
        if (it != g_own.end()) {
            it->second.mode = mode;
            return HIPBLAS_STATUS_SUCCESS;
        }
    }
    auto f = vendor<hipblasStatus_t (*)(hipblasHandle_t, hipblasPointerMode_t)>("hipblasSetPointerMode");
    return f ? f(handle, mode) : HIPBLAS_STATUS_NOT_INITIALIZED;
}

hipblasStatus_t hipblasGetPointerMode(hipblasHandle_t handle, hipblasPointerMode_t *mode) {
    if (!handle) return HIPBLAS_STATUS_HANDLE_IS_NULLPTR;
    if (!mode) return HIPBLAS_STATUS_INVALID_VALUE;
    hipStream_t s;
    return handle_state(handle, &s, mode);
}

// shim/hipblas_shim.cpp:251-290
hipblasStatus_t hipblasGemmEx(hipblasHandle_t handle, hipblasOperation_t transA, hipblasOperation_t transB, int m,
                              int n, int k, const void *alpha, const void *A, hipDataType aType, int lda,
                              const void *B, hipDataType bType, int ldb, const void *beta, void *C, hipDataType cType,
                              int ldc, hipblasComputeType_t computeType, hipblasGemmAlgo_t algo) {
    VKF_OR_VENDOR(gemm_one(handle, transA, transB, m, n, k, alpha, A, aType, lda, B, bType, ldb, beta, C, cType, ldc,
                           computeType),
                  "hipblasGemmEx", decltype(&hipblasGemmEx), handle, transA, transB, m, n, k, alpha, A, aType, lda, B,
                  bType, ldb, beta, C, cType, ldc, computeType, algo);
}

// shim/hipblas_shim.cpp:293-314.  One launch per up to 65535 matrices, each
// workgroup reading its matrices' addresses from the caller's device arrays
// of device pointers (hipBLAS's batched convention; the reference reads them
// on the host and dispatches once per matrix, shim/hipblas_shim.cpp:159-164).
static hipblasStatus_t gemm_batched(hipblasHandle_t handle, hipblasOperation_t transA, hipblasOperation_t transB,
                                    int m, int n, int k, const void *alpha, const void *const A[], hipDataType aType,
                                    int lda, const void *const B[], hipDataType bType, int ldb, const void *beta,
                                    void *const C[], hipDataType cType, int ldc, int batchCount,
                                    hipblasComputeType_t computeType) {
    if (batchCount < 0) return HIPBLAS_STATUS_INVALID_VALUE;
    Prepared p;
    hipblasStatus_t st = prepare(handle, transA, transB, m, n, k, alpha, nullptr, aType, lda, nullptr, bType, ldb,
                                 beta, nullptr, cType, ldc, computeType, &p);
    if (st != HIPBLAS_STATUS_SUCCESS || p.empty || batchCount == 0) return st;
    if (!A || !B || !C) return HIPBLAS_STATUS_INVALID_VALUE;
    for (int b0 = 0; b0 < batchCount; b0 += kMaxBatchPerLaunch) {
        VkfGemmArgs g = p.g;
        g.bpx = (const void *const *)(B + b0);  // X = op(B)^T, Y = op(A)
        g.bpy = (const void *const *)(A + b0);
        g.bpd = C + b0;
        const int nb = batchCount - b0 < kMaxBatchPerLaunch ? batchCount - b0 : kMaxBatchPerLaunch;
        st = to_status(vkf::launch_gemm(p.kid, g, p.stream, (uint32_t)nb));
        if (st != HIPBLAS_STATUS_SUCCESS) return st;
    }
    return HIPBLAS_STATUS_SUCCESS;
}

hipblasStatus_t hipblasGemmBatchedEx(hipblasHandle_t handle, hipblasOperation_t transA, hipblasOperation_t transB,
                                     int m, int n, int k, const void *alpha, const void *A[], hipDataType aType,
                                     int lda, const void *B[], hipDataType bType, int ldb, const void *beta,
                                     void *C[], hipDataType cType, int ldc, int batchCount,
                                     hipblasComputeType_t computeType, hipblasGemmAlgo_t algo) {
    VKF_OR_VENDOR(gemm_batched(handle, transA, transB, m, n, k, alpha, A, aType, lda, B, bType, ldb, beta, C, cType,
                               ldc, batchCount, computeType),
                  "hipblasGemmBatchedEx", decltype(&hipblasGemmBatchedEx), handle, transA, transB, m, n, k, alpha, A,
                  aType, lda, B, bType, ldb, beta, C, cType, ldc, batchCount, computeType, algo);
}

// shim/hipblas_shim.cpp:317-349.  One launch per up to 65535 matrices at
// constant strides, in elements of each operand's type (the reference
// strides int8 with 4-byte elements, 332-334, and dispatches once per matrix).
static hipblasStatus_t gemm_strided(hipblasHandle_t handle, hipblasOperation_t transA, hipblasOperation_t transB,
                                    int m, int n, int k, const void *alpha, const void *A, hipDataType aType, int lda,
                                    hipblasStride strideA, const void *B, hipDataType bType, int ldb,
                                    hipblasStride strideB, const void *beta, void *C, hipDataType cType, int ldc,
                                    hipblasStride strideC, int batchCount, hipblasComputeType_t computeType) {
    if (batchCount < 0 || strideA < 0 || strideB < 0 || strideC < 0) return HIPBLAS_STATUS_INVALID_VALUE;
    Prepared p;
    hipblasStatus_t st = prepare(handle, transA, transB, m, n, k, alpha, A, aType, lda, B, bType, ldb, beta, C, cType,
                                 ldc, computeType, &p);
    if (st != HIPBLAS_STATUS_SUCCESS || p.empty || batchCount == 0) return st;
    if (!A || !B || !C) return HIPBLAS_STATUS_INVALID_VALUE;
    const uint64_t sa = (uint64_t)strideA * dtype_bytes(aType), sb = (uint64_t)strideB * dtype_bytes(bType),
                   sc = (uint64_t)strideC * dtype_bytes(cType);
    for (int b0 = 0; b0 < batchCount; b0 += kMaxBatchPerLaunch) {
        VkfGemmArgs g = p.g;
        g.X = (const uint8_t *)B + b0 * sb;
        g.Y = (const uint8_t *)A + b0 * sa;
        g.D = (uint8_t *)C + b0 * sc;
        g.Cin = g.D;
        g.bsx = sb;
        g.bsy = sa;
        g.bsd = sc;
        g.bsc = sc;
        const int nb = batchCount - b0 < kMaxBatchPerLaunch ? batchCount - b0 : kMaxBatchPerLaunch;
        st = to_status(vkf::launch_gemm(p.kid, g, p.stream, (uint32_t)nb));
        if (st != HIPBLAS_STATUS_SUCCESS) return st;
    }
    return HIPBLAS_STATUS_SUCCESS;
}

hipblasStatus_t hipblasGemmStridedBatchedEx(hipblasHandle_t handle, hipblasOperation_t transA,
                                            hipblasOperation_t transB, int m, int n, int k, const void *alpha,
                                            const void *A, hipDataType aType, int lda, hipblasStride strideA,
                                            const void *B, hipDataType bType, int ldb, hipblasStride strideB,
                                            const void *beta, void *C, hipDataType cType, int ldc,
                                            hipblasStride strideC, int batchCount, hipblasComputeType_t computeType,
                                            hipblasGemmAlgo_t algo) {
    VKF_OR_VENDOR(gemm_strided(handle, transA, transB, m, n, k, alpha, A, aType, lda, strideA, B, bType, ldb, strideB,
                               beta, C, cType, ldc, strideC, batchCount, computeType),
                  "hipblasGemmStridedBatchedEx", decltype(&hipblasGemmStridedBatchedEx), handle, transA, transB, m, n,
                  k, alpha, A, aType, lda, strideA, B, bType, ldb, strideB, beta, C, cType, ldc, strideC, batchCount,
                  computeType, algo);
}

// shim/hipblas_shim.cpp:116-142 (fp16 in/out, fp16 scalars)
hipblasStatus_t hipblasHgemm(hipblasHandle_t handle, hipblasOperation_t transA, hipblasOperation_t transB, int m,
                             int n, int k, const hipblasHalf *alpha, const hipblasHalf *AP, int lda,
                             const hipblasHalf *BP, int ldb, const hipblasHalf *beta, hipblasHalf *CP, int ldc) {
    VKF_OR_VENDOR(gemm_one(handle, transA, transB, m, n, k, alpha, AP, HIP_R_16F, lda, BP, HIP_R_16F, ldb, beta, CP,
                           HIP_R_16F, ldc, HIPBLAS_COMPUTE_16F),
                  "hipblasHgemm", decltype(&hipblasHgemm), handle, transA, transB, m, n, k, alpha, AP, lda, BP, ldb,
                  beta, CP, ldc);
}

// shim/hipblas_shim.cpp:168-188
hipblasStatus_t hipblasHgemmBatched(hipblasHandle_t handle, hipblasOperation_t transA, hipblasOperation_t transB,
                                    int m, int n, int k, const hipblasHalf *alpha, const hipblasHalf *const AP[],
                                    int lda, const hipblasHalf *const BP[], int ldb, const hipblasHalf *beta,
                                    hipblasHalf *const CP[], int ldc, int batchCount) {
    VKF_OR_VENDOR(gemm_batched(handle, transA, transB, m, n, k, alpha, (const void *const *)AP, HIP_R_16F, lda,
                               (const void *const *)BP, HIP_R_16F, ldb, beta, (void *const *)CP, HIP_R_16F, ldc,
                               batchCount, HIPBLAS_COMPUTE_16F),
                  "hipblasHgemmBatched", decltype(&hipblasHgemmBatched), handle, transA, transB, m, n, k, alpha, AP,
                  lda, BP, ldb, beta, CP, ldc, batchCount);
}

// shim/hipblas_shim.cpp:219-245
hipblasStatus_t hipblasHgemmStridedBatched(hipblasHandle_t handle, hipblasOperation_t transA,
                                           hipblasOperation_t transB, int m, int n, int k, const hipblasHalf *alpha,
                                           const hipblasHalf *AP, int lda, long long strideA, const hipblasHalf *BP,
                                           int ldb, long long strideB, const hipblasHalf *beta, hipblasHalf *CP,
                                           int ldc, long long strideC, int batchCount) {
    VKF_OR_VENDOR(gemm_strided(handle, transA, transB, m, n, k, alpha, AP, HIP_R_16F, lda, strideA, BP, HIP_R_16F,
                               ldb, strideB, beta, CP, HIP_R_16F, ldc, strideC, batchCount, HIPBLAS_COMPUTE_16F),
                  "hipblasHgemmStridedBatched", decltype(&hipblasHgemmStridedBatched), handle, transA, transB, m, n, k,
                  alpha, AP, lda, strideA, BP, ldb, strideB, beta, CP, ldc, strideC, batchCount);
}

// shim/hipblas_shim.cpp:84-113 (fp32 in/out, fp32 scalars; the reference
// hands fp32 data to its fp16 shader)
hipblasStatus_t hipblasSgemm(hipblasHandle_t handle, hipblasOperation_t transA, hipblasOperation_t transB, int m,
                             int n, int k, const float *alpha, const float *AP, int lda, const float *BP, int ldb,
                             const float *beta, float *CP, int ldc) {
    VKF_OR_VENDOR(gemm_one(handle, transA, transB, m, n, k, alpha, AP, HIP_R_32F, lda, BP, HIP_R_32F, ldb, beta, CP,
                           HIP_R_32F, ldc, HIPBLAS_COMPUTE_32F),
                  "hipblasSgemm", decltype(&hipblasSgemm), handle, transA, transB, m, n, k, alpha, AP, lda, BP, ldb,
                  beta, CP, ldc);
}

// shim/hipblas_shim.cpp:145-166 (the reference also passes its own m and k
// as the leading dimensions; here the caller's are used)
hipblasStatus_t hipblasSgemmBatched(hipblasHandle_t handle, hipblasOperation_t transA, hipblasOperation_t transB,
                                    int m, int n, int k, const float *alpha, const float *const AP[], int lda,
                                    const float *const BP[], int ldb, const float *beta, float *const CP[], int ldc,
                                    int batchCount) {
    VKF_OR_VENDOR(gemm_batched(handle, transA, transB, m, n, k, alpha, (const void *const *)AP, HIP_R_32F, lda,
                               (const void *const *)BP, HIP_R_32F, ldb, beta, (void *const *)CP, HIP_R_32F, ldc,
                               batchCount, HIPBLAS_COMPUTE_32F),
                  "hipblasSgemmBatched", decltype(&hipblasSgemmBatched), handle, transA, transB, m, n, k, alpha, AP,
                  lda, BP, ldb, beta, CP, ldc, batchCount);
}

// shim/hipblas_shim.cpp:191-217
hipblasStatus_t hipblasSgemmStridedBatched(hipblasHandle_t handle, hipblasOperation_t transA,
                                           hipblasOperation_t transB, int m, int n, int k, const float *alpha,
                                           const float *AP, int lda, long long strideA, const float *BP, int ldb,
                                           long long strideB, const float *beta, float *CP, int ldc,
                                           long long strideC, int batchCount) {
    VKF_OR_VENDOR(gemm_strided(handle, transA, transB, m, n, k, alpha, AP, HIP_R_32F, lda, strideA, BP, HIP_R_32F,
                               ldb, strideB, beta, CP, HIP_R_32F, ldc, strideC, batchCount, HIPBLAS_COMPUTE_32F),
                  "hipblasSgemmStridedBatched", decltype(&hipblasSgemmStridedBatched), handle, transA, transB, m, n, k,
                  alpha, AP, lda, strideA, BP, ldb, strideB, beta, CP, ldc, strideC, batchCount);
}

}  // extern "C"
