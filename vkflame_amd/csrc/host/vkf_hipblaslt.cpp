// vkf_hipblaslt.cpp — hipBLASLt entry points over the gfx950 MFMA kernels.
//
// Same names, signatures and enum values as ROCm 7.2's hipblaslt.h (included,
// so every signature is compiler-checked), exported from libvkflame_amd.so.
// Replaces shim/hipblaslt_shim.cpp:99-426.  The reference reads M,N,K from the
// layouts assuming row-major, maps the epilogue to an activation and drops
// bias, A/B scales, alpha, beta, ld and order (shim/hipblaslt_shim.cpp:369-423,
// its own enum numbering, shim/hipblaslt_shim.cpp:20-50).  Here:
//   D = act( alpha * scaleA * scaleB * op(A) op(B) + beta * C + bias )
// with column-major (default) or row-major layouts, per-tensor scalar or
// OUTER_VEC_32F scales (a_scale per row of op(A), b_scale per column of
// op(B)), a bias vector over the rows of D, and the epilogues
// DEFAULT / RELU / BIAS / RELU_BIAS / GELU / GELU_BIAS / SWISH_EXT /
// SWISH_BIAS_EXT (GELU is the erf form, as in the reference's kernels).
// Types: fp16 x fp16 -> fp16 | fp32 (compute 32F) and int8 x int8 -> int32
// (compute 32I, raw accumulator) or -> fp16 | fp32 (compute 32I or 32F with
// the fp32 epilogue).  Batched layouts loop one launch per matrix.
#include <hipblaslt/hipblaslt.h>

#include <cstdint>
#include <cstring>
#include <new>

#include "vkf_runtime.h"

namespace {

struct Layout {
    hipDataType type;
    uint64_t rows, cols;
    int64_t ld;
    int32_t order;
    int32_t batch;
    int64_t stride;
};

struct Desc {
    hipblasComputeType_t compute;
    hipDataType scale_type;
    int32_t transA, transB;
    uint32_t epilogue;
    const void *bias;
    int32_t bias_type;  // -1: follow D
    const void *a_scale, *b_scale;
    int32_t a_scale_mode, b_scale_mode;
    int32_t pointer_mode;
};

struct Pref {
    uint64_t max_ws;
    uint32_t search_mode;
};

struct LtHandle {
    int magic;
};

template <class T>
hipblasStatus_t put(void *buf, size_t size, size_t *written, T v) {
    if (written) *written = sizeof(T);
    if (!buf) return written ? HIPBLAS_STATUS_SUCCESS : HIPBLAS_STATUS_INVALID_VALUE;
    if (size < sizeof(T)) return HIPBLAS_STATUS_INVALID_VALUE;
    std::memcpy(buf, &v, sizeof(T));
    return HIPBLAS_STATUS_SUCCESS;
}

template <class T>
hipblasStatus_t get(const void *buf, size_t size, T *out) {
    if (!buf || size != sizeof(T)) return HIPBLAS_STATUS_INVALID_VALUE;
    std::memcpy(out, buf, sizeof(T));
    return HIPBLAS_STATUS_SUCCESS;
}

hipblasStatus_t to_status(hipError_t e) {
    if (e == hipSuccess) return HIPBLAS_STATUS_SUCCESS;
    if (e == hipErrorInvalidValue) return HIPBLAS_STATUS_INVALID_VALUE;
    if (e == hipErrorNotSupported) return HIPBLAS_STATUS_NOT_SUPPORTED;
    return HIPBLAS_STATUS_EXECUTION_FAILED;
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

// epilogue -> (activation code, has bias); false if unsupported.
bool map_epilogue(uint32_t e, uint32_t *act, bool *bias) {
    switch (e) {
    case HIPBLASLT_EPILOGUE_DEFAULT: *act = VKF_ACT_NONE; *bias = false; return true;
    case HIPBLASLT_EPILOGUE_RELU: *act = VKF_ACT_RELU; *bias = false; return true;
    case HIPBLASLT_EPILOGUE_BIAS: *act = VKF_ACT_NONE; *bias = true; return true;
    case HIPBLASLT_EPILOGUE_RELU_BIAS: *act = VKF_ACT_RELU; *bias = true; return true;
    case HIPBLASLT_EPILOGUE_GELU: *act = VKF_ACT_GELU_ERF; *bias = false; return true;
    case HIPBLASLT_EPILOGUE_GELU_BIAS: *act = VKF_ACT_GELU_ERF; *bias = true; return true;
    case HIPBLASLT_EPILOGUE_SWISH_EXT: *act = VKF_ACT_SILU; *bias = false; return true;
    case HIPBLASLT_EPILOGUE_SWISH_BIAS_EXT: *act = VKF_ACT_SILU; *bias = true; return true;
    default: return false;
    }
}

}  // namespace

extern "C" {

hipblasStatus_t hipblasLtCreate(hipblasLtHandle_t *handle) {
    if (!handle) return HIPBLAS_STATUS_INVALID_VALUE;
    LtHandle *h = new (std::nothrow) LtHandle{0x564b464c};
    if (!h) return HIPBLAS_STATUS_ALLOC_FAILED;
    *handle = h;
    return HIPBLAS_STATUS_SUCCESS;
}

hipblasStatus_t hipblasLtDestroy(const hipblasLtHandle_t handle) {
    if (!handle) return HIPBLAS_STATUS_NOT_INITIALIZED;
    delete static_cast<LtHandle *>(handle);
    return HIPBLAS_STATUS_SUCCESS;
}

// shim/hipblaslt_shim.cpp:120-134 (the reference ignores ld and assumes row-major)
hipblasStatus_t hipblasLtMatrixLayoutCreate(hipblasLtMatrixLayout_t *matLayout, hipDataType type, uint64_t rows,
                                            uint64_t cols, int64_t ld) {
    if (!matLayout) return HIPBLAS_STATUS_INVALID_VALUE;
    Layout *l = new (std::nothrow) Layout{type, rows, cols, ld, HIPBLASLT_ORDER_COL, 1, 0};
    if (!l) return HIPBLAS_STATUS_ALLOC_FAILED;
    *matLayout = reinterpret_cast<hipblasLtMatrixLayout_t>(l);
    return HIPBLAS_STATUS_SUCCESS;
}

hipblasStatus_t hipblasLtMatrixLayoutDestroy(const hipblasLtMatrixLayout_t matLayout) {
    if (!matLayout) return HIPBLAS_STATUS_INVALID_VALUE;
    delete reinterpret_cast<Layout *>(matLayout);
    return HIPBLAS_STATUS_SUCCESS;
}

// shim/hipblaslt_shim.cpp:142-173
hipblasStatus_t hipblasLtMatrixLayoutSetAttribute(hipblasLtMatrixLayout_t matLayout,
                                                  hipblasLtMatrixLayoutAttribute_t attr, const void *buf,
                                                  size_t sizeInBytes) {
    if (!matLayout) return HIPBLAS_STATUS_INVALID_VALUE;
    Layout *l = reinterpret_cast<Layout *>(matLayout);
    switch (attr) {
    case HIPBLASLT_MATRIX_LAYOUT_BATCH_COUNT: return get(buf, sizeInBytes, &l->batch);
    case HIPBLASLT_MATRIX_LAYOUT_STRIDED_BATCH_OFFSET: return get(buf, sizeInBytes, &l->stride);
    case HIPBLASLT_MATRIX_LAYOUT_TYPE: {
        uint32_t t;
        hipblasStatus_t s = get(buf, sizeInBytes, &t);
        if (s == HIPBLAS_STATUS_SUCCESS) l->type = (hipDataType)t;
        return s;
    }
    case HIPBLASLT_MATRIX_LAYOUT_ORDER: return get(buf, sizeInBytes, &l->order);
    case HIPBLASLT_MATRIX_LAYOUT_ROWS: return get(buf, sizeInBytes, &l->rows);
    case HIPBLASLT_MATRIX_LAYOUT_COLS: return get(buf, sizeInBytes, &l->cols);
    case HIPBLASLT_MATRIX_LAYOUT_LD: return get(buf, sizeInBytes, &l->ld);
    default: return HIPBLAS_STATUS_INVALID_VALUE;
    }
}

// shim/hipblaslt_shim.cpp:175-209
hipblasStatus_t hipblasLtMatrixLayoutGetAttribute(hipblasLtMatrixLayout_t matLayout,
                                                  hipblasLtMatrixLayoutAttribute_t attr, void *buf,
                                                  size_t sizeInBytes, size_t *sizeWritten) {
    if (!matLayout) return HIPBLAS_STATUS_INVALID_VALUE;
    const Layout *l = reinterpret_cast<const Layout *>(matLayout);
    switch (attr) {
    case HIPBLASLT_MATRIX_LAYOUT_BATCH_COUNT: return put(buf, sizeInBytes, sizeWritten, l->batch);
    case HIPBLASLT_MATRIX_LAYOUT_STRIDED_BATCH_OFFSET: return put(buf, sizeInBytes, sizeWritten, l->stride);
    case HIPBLASLT_MATRIX_LAYOUT_TYPE: return put(buf, sizeInBytes, sizeWritten, (uint32_t)l->type);
    case HIPBLASLT_MATRIX_LAYOUT_ORDER: return put(buf, sizeInBytes, sizeWritten, l->order);
    case HIPBLASLT_MATRIX_LAYOUT_ROWS: return put(buf, sizeInBytes, sizeWritten, l->rows);
    case HIPBLASLT_MATRIX_LAYOUT_COLS: return put(buf, sizeInBytes, sizeWritten, l->cols);
    case HIPBLASLT_MATRIX_LAYOUT_LD: return put(buf, sizeInBytes, sizeWritten, l->ld);
    default: return HIPBLAS_STATUS_INVALID_VALUE;
    }
}

// shim/hipblaslt_shim.cpp:213-229
hipblasStatus_t hipblasLtMatmulDescCreate(hipblasLtMatmulDesc_t *matmulDesc, hipblasComputeType_t computeType,
                                          hipDataType scaleType) {
    if (!matmulDesc) return HIPBLAS_STATUS_INVALID_VALUE;
    Desc *d = new (std::nothrow) Desc{computeType,
                                      scaleType,
                                      HIPBLAS_OP_N,
                                      HIPBLAS_OP_N,
                                      HIPBLASLT_EPILOGUE_DEFAULT,
                                      nullptr,
                                      -1,
                                      nullptr,
                                      nullptr,
                                      HIPBLASLT_MATMUL_MATRIX_SCALE_SCALAR_32F,
                                      HIPBLASLT_MATMUL_MATRIX_SCALE_SCALAR_32F,
                                      HIPBLASLT_POINTER_MODE_HOST};
    if (!d) return HIPBLAS_STATUS_ALLOC_FAILED;
    *matmulDesc = reinterpret_cast<hipblasLtMatmulDesc_t>(d);
    return HIPBLAS_STATUS_SUCCESS;
}

hipblasStatus_t hipblasLtMatmulDescDestroy(const hipblasLtMatmulDesc_t matmulDesc) {
    if (!matmulDesc) return HIPBLAS_STATUS_INVALID_VALUE;
    delete reinterpret_cast<Desc *>(matmulDesc);
    return HIPBLAS_STATUS_SUCCESS;
}

// shim/hipblaslt_shim.cpp:237-267
hipblasStatus_t hipblasLtMatmulDescSetAttribute(hipblasLtMatmulDesc_t matmulDesc, hipblasLtMatmulDescAttributes_t attr,
                                                const void *buf, size_t sizeInBytes) {
    if (!matmulDesc) return HIPBLAS_STATUS_INVALID_VALUE;
    Desc *d = reinterpret_cast<Desc *>(matmulDesc);
    switch (attr) {
    case HIPBLASLT_MATMUL_DESC_TRANSA: return get(buf, sizeInBytes, &d->transA);
    case HIPBLASLT_MATMUL_DESC_TRANSB: return get(buf, sizeInBytes, &d->transB);
    case HIPBLASLT_MATMUL_DESC_EPILOGUE: return get(buf, sizeInBytes, &d->epilogue);
    case HIPBLASLT_MATMUL_DESC_BIAS_POINTER: return get(buf, sizeInBytes, &d->bias);
    case HIPBLASLT_MATMUL_DESC_BIAS_DATA_TYPE: return get(buf, sizeInBytes, &d->bias_type);
    case HIPBLASLT_MATMUL_DESC_A_SCALE_POINTER: return get(buf, sizeInBytes, &d->a_scale);
    case HIPBLASLT_MATMUL_DESC_B_SCALE_POINTER: return get(buf, sizeInBytes, &d->b_scale);
    case HIPBLASLT_MATMUL_DESC_A_SCALE_MODE: return get(buf, sizeInBytes, &d->a_scale_mode);
    case HIPBLASLT_MATMUL_DESC_B_SCALE_MODE: return get(buf, sizeInBytes, &d->b_scale_mode);
    case HIPBLASLT_MATMUL_DESC_POINTER_MODE: return get(buf, sizeInBytes, &d->pointer_mode);
    default: return HIPBLAS_STATUS_NOT_SUPPORTED;
    }
}

// shim/hipblaslt_shim.cpp:269-292
hipblasStatus_t hipblasLtMatmulDescGetAttribute(hipblasLtMatmulDesc_t matmulDesc, hipblasLtMatmulDescAttributes_t attr,
                                                void *buf, size_t sizeInBytes, size_t *sizeWritten) {
    if (!matmulDesc) return HIPBLAS_STATUS_INVALID_VALUE;
    const Desc *d = reinterpret_cast<const Desc *>(matmulDesc);
    switch (attr) {
    case HIPBLASLT_MATMUL_DESC_TRANSA: return put(buf, sizeInBytes, sizeWritten, d->transA);
    case HIPBLASLT_MATMUL_DESC_TRANSB: return put(buf, sizeInBytes, sizeWritten, d->transB);
    case HIPBLASLT_MATMUL_DESC_EPILOGUE: return put(buf, sizeInBytes, sizeWritten, d->epilogue);
    case HIPBLASLT_MATMUL_DESC_BIAS_POINTER: return put(buf, sizeInBytes, sizeWritten, d->bias);
    case HIPBLASLT_MATMUL_DESC_BIAS_DATA_TYPE: return put(buf, sizeInBytes, sizeWritten, d->bias_type);
    case HIPBLASLT_MATMUL_DESC_A_SCALE_POINTER: return put(buf, sizeInBytes, sizeWritten, d->a_scale);
    case HIPBLASLT_MATMUL_DESC_B_SCALE_POINTER: return put(buf, sizeInBytes, sizeWritten, d->b_scale);
    case HIPBLASLT_MATMUL_DESC_A_SCALE_MODE: return put(buf, sizeInBytes, sizeWritten, d->a_scale_mode);
    case HIPBLASLT_MATMUL_DESC_B_SCALE_MODE: return put(buf, sizeInBytes, sizeWritten, d->b_scale_mode);
    case HIPBLASLT_MATMUL_DESC_POINTER_MODE: return put(buf, sizeInBytes, sizeWritten, d->pointer_mode);
    default: return HIPBLAS_STATUS_NOT_SUPPORTED;
    }
}

// shim/hipblaslt_shim.cpp:296-319
hipblasStatus_t hipblasLtMatmulPreferenceCreate(hipblasLtMatmulPreference_t *pref) {
    if (!pref) return HIPBLAS_STATUS_INVALID_VALUE;
    Pref *p = new (std::nothrow) Pref{0, 0};
    if (!p) return HIPBLAS_STATUS_ALLOC_FAILED;
    *pref = reinterpret_cast<hipblasLtMatmulPreference_t>(p);
    return HIPBLAS_STATUS_SUCCESS;
}

hipblasStatus_t hipblasLtMatmulPreferenceDestroy(const hipblasLtMatmulPreference_t pref) {
    if (!pref) return HIPBLAS_STATUS_INVALID_VALUE;
    delete reinterpret_cast<Pref *>(pref);
    return HIPBLAS_STATUS_SUCCESS;
}

hipblasStatus_t hipblasLtMatmulPreferenceSetAttribute(hipblasLtMatmulPreference_t pref,
                                                      hipblasLtMatmulPreferenceAttributes_t attr, const void *buf,
                                                      size_t sizeInBytes) {
    if (!pref) return HIPBLAS_STATUS_INVALID_VALUE;
    Pref *p = reinterpret_cast<Pref *>(pref);
    switch (attr) {
    case HIPBLASLT_MATMUL_PREF_SEARCH_MODE: return get(buf, sizeInBytes, &p->search_mode);
    case HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES: return get(buf, sizeInBytes, &p->max_ws);
    default: return HIPBLAS_STATUS_INVALID_VALUE;
    }
}

// shim/hipblaslt_shim.cpp:323-343: one algorithm, no workspace.
hipblasStatus_t hipblasLtMatmulAlgoGetHeuristic(hipblasLtHandle_t handle, hipblasLtMatmulDesc_t matmulDesc,
                                                hipblasLtMatrixLayout_t Adesc, hipblasLtMatrixLayout_t Bdesc,
                                                hipblasLtMatrixLayout_t Cdesc, hipblasLtMatrixLayout_t Ddesc,
                                                hipblasLtMatmulPreference_t pref, int requestedAlgoCount,
                                                hipblasLtMatmulHeuristicResult_t heuristicResultsArray[],
                                                int *returnAlgoCount) {
    (void)pref;
    if (!handle) return HIPBLAS_STATUS_NOT_INITIALIZED;
    if (!matmulDesc || !Adesc || !Bdesc || !Cdesc || !Ddesc || !returnAlgoCount || requestedAlgoCount <= 0 ||
        !heuristicResultsArray)
        return HIPBLAS_STATUS_INVALID_VALUE;
    hipblasLtMatmulHeuristicResult_t r{};
    std::memcpy(r.algo.data, "vkf-mfma", 8);
    r.algo.max_workspace_bytes = 0;
    r.workspaceSize = 0;
    r.state = HIPBLAS_STATUS_SUCCESS;
    r.wavesCount = 1.0f;
    heuristicResultsArray[0] = r;
    *returnAlgoCount = 1;
    return HIPBLAS_STATUS_SUCCESS;
}

// shim/hipblaslt_shim.cpp:347-426
hipblasStatus_t hipblasLtMatmul(hipblasLtHandle_t handle, hipblasLtMatmulDesc_t matmulDesc, const void *alpha,
                                const void *A, hipblasLtMatrixLayout_t Adesc, const void *B,
                                hipblasLtMatrixLayout_t Bdesc, const void *beta, const void *C,
                                hipblasLtMatrixLayout_t Cdesc, void *D, hipblasLtMatrixLayout_t Ddesc,
                                const hipblasLtMatmulAlgo_t *algo, void *workspace, size_t workspaceSizeInBytes,
                                hipStream_t stream) {
    (void)algo;
    (void)workspace;
    (void)workspaceSizeInBytes;
    if (!handle) return HIPBLAS_STATUS_NOT_INITIALIZED;
    if (!matmulDesc || !Adesc || !Bdesc || !Cdesc || !Ddesc || !alpha || !beta) return HIPBLAS_STATUS_INVALID_VALUE;
    const Desc *d = reinterpret_cast<const Desc *>(matmulDesc);
    const Layout *la = reinterpret_cast<const Layout *>(Adesc), *lb = reinterpret_cast<const Layout *>(Bdesc),
                 *lc = reinterpret_cast<const Layout *>(Cdesc), *ld = reinterpret_cast<const Layout *>(Ddesc);
    if (d->pointer_mode != HIPBLASLT_POINTER_MODE_HOST) return HIPBLAS_STATUS_NOT_SUPPORTED;
    const bool row = ld->order == HIPBLASLT_ORDER_ROW;
    if (la->order != ld->order || lb->order != ld->order || lc->order != ld->order) return HIPBLAS_STATUS_NOT_SUPPORTED;
    if (!row && ld->order != HIPBLASLT_ORDER_COL) return HIPBLAS_STATUS_NOT_SUPPORTED;
    const bool a_n = d->transA == HIPBLAS_OP_N, b_n = d->transB == HIPBLAS_OP_N;
    const uint64_t m = ld->rows, n = ld->cols, k = a_n ? la->cols : la->rows;
    if ((a_n ? la->rows : la->cols) != m || (b_n ? lb->rows : lb->cols) != k || (b_n ? lb->cols : lb->rows) != n ||
        lc->rows != m || lc->cols != n)
        return HIPBLAS_STATUS_INVALID_VALUE;
    if (m > 0x7fffffffu || n > 0x7fffffffu || k > 0x7fffffffu) return HIPBLAS_STATUS_INVALID_VALUE;
    // Leading dimensions: column-major ld >= rows, row-major ld >= cols.
    auto ld_ok = [row](const Layout *l) { return l->ld >= (int64_t)(row ? l->cols : l->rows) && l->ld > 0; };
    if (!ld_ok(la) || !ld_ok(lb) || !ld_ok(lc) || !ld_ok(ld)) return HIPBLAS_STATUS_INVALID_VALUE;
    uint32_t act;
    bool has_bias;
    if (!map_epilogue(d->epilogue, &act, &has_bias)) return HIPBLAS_STATUS_NOT_SUPPORTED;
    if (m == 0 || n == 0) return HIPBLAS_STATUS_SUCCESS;
    if (!A || !B || !D) return HIPBLAS_STATUS_INVALID_VALUE;

    VkfGemmArgs g{};
    g.act = act;
    // Kernel core D[r,c] = sum_k X[r,k] Y[c,k].
    if (row) {  // r = i (row of D), c = j
        g.X = A; g.ldx = (uint64_t)la->ld; g.R = (uint32_t)m;
        g.Y = B; g.ldy = (uint64_t)lb->ld; g.Cn = (uint32_t)n;
        g.flags = (a_n ? 0u : VKF_GF_X_TRANS) | (b_n ? VKF_GF_Y_TRANS : 0u) | VKF_GF_BIAS_ROW;
        g.rs = (const float *)d->a_scale;
        g.cs = (const float *)d->b_scale;
        if (d->a_scale && d->a_scale_mode == HIPBLASLT_MATMUL_MATRIX_SCALE_SCALAR_32F) g.flags |= VKF_GF_RS_SCALAR;
        if (d->b_scale && d->b_scale_mode == HIPBLASLT_MATMUL_MATRIX_SCALE_SCALAR_32F) g.flags |= VKF_GF_CS_SCALAR;
    } else {    // column-major: r = j (column of D), c = i
        g.X = B; g.ldx = (uint64_t)lb->ld; g.R = (uint32_t)n;
        g.Y = A; g.ldy = (uint64_t)la->ld; g.Cn = (uint32_t)m;
        g.flags = (b_n ? 0u : VKF_GF_X_TRANS) | (a_n ? VKF_GF_Y_TRANS : 0u);
        g.rs = (const float *)d->b_scale;
        g.cs = (const float *)d->a_scale;
        if (d->b_scale && d->b_scale_mode == HIPBLASLT_MATMUL_MATRIX_SCALE_SCALAR_32F) g.flags |= VKF_GF_RS_SCALAR;
        if (d->a_scale && d->a_scale_mode == HIPBLASLT_MATMUL_MATRIX_SCALE_SCALAR_32F) g.flags |= VKF_GF_CS_SCALAR;
    }
    for (int32_t mode : {d->a_scale_mode, d->b_scale_mode})
        if (mode != HIPBLASLT_MATMUL_MATRIX_SCALE_SCALAR_32F && mode != HIPBLASLT_MATMUL_MATRIX_SCALE_OUTER_VEC_32F)
            return HIPBLAS_STATUS_NOT_SUPPORTED;
    g.K = (uint32_t)k;
    g.ldd = (uint64_t)ld->ld;
    g.ldc = (uint64_t)lc->ld;
    g.D = D;
    g.Cin = C;

    VkfKernelId kid;
    const hipDataType at = la->type, bt = lb->type, dt = ld->type;
    if (lc->type != dt) return HIPBLAS_STATUS_NOT_SUPPORTED;
    if (at == HIP_R_16F && bt == HIP_R_16F && (dt == HIP_R_16F || dt == HIP_R_32F)) {
        if (d->compute != HIPBLAS_COMPUTE_32F && d->compute != HIPBLAS_COMPUTE_32F_PEDANTIC)
            return HIPBLAS_STATUS_NOT_SUPPORTED;
        kid = VKF_K_GEMM_F16;
        g.alpha = *(const float *)alpha;
        g.beta = *(const float *)beta;
        if (dt == HIP_R_32F) g.flags |= VKF_GF_D_F32 | VKF_GF_CIN_F32;
    } else if (at == HIP_R_8I && bt == HIP_R_8I && dt == HIP_R_32I) {
        if (d->compute != HIPBLAS_COMPUTE_32I && d->compute != HIPBLAS_COMPUTE_32I_PEDANTIC)
            return HIPBLAS_STATUS_NOT_SUPPORTED;
        if (act != VKF_ACT_NONE || has_bias || d->a_scale || d->b_scale) return HIPBLAS_STATUS_NOT_SUPPORTED;
        kid = VKF_K_GEMM_I8;
        g.flags |= VKF_GF_D_I32;
        if (d->scale_type == HIP_R_32I) {
            g.alpha = (float)*(const int32_t *)alpha;
            g.beta = (float)*(const int32_t *)beta;
        } else {
            g.alpha = *(const float *)alpha;
            g.beta = *(const float *)beta;
        }
    } else if (at == HIP_R_8I && bt == HIP_R_8I && (dt == HIP_R_16F || dt == HIP_R_32F)) {
        if (d->compute != HIPBLAS_COMPUTE_32I && d->compute != HIPBLAS_COMPUTE_32I_PEDANTIC &&
            d->compute != HIPBLAS_COMPUTE_32F && d->compute != HIPBLAS_COMPUTE_32F_PEDANTIC)
            return HIPBLAS_STATUS_NOT_SUPPORTED;
        kid = VKF_K_GEMM_I8;
        g.alpha = *(const float *)alpha;
        g.beta = *(const float *)beta;
        if (dt == HIP_R_32F) g.flags |= VKF_GF_D_F32 | VKF_GF_CIN_F32;
    } else {
        return HIPBLAS_STATUS_NOT_SUPPORTED;
    }
    if (g.beta != 0.0f && !C) return HIPBLAS_STATUS_INVALID_VALUE;
    if (has_bias) {
        if (!d->bias) return HIPBLAS_STATUS_INVALID_VALUE;
        int32_t bty = d->bias_type >= 0 ? d->bias_type : (int32_t)dt;
        if (bty == HIP_R_32F) g.flags |= VKF_GF_BIAS_F32;
        else if (bty != HIP_R_16F) return HIPBLAS_STATUS_NOT_SUPPORTED;
        g.bias = d->bias;
    }

    const int32_t batch = ld->batch > 0 ? ld->batch : 1;
    const size_t ea = dtype_bytes(at), eb = dtype_bytes(bt), ec = dtype_bytes(dt);
    if (vkf::debug_enabled())
        vkf::debug_log("hipblasLtMatmul m=%llu n=%llu k=%llu order=%s batch=%d epi=%u", (unsigned long long)m,
                       (unsigned long long)n, (unsigned long long)k, row ? "row" : "col", batch, d->epilogue);
    for (int32_t b = 0; b < batch; b++) {
        VkfGemmArgs gb = g;
        const bool xa = row;  // X is A for row-major, B for column-major
        gb.X = (const char *)g.X + (int64_t)b * (xa ? la->stride * ea : lb->stride * eb);
        gb.Y = (const char *)g.Y + (int64_t)b * (xa ? lb->stride * eb : la->stride * ea);
        gb.Cin = C ? (const char *)C + (int64_t)b * lc->stride * ec : nullptr;
        gb.D = (char *)D + (int64_t)b * ld->stride * ec;
        hipblasStatus_t s = to_status(vkf::launch_gemm(kid, gb, stream));
        if (s != HIPBLAS_STATUS_SUCCESS) return s;
    }
    return HIPBLAS_STATUS_SUCCESS;
}

}  // extern "C"
