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
//
// Objects: with ROCm's hipBLASLt present and a GPU visible, the handle,
// layouts, descriptors and preferences are ROCm's own objects (created by
// ROCm's functions) and this library keeps a mirror of their attributes, so
// every hipBLASLt function it does not export works on them unchanged and a
// matmul its kernels do not take (an attribute or epilogue it does not model,
// device-pointer scalars, other types) is forwarded to ROCm's hipblasLtMatmul.
// Without ROCm's hipBLASLt the objects are the library's own and such calls
// return HIPBLAS_STATUS_NOT_SUPPORTED.
#include <hipblaslt/hipblaslt.h>

#include <cstdint>
#include <cstring>
#include <mutex>
#include <new>
#include <unordered_map>

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

// True when f is an integer in int32's range (so (int32_t)f loses nothing).
bool int32_exact(float f) { return f >= -2147483648.0f && f < 2147483648.0f && (float)(int64_t)f == f; }

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


// Mirrored state of a layout / descriptor (the library's own object, or a
// ROCm object whose attributes are mirrored as they are set).  `exotic`: an
// attribute was set that the mirror does not model, so the library's kernels
// leave the matmul to ROCm.
struct LayoutRec {
    Layout l;
    bool vendor, exotic;
};
struct DescRec {
    Desc d;
    bool vendor, exotic;
};

std::mutex g_mu;
std::unordered_map<void *, LayoutRec> g_layouts;
std::unordered_map<void *, DescRec> g_descs;
std::unordered_map<void *, Pref> g_prefs;     // the library's own preferences
std::unordered_map<void *, bool> g_handles;   // handle -> created by ROCm

template <class F>
F vendor(const char *name) {
    return reinterpret_cast<F>(vkf::vendor_symbol("libhipblaslt.so", name));
}
#define VENDOR(fn) vendor<decltype(&fn)>(#fn)

// A fresh key for an object of the library's own.
void *own_key() { return new (std::nothrow) char[1]; }

// Attribute writes on a mirror (the library's own object or a ROCm one's).
hipblasStatus_t set_layout_attr(Layout *l, hipblasLtMatrixLayoutAttribute_t attr, const void *buf, size_t size) {
    switch (attr) {
    case HIPBLASLT_MATRIX_LAYOUT_BATCH_COUNT: return get(buf, size, &l->batch);
    case HIPBLASLT_MATRIX_LAYOUT_STRIDED_BATCH_OFFSET: return get(buf, size, &l->stride);
    case HIPBLASLT_MATRIX_LAYOUT_TYPE: {
        uint32_t t;
        hipblasStatus_t s = get(buf, size, &t);
        if (s == HIPBLAS_STATUS_SUCCESS) l->type = (hipDataType)t;
        return s;
    }
    case HIPBLASLT_MATRIX_LAYOUT_ORDER: return get(buf, size, &l->order);
    case HIPBLASLT_MATRIX_LAYOUT_ROWS: return get(buf, size, &l->rows);
    case HIPBLASLT_MATRIX_LAYOUT_COLS: return get(buf, size, &l->cols);
    case HIPBLASLT_MATRIX_LAYOUT_LD: return get(buf, size, &l->ld);
    default: return HIPBLAS_STATUS_INVALID_VALUE;
    }
}

hipblasStatus_t get_layout_attr(const Layout *l, hipblasLtMatrixLayoutAttribute_t attr, void *buf, size_t size,
                                size_t *written) {
    switch (attr) {
    case HIPBLASLT_MATRIX_LAYOUT_BATCH_COUNT: return put(buf, size, written, l->batch);
    case HIPBLASLT_MATRIX_LAYOUT_STRIDED_BATCH_OFFSET: return put(buf, size, written, l->stride);
    case HIPBLASLT_MATRIX_LAYOUT_TYPE: return put(buf, size, written, (uint32_t)l->type);
    case HIPBLASLT_MATRIX_LAYOUT_ORDER: return put(buf, size, written, l->order);
    case HIPBLASLT_MATRIX_LAYOUT_ROWS: return put(buf, size, written, l->rows);
    case HIPBLASLT_MATRIX_LAYOUT_COLS: return put(buf, size, written, l->cols);
    case HIPBLASLT_MATRIX_LAYOUT_LD: return put(buf, size, written, l->ld);
    default: return HIPBLAS_STATUS_INVALID_VALUE;
    }
}

hipblasStatus_t set_desc_attr(Desc *d, hipblasLtMatmulDescAttributes_t attr, const void *buf, size_t size) {
    switch (attr) {
    case HIPBLASLT_MATMUL_DESC_TRANSA: return get(buf, size, &d->transA);
    case HIPBLASLT_MATMUL_DESC_TRANSB: return get(buf, size, &d->transB);
    case HIPBLASLT_MATMUL_DESC_EPILOGUE: return get(buf, size, &d->epilogue);
    case HIPBLASLT_MATMUL_DESC_BIAS_POINTER: return get(buf, size, &d->bias);
    case HIPBLASLT_MATMUL_DESC_BIAS_DATA_TYPE: return get(buf, size, &d->bias_type);
    case HIPBLASLT_MATMUL_DESC_A_SCALE_POINTER: return get(buf, size, &d->a_scale);
    case HIPBLASLT_MATMUL_DESC_B_SCALE_POINTER: return get(buf, size, &d->b_scale);
    case HIPBLASLT_MATMUL_DESC_A_SCALE_MODE: return get(buf, size, &d->a_scale_mode);
    case HIPBLASLT_MATMUL_DESC_B_SCALE_MODE: return get(buf, size, &d->b_scale_mode);
    case HIPBLASLT_MATMUL_DESC_POINTER_MODE: return get(buf, size, &d->pointer_mode);
    default: return HIPBLAS_STATUS_NOT_SUPPORTED;
    }
}

hipblasStatus_t get_desc_attr(const Desc *d, hipblasLtMatmulDescAttributes_t attr, void *buf, size_t size,
                              size_t *written) {
    switch (attr) {
    case HIPBLASLT_MATMUL_DESC_TRANSA: return put(buf, size, written, d->transA);
    case HIPBLASLT_MATMUL_DESC_TRANSB: return put(buf, size, written, d->transB);
    case HIPBLASLT_MATMUL_DESC_EPILOGUE: return put(buf, size, written, d->epilogue);
    case HIPBLASLT_MATMUL_DESC_BIAS_POINTER: return put(buf, size, written, d->bias);
    case HIPBLASLT_MATMUL_DESC_BIAS_DATA_TYPE: return put(buf, size, written, d->bias_type);
    case HIPBLASLT_MATMUL_DESC_A_SCALE_POINTER: return put(buf, size, written, d->a_scale);
    case HIPBLASLT_MATMUL_DESC_B_SCALE_POINTER: return put(buf, size, written, d->b_scale);
    case HIPBLASLT_MATMUL_DESC_A_SCALE_MODE: return put(buf, size, written, d->a_scale_mode);
    case HIPBLASLT_MATMUL_DESC_B_SCALE_MODE: return put(buf, size, written, d->b_scale_mode);
    case HIPBLASLT_MATMUL_DESC_POINTER_MODE: return put(buf, size, written, d->pointer_mode);
    default: return HIPBLAS_STATUS_NOT_SUPPORTED;
    }
}

Desc default_desc(hipblasComputeType_t computeType, hipDataType scaleType) {
    return Desc{computeType,
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
}

// The algorithm this library reports when ROCm has none to offer.
constexpr char kAlgoTag[8] = {'v', 'k', 'f', '-', 'm', 'f', 'm', 'a'};
bool our_algo(const hipblasLtMatmulAlgo_t *a) { return a && std::memcmp(a->data, kAlgoTag, 8) == 0; }

// The matmul on this library's kernels; HIPBLAS_STATUS_NOT_SUPPORTED (before
// any launch) for what they do not take.
hipblasStatus_t matmul_ours(const Desc *d, const void *alpha, const void *A, const Layout *la, const void *B,
                            const Layout *lb, const void *beta, const void *C, const Layout *lc, void *D,
                            const Layout *ld, hipStream_t stream) {
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
    bool beta_nonzero = false;
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
        // the int32 epilogue scales by integers: a float alpha / beta must be
        // an exact int32 value (0.5 would otherwise truncate to 0)
        int32_t ia, ib;
        if (d->scale_type == HIP_R_32I) {
            ia = *(const int32_t *)alpha;
            ib = *(const int32_t *)beta;
        } else {
            const float fa = *(const float *)alpha, fb = *(const float *)beta;
            if (!int32_exact(fa) || !int32_exact(fb)) return HIPBLAS_STATUS_NOT_SUPPORTED;
            ia = (int32_t)fa;
            ib = (int32_t)fb;
        }
        vkf_gemm_set_int_scalars(g, ia, ib);
        beta_nonzero = ib != 0;
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
    if (!(g.flags & VKF_GF_D_I32)) beta_nonzero = g.beta != 0.0f;
    if (beta_nonzero && !C) return HIPBLAS_STATUS_INVALID_VALUE;
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
    if (batch > 1 && (la->stride < 0 || lb->stride < 0 || lc->stride < 0 || ld->stride < 0))
        return HIPBLAS_STATUS_INVALID_VALUE;
    // all matrices of a batched layout in one launch (grid z), 65535 at most
    const bool xa = row;  // X is A for row-major, B for column-major
    g.bsx = (uint64_t)(xa ? la->stride * ea : lb->stride * eb);
    g.bsy = (uint64_t)(xa ? lb->stride * eb : la->stride * ea);
    g.bsd = (uint64_t)(ld->stride * ec);
    g.bsc = C ? (uint64_t)(lc->stride * ec) : 0;
    for (int32_t b0 = 0; b0 < batch; b0 += 65535) {
        VkfGemmArgs gb = g;
        gb.X = (const char *)g.X + b0 * g.bsx;
        gb.Y = (const char *)g.Y + b0 * g.bsy;
        gb.Cin = C ? (const char *)C + b0 * g.bsc : nullptr;
        gb.D = (char *)D + b0 * g.bsd;
        const int32_t nb = batch - b0 < 65535 ? batch - b0 : 65535;
        hipblasStatus_t s = to_status(vkf::launch_gemm(kid, gb, stream, (uint32_t)nb));
        if (s != HIPBLAS_STATUS_SUCCESS) return s;
    }
    return HIPBLAS_STATUS_SUCCESS;
}

}  // namespace

extern "C" {

hipblasStatus_t hipblasLtCreate(hipblasLtHandle_t *handle) {
    if (!handle) return HIPBLAS_STATUS_INVALID_VALUE;
    if (auto f = VENDOR(hipblasLtCreate)) {
        if (f(handle) == HIPBLAS_STATUS_SUCCESS) {
            std::lock_guard<std::mutex> lk(g_mu);
            g_handles[*handle] = true;
            return HIPBLAS_STATUS_SUCCESS;
        }
    }
    void *h = own_key();
    if (!h) return HIPBLAS_STATUS_ALLOC_FAILED;
    std::lock_guard<std::mutex> lk(g_mu);
    g_handles[h] = false;
    *handle = h;
    return HIPBLAS_STATUS_SUCCESS;
}

hipblasStatus_t hipblasLtDestroy(const hipblasLtHandle_t handle) {
    if (!handle) return HIPBLAS_STATUS_NOT_INITIALIZED;
    bool own = false;
    {
        std::lock_guard<std::mutex> lk(g_mu);
        auto it = g_handles.find(handle);
        if (it != g_handles.end()) {
            own = !it->second;
            g_handles.erase(it);
        }
    }
    if (own) {
        delete[] static_cast<char *>(handle);
        return HIPBLAS_STATUS_SUCCESS;
    }
    auto f = VENDOR(hipblasLtDestroy);
    return f ? f(handle) : HIPBLAS_STATUS_NOT_INITIALIZED;
}

// shim/hipblaslt_shim.cpp:120-134 (the reference ignores ld and assumes row-major)
hipblasStatus_t hipblasLtMatrixLayoutCreate(hipblasLtMatrixLayout_t *matLayout, hipDataType type, uint64_t rows,
                                            uint64_t cols, int64_t ld) {
    if (!matLayout) return HIPBLAS_STATUS_INVALID_VALUE;
    const Layout l{type, rows, cols, ld, HIPBLASLT_ORDER_COL, 1, 0};
    if (auto f = VENDOR(hipblasLtMatrixLayoutCreate)) {
        if (f(matLayout, type, rows, cols, ld) == HIPBLAS_STATUS_SUCCESS) {
            std::lock_guard<std::mutex> lk(g_mu);
            g_layouts[*matLayout] = LayoutRec{l, true, false};
            return HIPBLAS_STATUS_SUCCESS;
        }
    }
    void *k = own_key();
    if (!k) return HIPBLAS_STATUS_ALLOC_FAILED;
    std::lock_guard<std::mutex> lk(g_mu);
    g_layouts[k] = LayoutRec{l, false, false};
    *matLayout = reinterpret_cast<hipblasLtMatrixLayout_t>(k);
    return HIPBLAS_STATUS_SUCCESS;
}

hipblasStatus_t hipblasLtMatrixLayoutDestroy(const hipblasLtMatrixLayout_t matLayout) {
    if (!matLayout) return HIPBLAS_STATUS_INVALID_VALUE;
    bool own = false;
    {
        std::lock_guard<std::mutex> lk(g_mu);
        auto it = g_layouts.find(matLayout);
        if (it != g_layouts.end()) {
            own = !it->second.vendor;
            g_layouts.erase(it);
        }
    }
    if (own) {
        delete[] reinterpret_cast<char *>(matLayout);
        return HIPBLAS_STATUS_SUCCESS;
    }
    auto f = VENDOR(hipblasLtMatrixLayoutDestroy);
    return f ? f(matLayout) : HIPBLAS_STATUS_INVALID_VALUE;
}

// shim/hipblaslt_shim.cpp:142-173
hipblasStatus_t hipblasLtMatrixLayoutSetAttribute(hipblasLtMatrixLayout_t matLayout,
                                                  hipblasLtMatrixLayoutAttribute_t attr, const void *buf,
                                                  size_t sizeInBytes) {
    if (!matLayout) return HIPBLAS_STATUS_INVALID_VALUE;
    std::unique_lock<std::mutex> lk(g_mu);
    auto it = g_layouts.find(matLayout);
    if (it != g_layouts.end() && !it->second.vendor) return set_layout_attr(&it->second.l, attr, buf, sizeInBytes);
    lk.unlock();
    auto f = VENDOR(hipblasLtMatrixLayoutSetAttribute);
    if (!f) return HIPBLAS_STATUS_INVALID_VALUE;
    const hipblasStatus_t s = f(matLayout, attr, buf, sizeInBytes);
    if (s != HIPBLAS_STATUS_SUCCESS) return s;
    lk.lock();
    it = g_layouts.find(matLayout);
    if (it != g_layouts.end() && set_layout_attr(&it->second.l, attr, buf, sizeInBytes) != HIPBLAS_STATUS_SUCCESS)
        it->second.exotic = true;
    return s;
}

// shim/hipblaslt_shim.cpp:175-209
hipblasStatus_t hipblasLtMatrixLayoutGetAttribute(hipblasLtMatrixLayout_t matLayout,
                                                  hipblasLtMatrixLayoutAttribute_t attr, void *buf,
                                                  size_t sizeInBytes, size_t *sizeWritten) {
    if (!matLayout) return HIPBLAS_STATUS_INVALID_VALUE;
    {
        std::lock_guard<std::mutex> lk(g_mu);
        auto it = g_layouts.find(matLayout);
        if (it != g_layouts.end() && !it->second.vendor)
            return get_layout_attr(&it->second.l, attr, buf, sizeInBytes, sizeWritten);
    }
    auto f = VENDOR(hipblasLtMatrixLayoutGetAttribute);
    return f ? f(matLayout, attr, buf, sizeInBytes, sizeWritten) : HIPBLAS_STATUS_INVALID_VALUE;
}

// shim/hipblaslt_shim.cpp:213-229
hipblasStatus_t hipblasLtMatmulDescCreate(hipblasLtMatmulDesc_t *matmulDesc, hipblasComputeType_t computeType,
                                          hipDataType scaleType) {
    if (!matmulDesc) return HIPBLAS_STATUS_INVALID_VALUE;
    const Desc d = default_desc(computeType, scaleType);
    if (auto f = VENDOR(hipblasLtMatmulDescCreate)) {
        if (f(matmulDesc, computeType, scaleType) == HIPBLAS_STATUS_SUCCESS) {
            std::lock_guard<std::mutex> lk(g_mu);
            g_descs[*matmulDesc] = DescRec{d, true, false};
            return HIPBLAS_STATUS_SUCCESS;
        }
    }
    void *k = own_key();
    if (!k) return HIPBLAS_STATUS_ALLOC_FAILED;
    std::lock_guard<std::mutex> lk(g_mu);
    g_descs[k] = DescRec{d, false, false};
    *matmulDesc = reinterpret_cast<hipblasLtMatmulDesc_t>(k);
    return HIPBLAS_STATUS_SUCCESS;
}

hipblasStatus_t hipblasLtMatmulDescDestroy(const hipblasLtMatmulDesc_t matmulDesc) {
    if (!matmulDesc) return HIPBLAS_STATUS_INVALID_VALUE;
    bool own = false;
    {
        std::lock_guard<std::mutex> lk(g_mu);
        auto it = g_descs.find(matmulDesc);
        if (it != g_descs.end()) {
            own = !it->second.vendor;
            g_descs.erase(it);
        }
    }
    if (own) {
        delete[] reinterpret_cast<char *>(matmulDesc);
        return HIPBLAS_STATUS_SUCCESS;
    }
    auto f = VENDOR(hipblasLtMatmulDescDestroy);
    return f ? f(matmulDesc) : HIPBLAS_STATUS_INVALID_VALUE;
}

// shim/hipblaslt_shim.cpp:237-267
hipblasStatus_t hipblasLtMatmulDescSetAttribute(hipblasLtMatmulDesc_t matmulDesc, hipblasLtMatmulDescAttributes_t attr,
                                                const void *buf, size_t sizeInBytes) {
    if (!matmulDesc) return HIPBLAS_STATUS_INVALID_VALUE;
    std::unique_lock<std::mutex> lk(g_mu);
    auto it = g_descs.find(matmulDesc);
    if (it != g_descs.end() && !it->second.vendor) return set_desc_attr(&it->second.d, attr, buf, sizeInBytes);
    lk.unlock();
    auto f = VENDOR(hipblasLtMatmulDescSetAttribute);
    if (!f) return HIPBLAS_STATUS_INVALID_VALUE;
    const hipblasStatus_t s = f(matmulDesc, attr, buf, sizeInBytes);
    if (s != HIPBLAS_STATUS_SUCCESS) return s;
    lk.lock();
    it = g_descs.find(matmulDesc);
    if (it != g_descs.end() && set_desc_attr(&it->second.d, attr, buf, sizeInBytes) != HIPBLAS_STATUS_SUCCESS)
        it->second.exotic = true;
    return s;
}

// shim/hipblaslt_shim.cpp:269-292
hipblasStatus_t hipblasLtMatmulDescGetAttribute(hipblasLtMatmulDesc_t matmulDesc, hipblasLtMatmulDescAttributes_t attr,
                                                void *buf, size_t sizeInBytes, size_t *sizeWritten) {
    if (!matmulDesc) return HIPBLAS_STATUS_INVALID_VALUE;
    {
        std::lock_guard<std::mutex> lk(g_mu);
        auto it = g_descs.find(matmulDesc);
        if (it != g_descs.end() && !it->second.vendor)
            return get_desc_attr(&it->second.d, attr, buf, sizeInBytes, sizeWritten);
    }
    auto f = VENDOR(hipblasLtMatmulDescGetAttribute);
    return f ? f(matmulDesc, attr, buf, sizeInBytes, sizeWritten) : HIPBLAS_STATUS_INVALID_VALUE;
}

// shim/hipblaslt_shim.cpp:296-319
hipblasStatus_t hipblasLtMatmulPreferenceCreate(hipblasLtMatmulPreference_t *pref) {
    if (!pref) return HIPBLAS_STATUS_INVALID_VALUE;
    if (auto f = VENDOR(hipblasLtMatmulPreferenceCreate)) {
        if (f(pref) == HIPBLAS_STATUS_SUCCESS) return HIPBLAS_STATUS_SUCCESS;
    }
    void *k = own_key();
    if (!k) return HIPBLAS_STATUS_ALLOC_FAILED;
    std::lock_guard<std::mutex> lk(g_mu);
    g_prefs[k] = Pref{0, 0};
    *pref = reinterpret_cast<hipblasLtMatmulPreference_t>(k);
    return HIPBLAS_STATUS_SUCCESS;
}

hipblasStatus_t hipblasLtMatmulPreferenceDestroy(const hipblasLtMatmulPreference_t pref) {
    if (!pref) return HIPBLAS_STATUS_INVALID_VALUE;
    {
        std::lock_guard<std::mutex> lk(g_mu);
        if (g_prefs.erase(pref)) {
            delete[] reinterpret_cast<char *>(pref);
            return HIPBLAS_STATUS_SUCCESS;
        }
    }
    auto f = VENDOR(hipblasLtMatmulPreferenceDestroy);
    return f ? f(pref) : HIPBLAS_STATUS_INVALID_VALUE;
}

hipblasStatus_t hipblasLtMatmulPreferenceSetAttribute(hipblasLtMatmulPreference_t pref,
                                                      hipblasLtMatmulPreferenceAttributes_t attr, const void *buf,
                                                      size_t sizeInBytes) {
    if (!pref) return HIPBLAS_STATUS_INVALID_VALUE;
    {
        std::lock_guard<std::mutex> lk(g_mu);
        auto it = g_prefs.find(pref);
        if (it != g_prefs.end()) {
            switch (attr) {
            case HIPBLASLT_MATMUL_PREF_SEARCH_MODE: return get(buf, sizeInBytes, &it->second.search_mode);
            case HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES: return get(buf, sizeInBytes, &it->second.max_ws);
            default: return HIPBLAS_STATUS_INVALID_VALUE;
            }
        }
    }
    auto f = VENDOR(hipblasLtMatmulPreferenceSetAttribute);
    return f ? f(pref, attr, buf, sizeInBytes) : HIPBLAS_STATUS_INVALID_VALUE;
}

// shim/hipblaslt_shim.cpp:323-343: ROCm's candidates for a ROCm handle; one
// algorithm of this library's (no workspace) otherwise, or when ROCm has none.
hipblasStatus_t hipblasLtMatmulAlgoGetHeuristic(hipblasLtHandle_t handle, hipblasLtMatmulDesc_t matmulDesc,
                                                hipblasLtMatrixLayout_t Adesc, hipblasLtMatrixLayout_t Bdesc,
                                                hipblasLtMatrixLayout_t Cdesc, hipblasLtMatrixLayout_t Ddesc,
                                                hipblasLtMatmulPreference_t pref, int requestedAlgoCount,
                                                hipblasLtMatmulHeuristicResult_t heuristicResultsArray[],
                                                int *returnAlgoCount) {
    if (!handle) return HIPBLAS_STATUS_NOT_INITIALIZED;
    if (!matmulDesc || !Adesc || !Bdesc || !Cdesc || !Ddesc || !returnAlgoCount || requestedAlgoCount <= 0 ||
        !heuristicResultsArray)
        return HIPBLAS_STATUS_INVALID_VALUE;
    bool vendor_handle = true;
    {
        std::lock_guard<std::mutex> lk(g_mu);
        auto it = g_handles.find(handle);
        if (it != g_handles.end()) vendor_handle = it->second;
    }
    if (vendor_handle) {
        if (auto f = VENDOR(hipblasLtMatmulAlgoGetHeuristic)) {
            const hipblasStatus_t s = f(handle, matmulDesc, Adesc, Bdesc, Cdesc, Ddesc, pref, requestedAlgoCount,
                                        heuristicResultsArray, returnAlgoCount);
            if (s == HIPBLAS_STATUS_SUCCESS && *returnAlgoCount > 0) return s;
        }
    }
    hipblasLtMatmulHeuristicResult_t r{};
    std::memcpy(r.algo.data, kAlgoTag, 8);
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
    if (!handle) return HIPBLAS_STATUS_NOT_INITIALIZED;
    if (!matmulDesc || !Adesc || !Bdesc || !Cdesc || !Ddesc || !alpha || !beta) return HIPBLAS_STATUS_INVALID_VALUE;
    bool vendor_handle = true, mirrored = false;
    Desc d{};
    Layout la{}, lb{}, lc{}, ld{};
    {
        std::lock_guard<std::mutex> lk(g_mu);
        auto h = g_handles.find(handle);
        if (h != g_handles.end()) vendor_handle = h->second;
        auto di = g_descs.find(matmulDesc);
        auto ai = g_layouts.find(Adesc), bi = g_layouts.find(Bdesc), ci = g_layouts.find(Cdesc),
             oi = g_layouts.find(Ddesc);
        mirrored = di != g_descs.end() && ai != g_layouts.end() && bi != g_layouts.end() && ci != g_layouts.end() &&
                   oi != g_layouts.end() && !di->second.exotic && !ai->second.exotic && !bi->second.exotic &&
                   !ci->second.exotic && !oi->second.exotic;
        if (mirrored) {
            d = di->second.d;
            la = ai->second.l;
            lb = bi->second.l;
            lc = ci->second.l;
            ld = oi->second.l;
        }
    }
    hipblasStatus_t s = HIPBLAS_STATUS_NOT_SUPPORTED;
    if (mirrored) s = matmul_ours(&d, alpha, A, &la, B, &lb, beta, C, &lc, D, &ld, stream);
    if (s != HIPBLAS_STATUS_NOT_SUPPORTED || !vendor_handle || our_algo(algo)) return s;
    auto f = VENDOR(hipblasLtMatmul);
    if (!f) return s;
    if (vkf::debug_enabled()) vkf::debug_log("hipblasLtMatmul -> ROCm hipBLASLt");
    return f(handle, matmulDesc, alpha, A, Adesc, B, Bdesc, beta, C, Cdesc, D, Ddesc, algo, workspace,
             workspaceSizeInBytes, stream);
}

}  // extern "C"
