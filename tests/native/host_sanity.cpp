// host_sanity.cpp — TEST HELPER for tests/test_host_sanitizers.py, not part of
// the library.  Linked, with AddressSanitizer and UndefinedBehaviorSanitizer,
// against the library's host sources (kernel-name table, C-ABI argument
// checks, hipBLAS / hipBLASLt descriptor handling) and the CPU oracle, and run
// on a machine without a GPU: every call below returns before any launch, so
// the run exercises exactly the host-side logic.  Exits non-zero (or the
// sanitizers abort) on any failure.
#include <hipblas/hipblas.h>
#include <hipblaslt/hipblaslt.h>

#include <cstdint>
#include <cstdio>
#include <cstring>
#include <random>
#include <vector>

#include "../../include/vkflame_amd.h"
#include "../../oracle/vkf_oracle.h"

static int g_fail = 0;
#define CHECK(c)                                                         \
    do {                                                                 \
        if (!(c)) {                                                      \
            std::fprintf(stderr, "%s:%d: check failed: %s\n", __FILE__, __LINE__, #c); \
            g_fail = 1;                                                  \
        }                                                                \
    } while (0)

static void table() {
    void *p0 = (void *)0x1000, *p1 = (void *)0x2000, *p2 = (void *)0x3000;
    int32_t i3 = 4096, i4 = 11008, i5 = 4096, i6 = 7;
    int64_t k64 = 32 * 1000;
    void *args7[7] = {&p0, &p1, &p2, &i3, &i4, &i5, &i6};
    void *args3_64[3] = {&p0, &p1, &k64};
    VkflameLaunchPlan plan;
    CHECK(vkflame_resolve_launch("mul_mat_q4_K_q8_1", 1, 1, 1, 64, 1, 1, args7, &plan) == VKF_LAUNCH_MUL_MAT_Q);
    CHECK(plan.K == 4096 && plan.N == 11008 && plan.M == 7 && plan.quant_type == VKF_DEQUANT_Q4_K);
    CHECK(vkflame_resolve_launch("dequantize_mul_mat_vec_q4_0", 1, 1, 1, 64, 1, 1, args7, &plan) == VKF_LAUNCH_NONE);
    CHECK(vkflame_resolve_launch("dequantize_block_q8_0", 1, 1, 1, 256, 1, 1, args3_64, &plan) == VKF_LAUNCH_DEQUANT);
    CHECK(plan.n_blocks == 1000);
    CHECK(vkflame_resolve_launch("_Z21dequantize_block_q6_KI6__halfEvPKvPT_", 77, 1, 1, 64, 1, 1, args3_64, &plan) ==
          VKF_LAUNCH_DEQUANT);
    CHECK(plan.n_blocks == 77 && plan.out_dtype == VKF_DTYPE_FP16);
    const char *none[] = {"", "softmax_f32", "mul_mat_iq4_nl_q8_1", "get_rows_q4_0", "mul_mat_bf16"};
    for (const char *n : none) CHECK(vkflame_resolve_launch(n, 1, 1, 1, 64, 1, 1, args7, &plan) == VKF_LAUNCH_NONE);
    CHECK(vkflame_resolve_launch(nullptr, 1, 1, 1, 64, 1, 1, args7, &plan) == VKF_LAUNCH_NONE);
    CHECK(vkflame_resolve_launch("mul_mat_q4_0_q8_1", 1, 1, 1, 64, 1, 1, nullptr, &plan) == VKF_LAUNCH_NONE);
}

static void c_abi() {
    void *p = (void *)16;
    CHECK(vkflame_dispatch_dequant(p, p, 4, 9, VKF_DTYPE_FP32, nullptr) == 1);
    CHECK(vkflame_dispatch_dequant(p, p, 0, VKF_DEQUANT_Q4_K, VKF_DTYPE_FP32, nullptr) == 0);
    CHECK(vkflame_quantize_q8_1((const float *)p, p, 4, 33, 0, nullptr) == 1);
    CHECK(vkflame_dispatch_gemm_q(p, VKF_DEQUANT_Q8_1, 0, p, VKF_DTYPE_FP16, 0, (float *)p, 0, 1, 8, 256, nullptr) == 1);
    CHECK(vkflame_dispatch_gemm_q(p, VKF_DEQUANT_Q4_K, 0, p, VKF_DTYPE_FP16, 0, (float *)p, 0, 0, 8, 256, nullptr) == 0);
    CHECK(vkflame_dispatch_linear(p, p, nullptr, p, 4, 4, 4, VKF_DTYPE_FP16, 0, 0, 7, nullptr, nullptr, nullptr) == 1);
    float bad = -1.0f;
    CHECK(vkflame_dispatch_linear(p, p, nullptr, p, 4, 4, 4, VKF_DTYPE_INT8, 0, 1, 0, &bad, nullptr, nullptr) == 1);
    CHECK(vkflame_gemm_q_workspace_bytes(VKF_DEQUANT_Q6_K, VKF_DTYPE_Q8_1, 512, 4096, 5120) == (size_t)512 * 5120 * 2);
    CHECK(vkflame_gemm_q_workspace_bytes(VKF_DEQUANT_Q6_K, VKF_DTYPE_Q8_1, 16, 4096, 5120) == 0);
    CHECK(vkflame_gemm_q_workspace_bytes(VKF_DEQUANT_Q4_K, VKF_DTYPE_FP16, 8, 5120, 13824) == (size_t)3 * 8 * 5120 * 4);
    CHECK(vkflame_gemm_q_workspace_bytes(VKF_DEQUANT_Q4_K, VKF_DTYPE_FP16, 8, 5120, 5120) == 0);
    CHECK(vkflame_noalloc_scratch_bytes() == VKFLAME_NOALLOC_SCRATCH_BYTES);
    CHECK(vkflame_dispatch_gemm_q_noalloc(p, VKF_DEQUANT_Q6_K, 0, p, VKF_DTYPE_Q8_1, 0, (float *)p, 0, 2048, 64, 8192,
                                          nullptr) == 1);
}

static void blas() {
    hipblasHandle_t h = nullptr;
    CHECK(hipblasCreate(&h) == HIPBLAS_STATUS_SUCCESS);
    CHECK(hipblasSetStream(h, (hipStream_t)0x1234) == HIPBLAS_STATUS_SUCCESS);
    hipStream_t s = nullptr;
    CHECK(hipblasGetStream(h, &s) == HIPBLAS_STATUS_SUCCESS && s == (hipStream_t)0x1234);
    float one = 1.0f;
    CHECK(hipblasGemmEx(h, HIPBLAS_OP_T, HIPBLAS_OP_N, 8, 8, 8, &one, (void *)16, HIP_R_16BF, 8, (void *)16,
                        HIP_R_16BF, 8, &one, (void *)16, HIP_R_16BF, 8, HIPBLAS_COMPUTE_32F,
                        HIPBLAS_GEMM_DEFAULT) == HIPBLAS_STATUS_NOT_SUPPORTED);
    CHECK(hipblasSgemm(h, HIPBLAS_OP_N, HIPBLAS_OP_N, 8, 8, 8, &one, (const float *)16, 4, (const float *)16, 8,
                       &one, (float *)16, 8) == HIPBLAS_STATUS_INVALID_VALUE);
    CHECK(hipblasDestroy(h) == HIPBLAS_STATUS_SUCCESS);

    hipblasLtHandle_t lt = nullptr;
    CHECK(hipblasLtCreate(&lt) == HIPBLAS_STATUS_SUCCESS);
    hipblasLtMatrixLayout_t a, b, d;
    CHECK(hipblasLtMatrixLayoutCreate(&a, HIP_R_8I, 64, 32, 64) == HIPBLAS_STATUS_SUCCESS);
    CHECK(hipblasLtMatrixLayoutCreate(&b, HIP_R_8I, 64, 16, 64) == HIPBLAS_STATUS_SUCCESS);
    CHECK(hipblasLtMatrixLayoutCreate(&d, HIP_R_32I, 32, 16, 32) == HIPBLAS_STATUS_SUCCESS);
    int64_t ld = 0;
    size_t w = 0;
    CHECK(hipblasLtMatrixLayoutGetAttribute(a, HIPBLASLT_MATRIX_LAYOUT_LD, &ld, 8, &w) == HIPBLAS_STATUS_SUCCESS);
    CHECK(ld == 64 && w == 8);
    CHECK(hipblasLtMatrixLayoutSetAttribute(a, HIPBLASLT_MATRIX_LAYOUT_LD, &ld, 3) == HIPBLAS_STATUS_INVALID_VALUE);
    hipblasLtMatmulDesc_t desc;
    CHECK(hipblasLtMatmulDescCreate(&desc, HIPBLAS_COMPUTE_32I, HIP_R_32F) == HIPBLAS_STATUS_SUCCESS);
    int32_t t = HIPBLAS_OP_T;
    CHECK(hipblasLtMatmulDescSetAttribute(desc, HIPBLASLT_MATMUL_DESC_TRANSA, &t, 4) == HIPBLAS_STATUS_SUCCESS);
    float half = 0.5f, zero = 0.0f;
    CHECK(hipblasLtMatmul(lt, desc, &half, (void *)16, a, (void *)16, b, &zero, (void *)16, d, (void *)16, d, nullptr,
                          nullptr, 0, nullptr) == HIPBLAS_STATUS_NOT_SUPPORTED);
    hipblasLtMatmulPreference_t pref;
    CHECK(hipblasLtMatmulPreferenceCreate(&pref) == HIPBLAS_STATUS_SUCCESS);
    hipblasLtMatmulHeuristicResult_t res[2];
    int cnt = 0;
    CHECK(hipblasLtMatmulAlgoGetHeuristic(lt, desc, a, b, d, d, pref, 2, res, &cnt) == HIPBLAS_STATUS_SUCCESS);
    CHECK(cnt == 1);
    CHECK(hipblasLtMatmulPreferenceDestroy(pref) == HIPBLAS_STATUS_SUCCESS);
    for (auto l : {a, b, d}) CHECK(hipblasLtMatrixLayoutDestroy(l) == HIPBLAS_STATUS_SUCCESS);
    CHECK(hipblasLtMatmulDescDestroy(desc) == HIPBLAS_STATUS_SUCCESS);
    CHECK(hipblasLtDestroy(lt) == HIPBLAS_STATUS_SUCCESS);
}

static void oracle() {
    std::mt19937 rng(5);
    for (int qt = 0; qt < 8; qt++) {
        const int bb = vkfo_block_bytes(qt), be = vkfo_block_elems(qt), nb = 37;
        std::vector<uint8_t> src((size_t)bb * nb);
        for (auto &x : src) x = (uint8_t)rng();
        // fp16 fields with small finite values (exponent below 15)
        for (int i = 0; i < nb; i++) {
            uint8_t *blk = src.data() + (size_t)i * bb;
            const int off = qt == VKFO_Q6_K ? 208 : 0;
            blk[off + 1] &= 0x3b;
            if (qt == VKFO_Q4_1 || qt == VKFO_Q4_K || qt == VKFO_Q5_K || qt == VKFO_Q8_1) blk[3] &= 0x3b;
        }
        std::vector<float> f((size_t)be * nb);
        std::vector<uint16_t> h((size_t)be * nb);
        CHECK(vkfo_dequant_f32(qt, src.data(), nb, f.data()) == 0);
        CHECK(vkfo_dequant_f16(qt, src.data(), nb, h.data()) == 0);
        for (size_t i = 0; i < f.size(); i++) CHECK(vkfo_f2h(f[i]) == h[i]);
    }
    std::vector<float> x(64 * 3);
    for (auto &v : x) v = (float)((int)(rng() % 2001) - 1000) / 100.0f;
    std::vector<uint8_t> q(36 * 2 * 3);
    vkfo_quantize_q8_1(x.data(), x.size(), q.data());
    std::vector<int8_t> A(5 * 70), B(6 * 70);
    for (auto &v : A) v = (int8_t)(rng() % 255 - 127);
    for (auto &v : B) v = (int8_t)(rng() % 255 - 127);
    std::vector<int32_t> C(5 * 6);
    CHECK(vkfo_gemm_i8_nt(A.data(), B.data(), C.data(), 5, 6, 70) == 0);
    std::vector<int8_t> qr(3 * 64);
    std::vector<float> sc(3);
    vkfo_quantize_rows_i8(x.data(), 3, 64, qr.data(), sc.data());
    for (int a = 0; a < 4; a++) CHECK(vkfo_act(a, 0.0f) == 0.0f);
}

int main() {
    table();
    c_abi();
    blas();
    oracle();
    std::printf("host_sanity %s\n", g_fail ? "FAILED" : "ok");
    return g_fail;
}
