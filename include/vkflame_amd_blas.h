/*
 * vkflame_amd_blas.h — the hipBLAS / hipBLASLt entry points that
 * libvkflame_amd.so exports.
 *
 * The declarations are ROCm 7.2's own (this header includes hipblas.h and
 * hipblaslt.h), with ROCm's enum values, so a caller built against ROCm
 * links to this library unchanged when it comes first on the link line or in
 * LD_PRELOAD.  The list below names each exported function and the
 * reference (vkflame) shim function it replaces.
 *
 * Semantics beyond the reference (which swaps operands for op = N only and
 * ignores ld, alpha, beta and the hipBLASLt epilogue inputs,
 * shim/hipblas_shim.cpp:282-287, shim/hipblaslt_shim.cpp:418-423):
 *   - hipblasGemmEx: column-major C = alpha*op(A)*op(B) + beta*C for every
 *     op combination and ld; (16F,16F -> 16F or 32F, compute 32F),
 *     (32F,32F -> 32F, compute 32F) and (8I,8I -> 32I, compute 32I, exact).
 *   - hipblasSgemm*: fp32 on the fp32 matrix cores.
 *   - hipblasLtMatmul: D = act(alpha*(A.B)*a_scale[m]*b_scale[n] + beta*C +
 *     bias) with BIAS, A/B_SCALE_POINTER (OUTER_VEC_32F vectors or scalars),
 *     RELU / GELU / SILU epilogues, row- or column-major layouts.
 * With ROCm's hipBLAS / hipBLASLt present (and a GPU visible) the handles and
 * descriptors these functions create are ROCm's own objects: functions not
 * listed here reach ROCm with objects it created, and calls this library does
 * not run (other types, device-pointer scalars, epilogues it lacks) are
 * forwarded to ROCm's function of the same name.  Without ROCm's libraries
 * such calls return HIPBLAS_STATUS_NOT_SUPPORTED.
 */
#ifndef VKFLAME_AMD_BLAS_H
#define VKFLAME_AMD_BLAS_H

#include <hipblas/hipblas.h>
#include <hipblaslt/hipblaslt.h>

/* X(name, reference file:lines) */
#define VKFLAME_AMD_BLAS_EXPORTS(X)                                        \
    X(hipblasCreate, "shim/hipblas_shim.cpp:52-58")                        \
    X(hipblasDestroy, "shim/hipblas_shim.cpp:60-64")                       \
    X(hipblasSetStream, "shim/hipblas_shim.cpp:66-72")                     \
    X(hipblasGetStream, "shim/hipblas_shim.cpp:74-80")                     \
    X(hipblasSetPointerMode, "(no reference counterpart: device alpha/beta)") \
    X(hipblasGetPointerMode, "(no reference counterpart)")                 \
    X(hipblasGemmEx, "shim/hipblas_shim.cpp:251-291")                      \
    X(hipblasGemmBatchedEx, "shim/hipblas_shim.cpp:293-315")               \
    X(hipblasGemmStridedBatchedEx, "shim/hipblas_shim.cpp:317-349")        \
    X(hipblasHgemm, "shim/hipblas_shim.cpp:116-143")                        \
    X(hipblasHgemmBatched, "shim/hipblas_shim.cpp:168-189")                \
    X(hipblasHgemmStridedBatched, "shim/hipblas_shim.cpp:219-249")         \
    X(hipblasSgemm, "shim/hipblas_shim.cpp:84-113")                        \
    X(hipblasSgemmBatched, "shim/hipblas_shim.cpp:145-166")                \
    X(hipblasSgemmStridedBatched, "shim/hipblas_shim.cpp:191-217")         \
    X(hipblasLtCreate, "shim/hipblaslt_shim.cpp:104-110")                  \
    X(hipblasLtDestroy, "shim/hipblaslt_shim.cpp:112-116")                 \
    X(hipblasLtMatrixLayoutCreate, "shim/hipblaslt_shim.cpp:120-134")      \
    X(hipblasLtMatrixLayoutDestroy, "shim/hipblaslt_shim.cpp:136-140")     \
    X(hipblasLtMatrixLayoutSetAttribute, "shim/hipblaslt_shim.cpp:142-173") \
    X(hipblasLtMatrixLayoutGetAttribute, "shim/hipblaslt_shim.cpp:175-209") \
    X(hipblasLtMatmulDescCreate, "shim/hipblaslt_shim.cpp:213-229")        \
    X(hipblasLtMatmulDescDestroy, "shim/hipblaslt_shim.cpp:231-235")       \
    X(hipblasLtMatmulDescSetAttribute, "shim/hipblaslt_shim.cpp:237-267")  \
    X(hipblasLtMatmulDescGetAttribute, "shim/hipblaslt_shim.cpp:269-292")  \
    X(hipblasLtMatmulPreferenceCreate, "shim/hipblaslt_shim.cpp:296-302")  \
    X(hipblasLtMatmulPreferenceDestroy, "shim/hipblaslt_shim.cpp:304-308") \
    X(hipblasLtMatmulPreferenceSetAttribute, "shim/hipblaslt_shim.cpp:310-319") \
    X(hipblasLtMatmulAlgoGetHeuristic, "shim/hipblaslt_shim.cpp:323-343")  \
    X(hipblasLtMatmul, "shim/hipblaslt_shim.cpp:347-426")

#endif /* VKFLAME_AMD_BLAS_H */
