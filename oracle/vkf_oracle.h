/*
 * vkf_oracle.h — CPU restatement of vkflame's quantized-linear arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the shipped library links, loads or
 * calls this code; only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg use it, and only as the checker.
 *
 * Every function names the reference file:line whose arithmetic it restates
 * (paths relative to the vkflame source tree).  The reference implementation
 * of this path is GLSL for Vulkan and cannot be built or run in this image
 * (no glslc, no Vulkan loader), so the restatement is pinned by the checks in
 * tests/test_oracle_*.py: hand-computed known-answer blocks, round trips
 * through independent packers, exhaustive fp16 conversion against numpy, and
 * closed-form invariants.
 */
#ifndef VKF_ORACLE_H
#define VKF_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Quant type codes: identical to the reference's VKF_DEQUANT_* codes
 * (runtime/dispatch.h:14-21). */
enum {
    VKFO_Q4_0 = 0, VKFO_Q4_1 = 1, VKFO_Q8_0 = 2, VKFO_Q5_0 = 3,
    VKFO_Q4_K = 4, VKFO_Q5_K = 5, VKFO_Q6_K = 6, VKFO_Q8_1 = 7
};

/* Bytes per block / elements per block of each quant type. */
int vkfo_block_bytes(int qtype);
int vkfo_block_elems(int qtype);

/* IEEE binary16 <-> binary32.  h2f is exact; f2h rounds to nearest even and
 * keeps subnormals, infinities and NaN (quiet). */
float    vkfo_h2f(uint16_t h);
uint16_t vkfo_f2h(float f);

/* Dequantise n_blocks blocks of qtype into fp32 (the reference's only output
 * type, kernels/dequant_*.glsl).  Returns 0, or -1 for an unknown type. */
int vkfo_dequant_f32(int qtype, const uint8_t *src, size_t n_blocks, float *dst);
/* Same values rounded to fp16 (RNE of the fp32 value). */
int vkfo_dequant_f16(int qtype, const uint8_t *src, size_t n_blocks, uint16_t *dst);

/* fp32 -> Q8_1 blocks (36 B: fp16 d, fp16 s, int8 qs[32]).  n % 32 == 0.
 * Follows ggml's reference quantizer quantize_row_q8_1_ref (ggml is not
 * vendored in the reference; kernels/dequant_q8_1.glsl:2-4 names the format). */
void vkfo_quantize_q8_1(const float *x, size_t n, uint8_t *dst);
void vkfo_quantize_rows_i8(const float *x, int M, int K, int8_t *q, float *scale);

/* Integer GEMM, both operands K-contiguous: C[m,n] = sum_k A[m,k]*B[n,k].
 * Accumulates in int64; returns -1 if any result leaves int32 range. */
int vkfo_gemm_i8_nt(const int8_t *A, const int8_t *B, int32_t *C,
                    int M, int N, int K);

/* Q6_K weights [N, K] x Q8_1 activations [M, K]: exact integer partial of
 * every (m, n, 32-element block kb):
 *   P[(m*N + n)*(K/32) + kb] = sum_{k in kb} q8[m,k] * sc(n,k) * (q6[n,k]-32)
 * This is the integer core of ggml's vec_dot_q6_K_q8_1, with the element
 * order of kernels/dequant_q6_k.glsl:34-58. */
void vkfo_q6k_q8_1_partials(const uint8_t *w, const uint8_t *xq, int32_t *P,
                            int M, int N, int K);

/* The linear kernels' activation epilogue (0 none, 1 silu, 2 relu,
 * 3 gelu with the Abramowitz-Stegun 7.1.26 erf), in fp32:
 * kernels/linear_int8.glsl:26-46, kernels/linear_fp16.glsl:22-36. */
float vkfo_act(int act, float x);

#ifdef __cplusplus
}
#endif
#endif
