/*
 * vkflame_amd.h — C ABI of the MI355X (gfx950) quantized-linear library
 * (libvkflame_amd.so).
 *
 * Every entry point takes plain device pointers, sizes and a hipStream_t
 * (declared here as void* so the header needs no HIP include).  All work is
 * enqueued asynchronously on the given stream (0 = the legacy default
 * stream) and nothing synchronises.  One entry point allocates device memory:
 * vkflame_dispatch_gemm_q takes a stream-ordered workspace (hipMallocAsync /
 * hipFreeAsync) for Q8_1 activations at M > 16; callers that must not allocate
 * use vkflame_dispatch_gemm_q_ws (their own workspace) or
 * vkflame_dispatch_gemm_q_noalloc (the library's fixed array).  Every other
 * entry point allocates nothing.
 * Return value: 0 on success, otherwise a hipError_t code
 * (1 = hipErrorInvalidValue for bad arguments, 98 = hipErrorInvalidDeviceFunction
 * on a device that is not gfx950, or the HIP error of a failed launch).
 *
 * The integer codes are the reference's (runtime/dispatch.h:6-21 and the
 * activation codes of kernels/linear_fp16.glsl:19), so the reference's
 * callers keep their constants.
 *
 * Citations name the reference (vkflame) interface each entry replaces.
 */
#ifndef VKFLAME_AMD_H
#define VKFLAME_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* dtype codes: runtime/dispatch.h:7-11 */
#define VKF_DTYPE_FP32 0
#define VKF_DTYPE_FP16 1
#define VKF_DTYPE_INT8 2
#define VKF_DTYPE_BF16 3
#define VKF_DTYPE_FP16_FP32OUT 4
/* extra codes of this library (no reference counterpart) */
#define VKF_DTYPE_INT32 10
#define VKF_DTYPE_Q8_1 11  /* activations given as ggml Q8_1 blocks */
#define VKF_DTYPE_INT8_INT32OUT 12  /* int8 x int8 -> raw int32 (exact) */

/* quant type codes: runtime/dispatch.h:14-21 */
#define VKF_DEQUANT_Q4_0 0
#define VKF_DEQUANT_Q4_1 1
#define VKF_DEQUANT_Q8_0 2
#define VKF_DEQUANT_Q5_0 3
#define VKF_DEQUANT_Q4_K 4
#define VKF_DEQUANT_Q5_K 5
#define VKF_DEQUANT_Q6_K 6
#define VKF_DEQUANT_Q8_1 7

/* activation codes: kernels/linear_fp16.glsl:19, kernels/linear_int8.glsl:23 */
#define VKF_ACT_NONE 0
#define VKF_ACT_SILU 1
#define VKF_ACT_RELU 2
#define VKF_ACT_GELU_ERF 3

/* Library version string. */
const char *vkflame_version(void);

/* Load the gfx950 code objects on the current device.  Optional: every entry
 * point does it on first use.  Replaces vkflame_init (runtime/device.h:39-42,
 * runtime/device.cpp:131-372) and vkflame_pipelines_init
 * (runtime/pipeline.cpp:143-251). */
int vkflame_init(void);

/* Bytes / elements of one block of quant_type (-1 for an unknown code). */
int vkflame_block_bytes(int quant_type);
int vkflame_block_elems(int quant_type);

/* Dequantise n_blocks consecutive blocks at src into dst, fp32
 * (out_dtype = VKF_DTYPE_FP32) or fp16 (VKF_DTYPE_FP16, the fp32 value rounded
 * to nearest even).  Values are bit-identical to kernels/dequant_*.glsl.
 * src must be 4-byte aligned for Q4_1, Q4_K, Q5_K and Q8_1 and 2-byte aligned
 * otherwise; dst 16-byte aligned.
 * Replaces vkflame_dispatch_dequant(VKFContext*, VKFBuffer *src,
 * VKFBuffer *dst, uint32_t n_blocks, int quant_type) (runtime/dispatch.h:89-92,
 * runtime/dispatch.cpp:469-498): raw device pointers at any offset instead of
 * whole VkBuffers, an explicit output dtype, and the caller's stream. */
int vkflame_dispatch_dequant(const void *src, void *dst, uint64_t n_blocks, int quant_type, int out_dtype,
                             void *stream);

/* Quantise fp32 activations x[M, K] (row stride ldx elements, K % 32 == 0)
 * to ggml Q8_1 blocks dst[M, K/32] (36 B each: fp16 d, fp16 s = d*sum(q),
 * int8 q[32]).  ggml's quantize_row_q8_1_ref rule: d = max|x|/127,
 * q = roundf(x/d).  The reference decodes Q8_1 (kernels/dequant_q8_1.glsl)
 * but has no quantizer. */
int vkflame_quantize_q8_1(const float *x, void *dst, int M, int K, int64_t ldx, void *stream);

/* Symmetric per-row int8 quantisation of x[M, K] (x_dtype VKF_DTYPE_FP16 or
 * VKF_DTYPE_FP32, row stride ldx elements, 0 = K): scale[m] = max(max_k
 * |x[m,k]| / 127, 1e-8), q[m, k] = clamp(round_half_even(x[m,k] / scale[m]),
 * -127, 127), q packed [M, K].  The rule of the reference's per-output-channel
 * weight quantiser (tools/quantise.py:35-41), used here also per token for the
 * activations of the int8 linear (vkflame_dispatch_linear_int8's A and
 * a_scale). */
int vkflame_quantize_rows_i8(const void *x, int x_dtype, int M, int K, int64_t ldx, int8_t *q, float *scale,
                             void *stream);

/* y[M, N] (fp32, row stride ldy) = x[M, K] @ Wdeq[N, K]^T.
 * w: N rows of K/block_elems blocks of quant_type, row stride row_bytes
 *    (0 = packed: K/block_elems*block_bytes).
 * x: x_dtype VKF_DTYPE_FP16 or VKF_DTYPE_FP32 (row stride ldx elements), or
 *    VKF_DTYPE_Q8_1 (Q8_1 blocks, row stride ldx bytes; 0 = packed).
 * M <= 16 runs the HBM-bound decode GEMV kernels, larger M the MFMA GEMM with
 * the weight tile dequantised into LDS.  K % block_elems == 0.
 * With Q8_1 activations and M > 16, Q8_0 weights run on the int8 matrix
 * cores: each 32-element block's dot is an exact int32, scaled by dx*dw in fp32.
 * With Q8_1 activations at M = 1, Q6_K weights use the exact integer dot
 * product (v_dot4_i32_i8), Q4_0, Q4_1, Q8_0, Q4_K and Q5_K the fp32 values
 * dx*q put on a 14-bit grid per 64 elements (as fp32 activations are); at
 * 2 <= M <= 16 the matrix-core GEMV (Q4_0, Q4_1, Q8_0, Q4_K, Q5_K, Q6_K; Q5_0
 * from M = 1 when N gives two 16-row tiles per CU) and the GEMM take fp16(dx*q) (the GEMV after scaling each row
 * by a power of two, so no row overflows fp16), and fp32 activations on the
 * matrix-core GEMV are rounded to fp16 the same way.
 * This is the fused form of the reference's quant mul_mat path, which
 * dequantises W and the activations to temporaries and runs linear_fp16_fp32out
 * (shim/hip_runtime_shim.cpp:1102-1172). */
int vkflame_dispatch_gemm_q(const void *w, int quant_type, uint64_t row_bytes, const void *x, int x_dtype,
                            int64_t ldx, float *y, int64_t ldy, int M, int N, int K, void *stream);

/* vkflame_dispatch_gemm_q with a caller-supplied device workspace, in the
 * manner of hipblasLtMatmul's workspace argument, 16-byte aligned, of at
 * least vkflame_gemm_q_workspace_bytes(quant_type, x_dtype, M, N, K) bytes;
 * without one (NULL or too small) each route below runs its no-workspace
 * form.  Two routes use it:
 *  - Q8_1 activations, M > 16, packed rows (ldx = K/32*36): M*K*2 bytes
 *    receive the activations decoded once to fp16(d*q) and the
 *    fp16-activation GEMM runs on them (from M = 256 with 256-row tiles);
 *    without it the GEMM decodes activation tiles itself.  Both multiply the
 *    same fp16 operand values.
 *  - Q4_K (K > 5120) and Q4_0 / Q4_1 (K > 4096) weights at 2 <= M <= 16,
 *    Q8_0 (K > 6144) at 9 <= M <= 16, fp16 activations, at most 8 K slices
 *    (of 20 / 16 / 24 256-k groups): S*M*N*4
 *    bytes hold the partial products of S K slices, which run side by side
 *    on the matrix-core GEMV and are added in slice order by a second
 *    launch; without it the slices run one launch after another.
 * vkflame_dispatch_gemm_q allocates the workspace stream-ordered
 * (hipMallocAsync / hipFreeAsync) when the stream is not being captured,
 * and goes without it under capture.  No reference counterpart as an entry
 * point: the workspace stands for the temporaries of the reference's mul_mat
 * path (shim/hip_runtime_shim.cpp:1102-1172). */
int vkflame_dispatch_gemm_q_ws(const void *w, int quant_type, uint64_t row_bytes, const void *x, int x_dtype,
                               int64_t ldx, float *y, int64_t ldy, int M, int N, int K, void *workspace,
                               size_t workspace_bytes, void *stream);
/* Workspace bytes vkflame_dispatch_gemm_q_ws uses for these arguments (0: none). */
size_t vkflame_gemm_q_workspace_bytes(int quant_type, int x_dtype, int M, int N, int K);

/* vkflame_dispatch_gemm_q that allocates nothing: the scratch buffer of
 * that entry point (the fp16 copy of Q8_1 activations at M > 16, M*K*2 bytes;
 * the K-slice partials of the GEMV, S*M*N*4 bytes) is a fixed device array of
 * VKFLAME_NOALLOC_SCRATCH_BYTES inside the library, one per GPU, held until
 * the process ends.  No reference counterpart: it is for callers that cannot
 * call hipMalloc (code under HIP graph capture, tight serving loops, harnesses
 * that forbid allocation).  Same arguments and results as
 * vkflame_dispatch_gemm_q; returns hipErrorInvalidValue (and says so on
 * stderr) when M*K*2 exceeds the array (a GEMV whose K-slice partials exceed
 * it runs its slices one launch after another instead).  Every call on one GPU shares
 * that GPU's array: calls that overlap on one GPU (different streams, or
 * threads) race and must be ordered by the caller.  The first call on a device
 * looks the array up (hipGetSymbolAddress); make it outside graph capture. */
#define VKFLAME_NOALLOC_SCRATCH_BYTES (16u << 20)
int vkflame_dispatch_gemm_q_noalloc(const void *w, int quant_type, uint64_t row_bytes, const void *x, int x_dtype,
                                    int64_t ldx, float *y, int64_t ldy, int M, int N, int K, void *stream);
/* Size of that array in bytes (VKFLAME_NOALLOC_SCRATCH_BYTES). */
size_t vkflame_noalloc_scratch_bytes(void);

/* Integer partials of Q6_K weights w[N, K] x Q8_1 activations xq[M, K]:
 * P[(m*N + n)*(K/32) + kb] = sum over the 32 elements of block kb of
 * q8 * sc * (q6 - 32).  Exact int32; a test hook for the integer core of the
 * Q6_K x Q8_1 product. */
int vkflame_q6_k_q8_1_partials(const void *w, const void *xq, int32_t *P, int M, int N, int K, void *stream);

/* Integer partials of Q8_0 weights w[N, K] x Q8_1 activations xq[M, K] as the
 * prefill's int8 matrix-core kernel computes them (the same MFMA code path):
 * P[(m*N + n)*(K/32) + kb] = sum over block kb of q8x * q8w, exact int32.
 * A test hook for the integer core of the Q8_0 x Q8_1 GEMM. */
int vkflame_q8_0_q8_1_partials(const void *w, const void *xq, int32_t *P, int M, int N, int K, void *stream);

/* Measurement hook: reads bytes (a multiple of 16) from src (16-byte
 * aligned) once with coalesced 16-byte loads and nothing else; sink is a
 * device word that is written only if the folded data equals a constant.
 * Its duration is the measured HBM read-bandwidth reference for the decode
 * GEMVs' weight streams.  No reference counterpart (the reference has no
 * bandwidth probe). */
int vkflame_stream_read(const void *src, uint64_t bytes, uint32_t *sink, void *stream);

/* Row-major linear layer, the reference's vkflame_dispatch_linear
 * (runtime/dispatch.h:51-58, runtime/dispatch.cpp:253-326) with the arguments
 * it ignores honoured:
 *   D[M,N] = act( alpha * op(A) @ op(B) + beta * C )
 *   op(A) = A[M,K] (transA = 0) or A stored [K,M] (transA = 1)
 *   op(B) = B[K,N] (transB = 0) or B stored [N,K] (transB = 1)
 * dtype VKF_DTYPE_FP16: A, B, C, D fp16, fp32 accumulation.
 * dtype VKF_DTYPE_FP16_FP32OUT: A, B fp16; C, D fp32.
 * dtype VKF_DTYPE_FP32: A, B, C, D fp32 (fp32 matrix cores; the reference
 *   runs FP32 through its fp16 shader, runtime/dispatch.cpp:270-282).
 * dtype VKF_DTYPE_INT8: the reference's int8 linear (kernels/linear_int8.glsl
 *   :8-24, 60-100): A fp16, quantised in the kernel to
 *   q = clamp(round_half_even(A / act_scale), -127, 127); B int8 weights;
 *   act_scale = *alpha (float, NULL = 1; the reference's "caller may pass via
 *   alpha", runtime/dispatch.cpp:302); C = per-output-channel w_scale, fp32
 *   [N] (NULL = 1; the reference binds D in its place,
 *   runtime/dispatch.cpp:305-308); beta NULL or 0;
 *   D fp16 = f16(act(float(acc) * w_scale[n] * act_scale)), acc the exact
 *   int32 sum (the reference omits act_scale here and only passes 1).
 * dtype VKF_DTYPE_INT8_INT32OUT (no reference code): A, B int8, C, D int32,
 *   exact; activation must be 0; alpha/beta (int32*) as in hipblasGemmEx with
 *   HIPBLAS_COMPUTE_32I.
 * alpha/beta: host pointers to float (int32 for INT8_INT32OUT), NULL = 1 and 0.
 * VKF_DTYPE_BF16 returns hipErrorNotSupported.
 * C may be NULL when beta is 0.  Matrices are packed (ld = row length). */
int vkflame_dispatch_linear(const void *A, const void *B, const void *C, void *D, int M, int N, int K, int dtype,
                            int transA, int transB, int activation, const void *alpha, const void *beta,
                            void *stream);

/* int8 linear with per-row / per-channel scales and bias (the full contract of
 * kernels/linear_int8.glsl:48-101 plus the scales and bias the reference binds
 * but drops, shim/hipblaslt_shim.cpp:254-262 vs 418-423):
 *   acc[m,n] = sum_k A[m,k] * W[n,k]              (exact int32)
 *   D[m,n]   = act(float(acc) * a_scale[m] * w_scale[n] + bias[n])
 * A int8 [M,K], W int8 [N,K], a_scale/w_scale fp32 (NULL = 1), bias fp16 or
 * fp32 per bias_dtype (NULL = none), D fp16 or fp32 per d_dtype. */
int vkflame_dispatch_linear_int8(const int8_t *A, const float *a_scale, const int8_t *W, const float *w_scale,
                                 const void *bias, int bias_dtype, void *D, int d_dtype, int M, int N, int K,
                                 int activation, void *stream);

/* ---- kernel-name dispatch table (the reference's hipLaunchKernel table,
 *      shim/hip_runtime_shim.cpp:833-1213) ---- */

/* What a resolved launch does. */
#define VKF_LAUNCH_NONE 0         /* not ours: fall through to the real launch */
#define VKF_LAUNCH_DEQUANT 1      /* dequantize_block_* */
#define VKF_LAUNCH_MUL_MAT_Q 2    /* quantised weight x Q8_1 activations */
#define VKF_LAUNCH_MUL_MAT_F16 3  /* fp16 x fp16 mul_mat */

typedef struct VkflameLaunchPlan {
    int kind;          /* VKF_LAUNCH_* */
    int quant_type;    /* VKF_DEQUANT_* */
    int out_dtype;     /* VKF_DTYPE_FP32 / VKF_DTYPE_FP16 for dequant */
    int pad;
    const void *src;   /* dequant src / mul_mat weights (vx) */
    const void *src1;  /* mul_mat activations (vy) */
    void *dst;
    uint64_t n_blocks; /* dequant */
    int M, N, K;       /* mul_mat: M = nrows_y, N = nrows_x, K = ncols_x */
    int pad2;
} VkflameLaunchPlan;

/* Pure function: decode a kernel launch by device-function name.
 * args follow the HIP launch convention (args[i] points at argument i).
 * Returns plan->kind.  Rules (shim/hip_runtime_shim.cpp:896-952, 1096-1188):
 *   mul_mat + quant substring -> MUL_MAT_Q (vx, vy, dst, ncols_x=K, nrows_x=N,
 *     _, nrows_y=M); tested before the dequant substrings so it is reachable;
 *   mul_mat + f16 -> MUL_MAT_F16 (A, B, D, K = arg3, N = arg4, M = arg6);
 *   q4_0|q4K_0, q4_1, q5_0|q5K_0: nb32 = int32 arg2;
 *   q8_0: nb = int32 arg2 when blockDim.x == 32, else int64 arg2 / 32;
 *   q4_K|q4K, q5_K|q5K, q6_K|q6K: nb = gridDim.x.
 * Dequant output is fp16 when the name marks a half/_Float16 destination
 * ("half", "__half", "DF16_"), fp32 otherwise. */
int vkflame_resolve_launch(const char *name, unsigned grid_x, unsigned grid_y, unsigned grid_z, unsigned block_x,
                           unsigned block_y, unsigned block_z, void **args, VkflameLaunchPlan *plan);

/* Run a resolved plan on stream.  Returns 0 or a hipError_t. */
int vkflame_execute_launch(const VkflameLaunchPlan *plan, void *stream);

#ifdef __cplusplus
}
#endif
#endif /* VKFLAME_AMD_H */
