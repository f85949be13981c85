// vkf_kernargs.h — packed kernel-argument structs shared by the gfx950 code
// objects and the host launcher.
//
// Every kernel in the library takes exactly one by-value struct parameter from
// this file.  The host fills the struct and hands its address to
// hipModuleLaunchKernel as kernelParams[0]; the static_asserts pin the byte
// layout on both sides.  This replaces the reference's per-shader push-constant
// blocks (runtime/dispatch.cpp:31-42 LinearInt8PC/LinearFP16PC, the {nb}
// block of runtime/dispatch.cpp:481-484) and its descriptor-set bindings.
#pragma once
#include <stdint.h>

// Quant type codes: the reference's VKF_DEQUANT_* (runtime/dispatch.h:14-21).
enum VkfQType {
    VKF_Q4_0 = 0, VKF_Q4_1 = 1, VKF_Q8_0 = 2, VKF_Q5_0 = 3,
    VKF_Q4_K = 4, VKF_Q5_K = 5, VKF_Q6_K = 6, VKF_Q8_1 = 7
};

// Epilogue activation codes: kernels/linear_fp16.glsl:19 (same values as the
// public header's VKF_ACT_*).
#ifndef VKF_ACT_NONE
#define VKF_ACT_NONE 0
#define VKF_ACT_SILU 1
#define VKF_ACT_RELU 2
#define VKF_ACT_GELU_ERF 3
#endif

// Dequantise n_blocks whole blocks to fp32 or fp16 (one kernel per type and
// output dtype).
struct VkfDequantArgs {
    const uint8_t *src;
    void *dst;
    uint64_t n_blocks;
};

// fp32 rows -> Q8_1 blocks.  Row m of x starts at x + m*ldx; its K/32 blocks
// land at dst + m*(K/32)*36.
struct VkfQuantizeArgs {
    const float *x;
    uint8_t *dst;
    uint64_t ldx;
    uint32_t M, K;
};

// Symmetric per-row int8 quantisation: scale[m] = max(max_k |x[m,k]| / 127,
// 1e-8), q[m,k] = clamp(rint(x[m,k] / scale[m]), -127, 127).  x fp16 or fp32
// (x_f16), row stride ldx elements; q packed [M, K].
struct VkfQuantRowsArgs {
    const void *x;
    int8_t *q;
    float *scale;
    uint64_t ldx;
    uint32_t M, K;
    uint32_t x_f16, pad;
};

// Read-bandwidth measurement: n16 16-byte vectors read once from src.
struct VkfStreamArgs {
    const void *src;
    uint32_t *sink;
    uint64_t n16;
};

// Decode GEMV / small GEMM: y[m, n] = sum_k x[m, k] * W[n, k], M <= 16.
// W row n starts at w + n*row_bytes.  x is fp16 or fp32 (by kernel), or Q8_1
// blocks (row m at x + m*ldx bytes) for the Q6_K x Q8_1 kernel.
struct VkfGemvArgs {
    const uint8_t *w;
    const void *x;
    float *y;
    uint64_t row_bytes;
    uint64_t ldx;   // elements (bytes for Q8_1 activations)
    uint64_t ldy;   // elements
    uint32_t M, N, K;
    uint32_t flags; // bit 0: y += (accumulate) instead of y =
};

// Sum of the K-slice partials of a GEMV: y[m, n] = sum over s < S, in order,
// of part[(s*M + m)*N + n].
struct VkfSplitSumArgs {
    const float *part;
    float *y;
    uint64_t ldy;   // elements
    uint32_t M, N, S, pad;
};

// Dense GEMM core, both operands K-contiguous:
//   D[r, c] = epi( sum_k X[r, k] * Y[c, k] )   r < R, c < C
// X row r at X + r*ldx, Y row c at Y + c*ldy, D element at D + r*ldd + c.
// Epilogue (fp32): v = alpha * acc * (rs ? rs[r] : 1) * (cs ? cs[c] : 1)
//                  v += beta * Cin[r*ldc + c]   (if beta != 0)
//                  v += bias[c]                 (if bias)
//                  v  = act(v)
// Quantised-weight variants put the quantised operand in Y (rows of blocks).
struct VkfGemmArgs {
    const void *X;
    const void *Y;
    void *D;
    const void *Cin;
    const float *rs;       // per-row scale of X (length R) or null
    const float *cs;       // per-row scale of Y (length C) or null
    const void *bias;      // length C, fp16 or fp32 (flags) or null
    uint64_t ldx, ldy, ldd, ldc;  // elements (bytes for quantised Y rows)
    uint32_t R, Cn, K;
    uint32_t act;
    float alpha, beta;
    uint32_t flags;        // VKF_GF_* below
    float xscale;          // VKF_GF_X_F16Q: the activation quantisation scale
    // Batched launches of the dense kernels (vkf_gemm_f16 / _f32 / _i8 and
    // their _k2 forms): matrix b = blockIdx.z sits at X + b*bsx, Y + b*bsy,
    // D + b*bsd, Cin + b*bsc (byte strides), or, when bpx is set, at the
    // device pointer arrays bpx[b], bpy[b], bpd[b] with Cin = D (hipBLAS's
    // batched form).  Zero / null for one matrix.
    uint64_t bsx, bsy, bsd, bsc;
    const void *const *bpx;
    const void *const *bpy;
    void *const *bpd;
};

// VkfGemmArgs.flags
#define VKF_GF_D_F32     1u   // D is fp32 (else fp16; int32 kernels: int32)
#define VKF_GF_CIN_F32   2u   // Cin is fp32 (else fp16)
#define VKF_GF_BIAS_F32  4u   // bias is fp32 (else fp16)
#define VKF_GF_X_TRANS   8u   // X stored [K, R] (element (r,k) at X + k*ldx + r)
#define VKF_GF_Y_TRANS  16u   // Y stored [K, C] (element (c,k) at Y + k*ldy + c)
#define VKF_GF_BIAS_ROW 32u   // bias indexed by r (length R) instead of c
#define VKF_GF_D_I32    64u   // int8 kernel: store the raw int32 accumulator
                              // (alpha/beta applied as integers, Cin int32);
                              // alpha and beta then hold int32 bit patterns
                              // (vkf_gemm_set_int_scalars), not floats
#define VKF_GF_RS_SCALAR 128u // rs is one scalar (rs[0]) for every row
#define VKF_GF_CS_SCALAR 256u // cs is one scalar (cs[0]) for every column
#define VKF_GF_X_F16Q   512u  // int8 kernel: X holds fp16 values, quantised
                              // on load to clamp(rint(x / xscale), -127, 127)

#ifdef __cplusplus
// Integer alpha / beta of a VKF_GF_D_I32 launch, stored bit for bit in the
// float fields (every int32 value, including those above 2^24).
inline void vkf_gemm_set_int_scalars(VkfGemmArgs &g, int32_t alpha, int32_t beta) {
    __builtin_memcpy(&g.alpha, &alpha, 4);
    __builtin_memcpy(&g.beta, &beta, 4);
}
static_assert(sizeof(VkfDequantArgs) == 24, "VkfDequantArgs layout");
static_assert(sizeof(VkfQuantizeArgs) == 32, "VkfQuantizeArgs layout");
static_assert(sizeof(VkfStreamArgs) == 24, "VkfStreamArgs layout");
static_assert(sizeof(VkfSplitSumArgs) == 40, "VkfSplitSumArgs layout");
static_assert(sizeof(VkfQuantRowsArgs) == 48, "VkfQuantRowsArgs layout");
static_assert(sizeof(VkfGemvArgs) == 64, "VkfGemvArgs layout");
static_assert(sizeof(VkfGemmArgs) == 176, "VkfGemmArgs layout");
#endif
