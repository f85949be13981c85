// gemv.hip — decode GEMV / small GEMM (M <= 16) over ggml-quantised weights.
//
// y[m, n] = sum_k x[m, k] * Wdeq[n, k], Wdeq the reference's exact fp32
// dequantised value.  The reference has no fused kernel for this: its (dead)
// mul_mat branch dequantises the whole weight to a temporary fp32 buffer and
// runs a separate GEMM (shim/hip_runtime_shim.cpp:1127-1166).  Here the weight
// is read once, decoded in registers and consumed by FMAs, with no temporary.
//
// Regime: HBM-bound (arithmetic intensity <= 2*16/0.56 flop/B, far below the
// MFMA ridge), so the kernels are VALU-only: one wave per weight row, each
// lane decoding 32-element chunks and a 64-lane butterfly reduction.
#include "vkf_device.h"

#define GEMV_WAVES 4

// x kinds: 0 = fp16, 1 = fp32, 2 = Q8_1 blocks (exact fp32 values dx*q).
#define XK_F16 0
#define XK_F32 1
#define XK_Q81 2

// 32 activations of row m, elements 32c .. 32c+31, as fp32.
template <int XK>
__device__ __forceinline__ void load_x32(const void *x, uint64_t ldx, uint32_t m, uint32_t c, float xv[32]) {
    if (XK == XK_F32) {
        const vkf_f4 *p = (const vkf_f4 *)((const float *)x + m * ldx + 32ull * c);
#pragma unroll
        for (int i = 0; i < 8; i++) {
            vkf_f4 v = p[i];
            xv[4 * i] = v[0]; xv[4 * i + 1] = v[1]; xv[4 * i + 2] = v[2]; xv[4 * i + 3] = v[3];
        }
    } else if (XK == XK_F16) {
        const vkf_h8 *p = (const vkf_h8 *)((const _Float16 *)x + m * ldx + 32ull * c);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            vkf_h8 v = p[i];
#pragma unroll
            for (int j = 0; j < 8; j++) xv[8 * i + j] = (float)v[j];
        }
    } else {
        const uint8_t *b = (const uint8_t *)x + m * ldx + 36ull * c;
#pragma unroll
        for (int g = 0; g < 4; g++) decode8<VKF_Q8_1>(b, g, xv + 8 * g);
    }
}

// Generic path: every format, x fp16 / fp32 / Q8_1, 1 <= M <= 16.
template <int QT, int XK>
__device__ __forceinline__ void gemv_generic(const VkfGemvArgs &a) {
    constexpr int BB = QTraits<QT>::BB, CPB = QTraits<QT>::BE / 32;  // chunks per block
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t nchunk = a.K / 32;
    for (uint32_t n = blockIdx.x * GEMV_WAVES + wave; n < a.N; n += gridDim.x * GEMV_WAVES) {
        const uint8_t *row = a.w + (uint64_t)n * a.row_bytes;
        float acc[16];
#pragma unroll
        for (int m = 0; m < 16; m++) acc[m] = 0.0f;
        for (uint32_t c = lane; c < nchunk; c += 64) {
            uint32_t ib = c / CPB, sub = c - ib * CPB;
            const uint8_t *blk = row + (uint64_t)ib * BB;
            float wv[32];
#pragma unroll
            for (int g = 0; g < 4; g++) decode8<QT>(blk, sub * 4 + g, wv + 8 * g);
#pragma unroll
            for (int m = 0; m < 16; m++) {
                if (m < (int)a.M) {
                    float xv[32];
                    load_x32<XK>(a.x, a.ldx, m, c, xv);
                    float s = acc[m];
#pragma unroll
                    for (int i = 0; i < 32; i++) s = fmaf(xv[i], wv[i], s);
                    acc[m] = s;
                }
            }
        }
#pragma unroll
        for (int m = 0; m < 16; m++) {
            if (m < (int)a.M) {
                float s = wave_sum(acc[m]);
                if (lane == 0) {
                    float *yp = a.y + (uint64_t)m * a.ldy + n;
                    *yp = (a.flags & 1u) ? *yp + s : s;
                }
            }
        }
    }
}

#define VKF_GEMV_KERNELS(name, QT)                                                           \
    VKF_KERNEL void __launch_bounds__(256) vkf_gemv_##name##_f16(VkfGemvArgs a) {            \
        gemv_generic<QT, XK_F16>(a);                                                         \
    }                                                                                        \
    VKF_KERNEL void __launch_bounds__(256) vkf_gemv_##name##_f32(VkfGemvArgs a) {            \
        gemv_generic<QT, XK_F32>(a);                                                         \
    }                                                                                        \
    VKF_KERNEL void __launch_bounds__(256) vkf_gemv_##name##_q8_1(VkfGemvArgs a) {           \
        gemv_generic<QT, XK_Q81>(a);                                                         \
    }

VKF_GEMV_KERNELS(q4_0, VKF_Q4_0)
VKF_GEMV_KERNELS(q4_1, VKF_Q4_1)
VKF_GEMV_KERNELS(q8_0, VKF_Q8_0)
VKF_GEMV_KERNELS(q5_0, VKF_Q5_0)
VKF_GEMV_KERNELS(q4_k, VKF_Q4_K)
VKF_GEMV_KERNELS(q5_k, VKF_Q5_K)
VKF_GEMV_KERNELS(q6_k, VKF_Q6_K)

// ---------------------------------------------------------------------------
// Q6_K weights x Q8_1 activations, integer dot (ggml's vec_dot_q6_K_q8_1
// arithmetic on the reference's element order, kernels/dequant_q6_k.glsl).
// Per 32-element chunk c (one Q8_1 block, a quarter-half of a Q6_K block):
//   P = sc0 * sum_{l<16} q8*(u-32) + sc1 * sum_{l>=16} q8*(u-32)   (exact int)
//   y += (dw * dx) * float(P)
// u = 6-bit code; v_dot4_i32_i8 computes sum q8*u and sum q8 four lanes at a
// time and the -32 offset is applied to the integer sums.
// PARTIALS=true writes P[(m*N + n)*(K/32) + c] (int32) instead of y.
// ---------------------------------------------------------------------------
template <bool PARTIALS>
__device__ __forceinline__ void gemv_q6k_q81(const VkfGemvArgs &a) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t nchunk = a.K / 32;
    const uint8_t *xq = (const uint8_t *)a.x;
    for (uint32_t n = blockIdx.x * GEMV_WAVES + wave; n < a.N; n += gridDim.x * GEMV_WAVES) {
        const uint8_t *row = a.w + (uint64_t)n * a.row_bytes;
        float acc[16];
#pragma unroll
        for (int m = 0; m < 16; m++) acc[m] = 0.0f;
        for (uint32_t c = lane; c < nchunk; c += 64) {
            uint32_t sb = c >> 3, j = c & 7, ip = j >> 2, t = j & 3;
            const uint8_t *b = row + (uint64_t)sb * 210;
            const uint8_t *ql = b + 64 * ip + 32 * (t & 1);
            const uint8_t *qh = b + 128 + 32 * ip;
            int sc0 = (int)(int8_t)b[192 + 8 * ip + 2 * t];
            int sc1 = (int)(int8_t)b[192 + 8 * ip + 2 * t + 1];
            float dw = vkf_h2f(ld_u16(b + 208));
            uint32_t sh = (t >> 1) * 4, hs = 2 * t;
            uint32_t u[8];
#pragma unroll
            for (int i = 0; i < 8; i++) {
                uint32_t lo = (ld_u32_a2(ql + 4 * i) >> sh) & 0x0f0f0f0fu;
                uint32_t hi = ((ld_u32_a2(qh + 4 * i) >> hs) & 0x03030303u) << 4;
                u[i] = lo | hi;
            }
#pragma unroll
            for (int m = 0; m < 16; m++) {
                if (m < (int)a.M) {
                    const uint8_t *xb = xq + (uint64_t)m * a.ldx + 36ull * c;
                    float dx = vkf_h2f(ld_u16(xb));
                    int qv[8];
#pragma unroll
                    for (int i = 0; i < 8; i++) qv[i] = (int)ld_u32(xb + 4 + 4 * i);
                    int s0 = 0, s1 = 0, q0 = 0, q1 = 0;
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        s0 = __builtin_amdgcn_sdot4((int)u[i], qv[i], s0, false);
                        q0 = __builtin_amdgcn_sdot4(qv[i], 0x01010101, q0, false);
                        s1 = __builtin_amdgcn_sdot4((int)u[4 + i], qv[4 + i], s1, false);
                        q1 = __builtin_amdgcn_sdot4(qv[4 + i], 0x01010101, q1, false);
                    }
                    int P = sc0 * (s0 - 32 * q0) + sc1 * (s1 - 32 * q1);
                    if (PARTIALS) {
                        ((int32_t *)a.y)[((uint64_t)m * a.N + n) * nchunk + c] = P;
                    } else {
                        acc[m] = fmaf(dw * dx, (float)P, acc[m]);
                    }
                }
            }
        }
        if (!PARTIALS) {
#pragma unroll
            for (int m = 0; m < 16; m++) {
                if (m < (int)a.M) {
                    float s = wave_sum(acc[m]);
                    if (lane == 0) {
                        float *yp = a.y + (uint64_t)m * a.ldy + n;
                        *yp = (a.flags & 1u) ? *yp + s : s;
                    }
                }
            }
        }
    }
}

VKF_KERNEL void __launch_bounds__(256) vkf_gemv_q6_k_q8_1_int(VkfGemvArgs a) { gemv_q6k_q81<false>(a); }
VKF_KERNEL void __launch_bounds__(256) vkf_q6_k_q8_1_partials(VkfGemvArgs a) { gemv_q6k_q81<true>(a); }
