// gemm.hip — prefill GEMM (M >= 17) on the gfx950 matrix cores.
//
// Replaces kernels/linear_fp16.glsl, linear_fp16_fp32out.glsl, linear_coop.glsl
// (one thread or one 16x16 subgroup tile per output, no LDS reuse) and
// kernels/linear_int8.glsl (one thread per output, scalar int MACs).
//
// Core: D[r, c] = epi( sum_k X[r, k] * Y[c, k] ) with both operands
// K-contiguous.  A 256-thread workgroup owns a 128x128 tile of D; each of its
// four waves owns 64x64 = 4x4 MFMA 16x16 sub-tiles.  K advances in steps that
// are staged through double-buffered LDS, one barrier per step.
//
// Variants (all share the tiling):
//   vkf_gemm_f16        fp16 x fp16 -> fp32 acc, v_mfma_f32_16x16x32_f16
//   vkf_gemm_i8         int8 x int8 -> int32 acc, v_mfma_i32_16x16x64_i8
//   vkf_gemm_<q>_f16    fp16 activations x ggml weights: each weight tile is
//                       dequantised in registers to the reference's exact fp32
//                       value, rounded to fp16 and written to LDS, then the
//                       fp16 MFMA core runs (dequant fused into the GEMM)
//   vkf_gemm_q6_k_q8_1  Q8_1 activations x Q6_K weights, integer-exact: LDS
//                       holds q8 and sc*(q6-32) as fp16 (both exact integers),
//                       so each 32-deep MFMA yields the exact integer partial
//                       P[m,n,kb]; the fp32 epilogue applies dx per block and
//                       dw per super-block.
//
// MFMA 16x16 operand layout used throughout: lane l supplies row (l % 16) of
// A and column (l % 16) of B, with a K slice selected by l / 16; both operands
// use the same K slice map, so the product is independent of the hardware's
// internal K order.  Accumulator: lane l holds D[4*(l/16) + i][l % 16].
#include "vkf_device.h"

#define BM 128
#define BN 128

__device__ __forceinline__ void epi_store(const VkfGemmArgs &a, uint32_t r, uint32_t c, float v) {
    if (a.rs) v *= a.rs[(a.flags & VKF_GF_RS_SCALAR) ? 0 : r];
    if (a.cs) v *= a.cs[(a.flags & VKF_GF_CS_SCALAR) ? 0 : c];
    v *= a.alpha;
    if (a.beta != 0.0f) {
        float cin = (a.flags & VKF_GF_CIN_F32) ? ((const float *)a.Cin)[(uint64_t)r * a.ldc + c]
                                                : (float)((const _Float16 *)a.Cin)[(uint64_t)r * a.ldc + c];
        v = fmaf(a.beta, cin, v);
    }
    if (a.bias) {
        uint32_t bi = (a.flags & VKF_GF_BIAS_ROW) ? r : c;
        v += (a.flags & VKF_GF_BIAS_F32) ? ((const float *)a.bias)[bi] : (float)((const _Float16 *)a.bias)[bi];
    }
    v = vkf_act(a.act, v);
    if (a.flags & VKF_GF_D_F32)
        ((float *)a.D)[(uint64_t)r * a.ldd + c] = v;
    else
        ((_Float16 *)a.D)[(uint64_t)r * a.ldd + c] = vkf_to_f16(v);
}

// ---------------------------------------------------------------------------
// fp16 operand tiles: 128 rows x 32 k, LDS row pitch 40 halves (80 B) so the
// 16 rows read by one ds_read_b128 fall in distinct banks.
// ---------------------------------------------------------------------------
#define KF 32
#define PF 40

// Load one 128 x 32 fp16 tile into two 8-half registers per thread.
// Thread t covers (row, 8-wide k chunk) for idx = t and t + 256.
__device__ __forceinline__ void load_f16_tile(const _Float16 *P, uint64_t ld, bool trans, uint32_t nrows,
                                              uint32_t row0, uint32_t K, uint32_t k0, vkf_h8 v[2]) {
#pragma unroll
    for (int i = 0; i < 2; i++) {
        int idx = threadIdx.x + 256 * i;
        uint32_t r = row0 + (idx >> 2), k = k0 + 8 * (idx & 3);
        vkf_h8 t = {};
        if (r < nrows) {
            if (!trans && k + 8 <= K && ((ld & 7) == 0) && (((uintptr_t)P & 15) == 0)) {
                t = *(const vkf_h8 *)(P + (uint64_t)r * ld + k);
            } else {
#pragma unroll
                for (int j = 0; j < 8; j++)
                    if (k + j < K)
                        t[j] = trans ? P[(uint64_t)(k + j) * ld + r] : P[(uint64_t)r * ld + k + j];
            }
        }
        v[i] = t;
    }
}

__device__ __forceinline__ void store_f16_tile(_Float16 *lds, const vkf_h8 v[2]) {
#pragma unroll
    for (int i = 0; i < 2; i++) {
        int idx = threadIdx.x + 256 * i;
        *(vkf_h8 *)(lds + (idx >> 2) * PF + 8 * (idx & 3)) = v[i];
    }
}

// Dequantise a 128-row x 32-k tile of ggml weights to fp16.  Thread t covers
// row t/2, elements 16*(t&1) .. +15 of the 32-element chunk k0/32.
template <int QT>
__device__ __forceinline__ void load_q_tile(const uint8_t *W, uint64_t row_bytes, uint32_t nrows,
                                            uint32_t row0, uint32_t k0, vkf_h8 v[2]) {
    constexpr int BB = QTraits<QT>::BB, CPB = QTraits<QT>::BE / 32;
    uint32_t r = row0 + (threadIdx.x >> 1);
    int h = threadIdx.x & 1;
    v[0] = vkf_h8{};
    v[1] = vkf_h8{};
    if (r < nrows) {
        uint32_t ch = k0 / 32, ib = ch / CPB, sub = ch - ib * CPB;
        const uint8_t *blk = W + (uint64_t)r * row_bytes + (uint64_t)ib * BB;
#pragma unroll
        for (int i = 0; i < 2; i++) {
            float y[8];
            decode8<QT>(blk, sub * 4 + 2 * h + i, y);
#pragma unroll
            for (int j = 0; j < 8; j++) v[i][j] = vkf_to_f16(y[j]);
        }
    }
}

__device__ __forceinline__ void store_q_tile(_Float16 *lds, const vkf_h8 v[2]) {
    int row = threadIdx.x >> 1, h = threadIdx.x & 1;
    *(vkf_h8 *)(lds + row * PF + 16 * h) = v[0];
    *(vkf_h8 *)(lds + row * PF + 16 * h + 8) = v[1];
}

// One 32-deep step of the 64x64 wave tile.
__device__ __forceinline__ void mfma_step_f16(const _Float16 *ax, const _Float16 *ay, int wr, int wc,
                                              vkf_f4 acc[4][4]) {
    const int lane = threadIdx.x & 63, li = lane & 15, lg = lane >> 4;
    vkf_h8 fa[4], fb[4];
#pragma unroll
    for (int i = 0; i < 4; i++) fa[i] = *(const vkf_h8 *)(ax + (wr * 64 + 16 * i + li) * PF + 8 * lg);
#pragma unroll
    for (int j = 0; j < 4; j++) fb[j] = *(const vkf_h8 *)(ay + (wc * 64 + 16 * j + li) * PF + 8 * lg);
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(fa[i], fb[j], acc[i][j], 0, 0, 0);
}

__device__ __forceinline__ void store_acc_f32(const VkfGemmArgs &a, uint32_t r0, uint32_t c0, int wr, int wc,
                                              vkf_f4 acc[4][4]) {
    const int lane = threadIdx.x & 63, li = lane & 15, lg = lane >> 4;
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                uint32_t r = r0 + wr * 64 + 16 * i + 4 * lg + e, c = c0 + wc * 64 + 16 * j + li;
                if (r < a.R && c < a.Cn) epi_store(a, r, c, acc[i][j][e]);
            }
}

// XQT < 0: dense fp16 X, otherwise Q8_1 activation blocks (each tile value
// fp16(dx*q)).  QT < 0: dense fp16 Y; otherwise Y holds ggml blocks of type QT.
template <int XQT, int QT>
__device__ __forceinline__ void gemm_f16_body(const VkfGemmArgs &a) {
    __shared__ __attribute__((aligned(16))) _Float16 lx[2][BM * PF];
    __shared__ __attribute__((aligned(16))) _Float16 ly[2][BN * PF];
    const uint32_t r0 = blockIdx.y * BM, c0 = blockIdx.x * BN;
    const int wave = threadIdx.x >> 6, wr = wave >> 1, wc = wave & 1;
    const bool xt = a.flags & VKF_GF_X_TRANS, yt = a.flags & VKF_GF_Y_TRANS;
    vkf_f4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = vkf_f4{0, 0, 0, 0};

    const uint32_t nk = (a.K + KF - 1) / KF;
    vkf_h8 vx[2], vy[2];
    if constexpr (XQT < 0) load_f16_tile((const _Float16 *)a.X, a.ldx, xt, a.R, r0, a.K, 0, vx);
    else load_q_tile<XQT>((const uint8_t *)a.X, a.ldx, a.R, r0, 0, vx);
    if constexpr (QT < 0) load_f16_tile((const _Float16 *)a.Y, a.ldy, yt, a.Cn, c0, a.K, 0, vy);
    else load_q_tile<QT>((const uint8_t *)a.Y, a.ldy, a.Cn, c0, 0, vy);
    if constexpr (XQT < 0) store_f16_tile(lx[0], vx);
    else store_q_tile(lx[0], vx);
    if constexpr (QT < 0) store_f16_tile(ly[0], vy);
    else store_q_tile(ly[0], vy);
    __syncthreads();
    for (uint32_t kt = 0; kt < nk; kt++) {
        const int cur = kt & 1;
        const bool more = kt + 1 < nk;
        if (more) {
            uint32_t k1 = (kt + 1) * KF;
            if constexpr (XQT < 0) load_f16_tile((const _Float16 *)a.X, a.ldx, xt, a.R, r0, a.K, k1, vx);
            else load_q_tile<XQT>((const uint8_t *)a.X, a.ldx, a.R, r0, k1, vx);
            if constexpr (QT < 0) load_f16_tile((const _Float16 *)a.Y, a.ldy, yt, a.Cn, c0, a.K, k1, vy);
            else load_q_tile<QT>((const uint8_t *)a.Y, a.ldy, a.Cn, c0, k1, vy);
        }
        mfma_step_f16(lx[cur], ly[cur], wr, wc, acc);
        if (more) {
            if constexpr (XQT < 0) store_f16_tile(lx[cur ^ 1], vx);
            else store_q_tile(lx[cur ^ 1], vx);
            if constexpr (QT < 0) store_f16_tile(ly[cur ^ 1], vy);
            else store_q_tile(ly[cur ^ 1], vy);
        }
        __syncthreads();
    }
    store_acc_f32(a, r0, c0, wr, wc, acc);
}

VKF_KERNEL void __launch_bounds__(256) vkf_gemm_f16(VkfGemmArgs a) { gemm_f16_body<-1, -1>(a); }
#define VKF_GEMM_Q(name, QT)                                                                        \
    VKF_KERNEL void __launch_bounds__(256) vkf_gemm_##name##_f16(VkfGemmArgs a) { gemm_f16_body<-1, QT>(a); }
#define VKF_GEMM_Q_Q81(name, QT)                                                                    \
    VKF_KERNEL void __launch_bounds__(256) vkf_gemm_##name##_q8_1(VkfGemmArgs a) {                  \
        gemm_f16_body<VKF_Q8_1, QT>(a);                                                             \
    }
VKF_GEMM_Q(q4_0, VKF_Q4_0)
VKF_GEMM_Q(q4_1, VKF_Q4_1)
VKF_GEMM_Q(q8_0, VKF_Q8_0)
VKF_GEMM_Q(q5_0, VKF_Q5_0)
VKF_GEMM_Q(q4_k, VKF_Q4_K)
VKF_GEMM_Q(q5_k, VKF_Q5_K)
VKF_GEMM_Q(q6_k, VKF_Q6_K)
VKF_GEMM_Q_Q81(q4_0, VKF_Q4_0)
VKF_GEMM_Q_Q81(q4_1, VKF_Q4_1)
VKF_GEMM_Q_Q81(q8_0, VKF_Q8_0)
VKF_GEMM_Q_Q81(q5_0, VKF_Q5_0)
VKF_GEMM_Q_Q81(q4_k, VKF_Q4_K)
VKF_GEMM_Q_Q81(q5_k, VKF_Q5_K)

// ---------------------------------------------------------------------------
// int8 x int8 -> int32 (kernels/linear_int8.glsl:54-93, with int8 A).
// Tiles 128 x 64 int8, LDS pitch 80 B.  flags & VKF_GF_D_F32 selects the
// float epilogue with fp32 D; VKF_GF_D_I32 stores the raw int32 accumulator.
// ---------------------------------------------------------------------------
#define KI 64
#define PI 80

__device__ __forceinline__ void load_i8_tile(const int8_t *P, uint64_t ld, bool trans, uint32_t nrows, uint32_t row0,
                                             uint32_t K, uint32_t k0, vkf_i4 v[2]) {
#pragma unroll
    for (int i = 0; i < 2; i++) {
        int idx = threadIdx.x + 256 * i;
        uint32_t r = row0 + (idx >> 2), k = k0 + 16 * (idx & 3);
        vkf_i4 t = {0, 0, 0, 0};
        if (r < nrows) {
            if (!trans && k + 16 <= K && ((ld & 15) == 0) && (((uintptr_t)P & 15) == 0)) {
                t = *(const vkf_i4 *)(P + (uint64_t)r * ld + k);
            } else {
                uint8_t bytes[16];
#pragma unroll
                for (int j = 0; j < 16; j++)
                    bytes[j] = (k + j < K) ? (uint8_t)(trans ? P[(uint64_t)(k + j) * ld + r] : P[(uint64_t)r * ld + k + j]) : 0;
#pragma unroll
                for (int j = 0; j < 4; j++)
                    t[j] = (int)((uint32_t)bytes[4 * j] | ((uint32_t)bytes[4 * j + 1] << 8) |
                                 ((uint32_t)bytes[4 * j + 2] << 16) | ((uint32_t)bytes[4 * j + 3] << 24));
            }
        }
        v[i] = t;
    }
}

__device__ __forceinline__ void store_i8_tile(int8_t *lds, const vkf_i4 v[2]) {
#pragma unroll
    for (int i = 0; i < 2; i++) {
        int idx = threadIdx.x + 256 * i;
        *(vkf_i4 *)(lds + (idx >> 2) * PI + 16 * (idx & 3)) = v[i];
    }
}

VKF_KERNEL void __launch_bounds__(256) vkf_gemm_i8(VkfGemmArgs a) {
    __shared__ __attribute__((aligned(16))) int8_t lx[2][BM * PI];
    __shared__ __attribute__((aligned(16))) int8_t ly[2][BN * PI];
    const uint32_t r0 = blockIdx.y * BM, c0 = blockIdx.x * BN;
    const int wave = threadIdx.x >> 6, wr = wave >> 1, wc = wave & 1;
    const int lane = threadIdx.x & 63, li = lane & 15, lg = lane >> 4;
    const bool xt = a.flags & VKF_GF_X_TRANS, yt = a.flags & VKF_GF_Y_TRANS;
    vkf_i4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = vkf_i4{0, 0, 0, 0};
    const uint32_t nk = (a.K + KI - 1) / KI;
    vkf_i4 vx[2], vy[2];
    load_i8_tile((const int8_t *)a.X, a.ldx, xt, a.R, r0, a.K, 0, vx);
    load_i8_tile((const int8_t *)a.Y, a.ldy, yt, a.Cn, c0, a.K, 0, vy);
    store_i8_tile(lx[0], vx);
    store_i8_tile(ly[0], vy);
    __syncthreads();
    for (uint32_t kt = 0; kt < nk; kt++) {
        const int cur = kt & 1;
        const bool more = kt + 1 < nk;
        if (more) {
            load_i8_tile((const int8_t *)a.X, a.ldx, xt, a.R, r0, a.K, (kt + 1) * KI, vx);
            load_i8_tile((const int8_t *)a.Y, a.ldy, yt, a.Cn, c0, a.K, (kt + 1) * KI, vy);
        }
        vkf_i4 fa[4], fb[4];
#pragma unroll
        for (int i = 0; i < 4; i++) fa[i] = *(const vkf_i4 *)(lx[cur] + (wr * 64 + 16 * i + li) * PI + 16 * lg);
#pragma unroll
        for (int j = 0; j < 4; j++) fb[j] = *(const vkf_i4 *)(ly[cur] + (wc * 64 + 16 * j + li) * PI + 16 * lg);
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int j = 0; j < 4; j++) acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fa[i], fb[j], acc[i][j], 0, 0, 0);
        if (more) {
            store_i8_tile(lx[cur ^ 1], vx);
            store_i8_tile(ly[cur ^ 1], vy);
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                uint32_t r = r0 + wr * 64 + 16 * i + 4 * lg + e, c = c0 + wc * 64 + 16 * j + li;
                if (r < a.R && c < a.Cn) {
                    if (a.flags & VKF_GF_D_I32) {
                        int32_t *dp = (int32_t *)a.D + (uint64_t)r * a.ldd + c;
                        int32_t v = acc[i][j][e];
                        // integer alpha/beta (hipblasGemmEx with compute 32I)
                        if (a.alpha != 1.0f || a.beta != 0.0f) {
                            int32_t al = (int32_t)a.alpha, be = (int32_t)a.beta;
                            v = al * v + (be ? be * ((const int32_t *)a.Cin)[(uint64_t)r * a.ldc + c] : 0);
                        }
                        *dp = v;
                    } else {
                        epi_store(a, r, c, (float)acc[i][j][e]);
                    }
                }
            }
}

// ---------------------------------------------------------------------------
// Q6_K weights x Q8_1 activations, M >= 17.
// X: Q8_1 rows (ldx bytes per row), Y: Q6_K rows (ldy bytes per row).
// Per 32-deep step kb: LDS X = q8 (fp16, exact), Y = sc*(q6-32) (fp16,
// exact, |.| <= 4096); one MFMA chain from zero gives P exactly (|P| < 2^24);
//   accs += dx[m, kb] * P;  at each 256 boundary: acc += dw[n, sb] * accs.
// ---------------------------------------------------------------------------
VKF_KERNEL void __launch_bounds__(256) vkf_gemm_q6_k_q8_1_int(VkfGemmArgs a) {
    __shared__ __attribute__((aligned(16))) _Float16 lx[2][BM * PF];
    __shared__ __attribute__((aligned(16))) _Float16 ly[2][BN * PF];
    __shared__ float ldx[2][BM];
    __shared__ float ldw[2][BN];
    const uint32_t r0 = blockIdx.y * BM, c0 = blockIdx.x * BN;
    const int wave = threadIdx.x >> 6, wr = wave >> 1, wc = wave & 1;
    const int lane = threadIdx.x & 63, li = lane & 15, lg = lane >> 4;
    const uint8_t *X = (const uint8_t *)a.X, *Y = (const uint8_t *)a.Y;
    vkf_f4 acc[4][4], accs[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = accs[i][j] = vkf_f4{0, 0, 0, 0};
    const uint32_t nk = a.K / 32;

    // thread t: X row t/2 (16 q8 values), Y row t/2 (16 weights)
    const int trow = threadIdx.x >> 1, th = threadIdx.x & 1;
    auto load = [&](uint32_t kb, vkf_h8 vx[2], vkf_h8 vy[2], float &dx, float &dw) {
        uint32_t r = r0 + trow;
        vx[0] = vx[1] = vkf_h8{};
        dx = 0.0f;
        if (r < a.R) {
            const uint8_t *xb = X + (uint64_t)r * a.ldx + 36ull * kb;
            dx = vkf_h2f(ld_u16(xb));
#pragma unroll
            for (int i = 0; i < 2; i++) {
                uint32_t w0 = ld_u32(xb + 4 + 16 * th + 8 * i), w1 = ld_u32(xb + 8 + 16 * th + 8 * i);
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    vx[i][j] = (_Float16)(int8_t)(w0 >> (8 * j));
                    vx[i][4 + j] = (_Float16)(int8_t)(w1 >> (8 * j));
                }
            }
        }
        uint32_t c = c0 + trow;
        vy[0] = vy[1] = vkf_h8{};
        dw = 0.0f;
        if (c < a.Cn) {
            uint32_t sb = kb >> 3, j8 = kb & 7, ip = j8 >> 2, t = j8 & 3;
            const uint8_t *b = Y + (uint64_t)c * a.ldy + 210ull * sb;
            dw = vkf_h2f(ld_u16(b + 208));
            int sc = (int)(int8_t)b[192 + 8 * ip + 2 * t + th];
            const uint8_t *ql = b + 64 * ip + 32 * (t & 1) + 16 * th;
            const uint8_t *qh = b + 128 + 32 * ip + 16 * th;
            uint32_t sh = (t >> 1) * 4, hs = 2 * t;
#pragma unroll
            for (int i = 0; i < 2; i++) {
#pragma unroll
                for (int q = 0; q < 2; q++) {
                    uint32_t lo = ld_u32_a2(ql + 8 * i + 4 * q), hi = ld_u32_a2(qh + 8 * i + 4 * q);
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        int v = (int)(((lo >> (8 * j + sh)) & 0xfu) | (((hi >> (8 * j + hs)) & 3u) << 4)) - 32;
                        vy[i][4 * q + j] = (_Float16)(sc * v);
                    }
                }
            }
        }
    };
    auto store = [&](int buf, const vkf_h8 vx[2], const vkf_h8 vy[2], float dx, float dw) {
        *(vkf_h8 *)(lx[buf] + trow * PF + 16 * th) = vx[0];
        *(vkf_h8 *)(lx[buf] + trow * PF + 16 * th + 8) = vx[1];
        *(vkf_h8 *)(ly[buf] + trow * PF + 16 * th) = vy[0];
        *(vkf_h8 *)(ly[buf] + trow * PF + 16 * th + 8) = vy[1];
        if (th == 0) { ldx[buf][trow] = dx; ldw[buf][trow] = dw; }
    };
    vkf_h8 vx[2], vy[2];
    float dx, dw;
    load(0, vx, vy, dx, dw);
    store(0, vx, vy, dx, dw);
    __syncthreads();
    for (uint32_t kb = 0; kb < nk; kb++) {
        const int cur = kb & 1;
        const bool more = kb + 1 < nk;
        if (more) load(kb + 1, vx, vy, dx, dw);
        vkf_h8 fa[4], fb[4];
#pragma unroll
        for (int i = 0; i < 4; i++) fa[i] = *(const vkf_h8 *)(lx[cur] + (wr * 64 + 16 * i + li) * PF + 8 * lg);
#pragma unroll
        for (int j = 0; j < 4; j++) fb[j] = *(const vkf_h8 *)(ly[cur] + (wc * 64 + 16 * j + li) * PF + 8 * lg);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            float dxs[4];
#pragma unroll
            for (int e = 0; e < 4; e++) dxs[e] = ldx[cur][wr * 64 + 16 * i + 4 * lg + e];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                vkf_f4 p = __builtin_amdgcn_mfma_f32_16x16x32_f16(fa[i], fb[j], vkf_f4{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
                for (int e = 0; e < 4; e++) accs[i][j][e] = fmaf(dxs[e], p[e], accs[i][j][e]);
            }
        }
        if ((kb & 7) == 7) {  // super-block boundary: apply dw[n, sb]
#pragma unroll
            for (int j = 0; j < 4; j++) {
                float w = ldw[cur][wc * 64 + 16 * j + li];
#pragma unroll
                for (int i = 0; i < 4; i++)
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        acc[i][j][e] = fmaf(w, accs[i][j][e], acc[i][j][e]);
                        accs[i][j][e] = 0.0f;
                    }
            }
        }
        if (more) store(cur ^ 1, vx, vy, dx, dw);
        __syncthreads();
    }
    store_acc_f32(a, r0, c0, wr, wc, acc);
}
