// gemm.hip — prefill GEMM (M >= 17) on the gfx950 matrix cores.
//
// Replaces kernels/linear_fp16.glsl, linear_fp16_fp32out.glsl, linear_coop.glsl
// (one thread or one 16x16 subgroup tile per output, no LDS reuse) and
// kernels/linear_int8.glsl (one thread per output, scalar int MACs).
//
// Core: D[r, c] = epi( sum_k X[r, k] * Y[c, k] ) with both operands
// K-contiguous.  A 256-thread workgroup owns a 128x128 tile of D; each of its
// four waves owns 64x64 = 4x4 MFMA 16x16 sub-tiles.  K advances 128 bytes of
// each operand row per step through two LDS buffers, one barrier per step.
// Main loops (chosen per call, all sharing the tiling and the epilogue):
//   gemm_mainloop_dma   dense, aligned operands: global_load_lds straight
//                       into XOR-swizzled LDS tiles (fp16 and int8)
//   gemm_mainloop_qdma  dense fp16 activations by direct-to-LDS loads x ggml
//                       weight tiles loaded before and decoded after each
//                       step's MFMAs (QStage<format>)
//   gemm_mainloop_qq    Q8_1 activations x ggml weights, both decoded that way
//   gemm_mainloop       anything else (transposed, ragged K, unaligned):
//                       register-staged tiles, padded LDS rows
// Kernels:
//   vkf_gemm_f16        fp16 x fp16 -> fp32 acc, v_mfma_f32_16x16x32_f16
//   vkf_gemm_i8         int8 x int8 -> int32 acc (exact), v_mfma_i32_16x16x64_i8
//   vkf_gemm_<q>_f16    fp16 activations x ggml weights dequantised to the
//                       reference's exact fp32 value, rounded to fp16
//   vkf_gemm_<q>_q8_1   Q8_1 activations as fp16(d*q) x ggml weights as above
//                       (fp32 accumulation; the products of two fp16-rounded
//                       operands are within the float tolerance, not integer
//                       exact)
//
// MFMA 16x16 operand layout used throughout: lane l supplies row (l % 16) of
// A and column (l % 16) of B, with a K slice selected by l / 16; both operands
// use the same K slice map, so the product is independent of the hardware's
// internal K order.  Accumulator: lane l holds D[4*(l/16) + i][l % 16].
#include "vkf_device.h"

// ---------------------------------------------------------------------------
// Pipelined core shared by the fp16, int8 and quantised-weight kernels.
//
// Each K step moves 128 bytes of K per operand row (64 fp16 or 128 int8
// elements) into one of two LDS buffers (row pitch GP = 160 bytes: 16-byte
// fragment reads of 16 consecutive rows spread over the banks).  Step kt+2
// is loaded into registers while step kt is multiplied out of LDS[kt & 1]
// and step kt+1 is written to the other buffer: one barrier per step, 32
// MFMAs per wave between barriers.
// ---------------------------------------------------------------------------
#define GK 128  // bytes of K per step and operand row

typedef unsigned int vkf_u4a4 __attribute__((ext_vector_type(4), aligned(4)));
#define GP 160  // LDS row pitch (bytes)

struct TileRegs {
    vkf_i4 v[4];
};

// Dense operand tile: 128 rows x GK bytes of elements of ES bytes.  Thread t
// covers rows t/8 + 32p (p < 4), bytes 16*(t%8) .. +15 of the step.
template <int ES>
__device__ __forceinline__ void load_dense(const void *P, uint64_t ld, bool trans, bool fast, uint32_t nrows,
                                           uint32_t row0, uint32_t K, uint32_t k0, TileRegs &t) {
    constexpr int EPC = 16 / ES;  // elements per 16-byte piece
    const uint32_t k = k0 + EPC * (threadIdx.x & 7);
#pragma unroll
    for (int p = 0; p < 4; p++) {
        const uint32_t r = row0 + (threadIdx.x >> 3) + 32 * p;
        vkf_i4 v = {0, 0, 0, 0};
        if (r < nrows) {
            if (fast && k + EPC <= K) {
                v = *(const vkf_i4 *)((const uint8_t *)P + ((uint64_t)r * ld + k) * ES);
            } else {
                uint8_t bytes[16];
#pragma unroll
                for (int e = 0; e < EPC; e++) {
                    const uint64_t idx = trans ? (uint64_t)(k + e) * ld + r : (uint64_t)r * ld + k + e;
                    const bool in = k + e < K;
#pragma unroll
                    for (int q = 0; q < ES; q++) bytes[e * ES + q] = in ? ((const uint8_t *)P)[idx * ES + q] : 0;
                }
#pragma unroll
                for (int j = 0; j < 4; j++)
                    v[j] = (int)((uint32_t)bytes[4 * j] | ((uint32_t)bytes[4 * j + 1] << 8) |
                                 ((uint32_t)bytes[4 * j + 2] << 16) | ((uint32_t)bytes[4 * j + 3] << 24));
            }
        }
        t.v[p] = v;
    }
}

// Transposed dense operand (stored [K, rows]: element (r, k) at P + (k*ld +
// r)*ES, e.g. B [K, N] of an NN product): thread t covers rows 4*(t/8) + i
// (i < 4) of the tile and the 16-byte K piece t%8 of the step.  Its EPC
// values of k are loaded along the contiguous row direction (the 4 rows'
// elements of one k in one 4*ES-byte load) and transposed in registers into
// the same 16-byte row pieces the K-contiguous loads produce: fp16 one
// v_perm per output dword, int8 three, fp32 none.  vec: the row pitch and
// base allow those loads; groups of 4 rows that cross the last row, and
// unaligned operands, load element by element.
template <int ES>
__device__ __forceinline__ void load_dense_t(const void *P, uint64_t ld, bool vec, uint32_t nrows, uint32_t row0,
                                             uint32_t K, uint32_t k0, TileRegs &t) {
    constexpr int EPC = 16 / ES;
    const uint32_t kb = k0 + EPC * (threadIdx.x & 7), r = row0 + 4 * (threadIdx.x >> 3);
    const uint8_t *B = (const uint8_t *)P;
    if (vec && r + 4 <= nrows) {
        if constexpr (ES == 2) {
            uint32_t in[8][2];
#pragma unroll
            for (int e = 0; e < 8; e++) {
                if (kb + e < K) {
                    const uint2 v = *(const uint2 *)(B + ((uint64_t)(kb + e) * ld + r) * 2);
                    in[e][0] = v.x;
                    in[e][1] = v.y;
                } else {
                    in[e][0] = in[e][1] = 0;
                }
            }
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int d = 0; d < 4; d++)  // (row i, k 2d) low, (row i, k 2d+1) high
                    t.v[i][d] = (int)__builtin_amdgcn_perm(in[2 * d + 1][i >> 1], in[2 * d][i >> 1],
                                                           (i & 1) ? 0x07060302u : 0x05040100u);
        } else if constexpr (ES == 1) {
            uint32_t in[16];
#pragma unroll
            for (int e = 0; e < 16; e++) in[e] = kb + e < K ? *(const uint32_t *)(B + (uint64_t)(kb + e) * ld + r) : 0u;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                // bytes (row i of in[lo], row i of in[lo + 1]) in the low half
                const uint32_t sel = (uint32_t)i | ((uint32_t)(4 + i) << 8) | 0x0c0c0000u;
#pragma unroll
                for (int d = 0; d < 4; d++) {
                    const uint32_t a = __builtin_amdgcn_perm(in[4 * d + 1], in[4 * d], sel);
                    const uint32_t b = __builtin_amdgcn_perm(in[4 * d + 3], in[4 * d + 2], sel);
                    t.v[i][d] = (int)__builtin_amdgcn_perm(b, a, 0x05040100u);
                }
            }
        } else {
            vkf_i4 in[4];
#pragma unroll
            for (int e = 0; e < 4; e++)
                in[e] = kb + e < K ? *(const vkf_i4 *)(B + ((uint64_t)(kb + e) * ld + r) * 4) : vkf_i4{0, 0, 0, 0};
#pragma unroll
            for (int i = 0; i < 4; i++) t.v[i] = vkf_i4{in[0][i], in[1][i], in[2][i], in[3][i]};
        }
        return;
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        uint8_t bytes[16];
#pragma unroll
        for (int e = 0; e < EPC; e++) {
            const bool in = r + i < nrows && kb + e < K;
            const uint64_t idx = (uint64_t)(kb + e) * ld + r + i;
#pragma unroll
            for (int q = 0; q < ES; q++) bytes[e * ES + q] = in ? B[idx * ES + q] : 0;
        }
#pragma unroll
        for (int j = 0; j < 4; j++)
            t.v[i][j] = (int)((uint32_t)bytes[4 * j] | ((uint32_t)bytes[4 * j + 1] << 8) |
                              ((uint32_t)bytes[4 * j + 2] << 16) | ((uint32_t)bytes[4 * j + 3] << 24));
    }
}

__device__ __forceinline__ void store_dense(uint8_t *lds, const TileRegs &t) {
#pragma unroll
    for (int p = 0; p < 4; p++)
        *(vkf_i4 *)(lds + ((threadIdx.x >> 3) + 32 * p) * GP + 16 * (threadIdx.x & 7)) = t.v[p];
}

// The pieces of load_dense_t: rows 4*(t/8) + p.
__device__ __forceinline__ void store_dense_t(uint8_t *lds, const TileRegs &t) {
#pragma unroll
    for (int p = 0; p < 4; p++) *(vkf_i4 *)(lds + (4 * (threadIdx.x >> 3) + p) * GP + 16 * (threadIdx.x & 7)) = t.v[p];
}

// Quantised operand tile dequantised to fp16: 128 rows x 64 k.  Thread t
// covers row t/2, 32-element chunk k0/32 + (t&1): the reference's exact fp32
// values (decode8) rounded to fp16.  Chunks at or past K are zero.
template <int QT>
__device__ __forceinline__ void load_quant(const uint8_t *W, uint64_t row_bytes, uint32_t nrows, uint32_t row0,
                                           uint32_t K, uint32_t k0, TileRegs &t) {
    constexpr int BB = QTraits<QT>::BB, CPB = QTraits<QT>::BE / 32;
    const uint32_t r = row0 + (threadIdx.x >> 1), kc = k0 + 32 * (threadIdx.x & 1);
#pragma unroll
    for (int g = 0; g < 4; g++) t.v[g] = vkf_i4{0, 0, 0, 0};
    if (r < nrows && kc < K) {
        const uint32_t ch = kc / 32, ib = ch / CPB, sub = ch - ib * CPB;
        const uint8_t *blk = W + (uint64_t)r * row_bytes + (uint64_t)ib * BB;
#pragma unroll
        for (int g = 0; g < 4; g++) {
            float y[8];
            decode8<QT>(blk, sub * 4 + g, y);
            vkf_h8 h;
#pragma unroll
            for (int j = 0; j < 8; j++) h[j] = vkf_to_f16(y[j]);
            t.v[g] = __builtin_bit_cast(vkf_i4, h);
        }
    }
}

__device__ __forceinline__ void store_quant(uint8_t *lds, const TileRegs &t) {
    uint8_t *p = lds + (threadIdx.x >> 1) * GP + 64 * (threadIdx.x & 1);
#pragma unroll
    for (int g = 0; g < 4; g++) *(vkf_i4 *)(p + 16 * g) = t.v[g];
}

// Operand sources: dense fp16 / int8 or quantised blocks (QT >= 0).
template <int ES, int QT>
struct Operand {
    const void *P;
    uint64_t ld;  // elements (dense) or bytes per row (quantised)
    bool trans, fast;  // fast: K-contiguous 16-byte pieces; for trans, load_dense_t's vector loads
    uint32_t nrows, row0, K;
    __device__ __forceinline__ void load(uint32_t kt, TileRegs &t) const {
        if constexpr (QT >= 0) load_quant<QT>((const uint8_t *)P, ld, nrows, row0, K, kt * (GK / 2), t);
        else if (trans) load_dense_t<ES>(P, ld, fast, nrows, row0, K, kt * (GK / ES), t);
        else load_dense<ES>(P, ld, false, fast, nrows, row0, K, kt * (GK / ES), t);
    }
    __device__ __forceinline__ void store(uint8_t *lds, const TileRegs &t) const {
        if constexpr (QT >= 0) store_quant(lds, t);
        else if (trans) store_dense_t(lds, t);
        else store_dense(lds, t);
    }
};

template <int ES, int QT>
__device__ __forceinline__ Operand<ES, QT> make_operand(const void *P, uint64_t ld, bool trans, uint32_t nrows,
                                                        uint32_t row0, uint32_t K) {
    Operand<ES, QT> o;
    o.P = P;
    o.ld = ld;
    o.trans = trans;
    o.fast = trans ? ((ld * ES) % (4 * ES)) == 0 && (((uintptr_t)P % (4 * ES)) == 0)
                   : ((ld * ES) % 16) == 0 && (((uintptr_t)P & 15) == 0);
    o.nrows = nrows;
    o.row0 = row0;
    o.K = K;
    return o;
}

// fp16 operand quantised to int8 while it is staged (the int8 linear of
// kernels/linear_int8.glsl:63-70: q = clamp(round(x / act_scale), -127, 127),
// here round-half-even, v_rndne, and an IEEE division).  Same tile geometry
// as load_dense<1>: thread t covers rows t/8 + 32p, int8 elements
// 16*(t%8) .. +15 of the 128-element step, i.e. 32 bytes of fp16 source.
struct OperandF16Q {
    const _Float16 *P;
    uint64_t ld;  // elements
    bool trans, fast;
    uint32_t nrows, row0, K;
    float s;
    __device__ __forceinline__ static uint32_t q8(float x, float s) {
        const float q = fminf(fmaxf(__builtin_rintf(x / s), -127.0f), 127.0f);
        return (uint32_t)(int32_t)q & 0xffu;
    }
    __device__ __forceinline__ void load(uint32_t kt, TileRegs &t) const {
        const uint32_t k = kt * 128 + 16 * (threadIdx.x & 7);
#pragma unroll
        for (int p = 0; p < 4; p++) {
            const uint32_t r = row0 + (threadIdx.x >> 3) + 32 * p;
            uint32_t w[4] = {0, 0, 0, 0};
            if (r < nrows) {
                float x[16];
                if (fast && k + 16 <= K) {
                    const vkf_h8 h0 = *(const vkf_h8 *)(P + (uint64_t)r * ld + k);
                    const vkf_h8 h1 = *(const vkf_h8 *)(P + (uint64_t)r * ld + k + 8);
#pragma unroll
                    for (int e = 0; e < 8; e++) {
                        x[e] = (float)h0[e];
                        x[8 + e] = (float)h1[e];
                    }
                } else {
#pragma unroll
                    for (int e = 0; e < 16; e++) {
                        const uint64_t idx = trans ? (uint64_t)(k + e) * ld + r : (uint64_t)r * ld + k + e;
                        x[e] = k + e < K ? (float)P[idx] : 0.0f;
                    }
                }
#pragma unroll
                for (int e = 0; e < 16; e++) w[e >> 2] |= q8(x[e], s) << (8 * (e & 3));
            }
            t.v[p] = vkf_i4{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
        }
    }
    __device__ __forceinline__ void store(uint8_t *lds, const TileRegs &t) const { store_dense(lds, t); }
};

// One 16x16 sub-tile product of a fragment pair, 16 bytes of K per lane on
// both operands: one 16x16x32 fp16 MFMA, one 16x16x64 int8 MFMA, or for fp32
// four 16x16x4 MFMAs, the e-th taking element e of each lane's four (K index
// 4*(lane/16) + e of the 16-element slice, the same map on both operands).
template <int ES, class ACC>
__device__ __forceinline__ ACC mfma_frag(vkf_i4 a, vkf_i4 b, ACC c) {
    if constexpr (ES == 2) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(vkf_h8, a), __builtin_bit_cast(vkf_h8, b),
                                                      c, 0, 0, 0);
    } else if constexpr (ES == 1) {
        return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
    } else {
        const vkf_f4 fa = __builtin_bit_cast(vkf_f4, a), fb = __builtin_bit_cast(vkf_f4, b);
#pragma unroll
        for (int e = 0; e < 4; e++) c = __builtin_amdgcn_mfma_f32_16x16x4f32(fa[e], fb[e], c, 0, 0, 0);
        return c;
    }
}

// One K step of the wave's 64x64 tile from LDS: two 16x16x32 fp16 MFMAs or
// two 16x16x64 int8 MFMAs deep per 16x16 sub-tile.
template <int ES, class ACC>
__device__ __forceinline__ void mfma_step(const uint8_t *lx, const uint8_t *ly, int wr, int wc, ACC acc[4][4]) {
    const int lane = threadIdx.x & 63, li = lane & 15, lg = lane >> 4;
    // all 16 fragments first: the second slice's reads overlap the first
    // slice's MFMAs (LDS results return in issue order)
    vkf_i4 fa[2][4], fb[2][4];
#pragma unroll
    for (int s = 0; s < 2; s++) {
#pragma unroll
        for (int i = 0; i < 4; i++)
            fa[s][i] = *(const vkf_i4 *)(lx + (wr * 64 + 16 * i + li) * GP + 64 * s + 16 * lg);
#pragma unroll
        for (int j = 0; j < 4; j++)
            fb[s][j] = *(const vkf_i4 *)(ly + (wc * 64 + 16 * j + li) * GP + 64 * s + 16 * lg);
    }
    // raised issue priority for the MFMA burst: when both waves of a SIMD
    // are ready, this wave's MFMAs go first and the matrix pipe stays fed
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int s = 0; s < 2; s++)
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int j = 0; j < 4; j++) {
                acc[i][j] = mfma_frag<ES>(fa[s][i], fb[s][j], acc[i][j]);
            }
    __builtin_amdgcn_s_setprio(0);
}

// The pipelined K loop: acc += X[r0.., :] . Y[c0.., :]^T.  The loads of the
// next GNS steps are in flight in a ring of register sets while the current
// step is multiplied out of LDS.  smem: GEMM_LDS bytes (two buffers per
// operand).
#define GNS 2
#define GEMM_LDS (4 * 128 * GP)
// 256 threads, at most 256 registers per lane (two waves per SIMD).
#define GEMM_KERNEL VKF_KERNEL void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2)))
template <int ES, class OX, class OY, class ACC>
__device__ __forceinline__ void gemm_mainloop(const OX &ox, const OY &oy, uint32_t K, uint32_t kelem_per_step,
                                              ACC acc[4][4], uint8_t *smem) {
    uint8_t *lx[2] = {smem, smem + 128 * GP}, *ly[2] = {smem + 2 * 128 * GP, smem + 3 * 128 * GP};
    const int wave = threadIdx.x >> 6, wr = wave >> 1, wc = wave & 1;
    const uint32_t nk = (K + kelem_per_step - 1) / kelem_per_step;
    TileRegs rx[GNS], ry[GNS];
#pragma unroll
    for (int u = 0; u < GNS; u++) {
        if ((uint32_t)u < nk) {
            ox.load(u, rx[u]);
            oy.load(u, ry[u]);
        }
    }
    ox.store(lx[0], rx[0]);
    oy.store(ly[0], ry[0]);
    if (GNS < nk) {
        ox.load(GNS, rx[0]);
        oy.load(GNS, ry[0]);
    }
    __syncthreads();
    for (uint32_t kt0 = 0; kt0 < nk; kt0 += GNS) {
#pragma unroll
        for (int u = 0; u < GNS; u++) {  // GNS even: LDS parity = u & 1
            const uint32_t kt = kt0 + u;
            if (kt < nk) {
                mfma_step<ES>(lx[u & 1], ly[u & 1], wr, wc, acc);
                const int nslot = (u + 1) % GNS;
                if (kt + 1 < nk) {
                    ox.store(lx[(u + 1) & 1], rx[nslot]);
                    oy.store(ly[(u + 1) & 1], ry[nslot]);
                }
                if (kt + 1 + GNS < nk) {
                    ox.load(kt + 1 + GNS, rx[nslot]);
                    oy.load(kt + 1 + GNS, ry[nslot]);
                }
                __syncthreads();
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Direct-to-LDS pipeline for dense operands that are K-contiguous, 16-byte
// aligned rows, with K*ES a multiple of 128 (the common case; everything
// else takes gemm_mainloop).  global_load_lds_dwordx4 writes each lane's 16
// bytes straight into LDS (slot = lane), so no registers stage the tiles:
// the next step loads while this one is multiplied.  Tile layout per stage and operand: 128
// rows x 128 bytes, 16-byte chunk c of row r at r*128 + ((c ^ (r & 7)) * 16)
// (the XOR spreads the 16 rows of a fragment read over all banks); a load
// instruction covers 8 rows x 8 chunks, lane L taking chunk (L%8) ^ (row&7)
// of row L/8 so that its slot lands on that position.
// ---------------------------------------------------------------------------
#define GNST 2
// two stages (64 KiB) or the epilogue's fp32 tile (128 x 132 floats), the
// larger; two workgroups fit a CU (measured faster than three or four stages
// with one workgroup per CU)
#define GEMM_LDS_DMA (GNST * 32768 > 128 * 132 * 4 ? GNST * 32768 : 128 * 132 * 4)
#define GEMM_LDS_BOTH (GEMM_LDS_DMA > GEMM_LDS ? GEMM_LDS_DMA : GEMM_LDS)

template <int N>
__device__ __forceinline__ void wait_vm() {
    if constexpr (N == 0) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    else if constexpr (N == 8) asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
    else if constexpr (N == 16) asm volatile("s_waitcnt vmcnt(16)" ::: "memory");
    else asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

__device__ __forceinline__ bool dma_ok(const void *P, uint64_t ld, bool trans, uint32_t K, int ES) {
    return !trans && ((ld * ES) % 16) == 0 && (((uintptr_t)P & 15) == 0) && ((uint64_t)K * ES) % 128 == 0;
}

// One step (128 bytes of K) of the wave's 64x64 tile from swizzled LDS tiles.
// PRIO false: no priority raise around the MFMAs (steps whose MFMAs are
// interleaved with other work by sched_group_barrier hints)
template <int ES, class ACC, bool PRIO = true>
__device__ __forceinline__ void mfma_step_swz(const uint8_t *lx, const uint8_t *ly, int wr, int wc, ACC acc[4][4]) {
    const int lane = threadIdx.x & 63, li = lane & 15, lg = lane >> 4, sw = li & 7;
    vkf_i4 fa[2][4], fb[2][4];
#pragma unroll
    for (int s = 0; s < 2; s++) {
        const int c = 4 * s + lg;
#pragma unroll
        for (int i = 0; i < 4; i++)
            fa[s][i] = *(const vkf_i4 *)(lx + (wr * 64 + 16 * i + li) * 128 + ((c ^ sw) << 4));
#pragma unroll
        for (int j = 0; j < 4; j++)
            fb[s][j] = *(const vkf_i4 *)(ly + (wc * 64 + 16 * j + li) * 128 + ((c ^ sw) << 4));
    }
    // raised issue priority for the MFMA burst: when both waves of a SIMD
    // are ready, this wave's MFMAs go first and the matrix pipe stays fed
    if constexpr (PRIO) __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int s = 0; s < 2; s++)
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int j = 0; j < 4; j++) {
                acc[i][j] = mfma_frag<ES>(fa[s][i], fb[s][j], acc[i][j]);
            }
    if constexpr (PRIO) __builtin_amdgcn_s_setprio(0);
}

template <int ES, class ACC>
__device__ __forceinline__ void gemm_mainloop_dma(const VkfGemmArgs &a, uint32_t r0, uint32_t c0, ACC acc[4][4],
                                                  uint8_t *smem) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, wr = wave >> 1, wc = wave & 1;
    const uint32_t nk = (uint32_t)(((uint64_t)a.K * ES) / 128);
    const uint8_t *gx[4], *gy[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const uint32_t rr = (4 * wave + j) * 8 + (lane >> 3);
        const uint32_t ch = (lane & 7) ^ (rr & 7);
        const uint32_t rx = r0 + rr < a.R ? r0 + rr : a.R - 1;  // rows past the edge: any valid row
        const uint32_t ry = c0 + rr < a.Cn ? c0 + rr : a.Cn - 1;
        gx[j] = (const uint8_t *)a.X + (uint64_t)rx * a.ldx * ES + ch * 16;
        gy[j] = (const uint8_t *)a.Y + (uint64_t)ry * a.ldy * ES + ch * 16;
    }
    auto issue = [&](uint32_t kt, uint32_t stage) {
        uint8_t *sx = smem + stage * 32768, *sy = sx + 16384;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t off = (4 * wave + j) * 8 * 128;
            vkf_load_lds16(gx[j] + (uint64_t)kt * 128, sx + off);
            vkf_load_lds16(gy[j] + (uint64_t)kt * 128, sy + off);
        }
    };
#pragma unroll
    for (uint32_t s = 0; s + 1 < GNST; s++)
        if (s < nk) issue(s, s);
    for (uint32_t kt = 0; kt < nk; kt++) {
        // this thread's loads of step kt are done when at most the loads of
        // the (up to GNST-2) later steps are outstanding
        if (kt + GNST - 2 < nk) wait_vm<8 * (GNST - 2)>();
        else wait_vm<0>();
        __syncthreads();
        if (kt + GNST - 1 < nk) issue(kt + GNST - 1, (kt + GNST - 1) % GNST);
        const uint8_t *lx = smem + (kt % GNST) * 32768;
        mfma_step_swz<ES>(lx, lx + 16384, wr, wc, acc);
    }
    __syncthreads();  // LDS free for the epilogue
}

// ---------------------------------------------------------------------------
// Quantised-weight GEMM with dense fp16 activations: X by direct-to-LDS
// loads, the weight tile staged through registers.  Each 64-k step, thread
// t owns weight row t/2 and its 32-element chunk (t&1): QStage<QT>::load
// issues the chunk's global loads (before the MFMAs of the current step),
// ::decode turns them into the reference's exact fp32 values rounded to
// fp16 (after the MFMAs, so the load latency hides under them), and the
// tile is written to LDS in the same XOR-swizzled layout as X.
// ---------------------------------------------------------------------------
template <int QT>
struct QStage {  // any format: decode8 on the spot (load waits for its data)
    TileRegs t;
    __device__ __forceinline__ void load(const uint8_t *W, uint64_t row_bytes, uint32_t nrows, uint32_t row0,
                                         uint32_t K, uint32_t k0) {
        load_quant<QT>(W, row_bytes, nrows, row0, K, k0, t);
    }
    __device__ __forceinline__ void decode(TileRegs &out) { out = t; }
};

// Q4_K: one 32-element chunk = sub-block j of a super-block: header (dall,
// dmin, 6-bit scales) + the 32 qs bytes of the sub-block pair, nibble j&1
// (kernels/dequant_q4_k.glsl:16-24, 49-57).  Value = fma(dall*sc, q, -dmin*m)
// in fp32 (dall*sc and its product with q are exact, so this is the
// reference's single rounding), then fp16 round-to-nearest-even.
template <>
struct QStage<VKF_Q4_K> {
    vkf_u4 hdr, qa, qb;
    uint32_t j;
    bool live;
    __device__ __forceinline__ void load(const uint8_t *W, uint64_t row_bytes, uint32_t nrows, uint32_t row0,
                                         uint32_t K, uint32_t k0) {
        const uint32_t r = row0 + (threadIdx.x >> 1), kc = k0 + 32 * (threadIdx.x & 1);
        live = r < nrows && kc < K;
        const uint32_t rr = r < nrows ? r : nrows - 1, kk = kc < K ? kc : 0;
        const uint8_t *blk = W + (uint64_t)rr * row_bytes + 144ull * (kk / 256);
        j = (kk % 256) / 32;
        hdr = *(const vkf_u4 *)blk;
        const uint8_t *q = blk + 16 + 32 * (j >> 1);
        qa = *(const vkf_u4 *)q;
        qb = *(const vkf_u4 *)(q + 16);
    }
    __device__ __forceinline__ void decode(TileRegs &out) {
        const float dall = vkf_h2f(hdr[0] & 0xffffu), dmin = vkf_h2f(hdr[0] >> 16);
        const uint32_t s0 = hdr[1], s4 = hdr[2], s8 = hdr[3];
        const uint32_t scW = j < 4 ? (s0 & 0x3f3f3f3fu) : ((s8 & 0x0f0f0f0fu) | ((s0 >> 2) & 0x30303030u));
        const uint32_t mnW = j < 4 ? (s4 & 0x3f3f3f3fu) : (((s8 >> 4) & 0x0f0f0f0fu) | ((s4 >> 2) & 0x30303030u));
        const uint32_t sh = 8 * (j & 3);
        const float dsc = dall * (float)((scW >> sh) & 0xffu), dm = dmin * (float)((mnW >> sh) & 0xffu);
        const uint32_t nsh = 4 * (j & 1);
        uint32_t w[8] = {qa[0], qa[1], qa[2], qa[3], qb[0], qb[1], qb[2], qb[3]};
#pragma unroll
        for (int g = 0; g < 4; g++) {
            vkf_h8 h;
#pragma unroll
            for (int e = 0; e < 2; e++) {
                uint32_t n = (w[2 * g + e] >> nsh) & 0x0f0f0f0fu;
                // n in a register of its own: each code then converts with one
                // v_cvt_f32_ubyte<k> instead of a bit-field extract and a convert
                asm volatile("" : "+v"(n));
#pragma unroll
                for (int k = 0; k < 4; k++)
                    h[4 * e + k] = vkf_to_f16(fmaf(dsc, (float)((n >> (8 * k)) & 0xffu), -dm));
            }
            out.v[g] = live ? __builtin_bit_cast(vkf_i4, h) : vkf_i4{0, 0, 0, 0};
        }
    }
};

// Q5_K: as Q4_K with the fifth bit of element l of sub-block j in qh[l], bit
// j (kernels/dequant_q5_k.glsl:51-73; 176-byte super-blocks: header, qh[32]
// at 16, qs[128] at 48).  Value fma(dall*sc, q, -dmin*m) in fp32 (exact up to
// the one rounding), then fp16.
template <>
struct QStage<VKF_Q5_K> {
    vkf_u4 hdr, qa, qb, ha, hb;
    uint32_t j;
    bool live;
    __device__ __forceinline__ void load(const uint8_t *W, uint64_t row_bytes, uint32_t nrows, uint32_t row0,
                                         uint32_t K, uint32_t k0) {
        const uint32_t r = row0 + (threadIdx.x >> 1), kc = k0 + 32 * (threadIdx.x & 1);
        live = r < nrows && kc < K;
        const uint32_t rr = r < nrows ? r : nrows - 1, kk = kc < K ? kc : 0;
        const uint8_t *blk = W + (uint64_t)rr * row_bytes + 176ull * (kk / 256);
        j = (kk % 256) / 32;
        hdr = *(const vkf_u4a4 *)blk;
        ha = *(const vkf_u4a4 *)(blk + 16);
        hb = *(const vkf_u4a4 *)(blk + 32);
        const uint8_t *q = blk + 48 + 32 * (j >> 1);
        qa = *(const vkf_u4a4 *)q;
        qb = *(const vkf_u4a4 *)(q + 16);
    }
    __device__ __forceinline__ void decode(TileRegs &out) {
        const float dall = vkf_h2f(hdr[0] & 0xffffu), dmin = vkf_h2f(hdr[0] >> 16);
        const uint32_t s0 = hdr[1], s4 = hdr[2], s8 = hdr[3];
        const uint32_t scW = j < 4 ? (s0 & 0x3f3f3f3fu) : ((s8 & 0x0f0f0f0fu) | ((s0 >> 2) & 0x30303030u));
        const uint32_t mnW = j < 4 ? (s4 & 0x3f3f3f3fu) : (((s8 >> 4) & 0x0f0f0f0fu) | ((s4 >> 2) & 0x30303030u));
        const uint32_t sh = 8 * (j & 3);
        const float dsc = dall * (float)((scW >> sh) & 0xffu), dm = dmin * (float)((mnW >> sh) & 0xffu);
        const uint32_t nsh = 4 * (j & 1);
        const uint32_t w[8] = {qa[0], qa[1], qa[2], qa[3], qb[0], qb[1], qb[2], qb[3]};
        const uint32_t hq[8] = {ha[0], ha[1], ha[2], ha[3], hb[0], hb[1], hb[2], hb[3]};
#pragma unroll
        for (int g = 0; g < 4; g++) {
            vkf_h8 h;
#pragma unroll
            for (int e = 0; e < 2; e++) {
                const uint32_t n = ((w[2 * g + e] >> nsh) & 0x0f0f0f0fu) | (((hq[2 * g + e] >> j) & 0x01010101u) << 4);
#pragma unroll
                for (int k = 0; k < 4; k++)
                    h[4 * e + k] = vkf_to_f16(fmaf(dsc, (float)((n >> (8 * k)) & 0xffu), -dm));
            }
            out.v[g] = live ? __builtin_bit_cast(vkf_i4, h) : vkf_i4{0, 0, 0, 0};
        }
    }
};

// 32-element blocks at 2-byte aligned addresses (Q4_0 18 B, Q8_0 34 B): the
// block's bytes are loaded as the 4-byte aligned dwords that cover them and
// realigned by sh = block address & 3 (0 or 2); no load reaches past the
// block's last byte.
__device__ __forceinline__ uint32_t realign(uint32_t lo, uint32_t hi, uint32_t sh) {
    return __builtin_amdgcn_alignbyte(hi, lo, sh);
}

// Q4_0: value d*q + (-8d) (kernels/dequant_q4_0.glsl:30-35; d*q exact).
template <>
struct QStage<VKF_Q4_0> {
    uint32_t r[5], sh;
    bool live;
    __device__ __forceinline__ void load(const uint8_t *W, uint64_t row_bytes, uint32_t nrows, uint32_t row0,
                                         uint32_t K, uint32_t k0) {
        const uint32_t rw = row0 + (threadIdx.x >> 1), kc = k0 + 32 * (threadIdx.x & 1);
        live = rw < nrows && kc < K;
        const uint8_t *blk = W + (uint64_t)(rw < nrows ? rw : nrows - 1) * row_bytes + 18ull * ((kc < K ? kc : 0) / 32);
        sh = (uint32_t)(uintptr_t)blk & 3u;
        const uint8_t *a = blk - sh;
        const vkf_u4 v = *(const vkf_u4a4 *)a;
        r[0] = v[0]; r[1] = v[1]; r[2] = v[2]; r[3] = v[3];
        r[4] = sh ? *(const uint32_t *)(a + 16) : (uint32_t)*(const uint16_t *)(blk + 16);
    }
    __device__ __forceinline__ void decode(TileRegs &out) {
        // d at bytes sh..sh+1, qs at sh+2 .. sh+17
        const float d = vkf_h2f((uint16_t)(realign(r[0], r[1], sh) & 0xffffu)), dm = -8.0f * d;
        uint32_t q[4];
#pragma unroll
        for (int i = 0; i < 4; i++) q[i] = sh ? r[i + 1] : realign(r[i], r[i + 1], 2);
#pragma unroll
        for (int g = 0; g < 4; g++) {  // elements 8g .. 8g+7
            vkf_h8 h;
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const int el = 8 * g + e, byte = el & 15;
                const uint32_t nib = (q[byte >> 2] >> (8 * (byte & 3) + 4 * (el >> 4))) & 0xfu;
                h[e] = vkf_to_f16(fmaf(d, (float)nib, dm));
            }
            out.v[g] = live ? __builtin_bit_cast(vkf_i4, h) : vkf_i4{0, 0, 0, 0};
        }
    }
};

// Q4_1: value d*q + m (kernels/dequant_q4_1.glsl; 20-byte blocks are 4-byte
// aligned).
template <>
struct QStage<VKF_Q4_1> {
    uint32_t r[5];
    bool live;
    __device__ __forceinline__ void load(const uint8_t *W, uint64_t row_bytes, uint32_t nrows, uint32_t row0,
                                         uint32_t K, uint32_t k0) {
        const uint32_t rw = row0 + (threadIdx.x >> 1), kc = k0 + 32 * (threadIdx.x & 1);
        live = rw < nrows && kc < K;
        const uint8_t *blk = W + (uint64_t)(rw < nrows ? rw : nrows - 1) * row_bytes + 20ull * ((kc < K ? kc : 0) / 32);
        const vkf_u4 v = *(const vkf_u4a4 *)blk;
        r[0] = v[0]; r[1] = v[1]; r[2] = v[2]; r[3] = v[3];
        r[4] = *(const uint32_t *)(blk + 16);
    }
    __device__ __forceinline__ void decode(TileRegs &out) {
        const float d = vkf_h2f((uint16_t)(r[0] & 0xffffu)), m = vkf_h2f((uint16_t)(r[0] >> 16));
#pragma unroll
        for (int g = 0; g < 4; g++) {
            vkf_h8 h;
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const int el = 8 * g + e, byte = el & 15;
                const uint32_t nib = (r[1 + (byte >> 2)] >> (8 * (byte & 3) + 4 * (el >> 4))) & 0xfu;
                h[e] = vkf_to_f16(fmaf(d, (float)nib, m));
            }
            out.v[g] = live ? __builtin_bit_cast(vkf_i4, h) : vkf_i4{0, 0, 0, 0};
        }
    }
};

// Q8_0: value d*q (exact), 34-byte blocks.
template <>
struct QStage<VKF_Q8_0> {
    uint32_t r[9], sh;
    bool live;
    __device__ __forceinline__ void load(const uint8_t *W, uint64_t row_bytes, uint32_t nrows, uint32_t row0,
                                         uint32_t K, uint32_t k0) {
        const uint32_t rw = row0 + (threadIdx.x >> 1), kc = k0 + 32 * (threadIdx.x & 1);
        live = rw < nrows && kc < K;
        const uint8_t *blk = W + (uint64_t)(rw < nrows ? rw : nrows - 1) * row_bytes + 34ull * ((kc < K ? kc : 0) / 32);
        sh = (uint32_t)(uintptr_t)blk & 3u;
        const uint8_t *a = blk - sh;
        const vkf_u4 v0 = *(const vkf_u4a4 *)a, v1 = *(const vkf_u4a4 *)(a + 16);
        r[0] = v0[0]; r[1] = v0[1]; r[2] = v0[2]; r[3] = v0[3];
        r[4] = v1[0]; r[5] = v1[1]; r[6] = v1[2]; r[7] = v1[3];
        r[8] = sh ? *(const uint32_t *)(a + 32) : (uint32_t)*(const uint16_t *)(blk + 32);
    }
    __device__ __forceinline__ void decode(TileRegs &out) {
        const float d = vkf_h2f((uint16_t)(realign(r[0], r[1], sh) & 0xffffu));
#pragma unroll
        for (int g = 0; g < 4; g++) {
            vkf_h8 h;
#pragma unroll
            for (int e2 = 0; e2 < 2; e2++) {
                const int i = 2 * g + e2;  // qs dword i = bytes sh+2+4i ..
                const uint32_t q = sh ? r[i + 1] : realign(r[i], r[i + 1], 2);
#pragma unroll
                for (int k = 0; k < 4; k++) h[4 * e2 + k] = vkf_to_f16(d * (float)(int8_t)(q >> (8 * k)));
            }
            out.v[g] = live ? __builtin_bit_cast(vkf_i4, h) : vkf_i4{0, 0, 0, 0};
        }
    }
};

// Q8_1 activation blocks (36 bytes, 4-byte aligned: fp16 d, fp16 s, int8
// q[32]) as an fp16 operand: fp16(d*q), the RNE of the exact product.
template <>
struct QStage<VKF_Q8_1> {
    uint32_t r[9];
    bool live;
    __device__ __forceinline__ void load(const uint8_t *W, uint64_t row_bytes, uint32_t nrows, uint32_t row0,
                                         uint32_t K, uint32_t k0) {
        const uint32_t rw = row0 + (threadIdx.x >> 1), kc = k0 + 32 * (threadIdx.x & 1);
        live = rw < nrows && kc < K;
        const uint8_t *blk = W + (uint64_t)(rw < nrows ? rw : nrows - 1) * row_bytes + 36ull * ((kc < K ? kc : 0) / 32);
        const vkf_u4 v0 = *(const vkf_u4a4 *)blk, v1 = *(const vkf_u4a4 *)(blk + 16);
        r[0] = v0[0]; r[1] = v0[1]; r[2] = v0[2]; r[3] = v0[3];
        r[4] = v1[0]; r[5] = v1[1]; r[6] = v1[2]; r[7] = v1[3];
        r[8] = *(const uint32_t *)(blk + 32);
    }
    __device__ __forceinline__ void decode(TileRegs &out) {
        const float d = vkf_h2f((uint16_t)(r[0] & 0xffffu));
#pragma unroll
        for (int g = 0; g < 4; g++) {
            vkf_h8 h;
#pragma unroll
            for (int e2 = 0; e2 < 2; e2++) {
                const uint32_t q = r[1 + 2 * g + e2];
#pragma unroll
                for (int k = 0; k < 4; k++) h[4 * e2 + k] = vkf_to_f16(d * (float)(int8_t)(q >> (8 * k)));
            }
            out.v[g] = live ? __builtin_bit_cast(vkf_i4, h) : vkf_i4{0, 0, 0, 0};
        }
    }
};

// Q6_K: 32-element block t of half ip of a 210-byte super-block
// (kernels/dequant_q6_k.glsl:34-58): u = low or high nibble of
// ql[64ip + 32(t&1) + l] | bits 2t, 2t+1 of qh[32ip + l] << 4, value
// d * sc * (u - 32) with sc = scales[8ip + 2t + l/16] (exact in fp32; the
// fma below forms it without rounding), then fp16.  Fields are 2-byte
// aligned: loaded as covering dwords and realigned, scales and d as 2-byte
// loads, nothing past the super-block.
template <>
struct QStage<VKF_Q6_K> {
    uint32_t ql[9], qh[9], sc, dd, sh, t;
    bool live;
    __device__ __forceinline__ void load(const uint8_t *W, uint64_t row_bytes, uint32_t nrows, uint32_t row0,
                                         uint32_t K, uint32_t k0) {
        const uint32_t rw = row0 + (threadIdx.x >> 1), kc = k0 + 32 * (threadIdx.x & 1);
        live = rw < nrows && kc < K;
        const uint32_t kk = kc < K ? kc : 0, j8 = (kk % 256) / 32, ip = j8 >> 2;
        t = j8 & 3;
        const uint8_t *blk = W + (uint64_t)(rw < nrows ? rw : nrows - 1) * row_bytes + 210ull * (kk / 256);
        sh = (uint32_t)(uintptr_t)blk & 3u;
        const uint8_t *a = blk - sh;  // 4-byte aligned
        const uint8_t *pl = a + 64 * ip + 32 * (t & 1), *ph = a + 128 + 32 * ip;
        const vkf_u4 l0 = *(const vkf_u4a4 *)pl, l1 = *(const vkf_u4a4 *)(pl + 16);
        const vkf_u4 h0 = *(const vkf_u4a4 *)ph, h1 = *(const vkf_u4a4 *)(ph + 16);
        ql[0] = l0[0]; ql[1] = l0[1]; ql[2] = l0[2]; ql[3] = l0[3];
        ql[4] = l1[0]; ql[5] = l1[1]; ql[6] = l1[2]; ql[7] = l1[3];
        qh[0] = h0[0]; qh[1] = h0[1]; qh[2] = h0[2]; qh[3] = h0[3];
        qh[4] = h1[0]; qh[5] = h1[1]; qh[6] = h1[2]; qh[7] = h1[3];
        // the dword after each field: inside the super-block (ql ends at
        // byte <= 132, qh at <= 196); only needed when sh = 2
        ql[8] = *(const uint32_t *)(pl + 32);
        qh[8] = *(const uint32_t *)(ph + 32);
        sc = *(const uint16_t *)(blk + 192 + 8 * ip + 2 * t);
        dd = *(const uint16_t *)(blk + 208);
    }
    __device__ __forceinline__ void decode(TileRegs &out) {
        const float d = vkf_h2f((uint16_t)dd);
        const float ds0 = d * (float)(int8_t)(sc & 0xffu), ds1 = d * (float)(int8_t)(sc >> 8);
        const uint32_t nsh = 4 * (t >> 1), hsh = 2 * t;
#pragma unroll
        for (int g = 0; g < 4; g++) {
            const float ds = g < 2 ? ds0 : ds1, off = -32.0f * ds;
            vkf_h8 h;
#pragma unroll
            for (int e2 = 0; e2 < 2; e2++) {
                const int i = 2 * g + e2;
                const uint32_t l = realign(ql[i], ql[i + 1], sh), hb = realign(qh[i], qh[i + 1], sh);
                const uint32_t u = ((l >> nsh) & 0x0f0f0f0fu) | (((hb >> hsh) & 0x03030303u) << 4);
#pragma unroll
                for (int k = 0; k < 4; k++) h[4 * e2 + k] = vkf_to_f16(fmaf(ds, (float)((u >> (8 * k)) & 0xffu), off));
            }
            out.v[g] = live ? __builtin_bit_cast(vkf_i4, h) : vkf_i4{0, 0, 0, 0};
        }
    }
};

// Half-chunk weight decoders for the 512-thread wide GEMM: thread t decodes
// 16 elements -- row t/4 of the 128-row tile, elements 16*(t&3) .. +15 of
// the 64-k step -- so that all eight waves share the decode.  Same values,
// bit for bit, as the 32-element QStage decoders above.
template <int QT>
struct QHalf;

// Q4_K: half h of sub-block j: qs bytes 16 + 32(j/2) + 16h .. +15, nibble j&1.
template <>
struct QHalf<VKF_Q4_K> {
    vkf_u4 hdr, qs;
    uint32_t j;
    bool live;
    __device__ __forceinline__ void load(const uint8_t *W, uint64_t row_bytes, uint32_t nrows, uint32_t row0,
                                         uint32_t K, uint32_t k0) {
        const uint32_t r = row0 + (threadIdx.x >> 2), kc = k0 + 32 * ((threadIdx.x >> 1) & 1);
        const uint32_t h = threadIdx.x & 1;
        live = r < nrows && kc < K;
        const uint32_t rr = r < nrows ? r : nrows - 1, kk = kc < K ? kc : 0;
        const uint8_t *blk = W + (uint64_t)rr * row_bytes + 144ull * (kk / 256);
        j = (kk % 256) / 32;
        hdr = *(const vkf_u4 *)blk;
        qs = *(const vkf_u4 *)(blk + 16 + 32 * (j >> 1) + 16 * h);
    }
    __device__ __forceinline__ void decode(vkf_i4 out[2]) {
        const float dall = vkf_h2f(hdr[0] & 0xffffu), dmin = vkf_h2f(hdr[0] >> 16);
        const uint32_t s0 = hdr[1], s4 = hdr[2], s8 = hdr[3];
        const uint32_t scW = j < 4 ? (s0 & 0x3f3f3f3fu) : ((s8 & 0x0f0f0f0fu) | ((s0 >> 2) & 0x30303030u));
        const uint32_t mnW = j < 4 ? (s4 & 0x3f3f3f3fu) : (((s8 >> 4) & 0x0f0f0f0fu) | ((s4 >> 2) & 0x30303030u));
        const uint32_t sh = 8 * (j & 3);
        const float dsc = dall * (float)((scW >> sh) & 0xffu), dm = dmin * (float)((mnW >> sh) & 0xffu);
        const uint32_t nsh = 4 * (j & 1);
#pragma unroll
        for (int g = 0; g < 2; g++) {
            vkf_h8 v;
#pragma unroll
            for (int e = 0; e < 2; e++) {
                uint32_t n = (qs[2 * g + e] >> nsh) & 0x0f0f0f0fu;
                asm volatile("" : "+v"(n));  // one v_cvt_f32_ubyte<k> per code (as QStage<VKF_Q4_K>)
#pragma unroll
                for (int k = 0; k < 4; k++)
                    v[4 * e + k] = vkf_to_f16(fmaf(dsc, (float)((n >> (8 * k)) & 0xffu), -dm));
            }
            out[g] = live ? __builtin_bit_cast(vkf_i4, v) : vkf_i4{0, 0, 0, 0};
        }
    }
};

// Q5_K: half h of sub-block j: qs bytes 48 + 32(j/2) + 16h .., qh bytes 16 +
// 16h .. (bit j), as QStage<VKF_Q5_K>.
template <>
struct QHalf<VKF_Q5_K> {
    vkf_u4 hdr, qs, qh;
    uint32_t j;
    bool live;
    __device__ __forceinline__ void load(const uint8_t *W, uint64_t row_bytes, uint32_t nrows, uint32_t row0,
                                         uint32_t K, uint32_t k0) {
        const uint32_t r = row0 + (threadIdx.x >> 2), kc = k0 + 32 * ((threadIdx.x >> 1) & 1);
        const uint32_t h = threadIdx.x & 1;
        live = r < nrows && kc < K;
        const uint32_t rr = r < nrows ? r : nrows - 1, kk = kc < K ? kc : 0;
        const uint8_t *blk = W + (uint64_t)rr * row_bytes + 176ull * (kk / 256);
        j = (kk % 256) / 32;
        hdr = *(const vkf_u4a4 *)blk;
        qh = *(const vkf_u4a4 *)(blk + 16 + 16 * h);
        qs = *(const vkf_u4a4 *)(blk + 48 + 32 * (j >> 1) + 16 * h);
    }
    __device__ __forceinline__ void decode(vkf_i4 out[2]) {
        const float dall = vkf_h2f(hdr[0] & 0xffffu), dmin = vkf_h2f(hdr[0] >> 16);
        const uint32_t s0 = hdr[1], s4 = hdr[2], s8 = hdr[3];
        const uint32_t scW = j < 4 ? (s0 & 0x3f3f3f3fu) : ((s8 & 0x0f0f0f0fu) | ((s0 >> 2) & 0x30303030u));
        const uint32_t mnW = j < 4 ? (s4 & 0x3f3f3f3fu) : (((s8 >> 4) & 0x0f0f0f0fu) | ((s4 >> 2) & 0x30303030u));
        const uint32_t sh = 8 * (j & 3);
        const float dsc = dall * (float)((scW >> sh) & 0xffu), dm = dmin * (float)((mnW >> sh) & 0xffu);
        const uint32_t nsh = 4 * (j & 1);
#pragma unroll
        for (int g = 0; g < 2; g++) {
            vkf_h8 v;
#pragma unroll
            for (int e = 0; e < 2; e++) {
                const uint32_t n = ((qs[2 * g + e] >> nsh) & 0x0f0f0f0fu) | (((qh[2 * g + e] >> j) & 0x01010101u) << 4);
#pragma unroll
                for (int k = 0; k < 4; k++)
                    v[4 * e + k] = vkf_to_f16(fmaf(dsc, (float)((n >> (8 * k)) & 0xffu), -dm));
            }
            out[g] = live ? __builtin_bit_cast(vkf_i4, v) : vkf_i4{0, 0, 0, 0};
        }
    }
};

// Q6_K: half h (elements 16h .. 16h+15, one scale) of 32-element block t of
// half ip: ql bytes 64ip + 32(t&1) + 16h .., qh bytes 128 + 32ip + 16h ..,
// each loaded as the five aligned dwords that cover it (inside the
// super-block) and realigned.
template <>
struct QHalf<VKF_Q6_K> {
    uint32_t ql[5], qh[5], sc, dd, sh, t, h;
    bool live;
    __device__ __forceinline__ void load(const uint8_t *W, uint64_t row_bytes, uint32_t nrows, uint32_t row0,
                                         uint32_t K, uint32_t k0) {
        const uint32_t rw = row0 + (threadIdx.x >> 2), kc = k0 + 32 * ((threadIdx.x >> 1) & 1);
        h = threadIdx.x & 1;
        live = rw < nrows && kc < K;
        const uint32_t kk = kc < K ? kc : 0, j8 = (kk % 256) / 32, ip = j8 >> 2;
        t = j8 & 3;
        const uint8_t *blk = W + (uint64_t)(rw < nrows ? rw : nrows - 1) * row_bytes + 210ull * (kk / 256);
        sh = (uint32_t)(uintptr_t)blk & 3u;
        const uint8_t *a = blk - sh;  // 4-byte aligned
        const uint8_t *pl = a + 64 * ip + 32 * (t & 1) + 16 * h, *ph = a + 128 + 32 * ip + 16 * h;
        const vkf_u4 l0 = *(const vkf_u4a4 *)pl, h0 = *(const vkf_u4a4 *)ph;
        ql[0] = l0[0]; ql[1] = l0[1]; ql[2] = l0[2]; ql[3] = l0[3];
        qh[0] = h0[0]; qh[1] = h0[1]; qh[2] = h0[2]; qh[3] = h0[3];
        ql[4] = *(const uint32_t *)(pl + 16);  // ends at byte <= 132 of the super-block
        qh[4] = *(const uint32_t *)(ph + 16);  // ends at byte <= 196
        sc = *(const uint16_t *)(blk + 192 + 8 * ip + 2 * t);
        dd = *(const uint16_t *)(blk + 208);
    }
    __device__ __forceinline__ void decode(vkf_i4 out[2]) {
        const float d = vkf_h2f((uint16_t)dd);
        const float ds = d * (float)(int8_t)(h ? (sc >> 8) : (sc & 0xffu)), off = -32.0f * ds;
        const uint32_t nsh = 4 * (t >> 1), hsh = 2 * t;
#pragma unroll
        for (int g = 0; g < 2; g++) {
            vkf_h8 v;
#pragma unroll
            for (int e2 = 0; e2 < 2; e2++) {
                const int i = 2 * g + e2;
                const uint32_t l = realign(ql[i], ql[i + 1], sh), hb = realign(qh[i], qh[i + 1], sh);
                const uint32_t u = ((l >> nsh) & 0x0f0f0f0fu) | (((hb >> hsh) & 0x03030303u) << 4);
#pragma unroll
                for (int k = 0; k < 4; k++) v[4 * e2 + k] = vkf_to_f16(fmaf(ds, (float)((u >> (8 * k)) & 0xffu), off));
            }
            out[g] = live ? __builtin_bit_cast(vkf_i4, v) : vkf_i4{0, 0, 0, 0};
        }
    }
};

template <int QT> constexpr bool has_qhalf() { return QT == VKF_Q4_K || QT == VKF_Q5_K || QT == VKF_Q6_K; }
// Both operands quantised (Q8_1 activations x ggml weights): both tiles are
// staged through registers with the same load-before / decode-after split.
template <int XQT, int QT>
__device__ __forceinline__ void gemm_mainloop_qq(const VkfGemmArgs &a, uint32_t r0, uint32_t c0, vkf_f4 acc[4][4],
                                                 uint8_t *smem) {
    const int wave = threadIdx.x >> 6, wr = wave >> 1, wc = wave & 1;
    const uint32_t nk = (a.K + 63) / 64;
    const uint32_t tr = threadIdx.x >> 1, th = threadIdx.x & 1;
    auto store = [&](uint8_t *tile, const TileRegs &t) {
        uint8_t *p = tile + tr * 128;
#pragma unroll
        for (int g = 0; g < 4; g++) *(vkf_i4 *)(p + (((4 * th + g) ^ (tr & 7)) << 4)) = t.v[g];
    };
    QStage<XQT> qx;
    QStage<QT> qy;
    TileRegs tx, ty;
    qx.load((const uint8_t *)a.X, a.ldx, a.R, r0, a.K, 0);
    qy.load((const uint8_t *)a.Y, a.ldy, a.Cn, c0, a.K, 0);
    qx.decode(tx);
    qy.decode(ty);
    store(smem, tx);
    store(smem + 16384, ty);
    __syncthreads();
    for (uint32_t kt = 0; kt < nk; kt++) {
        const uint32_t cur = kt & 1;
        if (kt + 1 < nk) {
            qx.load((const uint8_t *)a.X, a.ldx, a.R, r0, a.K, (kt + 1) * 64);
            qy.load((const uint8_t *)a.Y, a.ldy, a.Cn, c0, a.K, (kt + 1) * 64);
        }
        const uint8_t *lx = smem + cur * 32768;
        mfma_step_swz<2>(lx, lx + 16384, wr, wc, acc);
        if (kt + 1 < nk) {
            qx.decode(tx);
            qy.decode(ty);
            store(smem + (cur ^ 1) * 32768, tx);
            store(smem + (cur ^ 1) * 32768 + 16384, ty);
        }
        __syncthreads();
    }
}

template <int QT>
__device__ __forceinline__ void gemm_mainloop_qdma(const VkfGemmArgs &a, uint32_t r0, uint32_t c0, vkf_f4 acc[4][4],
                                                   uint8_t *smem) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, wr = wave >> 1, wc = wave & 1;
    const uint32_t nk = a.K / 64;
    const uint8_t *gx[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const uint32_t rr = (4 * wave + j) * 8 + (lane >> 3);
        const uint32_t ch = (lane & 7) ^ (rr & 7);
        const uint32_t rx = r0 + rr < a.R ? r0 + rr : a.R - 1;
        gx[j] = (const uint8_t *)a.X + (uint64_t)rx * a.ldx * 2 + ch * 16;
    }
    auto issue_x = [&](uint32_t kt, uint32_t stage) {
        uint8_t *sx = smem + stage * 32768;
#pragma unroll
        for (int j = 0; j < 4; j++)
            vkf_load_lds16(gx[j] + (uint64_t)kt * 128, sx + (4 * wave + j) * 1024);
    };
    const uint32_t yr = threadIdx.x >> 1, yh = threadIdx.x & 1;
    auto store_y = [&](uint32_t stage, const TileRegs &t) {
        uint8_t *sy = smem + stage * 32768 + 16384 + yr * 128;
#pragma unroll
        for (int g = 0; g < 4; g++) *(vkf_i4 *)(sy + (((4 * yh + g) ^ (yr & 7)) << 4)) = t.v[g];
    };
    QStage<QT> q;
    TileRegs ty;
    issue_x(0, 0);
    q.load((const uint8_t *)a.Y, a.ldy, a.Cn, c0, a.K, 0);
    q.decode(ty);
    store_y(0, ty);
    wait_vm<0>();
    __syncthreads();
    for (uint32_t kt = 0; kt < nk; kt++) {
        const uint32_t cur = kt & 1;
        if (kt + 1 < nk) {
            issue_x(kt + 1, cur ^ 1);
            q.load((const uint8_t *)a.Y, a.ldy, a.Cn, c0, a.K, (kt + 1) * 64);
        }
        const uint8_t *lx = smem + cur * 32768;
        mfma_step_swz<2>(lx, lx + 16384, wr, wc, acc);
        if (kt + 1 < nk) {
            q.decode(ty);
            store_y(cur ^ 1, ty);
        }
        wait_vm<0>();
        __syncthreads();
    }
}

// fp16 Y stored [K, C] (an NN product's B [K, N]; torch.mm(a, b) with a
// contiguous b) with both operands on direct-to-LDS loads: Y's tile is
// copied as it lies, 64 k-rows of 128 columns (256 bytes each), and the
// MFMA operand (8 consecutive k of one column per lane) is read back with
// ds_read_b64_tr_b16.  That instruction works on groups of 16 lanes: with
// R[s][e] the e-th 16-bit element at lane s's address, lane j receives
// R[4e + (j >> 2)][j & 3], e = 0..3 (measured on MI355X).  So lane s of a
// group points at row k0 + (s >> 2), columns 4(s & 3) .. +3 of a 16-column
// block, and lane j gets column j, rows k0 .. k0+3; two such reads make the
// 8 k of lane (column j, k-slice g) for the 16x16x32 MFMA.  Row k's 16-byte
// piece p sits at slot p ^ 2(k & 3) (the direct loads fetch piece
// slot ^ 2(k & 3) into each slot), so the 4 rows of a 16-lane read fall on
// different banks.  Needs C % 8 == 0 (no piece straddles the last column),
// 16-byte aligned Y and row pitch, K % 64 == 0.
__device__ __forceinline__ bool dma_trb_ok(const void *P, uint64_t ld, uint32_t C, uint32_t K) {
    return ((ld * 2) % 16) == 0 && (((uintptr_t)P & 15) == 0) && (C % 8) == 0 && (K % 64) == 0;
}

typedef short vkf_s4 __attribute__((ext_vector_type(4)));

// 4 k of one column: the ds_read_b64_tr_b16 of this lane's address p (LDS)
__device__ __forceinline__ vkf_i2 lds_read_tr16(const uint8_t *p) {
    const vkf_s4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) vkf_s4 *)(p));
    return __builtin_bit_cast(vkf_i2, v);
}

// One 64-k step of the wave's 64x64 tile: X fragments as mfma_step_swz,
// Y fragments by transposed reads of the [k][column] tile ly.
template <class ACC>
__device__ __forceinline__ void mfma_step_trb(const uint8_t *lx, const uint8_t *ly, int wr, int wc, ACC acc[4][4]) {
    const int lane = threadIdx.x & 63, li = lane & 15, lg = lane >> 4, sw = li & 7;
    const int rsub = li >> 2, hb = (li & 1) * 8;  // this lane's row in a 4-row read, half of its piece
    vkf_i4 fa[2][4], fb[2][4];
#pragma unroll
    for (int s = 0; s < 2; s++) {
        const int c = 4 * s + lg;
#pragma unroll
        for (int i = 0; i < 4; i++)
            fa[s][i] = *(const vkf_i4 *)(lx + (wr * 64 + 16 * i + li) * 128 + ((c ^ sw) << 4));
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int slot = (8 * wc + 2 * j + ((li & 3) >> 1)) ^ (2 * rsub);
            const uint8_t *q = ly + (32 * s + 8 * lg + rsub) * 256 + slot * 16 + hb;
            const vkf_i2 lo = lds_read_tr16(q), hi = lds_read_tr16(q + 4 * 256);
            fb[s][j] = vkf_i4{lo[0], lo[1], hi[0], hi[1]};
        }
    }
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int s = 0; s < 2; s++)
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int j = 0; j < 4; j++) acc[i][j] = mfma_frag<2>(fa[s][i], fb[s][j], acc[i][j]);
    __builtin_amdgcn_s_setprio(0);
}

template <class ACC>
__device__ __forceinline__ void gemm_mainloop_dma_trb(const VkfGemmArgs &a, uint32_t r0, uint32_t c0, ACC acc[4][4],
                                                      uint8_t *smem) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, wr = wave >> 1, wc = wave & 1;
    const uint32_t nk = a.K / 64;
    const uint8_t *gx[4], *gy[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const uint32_t rr = (4 * wave + j) * 8 + (lane >> 3);
        const uint32_t ch = (lane & 7) ^ (rr & 7);
        const uint32_t rx = r0 + rr < a.R ? r0 + rr : a.R - 1;  // rows past the edge: any valid row
        gx[j] = (const uint8_t *)a.X + (uint64_t)rx * a.ldx * 2 + ch * 16;
        // k-row kr of the step, slot lane & 15: columns of piece slot ^ 2(kr & 3)
        const uint32_t kr = 16 * wave + 4 * j + (lane >> 4), p = (lane & 15) ^ (2 * (kr & 3));
        const uint32_t col = c0 + 8 * p < a.Cn ? c0 + 8 * p : a.Cn - 8;  // pieces past the edge: any valid one
        gy[j] = (const uint8_t *)a.Y + ((uint64_t)kr * a.ldy + col) * 2;
    }
    const uint64_t ystep = (uint64_t)64 * a.ldy * 2;
    auto issue = [&](uint32_t kt, uint32_t stage) {
        uint8_t *sx = smem + stage * 32768, *sy = sx + 16384;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            vkf_load_lds16(gx[j] + (uint64_t)kt * 128, sx + (4 * wave + j) * 8 * 128);
            vkf_load_lds16(gy[j] + kt * ystep, sy + (16 * wave + 4 * j) * 256);
        }
    };
#pragma unroll
    for (uint32_t s = 0; s + 1 < GNST; s++)
        if (s < nk) issue(s, s);
    for (uint32_t kt = 0; kt < nk; kt++) {
        if (kt + GNST - 2 < nk) wait_vm<8 * (GNST - 2)>();
        else wait_vm<0>();
        __syncthreads();
        if (kt + GNST - 1 < nk) issue(kt + GNST - 1, (kt + GNST - 1) % GNST);
        const uint8_t *lx = smem + (kt % GNST) * 32768;
        mfma_step_trb(lx, lx + 16384, wr, wc, acc);
    }
    __syncthreads();  // LDS free for the epilogue
}

// Dense X K-contiguous (direct-to-LDS tiles) and Y transposed (stored
// [K, C], e.g. B [K, N] of an NN product, torch.mm(a, b) with contiguous b):
// Y's 16-byte row pieces come from load_dense_t (loads along Y's contiguous
// direction, transposed in registers), loaded a step ahead and stored into
// the swizzled LDS layout after the step's MFMAs, as the quantised weight
// tiles of gemm_mainloop_qdma.  K*ES a multiple of 128 (X's condition).
template <int ES, class ACC>
__device__ __forceinline__ void gemm_mainloop_tdma(const VkfGemmArgs &a, uint32_t r0, uint32_t c0, ACC acc[4][4],
                                                   uint8_t *smem) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, wr = wave >> 1, wc = wave & 1;
    const uint32_t nk = (uint32_t)(((uint64_t)a.K * ES) / 128);
    const uint8_t *gx[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const uint32_t rr = (4 * wave + j) * 8 + (lane >> 3);
        const uint32_t ch = (lane & 7) ^ (rr & 7);
        const uint32_t rx = r0 + rr < a.R ? r0 + rr : a.R - 1;
        gx[j] = (const uint8_t *)a.X + (uint64_t)rx * a.ldx * ES + ch * 16;
    }
    auto issue_x = [&](uint32_t kt, uint32_t stage) {
        uint8_t *sx = smem + stage * 32768;
#pragma unroll
        for (int j = 0; j < 4; j++) vkf_load_lds16(gx[j] + (uint64_t)kt * 128, sx + (4 * wave + j) * 1024);
    };
    const auto oy = make_operand<ES, -1>(a.Y, a.ldy, true, a.Cn, c0, a.K);
    const uint32_t yr = 4 * (threadIdx.x >> 3), yc = threadIdx.x & 7;
    auto store_y = [&](uint32_t stage, const TileRegs &t) {
        uint8_t *sy = smem + stage * 32768 + 16384;
#pragma unroll
        for (int p = 0; p < 4; p++) {
            const uint32_t r = yr + p;
            *(vkf_i4 *)(sy + r * 128 + ((yc ^ (r & 7)) << 4)) = t.v[p];
        }
    };
    TileRegs ty;
    issue_x(0, 0);
    oy.load(0, ty);
    store_y(0, ty);
    wait_vm<0>();
    __syncthreads();
    for (uint32_t kt = 0; kt < nk; kt++) {
        const uint32_t cur = kt & 1;
        if (kt + 1 < nk) {
            issue_x(kt + 1, cur ^ 1);
            oy.load(kt + 1, ty);
        }
        const uint8_t *lx = smem + cur * 32768;
        mfma_step_swz<ES>(lx, lx + 16384, wr, wc, acc);
        if (kt + 1 < nk) store_y(cur ^ 1, ty);
        wait_vm<0>();
        __syncthreads();
    }
}

// Float epilogue of the workgroup's 128x128 tile (v = alpha * acc * rs[r] *
// cs[c] + beta * Cin + bias, then the activation):
// each lane finishes its 64 values, the tile is staged as fp32 rows in LDS
// (pitch 132 floats) and written out as 16-byte row vectors when D's rows
// allow it, element by element otherwise.  smem must be free (the main loop
// ends with a barrier).
// epi_stage: one wave's 64x64 values (position wr, wc inside the 128x128
// tile at r0, c0) finished and written to the fp32 staging tile.
// The epilogue's per-column scale and bias and per-row scale of one wave's
// 64x64 values, loaded ahead (before the main loop) so that their latency
// hides under the MFMAs instead of following them.
struct EpiPre {
    float cs[4], bc[4], rs[16];
};
__device__ __forceinline__ EpiPre epi_prefetch(const VkfGemmArgs &a, uint32_t r0, uint32_t c0, int wr, int wc) {
    const int lane = threadIdx.x & 63, li = lane & 15, lg = lane >> 4;
    EpiPre p;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const uint32_t c = c0 + wc * 64 + 16 * j + li, cc = c < a.Cn ? c : a.Cn - 1;
        p.cs[j] = a.cs ? a.cs[(a.flags & VKF_GF_CS_SCALAR) ? 0 : cc] : 1.0f;
        p.bc[j] = 0.0f;
        if (a.bias && !(a.flags & VKF_GF_BIAS_ROW))
            p.bc[j] = (a.flags & VKF_GF_BIAS_F32) ? ((const float *)a.bias)[cc] : (float)((const _Float16 *)a.bias)[cc];
    }
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const uint32_t r = r0 + wr * 64 + 16 * i + 4 * lg + e, rr = r < a.R ? r : a.R - 1;
            p.rs[4 * i + e] = a.rs ? a.rs[(a.flags & VKF_GF_RS_SCALAR) ? 0 : rr] : 1.0f;
        }
    return p;
}

// NI < 4: the wave holds only 16-row groups i0 .. i0 + NI - 1 of its 64 rows.
template <int NI = 4, class ACC>
__device__ __forceinline__ void epi_stage(const VkfGemmArgs &a, uint32_t r0, uint32_t c0, const ACC acc[][4],
                                          float *tile, int wr, int wc, const EpiPre *pre = nullptr, int i0 = 0) {
    constexpr int TP = 132;
    const int lane = threadIdx.x & 63, li = lane & 15, lg = lane >> 4;
    const EpiPre p = pre ? *pre : epi_prefetch(a, r0, c0, wr, wc);
    const float *csv = p.cs, *bcv = p.bc;
#pragma unroll
    for (int i = 0; i < NI; i++)
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int tr = wr * 64 + 16 * (i0 + i) + 4 * lg + e;
            const uint32_t r = r0 + tr, rr = r < a.R ? r : a.R - 1;
            const float rsv = p.rs[4 * (i0 + i) + e];
            float brv = 0.0f;
            if (a.bias && (a.flags & VKF_GF_BIAS_ROW))
                brv = (a.flags & VKF_GF_BIAS_F32) ? ((const float *)a.bias)[rr] : (float)((const _Float16 *)a.bias)[rr];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const uint32_t c = c0 + wc * 64 + 16 * j + li;
                float v = (float)acc[i][j][e];
                if (a.rs) v *= rsv;
                if (a.cs) v *= csv[j];
                v *= a.alpha;
                if (a.beta != 0.0f && r < a.R && c < a.Cn) {
                    const float cin = (a.flags & VKF_GF_CIN_F32)
                                          ? ((const float *)a.Cin)[(uint64_t)r * a.ldc + c]
                                          : (float)((const _Float16 *)a.Cin)[(uint64_t)r * a.ldc + c];
                    v = fmaf(a.beta, cin, v);
                }
                if (a.bias) v += (a.flags & VKF_GF_BIAS_ROW) ? brv : bcv[j];
                tile[tr * TP + wc * 64 + 16 * j + li] = vkf_act(a.act, v);
            }
        }
}

// epi_store: the staged 128x128 tile to D by all NT threads of the workgroup.
template <int NT>
__device__ __forceinline__ void epi_store(const VkfGemmArgs &a, uint32_t r0, uint32_t c0, const float *tile) {
    constexpr int TP = 132;
    const bool f32 = (a.flags & VKF_GF_D_F32) != 0;
    const uint32_t vec = f32 ? 4 : 8;  // elements per 16-byte store
    const bool vok = (a.ldd % vec) == 0 && (((uintptr_t)a.D & 15) == 0);
    const uint32_t per_row = 128 / vec;
    for (uint32_t q = threadIdx.x; q < 128 * per_row; q += NT) {
        const uint32_t tr = q / per_row, tc = (q % per_row) * vec;
        const uint32_t r = r0 + tr, c = c0 + tc;
        if (r >= a.R || c >= a.Cn) continue;
        const float *src = tile + tr * TP + tc;
        if (vok && c + vec <= a.Cn) {
            if (f32) {
                *(vkf_f4 *)((float *)a.D + (uint64_t)r * a.ldd + c) = *(const vkf_f4 *)src;
            } else {
                vkf_h8 h;
#pragma unroll
                for (int k = 0; k < 8; k++) h[k] = vkf_to_f16(src[k]);
                *(vkf_h8 *)((_Float16 *)a.D + (uint64_t)r * a.ldd + c) = h;
            }
        } else {
            for (uint32_t k = 0; k < vec && c + k < a.Cn; k++) {
                if (f32) ((float *)a.D)[(uint64_t)r * a.ldd + c + k] = src[k];
                else ((_Float16 *)a.D)[(uint64_t)r * a.ldd + c + k] = vkf_to_f16(src[k]);
            }
        }
    }
}

template <class ACC>
__device__ __forceinline__ void epilogue_tile(const VkfGemmArgs &a, uint32_t r0, uint32_t c0, const ACC acc[4][4],
                                              uint8_t *smem) {
    const int wave = threadIdx.x >> 6;
    epi_stage(a, r0, c0, acc, (float *)smem, wave >> 1, wave & 1);
    __syncthreads();
    epi_store<256>(a, r0, c0, (const float *)smem);
}

// The matrix of batch blockIdx.z of a dense launch (strided or through the
// device pointer arrays).
__device__ __forceinline__ VkfGemmArgs gemm_batch(const VkfGemmArgs &a0) {
    VkfGemmArgs a = a0;
    const uint32_t b = blockIdx.z;
    if (a.bpx) {
        a.X = a.bpx[b];
        a.Y = a.bpy[b];
        a.D = a.bpd[b];
        a.Cin = a.D;
    } else if (b) {
        a.X = (const uint8_t *)a.X + b * a.bsx;
        a.Y = (const uint8_t *)a.Y + b * a.bsy;
        a.D = (uint8_t *)a.D + b * a.bsd;
        if (a.Cin) a.Cin = (const uint8_t *)a.Cin + b * a.bsc;
    }
    return a;
}

// Workgroup -> 128 x 128 tile, XCD-aware.  Workgroups are dispatched to the
// 8 XCDs round-robin (id % 8), each XCD with its own L2.  Columns (Y tiles)
// are dealt to XCDs round-robin and an XCD runs all row tiles of a column
// back to back, so a Y tile is fetched into one L2 and reused there by every
// row tile (for the vocabulary projection, 512 x 152064 x 5120, that is 4x
// fewer weight bytes from HBM than a row-major order).  Columns past the
// last multiple of 8 go in plain order.
template <uint32_t RT = 128>
__device__ __forceinline__ void gemm_tile_of(uint32_t &r0, uint32_t &c0) {
    const uint32_t nc = gridDim.x, nr = gridDim.y, id = blockIdx.x + nc * blockIdx.y;
    const uint32_t full = nc & ~7u;
    uint32_t r, c;
    if (id < full * nr) {
        const uint32_t x = id & 7u, sl = id >> 3;
        c = (sl / nr) * 8 + x;
        r = sl % nr;
    } else {
        const uint32_t j = id - full * nr;
        c = full + j / nr;
        r = j % nr;
    }
    r0 = r * RT;
    c0 = c * 128;
}

// XQT < 0: dense fp16 X, otherwise Q8_1 activation blocks (each tile value
// fp16(dx*q)).  QT < 0: dense fp16 Y; otherwise Y holds ggml blocks of type QT.
template <int XQT, int QT>
__device__ __forceinline__ void gemm_f16_body(const VkfGemmArgs &a) {
    uint32_t r0, c0;
    gemm_tile_of(r0, c0);
    vkf_f4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = vkf_f4{0, 0, 0, 0};
    // kernels with dense fp16 X hold either main loop's buffers
    __shared__ __attribute__((aligned(16))) uint8_t smem[XQT < 0 ? GEMM_LDS_BOTH : GEMM_LDS];
    if constexpr (XQT < 0 && QT < 0) {
        if (dma_ok(a.X, a.ldx, (a.flags & VKF_GF_X_TRANS) != 0, a.K, 2)) {
            if (dma_ok(a.Y, a.ldy, (a.flags & VKF_GF_Y_TRANS) != 0, a.K, 2)) gemm_mainloop_dma<2>(a, r0, c0, acc, smem);
            else if ((a.flags & VKF_GF_Y_TRANS) && dma_trb_ok(a.Y, a.ldy, a.Cn, a.K))
                gemm_mainloop_dma_trb(a, r0, c0, acc, smem);
            else if (a.flags & VKF_GF_Y_TRANS) gemm_mainloop_tdma<2>(a, r0, c0, acc, smem);
            else goto general;
            epilogue_tile(a, r0, c0, acc, smem);
            return;
        }
    general:;
    }
    if constexpr (XQT < 0 && QT >= 0) {
        if (dma_ok(a.X, a.ldx, (a.flags & VKF_GF_X_TRANS) != 0, a.K, 2)) {
            gemm_mainloop_qdma<QT>(a, r0, c0, acc, smem);
            epilogue_tile(a, r0, c0, acc, smem);
            return;
        }
    }
    if constexpr (XQT >= 0 && QT >= 0) {  // K is a multiple of 32 here
        gemm_mainloop_qq<XQT, QT>(a, r0, c0, acc, smem);
        epilogue_tile(a, r0, c0, acc, smem);
        return;
    }
    const auto ox = make_operand<2, XQT>(a.X, a.ldx, (a.flags & VKF_GF_X_TRANS) != 0, a.R, r0, a.K);
    const auto oy = make_operand<2, QT>(a.Y, a.ldy, (a.flags & VKF_GF_Y_TRANS) != 0, a.Cn, c0, a.K);
    gemm_mainloop<2>(ox, oy, a.K, 64, acc, smem);
    epilogue_tile(a, r0, c0, acc, smem);
}

GEMM_KERNEL vkf_gemm_f16(VkfGemmArgs a0) { gemm_f16_body<-1, -1>(gemm_batch(a0)); }
#define VKF_GEMM_Q(name, QT)                                                                        \
    GEMM_KERNEL vkf_gemm_##name##_f16(VkfGemmArgs a) { gemm_f16_body<-1, QT>(a); }
#define VKF_GEMM_Q_Q81(name, QT)                                                                    \
    GEMM_KERNEL vkf_gemm_##name##_q8_1(VkfGemmArgs a) {                                            \
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
VKF_GEMM_Q_Q81(q6_k, VKF_Q6_K)

// ---------------------------------------------------------------------------
// Wide quantised-weight GEMM with fp16 activations: 512 threads, a 256 x 128
// tile (activation rows x weight rows), eight waves of 64 x 64 (wave w: rows
// 64*(w/2), columns 64*(w%2)).  Against two 128 x 128 workgroups, each weight
// tile is loaded and decoded once per 256 activation rows instead of once
// per 128, which halves the decode work per MAC; the decode's VALU time is
// what bounds these GEMMs (Q6_K 512 x 152064 x 5120 on MI355X: 1.56 ms here
// against 1.75 ms with 128 x 128 tiles).  Waves 0-3 decode the weight tile
// (QStage, thread t: row t/2, chunk t&1); the activation tile comes by
// direct-to-LDS loads from all eight waves.  Two stages of 48 KiB (32 KiB
// activations + 16 KiB weights); the epilogue's 256-row fp32 staging tile
// (132 KiB) sets the LDS size.
// ---------------------------------------------------------------------------
#define GEMM_W_STAGE 49152
#define GEMM_W_LDS (2 * GEMM_W_STAGE)
#define GEMM_KERNEL_W VKF_KERNEL void __launch_bounds__(512)

template <int QT>
__device__ __forceinline__ void gemm_mainloop_wide(const VkfGemmArgs &a, uint32_t r0, uint32_t c0, vkf_f4 acc[4][4],
                                                   uint8_t *smem) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, wr = wave >> 1, wc = wave & 1;
    const bool ywave = threadIdx.x < 256;  // wave-uniform
    const uint32_t nk = a.K / 64;
    const uint8_t *gx[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const uint32_t rr = (4 * wave + j) * 8 + (lane >> 3);  // 0..255
        const uint32_t ch = (lane & 7) ^ (rr & 7);
        const uint32_t rx = r0 + rr < a.R ? r0 + rr : a.R - 1;
        gx[j] = (const uint8_t *)a.X + (uint64_t)rx * a.ldx * 2 + ch * 16;
    }
    auto issue_x = [&](uint32_t kt, uint32_t stage) {
        uint8_t *sx = smem + stage * GEMM_W_STAGE;
#pragma unroll
        for (int j = 0; j < 4; j++) vkf_load_lds16(gx[j] + (uint64_t)kt * 128, sx + (4 * wave + j) * 1024);
    };
    const uint32_t yr = threadIdx.x >> 1, yh = threadIdx.x & 1;
    auto store_y = [&](uint32_t stage, const TileRegs &t) {
        uint8_t *sy = smem + stage * GEMM_W_STAGE + 32768 + yr * 128;
#pragma unroll
        for (int g = 0; g < 4; g++) *(vkf_i4 *)(sy + (((4 * yh + g) ^ (yr & 7)) << 4)) = t.v[g];
    };
    if constexpr (has_qhalf<QT>()) {
        // all eight waves decode: thread t -> row t/4, elements 16(t&3) ..
        // Weight chunks are loaded two steps ahead of their MFMA step, into
        // two alternating register sets, so that a chunk's HBM latency hides
        // under two MFMA steps; activation tiles (mostly L2 hits) one step
        // ahead.  Step kt issues activation tile kt+1, then weight chunk
        // kt+2, so the compiler's s_waitcnt before the decode of chunk kt+1
        // (which lets only chunk kt+2's loads stay in flight; loads return
        // in order) also covers activation tile kt+1 before the barrier.
        const uint32_t hr = threadIdx.x >> 2, hq = threadIdx.x & 3;
        auto store_h = [&](uint32_t stage, const vkf_i4 v[2]) {
            uint8_t *sy = smem + stage * GEMM_W_STAGE + 32768 + hr * 128;
#pragma unroll
            for (int g = 0; g < 2; g++) *(vkf_i4 *)(sy + (((2 * hq + g) ^ (hr & 7)) << 4)) = v[g];
        };
        const uint8_t *W = (const uint8_t *)a.Y;
        QHalf<QT> qa, qb;
        vkf_i4 tv[2];
        issue_x(0, 0);
        qa.load(W, a.ldy, a.Cn, c0, a.K, 0);
        qb.load(W, a.ldy, a.Cn, c0, a.K, 64);
        qa.decode(tv);
        store_h(0, tv);
        wait_vm<0>();
        __syncthreads();
        // qn holds chunk kt+1 (loaded a step earlier), qf is free.  The
        // weight loads and decodes are unconditional (chunks past the end
        // are clamped in-bounds loads decoded to zeros into a stage that is
        // not read again), so that the compiler's wait analysis sees the
        // same loads in flight on every path and never falls back to
        // vmcnt(0) at a merge point.  K is whole 256-element super-blocks,
        // so nk is a multiple of 4 and the loop runs its steps in pairs.
        auto step = [&](uint32_t kt, QHalf<QT> &qn, QHalf<QT> &qf) {
            const uint32_t cur = kt & 1;
            if (kt + 1 < nk) issue_x(kt + 1, cur ^ 1);
            qf.load(W, a.ldy, a.Cn, c0, a.K, (kt + 2) * 64);
            const uint8_t *lx = smem + cur * GEMM_W_STAGE;
            mfma_step_swz<2, vkf_f4, false>(lx, lx + 32768, wr, wc, acc);
            qn.decode(tv);
            store_h(cur ^ 1, tv);
            // the decode's VALU between the MFMAs: fragment reads first, then
            // one MFMA and two VALU instructions at a time, the tile stores last
            __builtin_amdgcn_sched_group_barrier(0x020, 8, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 16, 0);
#pragma unroll
            for (int i = 0; i < 32; i++) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);
            }
            __builtin_amdgcn_sched_group_barrier(0x200, 2, 0);
            __syncthreads();
        };
        for (uint32_t kt = 0; kt < nk; kt += 2) {
            step(kt, qb, qa);
            step(kt + 1, qa, qb);
        }
        return;
    }
    QStage<QT> q;
    TileRegs ty;
    issue_x(0, 0);
    if (ywave) {
        q.load((const uint8_t *)a.Y, a.ldy, a.Cn, c0, a.K, 0);
        q.decode(ty);
        store_y(0, ty);
    }
    wait_vm<0>();
    __syncthreads();
    for (uint32_t kt = 0; kt < nk; kt++) {
        const uint32_t cur = kt & 1;
        if (kt + 1 < nk) {
            issue_x(kt + 1, cur ^ 1);
            if (ywave) q.load((const uint8_t *)a.Y, a.ldy, a.Cn, c0, a.K, (kt + 1) * 64);
        }
        const uint8_t *lx = smem + cur * GEMM_W_STAGE;
        mfma_step_swz<2>(lx, lx + 32768, wr, wc, acc);
        if (kt + 1 < nk && ywave) {
            q.decode(ty);
            store_y(cur ^ 1, ty);
        }
        wait_vm<0>();
        __syncthreads();
    }
}

template <int QT>
__device__ __forceinline__ void gemm_wide_body(const VkfGemmArgs &a) {
    uint32_t r0, c0;
    gemm_tile_of<256>(r0, c0);
    vkf_f4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = vkf_f4{0, 0, 0, 0};
    __shared__ __attribute__((aligned(16))) uint8_t smem[GEMM_W_LDS > 256 * 132 * 4 ? GEMM_W_LDS : 256 * 132 * 4];
    gemm_mainloop_wide<QT>(a, r0, c0, acc, smem);
    // epilogue: both 128-row halves staged at once (256 x 132 fp32; staging
    // them one after the other costs the kernel its registers)
    const int wave = threadIdx.x >> 6, wr = wave >> 1, wc = wave & 1;
    float *tile = (float *)smem + (wr >> 1) * 128 * 132;
    epi_stage(a, r0 + 128 * (wr >> 1), c0, acc, tile, wr & 1, wc);
    __syncthreads();
    epi_store<512>(a, r0, c0, (const float *)smem);
    epi_store<512>(a, r0 + 128, c0, (const float *)smem + 128 * 132);
}

// dense fp16 activations only: 16-byte aligned rows, K % 64 == 0
#define VKF_GEMM_W(name, QT) \
    GEMM_KERNEL_W vkf_gemm_##name##_f16_w(VkfGemmArgs a) { gemm_wide_body<QT>(a); }
VKF_GEMM_W(q4_0, VKF_Q4_0)
VKF_GEMM_W(q4_1, VKF_Q4_1)
VKF_GEMM_W(q8_0, VKF_Q8_0)
VKF_GEMM_W(q5_0, VKF_Q5_0)
VKF_GEMM_W(q4_k, VKF_Q4_K)
VKF_GEMM_W(q5_k, VKF_Q5_K)
VKF_GEMM_W(q6_k, VKF_Q6_K)

// ---------------------------------------------------------------------------
// Q8_1 activations x Q8_0 weights on the int8 matrix cores
// (vkf_gemm_q8_0_q8_1_i8): ggml's block dot, y[m, n] = sum over 32-element
// blocks kb of dx[m,kb] * dw[n,kb] * P[m,n,kb], with P = sum q8x * q8w the
// exact int32 dot of the block's codes (kernels/dequant_q8_1.glsl:21-32,
// kernels/dequant_q8_0.glsl:18-28; shim/hip_runtime_shim.cpp:1151-1166 is the
// reference's quantised mul_mat that dequantises both to fp32 instead).
// One v_mfma_i32_16x16x32_i8 per 16x16 sub-tile and block yields P exactly
// (|P| <= 32 * 128 * 128 = 2^19); the block's scales are applied to it in
// fp32: acc += float(P) * (dx * dw).  The fold is three VALU operations per
// output and block (convert, scale product, fma), three times the MFMA time
// of the block, so the kernel is built to keep the VALU busy: a 128 x 128
// tile per 512-thread workgroup, eight waves of 32 x 64 (two per SIMD, so
// that one wave's fold issues while the other waits on its MFMAs and LDS
// reads).  Wave w covers columns 64 * (w & 1) and rows 64 * ((w >> 1) & 1)
// + 32 * (w >> 2) of the tile.  K advances 4 blocks per step: thread t loads
// block t & 3 of activation row t >> 2 and of weight row t >> 2 into
// registers before the step's MFMAs and writes its codes (XOR-swizzled as
// in the direct-to-LDS tiles) and scales to the other LDS stage after them.
// PARTIALS: store every P (int32) at D[(m*N + n)*(K/32) + kb] instead (the
// integer core, for tests).
// ---------------------------------------------------------------------------
#define QI_STAGE (2 * 16384 + 2 * 2048)  // X codes, Y codes, dx[4][128], dw[4][128]
#define QI_LDS (2 * QI_STAGE > 128 * 132 * 4 ? 2 * QI_STAGE : 128 * 132 * 4)

struct Q8Stage {
    uint32_t x[9], w[9], wsh;
    bool xv, wv;
};

__device__ __forceinline__ void q8_stage_load(const VkfGemmArgs &a, uint32_t r0, uint32_t c0, uint32_t kt,
                                              Q8Stage &s) {
    const uint32_t tr = threadIdx.x >> 2, nb = a.K / 32, kb = 4 * kt + (threadIdx.x & 3);
    const uint32_t rx = r0 + tr < a.R ? r0 + tr : a.R - 1, ry = c0 + tr < a.Cn ? c0 + tr : a.Cn - 1;
    const uint32_t kk = kb < nb ? kb : nb - 1;
    s.xv = kb < nb && r0 + tr < a.R;
    s.wv = kb < nb && c0 + tr < a.Cn;
    // Q8_1: 36-byte blocks, 4-byte aligned: fp16 d, fp16 s, int8 q[32]
    const uint8_t *px = (const uint8_t *)a.X + (uint64_t)rx * a.ldx + 36ull * kk;
    const vkf_u4 x0 = *(const vkf_u4a4 *)px, x1 = *(const vkf_u4a4 *)(px + 16);
    s.x[0] = x0[0]; s.x[1] = x0[1]; s.x[2] = x0[2]; s.x[3] = x0[3];
    s.x[4] = x1[0]; s.x[5] = x1[1]; s.x[6] = x1[2]; s.x[7] = x1[3];
    s.x[8] = *(const uint32_t *)(px + 32);
    // Q8_0: 34-byte blocks, 2-byte aligned: the covering dwords, realigned
    // when stored; nothing past the block's last byte is read
    const uint8_t *pw = (const uint8_t *)a.Y + (uint64_t)ry * a.ldy + 34ull * kk;
    const uint32_t sh = (uint32_t)(uintptr_t)pw & 3u;
    const uint8_t *aw = pw - sh;
    const vkf_u4 w0 = *(const vkf_u4a4 *)aw, w1 = *(const vkf_u4a4 *)(aw + 16);
    s.w[0] = w0[0]; s.w[1] = w0[1]; s.w[2] = w0[2]; s.w[3] = w0[3];
    s.w[4] = w1[0]; s.w[5] = w1[1]; s.w[6] = w1[2]; s.w[7] = w1[3];
    s.w[8] = sh ? *(const uint32_t *)(aw + 32) : (uint32_t)*(const uint16_t *)(pw + 32);
    s.wsh = sh;
}

__device__ __forceinline__ void q8_stage_store(uint8_t *stage, const Q8Stage &s) {
    const uint32_t tr = threadIdx.x >> 2, bi = threadIdx.x & 3;
    uint8_t *cx = stage + tr * 128, *cw = stage + 16384 + tr * 128;
    float *dx = (float *)(stage + 32768), *dw = (float *)(stage + 32768 + 2048);
    const uint32_t *xq = &s.x[1];
    uint32_t wq[8];
#pragma unroll
    for (int i = 0; i < 8; i++) wq[i] = s.wsh ? s.w[i + 1] : realign(s.w[i], s.w[i + 1], 2);
    const uint32_t dwb = realign(s.w[0], s.w[1], s.wsh) & 0xffffu;
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const uint32_t off = ((2 * bi + h) ^ (tr & 7)) << 4;
        *(vkf_u4 *)(cx + off) = s.xv ? vkf_u4{xq[4 * h], xq[4 * h + 1], xq[4 * h + 2], xq[4 * h + 3]}
                                     : vkf_u4{0, 0, 0, 0};
        *(vkf_u4 *)(cw + off) = s.wv ? vkf_u4{wq[4 * h], wq[4 * h + 1], wq[4 * h + 2], wq[4 * h + 3]}
                                     : vkf_u4{0, 0, 0, 0};
    }
    dx[bi * 128 + tr] = s.xv ? vkf_h2f((uint16_t)(s.x[0] & 0xffffu)) : 0.0f;
    dw[bi * 128 + tr] = s.wv ? vkf_h2f((uint16_t)dwb) : 0.0f;
}

template <bool PARTIALS>
__device__ __forceinline__ void gemm_q8_i8_body(const VkfGemmArgs &a) {
    __shared__ __attribute__((aligned(16))) uint8_t smem[QI_LDS];
    uint32_t r0, c0;
    gemm_tile_of(r0, c0);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int wc = wave & 1, wr = (wave >> 1) & 1, i0 = 2 * (wave >> 2);
    const int li = lane & 15, lg = lane >> 4;
    const uint32_t nb = a.K / 32, nk = (nb + 3) / 4;
    vkf_f4 acc[2][4];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = vkf_f4{0, 0, 0, 0};
    Q8Stage st;
    q8_stage_load(a, r0, c0, 0, st);
    q8_stage_store(smem, st);
    __syncthreads();
    for (uint32_t kt = 0; kt < nk; kt++) {
        if (kt + 1 < nk) q8_stage_load(a, r0, c0, kt + 1, st);
        const uint8_t *stage = smem + (kt & 1) * QI_STAGE;
        const float *dx = (const float *)(stage + 32768), *dw = (const float *)(stage + 32768 + 2048);
#pragma unroll 1
        for (int b = 0; b < 4; b++) {
            // 8 bytes of the block per lane: k-slice 8*lg, inside chunk 2b + lg/2
            const uint32_t c = 2 * b + (lg >> 1), off = 8 * (lg & 1);
            long fb[4];
            float sw[4];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const uint32_t cc = wc * 64 + 16 * j + li;
                fb[j] = *(const long *)(stage + 16384 + cc * 128 + ((c ^ (cc & 7)) << 4) + off);
                sw[j] = dw[b * 128 + cc];
            }
            // the block's 8 dots first (independent results, so the MFMAs
            // issue back to back), then their folds
            vkf_i4 P[2][4];
            vkf_f4 sx[2];
#pragma unroll
            for (int i = 0; i < 2; i++) {
                const uint32_t rr = wr * 64 + 16 * (i0 + i) + li;
                const long fa = *(const long *)(stage + rr * 128 + ((c ^ (rr & 7)) << 4) + off);
                sx[i] = *(const vkf_f4 *)(dx + b * 128 + wr * 64 + 16 * (i0 + i) + 4 * lg);
#pragma unroll
                for (int j = 0; j < 4; j++)
                    P[i][j] = __builtin_amdgcn_mfma_i32_16x16x32_i8(fa, fb[j], vkf_i4{0, 0, 0, 0}, 0, 0, 0);
            }
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    if constexpr (PARTIALS) {
                        const uint32_t kb = 4 * kt + b, n = c0 + wc * 64 + 16 * j + li;
#pragma unroll
                        for (int e = 0; e < 4; e++) {
                            const uint32_t m = r0 + wr * 64 + 16 * (i0 + i) + 4 * lg + e;
                            if (m < a.R && n < a.Cn && kb < nb)
                                ((int32_t *)a.D)[((uint64_t)m * a.Cn + n) * nb + kb] = P[i][j][e];
                        }
                    } else {
#pragma unroll
                        for (int e = 0; e < 4; e++)
                            acc[i][j][e] = fmaf((float)P[i][j][e], sx[i][e] * sw[j], acc[i][j][e]);
                    }
                }
        }
        if (kt + 1 < nk) q8_stage_store(smem + ((kt + 1) & 1) * QI_STAGE, st);
        __syncthreads();
    }
    if constexpr (!PARTIALS) {
        epi_stage<2>(a, r0, c0, acc, (float *)smem, wr, wc, nullptr, i0);
        __syncthreads();
        epi_store<512>(a, r0, c0, (const float *)smem);
    }
}

GEMM_KERNEL_W vkf_gemm_q8_0_q8_1_i8(VkfGemmArgs a) { gemm_q8_i8_body<false>(a); }
GEMM_KERNEL_W vkf_q8_0_q8_1_partials_mfma(VkfGemmArgs a) { gemm_q8_i8_body<true>(a); }

// ---------------------------------------------------------------------------
// fp32 x fp32 -> fp32 (hipblasSgemm and the fp32 hipblasGemmEx /
// vkflame_dispatch_linear(FP32) the reference routes to its fp16 shader,
// shim/hipblas_shim.cpp:84-113): v_mfma_f32_16x16x4_f32, 32 K per 128-byte
// step, fp32 epilogue and fp32 D.
// ---------------------------------------------------------------------------
GEMM_KERNEL vkf_gemm_f32(VkfGemmArgs a0) {
    const VkfGemmArgs a = gemm_batch(a0);
    __shared__ __attribute__((aligned(16))) uint8_t smem[GEMM_LDS_BOTH];
    uint32_t r0, c0;
    gemm_tile_of(r0, c0);
    vkf_f4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = vkf_f4{0, 0, 0, 0};
    if (dma_ok(a.X, a.ldx, (a.flags & VKF_GF_X_TRANS) != 0, a.K, 4) &&
        dma_ok(a.Y, a.ldy, (a.flags & VKF_GF_Y_TRANS) != 0, a.K, 4)) {
        gemm_mainloop_dma<4>(a, r0, c0, acc, smem);
    } else if (dma_ok(a.X, a.ldx, (a.flags & VKF_GF_X_TRANS) != 0, a.K, 4) && (a.flags & VKF_GF_Y_TRANS)) {
        gemm_mainloop_tdma<4>(a, r0, c0, acc, smem);
    } else {
        const auto ox = make_operand<4, -1>(a.X, a.ldx, (a.flags & VKF_GF_X_TRANS) != 0, a.R, r0, a.K);
        const auto oy = make_operand<4, -1>(a.Y, a.ldy, (a.flags & VKF_GF_Y_TRANS) != 0, a.Cn, c0, a.K);
        gemm_mainloop<4>(ox, oy, a.K, 32, acc, smem);
    }
    epilogue_tile(a, r0, c0, acc, smem);
}

// ---------------------------------------------------------------------------
// int8 x int8 -> int32 (kernels/linear_int8.glsl:54-93, with int8 A).
// flags & VKF_GF_D_F32 selects the float epilogue with fp32 D; VKF_GF_D_I32
// stores the raw int32 accumulator.
// ---------------------------------------------------------------------------
GEMM_KERNEL vkf_gemm_i8(VkfGemmArgs a0) {
    const VkfGemmArgs a = gemm_batch(a0);
    __shared__ __attribute__((aligned(16))) uint8_t smem[GEMM_LDS_BOTH];
    uint32_t r0, c0;
    gemm_tile_of(r0, c0);
    vkf_i4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = vkf_i4{0, 0, 0, 0};
    if (a.flags & VKF_GF_X_F16Q) {  // fp16 activations quantised as they are staged
        OperandF16Q ox;
        ox.P = (const _Float16 *)a.X;
        ox.ld = a.ldx;
        ox.trans = (a.flags & VKF_GF_X_TRANS) != 0;
        ox.fast = !ox.trans && (a.ldx % 8) == 0 && (((uintptr_t)a.X & 15) == 0);
        ox.nrows = a.R;
        ox.row0 = r0;
        ox.K = a.K;
        ox.s = a.xscale;
        const auto oy = make_operand<1, -1>(a.Y, a.ldy, (a.flags & VKF_GF_Y_TRANS) != 0, a.Cn, c0, a.K);
        gemm_mainloop<1>(ox, oy, a.K, 128, acc, smem);
    } else if (dma_ok(a.X, a.ldx, (a.flags & VKF_GF_X_TRANS) != 0, a.K, 1) &&
               dma_ok(a.Y, a.ldy, (a.flags & VKF_GF_Y_TRANS) != 0, a.K, 1)) {
        gemm_mainloop_dma<1>(a, r0, c0, acc, smem);
    } else if (dma_ok(a.X, a.ldx, (a.flags & VKF_GF_X_TRANS) != 0, a.K, 1) && (a.flags & VKF_GF_Y_TRANS)) {
        gemm_mainloop_tdma<1>(a, r0, c0, acc, smem);
    } else {
        const auto ox = make_operand<1, -1>(a.X, a.ldx, (a.flags & VKF_GF_X_TRANS) != 0, a.R, r0, a.K);
        const auto oy = make_operand<1, -1>(a.Y, a.ldy, (a.flags & VKF_GF_Y_TRANS) != 0, a.Cn, c0, a.K);
        gemm_mainloop<1>(ox, oy, a.K, 128, acc, smem);
    }
    if (!(a.flags & VKF_GF_D_I32)) {
        epilogue_tile(a, r0, c0, acc, smem);
        return;
    }
    // raw int32 accumulator with integer alpha/beta (hipblasGemmEx, compute 32I)
    const int wave = threadIdx.x >> 6, wr = wave >> 1, wc = wave & 1;
    const int lane = threadIdx.x & 63, li = lane & 15, lg = lane >> 4;
    const int32_t al = __builtin_bit_cast(int32_t, a.alpha), be = __builtin_bit_cast(int32_t, a.beta);
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const uint32_t r = r0 + wr * 64 + 16 * i + 4 * lg + e, c = c0 + wc * 64 + 16 * j + li;
                if (r < a.R && c < a.Cn) {
                    int32_t v = acc[i][j][e];
                    if (al != 1 || be != 0)
                        v = al * v + (be ? be * ((const int32_t *)a.Cin)[(uint64_t)r * a.ldc + c] : 0);
                    ((int32_t *)a.D)[(uint64_t)r * a.ldd + c] = v;
                }
            }
}


// ---------------------------------------------------------------------------
// Dense GEMM with the K loop split inside the workgroup, for grids with no
// more 128 x 128 tiles than the chip has CUs (M = 512 x N = 5120: 160 tiles
// on 256 CUs).  There the 256-thread kernel runs one workgroup, one wave per
// SIMD, on each busy CU, and nothing overlaps a wave's LDS fragment reads
// with its MFMAs.  Here 512 threads hold the same 128 x 128 tile: waves 0-3
// (group 0) take the even 128-byte K steps, waves 4-7 (group 1) the odd
// ones, each wave a 64 x 64 quadrant as in the 256-thread kernel, so every
// SIMD runs two waves.  Both groups' tiles of a step pair arrive by
// direct-to-LDS loads (two stages of 2 x 32 KiB); at the end group 1's
// accumulators go through LDS and group 0 adds them, the same order on every
// run (int32 sums are exact, fp32 ones differ from the sequential K order
// only in rounding).  Aligned K-contiguous operands with K*ES a multiple of
// 128 only (the host checks this before it picks these kernels).
// ---------------------------------------------------------------------------
#define GEMM_K2_LDS (2 * 65536)
#define GEMM_KERNEL_K2 VKF_KERNEL void __launch_bounds__(512)

// Split-K workgroups: group 1's (waves 4-7) accumulators -> LDS (lane-major,
// 64 KiB), group 0 adds them; ends with LDS free.  smem must be free.
template <class ACC>
__device__ __forceinline__ void k2_group_sum(ACC acc[4][4], uint8_t *smem) {
    const int wave = threadIdx.x >> 6, g = wave >> 2, wq = wave & 3, lane = threadIdx.x & 63;
    vkf_i4 *red = (vkf_i4 *)smem;
    if (g == 1) {
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int j = 0; j < 4; j++) red[(wq * 16 + 4 * i + j) * 64 + lane] = __builtin_bit_cast(vkf_i4, acc[i][j]);
    }
    __syncthreads();
    if (g == 0) {
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int j = 0; j < 4; j++) acc[i][j] += __builtin_bit_cast(ACC, red[(wq * 16 + 4 * i + j) * 64 + lane]);
    }
    __syncthreads();  // LDS free for the epilogue
}

template <int ES, class ACC>
__device__ __forceinline__ void gemm_mainloop_dma_k2(const VkfGemmArgs &a, uint32_t r0, uint32_t c0, ACC acc[4][4],
                                                     uint8_t *smem) {
    const int wave = threadIdx.x >> 6, g = wave >> 2, wq = wave & 3, lane = threadIdx.x & 63;
    const int wr = wq >> 1, wc = wq & 1;
    const uint32_t nk = (uint32_t)(((uint64_t)a.K * ES) / 128);
    const uint8_t *gx[4], *gy[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const uint32_t rr = (4 * wq + j) * 8 + (lane >> 3);
        const uint32_t ch = (lane & 7) ^ (rr & 7);
        const uint32_t rx = r0 + rr < a.R ? r0 + rr : a.R - 1;  // rows past the edge: any valid row
        const uint32_t ry = c0 + rr < a.Cn ? c0 + rr : a.Cn - 1;
        gx[j] = (const uint8_t *)a.X + (uint64_t)rx * a.ldx * ES + ch * 16;
        gy[j] = (const uint8_t *)a.Y + (uint64_t)ry * a.ldy * ES + ch * 16;
    }
    // step kt of this group into its half of stage st
    auto issue = [&](uint32_t kt, uint32_t st) {
        uint8_t *sx = smem + st * 65536 + g * 32768, *sy = sx + 16384;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t off = (4 * wq + j) * 8 * 128;
            vkf_load_lds16(gx[j] + (uint64_t)kt * 128, sx + off);
            vkf_load_lds16(gy[j] + (uint64_t)kt * 128, sy + off);
        }
    };
    const uint32_t npair = (nk + 1) / 2;
    if ((uint32_t)g < nk) issue(g, 0);
    for (uint32_t t = 0; t < npair; t++) {
        wait_vm<0>();  // this thread's loads of pair t are the only ones in flight
        __syncthreads();
        const uint32_t kn = 2 * (t + 1) + g;
        if (kn < nk) issue(kn, (t + 1) & 1);
        if (2 * t + g < nk) {
            const uint8_t *lx = smem + (t & 1) * 65536 + g * 32768;
            mfma_step_swz<ES>(lx, lx + 16384, wr, wc, acc);
        }
    }
    __syncthreads();  // LDS free for the reduction
    k2_group_sum(acc, smem);
}

// epilogue of the split-K kernels: group 0 stages the tile, all 512 threads store it
template <class ACC>
__device__ __forceinline__ void epilogue_tile_k2(const VkfGemmArgs &a, uint32_t r0, uint32_t c0, const ACC acc[4][4],
                                                 uint8_t *smem, const EpiPre *pre = nullptr) {
    const int wave = threadIdx.x >> 6;
    if (wave < 4) epi_stage(a, r0, c0, acc, (float *)smem, (wave & 3) >> 1, wave & 1, pre);
    __syncthreads();
    epi_store<512>(a, r0, c0, (const float *)smem);
}

GEMM_KERNEL_K2 vkf_gemm_f16_k2(VkfGemmArgs a0) {
    const VkfGemmArgs a = gemm_batch(a0);
    __shared__ __attribute__((aligned(16))) uint8_t smem[GEMM_K2_LDS];
    uint32_t r0, c0;
    gemm_tile_of(r0, c0);
    vkf_f4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = vkf_f4{0, 0, 0, 0};
    const int wave = threadIdx.x >> 6;
    EpiPre pre{};
    if (wave < 4) pre = epi_prefetch(a, r0, c0, wave >> 1, wave & 1);  // group 0 stages the tile
    gemm_mainloop_dma_k2<2>(a, r0, c0, acc, smem);
    epilogue_tile_k2(a, r0, c0, acc, smem, &pre);
}

GEMM_KERNEL_K2 vkf_gemm_i8_k2(VkfGemmArgs a0) {
    const VkfGemmArgs a = gemm_batch(a0);
    __shared__ __attribute__((aligned(16))) uint8_t smem[GEMM_K2_LDS];
    uint32_t r0, c0;
    gemm_tile_of(r0, c0);
    vkf_i4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = vkf_i4{0, 0, 0, 0};
    const int wv = threadIdx.x >> 6;
    EpiPre pre{};
    if (wv < 4 && !(a.flags & VKF_GF_D_I32)) pre = epi_prefetch(a, r0, c0, wv >> 1, wv & 1);
    gemm_mainloop_dma_k2<1>(a, r0, c0, acc, smem);
    if (!(a.flags & VKF_GF_D_I32)) {
        epilogue_tile_k2(a, r0, c0, acc, smem, &pre);
        return;
    }
    if (threadIdx.x >= 256) return;  // group 0 holds the sums; no barrier follows
    // raw int32 accumulator with integer alpha/beta (hipblasGemmEx, compute 32I)
    const int wave = threadIdx.x >> 6, wr = wave >> 1, wc = wave & 1;
    const int lane = threadIdx.x & 63, li = lane & 15, lg = lane >> 4;
    const int32_t al = __builtin_bit_cast(int32_t, a.alpha), be = __builtin_bit_cast(int32_t, a.beta);
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const uint32_t r = r0 + wr * 64 + 16 * i + 4 * lg + e, c = c0 + wc * 64 + 16 * j + li;
                if (r < a.R && c < a.Cn) {
                    int32_t v = acc[i][j][e];
                    if (al != 1 || be != 0)
                        v = al * v + (be ? be * ((const int32_t *)a.Cin)[(uint64_t)r * a.ldc + c] : 0);
                    ((int32_t *)a.D)[(uint64_t)r * a.ldd + c] = v;
                }
            }
}

// ---------------------------------------------------------------------------
// Quantised-weight GEMM with fp16 activations, K split inside the workgroup
// as in vkf_gemm_f16_k2: for grids of at most one 128 x 128 tile per CU
// (the down projections of a prefill, N = 4096..5120 at M = 512).  Group g
// (waves 4g..4g+3) loads the activation tile and decodes the weight tile of
// the K steps kt = g (mod 2) into its own half of each stage (QStage, the
// same values as the 256-thread kernel; group 1's threads see rows from
// threadIdx.x / 2 - 128 through row0 - 128); the two partial tiles meet in
// LDS at the end.  Needs the direct-to-LDS activation loads (16-byte aligned
// rows, K % 64 == 0; the host checks).
// ---------------------------------------------------------------------------
template <int QT>
__device__ __forceinline__ void gemm_mainloop_qdma_k2(const VkfGemmArgs &a, uint32_t r0, uint32_t c0,
                                                      vkf_f4 acc[4][4], uint8_t *smem) {
    const int wave = threadIdx.x >> 6, g = wave >> 2, wq = wave & 3, lane = threadIdx.x & 63;
    const int wr = wq >> 1, wc = wq & 1;
    const uint32_t nk = a.K / 64, npair = (nk + 1) / 2;
    const uint8_t *gx[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const uint32_t rr = (4 * wq + j) * 8 + (lane >> 3);
        const uint32_t ch = (lane & 7) ^ (rr & 7);
        const uint32_t rx = r0 + rr < a.R ? r0 + rr : a.R - 1;
        gx[j] = (const uint8_t *)a.X + (uint64_t)rx * a.ldx * 2 + ch * 16;
    }
    auto issue_x = [&](uint32_t kt, uint32_t st) {
        uint8_t *sx = smem + st * 65536 + g * 32768;
#pragma unroll
        for (int j = 0; j < 4; j++)
            vkf_load_lds16(gx[j] + (uint64_t)kt * 128, sx + (4 * wq + j) * 1024);
    };
    const uint32_t yr = (threadIdx.x & 255) >> 1, yh = threadIdx.x & 1;
    auto store_y = [&](uint32_t st, const TileRegs &t) {
        uint8_t *sy = smem + st * 65536 + g * 32768 + 16384 + yr * 128;
#pragma unroll
        for (int k = 0; k < 4; k++) *(vkf_i4 *)(sy + (((4 * yh + k) ^ (yr & 7)) << 4)) = t.v[k];
    };
    const uint32_t qrow0 = c0 - 128u * (uint32_t)g;  // + threadIdx.x / 2 (mod 2^32) = c0 + row in the tile
    QStage<QT> q;
    TileRegs ty;
    if ((uint32_t)g < nk) {
        issue_x(g, 0);
        q.load((const uint8_t *)a.Y, a.ldy, a.Cn, qrow0, a.K, 64u * g);
        q.decode(ty);
        store_y(0, ty);
    }
    wait_vm<0>();
    __syncthreads();
    for (uint32_t t = 0; t < npair; t++) {
        const uint32_t cur = t & 1, kn = 2 * (t + 1) + g;
        if (kn < nk) {
            issue_x(kn, cur ^ 1);
            q.load((const uint8_t *)a.Y, a.ldy, a.Cn, qrow0, a.K, kn * 64);
        }
        if (2 * t + g < nk) {
            const uint8_t *lx = smem + cur * 65536 + g * 32768;
            mfma_step_swz<2>(lx, lx + 16384, wr, wc, acc);
        }
        if (kn < nk) {
            q.decode(ty);
            store_y(cur ^ 1, ty);
        }
        wait_vm<0>();
        __syncthreads();
    }
    k2_group_sum(acc, smem);
}

template <int QT>
__device__ __forceinline__ void gemm_q_k2_body(const VkfGemmArgs &a) {
    __shared__ __attribute__((aligned(16))) uint8_t smem[GEMM_K2_LDS];
    uint32_t r0, c0;
    gemm_tile_of(r0, c0);
    vkf_f4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = vkf_f4{0, 0, 0, 0};
    // (no epilogue prefetch here: the 24 registers it holds through the main
    // loop made these kernels 10-14 % slower on MI355X)
    gemm_mainloop_qdma_k2<QT>(a, r0, c0, acc, smem);
    epilogue_tile_k2(a, r0, c0, acc, smem);
}

#define VKF_GEMM_Q_K2(name, QT) \
    GEMM_KERNEL_K2 vkf_gemm_##name##_f16_k2(VkfGemmArgs a) { gemm_q_k2_body<QT>(a); }
VKF_GEMM_Q_K2(q4_0, VKF_Q4_0)
VKF_GEMM_Q_K2(q4_1, VKF_Q4_1)
VKF_GEMM_Q_K2(q8_0, VKF_Q8_0)
VKF_GEMM_Q_K2(q5_0, VKF_Q5_0)
VKF_GEMM_Q_K2(q4_k, VKF_Q4_K)
VKF_GEMM_Q_K2(q5_k, VKF_Q5_K)
VKF_GEMM_Q_K2(q6_k, VKF_Q6_K)

// ---------------------------------------------------------------------------
// Skinny fp16 GEMM: at most 64 rows of X (decode-sized batches, torch.mm of
// a few rows).  So few rows give a 128-row tile nothing to reuse: the kernel
// is a stream of Y at HBM speed with the rows of X alongside.  One 1024-
// thread workgroup per 16 columns of Y; its 16 waves split K in 32-k steps,
// each wave accumulating 16 columns x up to 64 rows on 16x16x32 MFMAs, and
// the 16 partial tiles are summed in LDS in wave order (a fixed order: the
// result is repeatable).  Per step a lane loads its 16 bytes of X straight
// from global memory (rows past R: zero operands, no load) and its B
// fragment:
//   Y stored [C, K] (NT): Y[c0 + j][32t + 8g .. +7], one 16-byte load;
//   Y stored [K, C] (NN): the step's 32 k-rows x 16 columns (32 bytes each)
//     go to the wave's LDS by one direct load (lane L: row L/2, columns
//     8(L&1) ..), read back as the fragment by two ds_read_b64_tr_b16 (the
//     lane layout of mfma_step_trb; 32-byte rows fall on distinct banks).
// A wave loads CH steps, then multiplies them; 16 waves per CU keep the
// loads of the others in flight meanwhile.  Workgroups b, b+8, b+16, ...
// share an XCD and take consecutive column tiles, so tiles that share Y's
// lines (NN: four per 128-byte line) share that XCD's L2.  Conditions
// (host): X K-contiguous, 16-byte aligned, ldx % 8 == 0; K % 32 == 0; Y
// 16-byte aligned with ldy % 8 == 0, and C % 8 == 0 for NN.
// ---------------------------------------------------------------------------
#define SK_WAVES 16

__device__ __forceinline__ float epi_one(const VkfGemmArgs &a, uint32_t r, uint32_t c, float v) {
    // the per-value epilogue of epi_stage, in the same order
    if (a.rs) v *= a.rs[(a.flags & VKF_GF_RS_SCALAR) ? 0 : r];
    if (a.cs) v *= a.cs[(a.flags & VKF_GF_CS_SCALAR) ? 0 : c];
    v *= a.alpha;
    if (a.beta != 0.0f) {
        const float cin = (a.flags & VKF_GF_CIN_F32) ? ((const float *)a.Cin)[(uint64_t)r * a.ldc + c]
                                                     : (float)((const _Float16 *)a.Cin)[(uint64_t)r * a.ldc + c];
        v = fmaf(a.beta, cin, v);
    }
    if (a.bias) {
        const uint32_t bi = (a.flags & VKF_GF_BIAS_ROW) ? r : c;
        v += (a.flags & VKF_GF_BIAS_F32) ? ((const float *)a.bias)[bi] : (float)((const _Float16 *)a.bias)[bi];
    }
    return vkf_act(a.act, v);
}

template <int MB, bool YT>
__device__ __forceinline__ void gemm_skinny(const VkfGemmArgs &a, uint8_t *smem) {
    constexpr int CH = MB <= 2 ? 8 : 4;  // 32-k steps per load batch
    const int lane = threadIdx.x & 63, li = lane & 15, lg = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    uint32_t tile = blockIdx.x;
    {
        const uint32_t per = gridDim.x / 8;
        if (blockIdx.x < per * 8) tile = (blockIdx.x % 8) * per + blockIdx.x / 8;
    }
    const uint32_t c0 = tile * 16;
    const uint32_t ns = a.K / 32, s0 = wave * ns / SK_WAVES, s1 = (wave + 1) * ns / SK_WAVES;

    const uint8_t *xrow[MB];
    bool xlive[MB];
#pragma unroll
    for (int m = 0; m < MB; m++) {
        const uint32_t r = 16 * m + li;
        xlive[m] = r < a.R;
        xrow[m] = (const uint8_t *)a.X + (uint64_t)(xlive[m] ? r : 0) * a.ldx * 2 + 16 * lg;
    }
    const uint8_t *yp;
    uint64_t ystep;  // bytes per 32-k step
    if constexpr (YT) {
        const uint32_t col = c0 + 8 * (lane & 1) < a.Cn ? c0 + 8 * (lane & 1) : a.Cn - 8;  // past the edge: any valid
        yp = (const uint8_t *)a.Y + ((uint64_t)(lane >> 1) * a.ldy + col) * 2;
        ystep = (uint64_t)32 * a.ldy * 2;
    } else {
        const uint32_t c = c0 + li < a.Cn ? c0 + li : a.Cn - 1;
        yp = (const uint8_t *)a.Y + (uint64_t)c * a.ldy * 2 + 16 * lg;
        ystep = 64;
    }
    uint8_t *ring = smem + wave * CH * 1024;  // NN: this wave's staged steps
    const int rsub = li >> 2, hb = (li & 1) * 8, pcol = ((li & 3) >> 1) * 16;

    vkf_f4 acc[MB];
#pragma unroll
    for (int m = 0; m < MB; m++) acc[m] = vkf_f4{0, 0, 0, 0};
    for (uint32_t t0 = s0; t0 < s1; t0 += CH) {  // wave-uniform
        const uint32_t n = s1 - t0 < CH ? s1 - t0 : CH;
        vkf_i4 xa[CH][MB], yb[CH];
        if constexpr (YT) {
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the ring's previous reads are done
#pragma unroll
            for (int q = 0; q < CH; q++)
                if (q < (int)n) vkf_load_lds16_nt(yp + (t0 + q) * ystep, ring + q * 1024);
        }
#pragma unroll
        for (int q = 0; q < CH; q++) {
            if (q < (int)n) {
                if constexpr (!YT) yb[q] = *(const vkf_i4 *)(yp + (t0 + q) * ystep);
#pragma unroll
                for (int m = 0; m < MB; m++)
                    xa[q][m] = xlive[m] ? *(const vkf_i4 *)(xrow[m] + (uint64_t)(t0 + q) * 64) : vkf_i4{0, 0, 0, 0};
            }
        }
        if constexpr (YT) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
        for (int q = 0; q < CH; q++) {
            if (q < (int)n) {
                vkf_i4 fb;
                if constexpr (YT) {
                    // rows 8g + 4h + (li >> 2) of the step, columns 4(li & 3) ..
                    const uint8_t *p = ring + q * 1024 + (8 * lg + rsub) * 32 + pcol + hb;
                    const vkf_i2 lo = lds_read_tr16(p), hi = lds_read_tr16(p + 4 * 32);
                    fb = vkf_i4{lo[0], lo[1], hi[0], hi[1]};
                } else {
                    fb = yb[q];
                }
#pragma unroll
                for (int m = 0; m < MB; m++) acc[m] = mfma_frag<2>(xa[q][m], fb, acc[m]);
            }
        }
    }
    // partial tiles of the 16 waves summed in wave order
    __syncthreads();
    float *red = (float *)smem;  // [wave][m][lane][4]
#pragma unroll
    for (int m = 0; m < MB; m++) *(vkf_f4 *)(red + ((wave * MB + m) * 64 + lane) * 4) = acc[m];
    __syncthreads();
    if (wave < MB) {
        const int m = wave;
        vkf_f4 s = *(const vkf_f4 *)(red + (m * 64 + lane) * 4);
        for (int w = 1; w < SK_WAVES; w++) {
            const vkf_f4 v = *(const vkf_f4 *)(red + ((w * MB + m) * 64 + lane) * 4);
#pragma unroll
            for (int e = 0; e < 4; e++) s[e] += v[e];
        }
        const uint32_t c = c0 + li;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const uint32_t r = 16 * m + 4 * lg + e;
            if (r < a.R && c < a.Cn) {
                const float v = epi_one(a, r, c, s[e]);
                if (a.flags & VKF_GF_D_F32) ((float *)a.D)[(uint64_t)r * a.ldd + c] = v;
                else ((_Float16 *)a.D)[(uint64_t)r * a.ldd + c] = vkf_to_f16(v);
            }
        }
    }
}

// LDS: the NN staging ring (16 waves x CH KiB) or the partial tiles
// (16 waves x MB KiB), the larger: 128 KiB
VKF_KERNEL void __launch_bounds__(64 * SK_WAVES) vkf_gemm_f16_skinny(VkfGemmArgs a0) {
    extern __shared__ __attribute__((aligned(16))) uint8_t sk_smem[];
    const VkfGemmArgs a = gemm_batch(a0);
    const bool yt = (a.flags & VKF_GF_Y_TRANS) != 0;
    if (a.R <= 16) {
        if (yt) gemm_skinny<1, true>(a, sk_smem);
        else gemm_skinny<1, false>(a, sk_smem);
    } else if (a.R <= 32) {
        if (yt) gemm_skinny<2, true>(a, sk_smem);
        else gemm_skinny<2, false>(a, sk_smem);
    } else {
        if (yt) gemm_skinny<4, true>(a, sk_smem);
        else gemm_skinny<4, false>(a, sk_smem);
    }
}

// ---------------------------------------------------------------------------
// Dense GEMM on narrow tiles for grids of fewer 128 x 128 tiles than CUs:
// 128 x 16·NB tiles (NB = 4 or 5: 64 or 80 columns), NB picked on the host
// as the narrowest tile whose grid still fits one tile per CU (M = 512,
// N = 5120: 4 x 64 = 256 tiles of 128 x 80, where 128 x 128 tiles give 160
// and leave 96 CUs idle).  At these sizes a CU's time is its tile traffic
// over the rate one CU can pull from L2 / MALL, which is set by the bytes it
// keeps in flight; the narrower tile moves (128 + 16·NB)·K instead of 256·K
// elements per CU, on every CU, and leaves room for three stages.
// K is split inside the workgroup as in the split-K kernels: waves 0-3 take
// the even 128-byte K steps and waves 4-7 the odd ones; wave q of a group
// owns rows 32q .. 32q + 31 of the tile and all its columns (2 x NB
// fragments of 16 x 16).  Three stages of both groups' steps (3 x 52 KiB
// for NB = 5) keep two pairs of steps in flight while one is multiplied.
// The group partials meet in LDS, each group then finishing half the tile
// (int32 exact; fp32 the same bits as one group adding both).  Conditions
// (host): X and Y K-contiguous (or, fp16 only, Y stored [K, C]: the NN
// variant), 16-byte aligned, 16-byte rows, K·ES % 256 == 0 (whole pairs of
// steps).  Dynamic LDS: 3 stages x 2 groups x (16 KiB + NB·2 KiB).
// ---------------------------------------------------------------------------

template <int ES, int NB, class ACC>
__device__ __forceinline__ void mfma_step_n(const uint8_t *lx, const uint8_t *ly, int wq, ACC acc[2][NB]) {
    const int lane = threadIdx.x & 63, li = lane & 15, lg = lane >> 4, sw = li & 7;
    vkf_i4 fa[2][2], fb[2][NB];
#pragma unroll
    for (int s = 0; s < 2; s++) {
        const int c = 4 * s + lg;
#pragma unroll
        for (int i = 0; i < 2; i++)
            fa[s][i] = *(const vkf_i4 *)(lx + (wq * 32 + 16 * i + li) * 128 + ((c ^ sw) << 4));
#pragma unroll
        for (int j = 0; j < NB; j++) fb[s][j] = *(const vkf_i4 *)(ly + (16 * j + li) * 128 + ((c ^ sw) << 4));
    }
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int s = 0; s < 2; s++)
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int j = 0; j < NB; j++) acc[i][j] = mfma_frag<ES>(fa[s][i], fb[s][j], acc[i][j]);
    __builtin_amdgcn_s_setprio(0);
}

// The same step with Y stored [K, C] (fp16, NN): the step's 64 k-rows of
// the tile's 16·NB columns lie in LDS as rows of 32·NB bytes, and each B
// fragment is read by two ds_read_b64_tr_b16 (the lane layout of
// mfma_step_trb: the 4 rows of a 16-lane read must fall on different
// banks).  NB = 4: 128-byte rows, row k's 16-byte piece p in slot
// p ^ 2(k & 3); NB = 2 and 5: 64- and 160-byte rows as they lie (rows 16
// or 40 dwords apart already fall on different banks).
template <int NB>
__device__ __forceinline__ uint32_t trb_slot(uint32_t p, uint32_t k) {
    static_assert(NB >= 1 && NB <= 5, "NN narrow tiles: 16 to 80 columns");
    return NB == 4 ? p ^ (2 * (k & 3)) : p;
}
template <int NB, class ACC>
__device__ __forceinline__ void mfma_step_n_trb(const uint8_t *lx, const uint8_t *ly, int wq, ACC acc[2][NB]) {
    constexpr int PR = 32 * NB;  // bytes per k-row
    const int lane = threadIdx.x & 63, li = lane & 15, lg = lane >> 4, sw = li & 7;
    const int rsub = li >> 2, hb = (li & 1) * 8;  // this lane's row in a 4-row read, half of its piece
    vkf_i4 fa[2][2], fb[2][NB];
#pragma unroll
    for (int s = 0; s < 2; s++) {
        const int c = 4 * s + lg;
#pragma unroll
        for (int i = 0; i < 2; i++)
            fa[s][i] = *(const vkf_i4 *)(lx + (wq * 32 + 16 * i + li) * 128 + ((c ^ sw) << 4));
#pragma unroll
        for (int j = 0; j < NB; j++) {
            const int slot = trb_slot<NB>(2 * j + ((li & 3) >> 1), rsub);
            const uint8_t *q = ly + (32 * s + 8 * lg + rsub) * PR + slot * 16 + hb;
            const vkf_i2 lo = lds_read_tr16(q), hi = lds_read_tr16(q + 4 * PR);
            fb[s][j] = vkf_i4{lo[0], lo[1], hi[0], hi[1]};
        }
    }
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int s = 0; s < 2; s++)
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int j = 0; j < NB; j++) acc[i][j] = mfma_frag<2>(fa[s][i], fb[s][j], acc[i][j]);
    __builtin_amdgcn_s_setprio(0);
}

template <int ES, int NB, bool YT, class ACC>
__device__ __forceinline__ void gemm_mainloop_n(const VkfGemmArgs &a, uint32_t r0, uint32_t c0, ACC acc[2][NB],
                                                uint8_t *smem) {
    constexpr uint32_t SX = 16384, SG = SX + NB * 16 * 128, SP = 2 * SG;
    constexpr int NCH = 2 * NB;             // 8-row chunks of the Y tile
    constexpr int NYC = (NCH + 3) / 4;      // the most chunks one wave loads
    const int wave = threadIdx.x >> 6, g = wave >> 2, wq = wave & 3, lane = threadIdx.x & 63;
    const int ny = (NCH - wq + 3) / 4;      // this wave's chunks: wq, wq + 4, ...
    const uint32_t npair = (uint32_t)(((uint64_t)a.K * ES) / 256);
    const uint8_t *gx[4], *gy[NYC];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const uint32_t rr = (4 * wq + j) * 8 + (lane >> 3);
        const uint32_t ch = (lane & 7) ^ (rr & 7);
        const uint32_t rx = r0 + rr < a.R ? r0 + rr : a.R - 1;  // rows past the edge: any valid row
        gx[j] = (const uint8_t *)a.X + (uint64_t)rx * a.ldx * ES + ch * 16;
    }
#pragma unroll
    for (int j = 0; j < NYC; j++) {
        if constexpr (YT) {
            // NN: the chunk's 64 lanes fill LDS pieces 64c .. 64c + 63 of the
            // step's 64 k-rows of 2·NB pieces; piece P = k-row P / (2·NB), slot
            // P % (2·NB), which holds the columns of piece trb_slot(slot, kr)
            const uint32_t P = (wq + 4 * j) * 64 + lane, kr = P / (2 * NB);
            const uint32_t pc = trb_slot<NB>(P % (2 * NB), kr);
            const uint32_t col = c0 + 8 * pc < a.Cn ? c0 + 8 * pc : a.Cn - 8;  // pieces past the edge: any valid one
            gy[j] = (const uint8_t *)a.Y + ((uint64_t)kr * a.ldy + col) * 2;
        } else {
            const uint32_t rr = (wq + 4 * j) * 8 + (lane >> 3);
            const uint32_t ch = (lane & 7) ^ (rr & 7);
            const uint32_t ry = c0 + rr < a.Cn ? c0 + rr : a.Cn - 1;
            gy[j] = (const uint8_t *)a.Y + (uint64_t)ry * a.ldy * ES + ch * 16;
        }
    }
    // this group's step of pair p into stage st
    auto issue = [&](uint32_t p, uint32_t st) {
        const uint64_t ko = (uint64_t)(2 * p + g) * 128;
        const uint64_t yo = YT ? (uint64_t)(2 * p + g) * 64 * a.ldy * 2 : ko;
        uint8_t *sx = smem + st * SP + g * SG, *sy = sx + SX;
#pragma unroll
        for (int j = 0; j < 4; j++) vkf_load_lds16(gx[j] + ko, sx + (4 * wq + j) * 1024);
#pragma unroll
        for (int j = 0; j < NYC; j++)
            if (j < ny) vkf_load_lds16(gy[j] + yo, sy + (wq + 4 * j) * 1024);
    };
    if (npair > 0) issue(0, 0);
    if (npair > 1) issue(1, 1);
    uint32_t st = 0;  // stage of pair t
    for (uint32_t t = 0; t < npair; t++) {
        // pair t landed; pair t + 1 (4 + ny loads of this wave) may stay in flight
        if (t + 1 < npair) {
            if (ny == NYC) wait_vm<4 + NYC>();
            else wait_vm<4 + NYC - 1>();
        } else {
            wait_vm<0>();
        }
        __syncthreads();  // every wave's part of pair t is in LDS; pair t - 1's stage is free
        if (t + 2 < npair) issue(t + 2, st == 0 ? 2 : st - 1);
        const uint8_t *lx = smem + st * SP + g * SG;
        if constexpr (YT) mfma_step_n_trb<NB>(lx, lx + SX, wq, acc);
        else mfma_step_n<ES, NB>(lx, lx + SX, wq, acc);
        st = st == 2 ? 0 : st + 1;
    }
    __syncthreads();  // LDS free for the group sums
}

// The two groups' partial tiles meet in LDS: group g keeps its 16-row
// fragment row i = g (rows 32q + 16g .. + 15 of wave q's 32), sends the
// other to LDS and adds the other group's partial of its own, so each group
// then holds the sums of half the tile (fp32: a + b == b + a, the same bits
// whichever group adds).
template <int NB, class ACC>
__device__ __forceinline__ void gemm_group_exchange_n(ACC acc[2][NB], ACC mine[NB], uint8_t *smem) {
    const int wave = threadIdx.x >> 6, g = wave >> 2, wq = wave & 3, lane = threadIdx.x & 63;
    vkf_i4 *red = (vkf_i4 *)smem;  // [group that sends][wave][NB][64 lanes]
    const bool g1 = g != 0;
    // element-wise selects (no indexing of acc by g, which would put it in scratch)
#pragma unroll
    for (int j = 0; j < NB; j++) {
        const vkf_i4 a0 = __builtin_bit_cast(vkf_i4, acc[0][j]), a1 = __builtin_bit_cast(vkf_i4, acc[1][j]);
        vkf_i4 snd, keep;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            snd[e] = g1 ? a0[e] : a1[e];
            keep[e] = g1 ? a1[e] : a0[e];
        }
        red[((g * 4 + wq) * NB + j) * 64 + lane] = snd;
        mine[j] = __builtin_bit_cast(ACC, keep);
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < NB; j++) mine[j] += __builtin_bit_cast(ACC, red[(((g ^ 1) * 4 + wq) * NB + j) * 64 + lane]);
    __syncthreads();  // LDS free for the epilogue
}

// Workgroup -> RTT x CT tile, XCD-aware as gemm_tile_of: column tiles dealt
// to the 8 XCDs round-robin, each XCD running all row tiles of a column.
template <uint32_t CT, uint32_t RTT = 128>
__device__ __forceinline__ void gemm_tile_of_n(uint32_t &r0, uint32_t &c0) {
    const uint32_t nc = gridDim.x, nr = gridDim.y, id = blockIdx.x + nc * blockIdx.y;
    const uint32_t full = nc & ~7u;
    uint32_t r, c;
    if (id < full * nr) {
        const uint32_t x = id & 7u, sl = id >> 3;
        c = (sl / nr) * 8 + x;
        r = sl % nr;
    } else {
        const uint32_t j = id - full * nr;
        c = full + j / nr;
        r = j % nr;
    }
    r0 = r * RTT;
    c0 = c * CT;
}

// A thread's row and column factors of the epilogue (row scale, column
// scale, bias) for the 4 rows x NB columns it finishes, loaded before the
// main loop so that their latency is hidden.
template <int NB>
struct EpiPreN {
    float rs[4], br[4], cs[NB], bc[NB];
};
template <int NB>
__device__ __forceinline__ EpiPreN<NB> epi_prefetch_n(const VkfGemmArgs &a, uint32_t r0, uint32_t c0) {
    const int wave = threadIdx.x >> 6, g = wave >> 2, wq = wave & 3, lane = threadIdx.x & 63, li = lane & 15,
              lg = lane >> 4;
    const bool bf32 = (a.flags & VKF_GF_BIAS_F32) != 0, brow = (a.flags & VKF_GF_BIAS_ROW) != 0;
    EpiPreN<NB> p;
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const uint32_t tr = wq * 32 + 16 * g + 4 * lg + e, r = r0 + tr < a.R ? r0 + tr : a.R - 1;
        p.rs[e] = a.rs ? a.rs[(a.flags & VKF_GF_RS_SCALAR) ? 0 : r] : 1.0f;
        p.br[e] = (a.bias && brow) ? (bf32 ? ((const float *)a.bias)[r] : (float)((const _Float16 *)a.bias)[r]) : 0.0f;
    }
#pragma unroll
    for (int j = 0; j < NB; j++) {
        const uint32_t tc = 16 * j + li, c = c0 + tc < a.Cn ? c0 + tc : a.Cn - 1;
        p.cs[j] = a.cs ? a.cs[(a.flags & VKF_GF_CS_SCALAR) ? 0 : c] : 1.0f;
        p.bc[j] = (a.bias && !brow) ? (bf32 ? ((const float *)a.bias)[c] : (float)((const _Float16 *)a.bias)[c]) : 0.0f;
    }
    return p;
}

// The float epilogue (epi_one's steps per value) of each group's half of
// the sums through an fp32 tile in LDS, then 16-byte row stores by all 512
// threads.  D_I32: each group stores its raw int32 sums with integer
// alpha / beta.
template <int ES, int NB, class ACC>
__device__ __forceinline__ void gemm_epilogue_n(const VkfGemmArgs &a, uint32_t r0, uint32_t c0, const ACC mine[NB],
                                                uint8_t *smem, const EpiPreN<NB> &pre) {
    constexpr uint32_t CT = 16 * NB, TP = CT + 4;
    const int wave = threadIdx.x >> 6, g = wave >> 2, wq = wave & 3, lane = threadIdx.x & 63, li = lane & 15,
              lg = lane >> 4;
    if constexpr (ES == 1) {
        if (a.flags & VKF_GF_D_I32) {
            const int32_t al = __builtin_bit_cast(int32_t, a.alpha), be = __builtin_bit_cast(int32_t, a.beta);
#pragma unroll
            for (int j = 0; j < NB; j++)
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const uint32_t r = r0 + wq * 32 + 16 * g + 4 * lg + e, c = c0 + 16 * j + li;
                    if (r < a.R && c < a.Cn) {
                        int32_t v = mine[j][e];
                        if (al != 1 || be != 0)
                            v = al * v + (be ? be * ((const int32_t *)a.Cin)[(uint64_t)r * a.ldc + c] : 0);
                        ((int32_t *)a.D)[(uint64_t)r * a.ldd + c] = v;
                    }
                }
            return;  // no barrier follows
        }
    }
    float *tile = (float *)smem;
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const uint32_t tr = wq * 32 + 16 * g + 4 * lg + e, r = r0 + tr < a.R ? r0 + tr : a.R - 1;
#pragma unroll
        for (int j = 0; j < NB; j++) {
            const uint32_t tc = 16 * j + li, c = c0 + tc < a.Cn ? c0 + tc : a.Cn - 1;
            // epi_one's steps, with the row and column factors from registers
            float v = (float)mine[j][e];
            if (a.rs) v *= pre.rs[e];
            if (a.cs) v *= pre.cs[j];
            v *= a.alpha;
            if (a.beta != 0.0f) {
                const float cin = (a.flags & VKF_GF_CIN_F32) ? ((const float *)a.Cin)[(uint64_t)r * a.ldc + c]
                                                             : (float)((const _Float16 *)a.Cin)[(uint64_t)r * a.ldc + c];
                v = fmaf(a.beta, cin, v);
            }
            if (a.bias) v += (a.flags & VKF_GF_BIAS_ROW) ? pre.br[e] : pre.bc[j];
            tile[tr * TP + tc] = vkf_act(a.act, v);
        }
    }
    __syncthreads();
    const bool f32 = (a.flags & VKF_GF_D_F32) != 0;
    const uint32_t vec = f32 ? 4 : 8;  // elements per 16-byte store
    const bool vok = (a.ldd % vec) == 0 && (((uintptr_t)a.D & 15) == 0);
    const uint32_t per_row = CT / vec;
    for (uint32_t q = threadIdx.x; q < 128 * per_row; q += 512) {
        const uint32_t tr = q / per_row, tc = (q % per_row) * vec;
        const uint32_t r = r0 + tr, c = c0 + tc;
        if (r >= a.R || c >= a.Cn) continue;
        const float *src = tile + tr * TP + tc;
        if (vok && c + vec <= a.Cn) {
            if (f32) {
                *(vkf_f4 *)((float *)a.D + (uint64_t)r * a.ldd + c) = *(const vkf_f4 *)src;
            } else {
                vkf_h8 h;
#pragma unroll
                for (int k = 0; k < 8; k++) h[k] = vkf_to_f16(src[k]);
                *(vkf_h8 *)((_Float16 *)a.D + (uint64_t)r * a.ldd + c) = h;
            }
        } else {
            for (uint32_t k = 0; k < vec && c + k < a.Cn; k++) {
                if (f32) ((float *)a.D)[(uint64_t)r * a.ldd + c + k] = src[k];
                else ((_Float16 *)a.D)[(uint64_t)r * a.ldd + c + k] = vkf_to_f16(src[k]);
            }
        }
    }
}

template <int ES, int NB, class ACC, bool YT = false>
__device__ __forceinline__ void gemm_n_body(const VkfGemmArgs &a0, uint8_t *smem) {
    const VkfGemmArgs a = gemm_batch(a0);
    uint32_t r0, c0;
    gemm_tile_of_n<16 * NB>(r0, c0);
    ACC acc[2][NB];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < NB; j++) acc[i][j] = ACC{0, 0, 0, 0};
    EpiPreN<NB> pre{};
    if (!(ES == 1 && (a.flags & VKF_GF_D_I32))) pre = epi_prefetch_n<NB>(a, r0, c0);
    gemm_mainloop_n<ES, NB, YT>(a, r0, c0, acc, smem);
    ACC mine[NB];
    gemm_group_exchange_n<NB>(acc, mine, smem);
    gemm_epilogue_n<ES, NB>(a, r0, c0, mine, smem, pre);
}

// dynamic LDS: 3 x 2 x (16 KiB + NB·2 KiB) (156 KiB for NB = 5)
#define VKF_GEMM_N(name, ES, ACC, NB)                                                \
    VKF_KERNEL void __launch_bounds__(512) vkf_gemm_##name##_n##NB(VkfGemmArgs a) { \
        extern __shared__ __attribute__((aligned(16))) uint8_t gn_smem[];          \
        gemm_n_body<ES, NB, ACC>(a, gn_smem);                                        \
    }
VKF_GEMM_N(f16, 2, vkf_f4, 1)
VKF_GEMM_N(f16, 2, vkf_f4, 2)
VKF_GEMM_N(f16, 2, vkf_f4, 3)
VKF_GEMM_N(f16, 2, vkf_f4, 4)
VKF_GEMM_N(f16, 2, vkf_f4, 5)
VKF_GEMM_N(i8, 1, vkf_i4, 1)
VKF_GEMM_N(i8, 1, vkf_i4, 2)
VKF_GEMM_N(i8, 1, vkf_i4, 3)
VKF_GEMM_N(i8, 1, vkf_i4, 4)
VKF_GEMM_N(i8, 1, vkf_i4, 5)
// fp16 with Y stored [K, C] (NN), 128 x 16, 32, 64 or 80 tiles; Y: 16-byte
// aligned, ldy % 8 == 0, C % 8 == 0
VKF_KERNEL void __launch_bounds__(512) vkf_gemm_f16_n1t(VkfGemmArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t gn_smem[];
    gemm_n_body<2, 1, vkf_f4, true>(a, gn_smem);
}
VKF_KERNEL void __launch_bounds__(512) vkf_gemm_f16_n2t(VkfGemmArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t gn_smem[];
    gemm_n_body<2, 2, vkf_f4, true>(a, gn_smem);
}
VKF_KERNEL void __launch_bounds__(512) vkf_gemm_f16_n4t(VkfGemmArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t gn_smem[];
    gemm_n_body<2, 4, vkf_f4, true>(a, gn_smem);
}
VKF_KERNEL void __launch_bounds__(512) vkf_gemm_f16_n5t(VkfGemmArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t gn_smem[];
    gemm_n_body<2, 5, vkf_f4, true>(a, gn_smem);
}

// ---------------------------------------------------------------------------
// Q4_K weights x fp16 activations on narrow tiles (128 x 16·NB, NB = 4 or
// 5) for grids of fewer 128 x 128 tiles than CUs, the down projections of a
// prefill (M = 512, N = 5120, K = 13824: 256 tiles of 128 x 80).  As in the
// dense narrow kernel the two wave groups take alternate 64-k steps and X
// moves by direct-to-LDS loads three stages deep; here the weights move the
// same way, as raw Q4_K bytes, so that every global load of the main loop
// is counted by hand and none waits for another: per row and 64-k step the
// super-block header and the step's 32 bytes of codes (three 16-byte
// pieces; lane L of wave q loads piece L % 3 of row 4·NB·q + L / 3), three
// steps ahead.  Each step's pieces are decoded (QStage<VKF_Q4_K>: the
// reference's fp32 value, rounded to fp16) from LDS into a double-buffered
// fp16 tile in the MFMA layout one step ahead of the MFMAs that read it.
// LDS: X 3 x 2 x 16 KiB, fp16 weights 2 x 2 x NB·2 KiB, raw 3 x 2 x NB·768
// bytes (158.5 KiB at NB = 5).  Conditions (host): X K-contiguous, 16-byte
// aligned, 16-byte rows; W 16-byte aligned rows; K % 256 == 0.
// ---------------------------------------------------------------------------
template <int NB>
struct QnLayout {
    static constexpr uint32_t XS = 2 * 16384;                      // X, per stage (both groups)
    static constexpr uint32_t Y16 = 3 * XS, YG = NB * 16 * 128;     // fp16 weights, per group
    static constexpr uint32_t YS = 2 * YG;
    static constexpr uint32_t RAW = Y16 + 2 * YS, RG = NB * 16 * 48; // raw Q4_K pieces, per group
    static constexpr uint32_t RS = 2 * RG;
    static constexpr uint32_t BYTES = RAW + 3 * RS;
};

template <int NB>
__device__ __forceinline__ void gemm_mainloop_q4k_n(const VkfGemmArgs &a, uint32_t r0, uint32_t c0,
                                                    vkf_f4 acc[2][NB], uint8_t *smem) {
    using L = QnLayout<NB>;
    constexpr int RW = 4 * NB;  // weight rows per wave (raw loads and decode)
    const int wave = threadIdx.x >> 6, g = wave >> 2, wq = wave & 3, lane = threadIdx.x & 63;
    const uint32_t npair = a.K / 128;
    const uint8_t *gx[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const uint32_t rr = (4 * wq + j) * 8 + (lane >> 3);
        const uint32_t ch = (lane & 7) ^ (rr & 7);
        const uint32_t rx = r0 + rr < a.R ? r0 + rr : a.R - 1;  // rows past the edge: any valid row
        gx[j] = (const uint8_t *)a.X + (uint64_t)rx * a.ldx * 2 + ch * 16;
    }
    // raw pieces: lane L < 3·RW loads piece L % 3 of tile row RW·wq + L / 3
    const bool rlive = lane < 3 * RW;
    const uint32_t rrow = RW * wq + (rlive ? (uint32_t)lane / 3 : 0u), rpc = (uint32_t)lane % 3;
    const uint32_t wrow = c0 + rrow < a.Cn ? c0 + rrow : a.Cn - 1;
    const uint8_t *wsrc = (const uint8_t *)a.Y + (uint64_t)wrow * a.ldy + 16 * rpc;
    // decode: lane L < 2·RW of wave q takes half (L & 1) of tile row RW·wq + L / 2
    const bool dlive = lane < 2 * RW;
    const uint32_t yr = RW * wq + (dlive ? (uint32_t)lane >> 1 : 0u), yh = lane & 1;
    auto issue_x = [&](uint32_t p, uint32_t st) {
        const uint64_t ko = (uint64_t)(2 * p + g) * 128;
        uint8_t *sx = smem + st * L::XS + g * 16384;
#pragma unroll
        for (int j = 0; j < 4; j++) vkf_load_lds16(gx[j] + ko, sx + (4 * wq + j) * 1024);
    };
    auto issue_raw = [&](uint32_t p, uint32_t slot) {
        const uint32_t ks = 2 * p + g;  // this group's 64-k step: super-block ks / 4, code run ks % 4
        const uint8_t *src = wsrc + 144ull * (ks >> 2) + (rpc ? 32 * (ks & 3) : 0);
        if (rlive) vkf_load_lds16(src, smem + L::RAW + slot * L::RS + g * L::RG + wq * (3 * RW * 16));
    };
    auto decode = [&](uint32_t p, uint32_t slot, uint32_t buf) {
        if (!dlive) return;
        const uint32_t ks = 2 * p + g;
        const uint8_t *rw = smem + L::RAW + slot * L::RS + g * L::RG + yr * 48;
        QStage<VKF_Q4_K> q;
        q.hdr = *(const vkf_u4 *)rw;
        q.qa = *(const vkf_u4 *)(rw + 16);
        q.qb = *(const vkf_u4 *)(rw + 32);
        q.j = 2 * (ks & 3) + yh;
        q.live = c0 + yr < a.Cn;
        TileRegs t;
        q.decode(t);
        uint8_t *sy = smem + L::Y16 + buf * L::YS + g * L::YG + yr * 128;
#pragma unroll
        for (int k = 0; k < 4; k++) *(vkf_i4 *)(sy + (((4 * yh + k) ^ (yr & 7)) << 4)) = t.v[k];
    };
    // prologue: pair 0 decoded, X of pair 1 and the raw pieces of pair 2 in flight
    issue_x(0, 0);
    issue_raw(0, 0);
    if (npair > 1) issue_raw(1, 1);
    wait_vm<0>();
    __syncthreads();
    decode(0, 0, 0);
    if (npair > 1) issue_x(1, 1);
    if (npair > 2) issue_raw(2, 2);
    uint32_t sx = 0, sr = 1;  // X stage of pair t, raw slot of pair t + 1
    for (uint32_t t = 0; t < npair; t++) {
        // X of pair t and the raw pieces of pair t + 1 landed; the previous
        // iteration's loads (X of t + 1: 4, raw of t + 2: 1 per wave) may stay in flight
        if (t + 2 < npair) wait_vm<5>();
        else if (t + 1 < npair) wait_vm<4>();
        else wait_vm<0>();
        __syncthreads();
        const uint32_t sx2 = sx == 0 ? 2 : sx - 1, sr2 = sr == 0 ? 2 : sr - 1;  // (t + 2) % 3, (t + 3) % 3
        if (t + 2 < npair) issue_x(t + 2, sx2);
        if (t + 3 < npair) issue_raw(t + 3, sr2);
        const uint8_t *lx = smem + sx * L::XS + g * 16384;
        mfma_step_n<2, NB>(lx, smem + L::Y16 + (t & 1) * L::YS + g * L::YG, wq, acc);
        if (t + 1 < npair) decode(t + 1, sr, (t + 1) & 1);
        sx = sx == 2 ? 0 : sx + 1;
        sr = sr == 2 ? 0 : sr + 1;
    }
    __syncthreads();  // LDS free for the group sums
}

template <int NB>
__device__ __forceinline__ void gemm_q4k_n_body(const VkfGemmArgs &a, uint8_t *smem) {
    uint32_t r0, c0;
    gemm_tile_of_n<16 * NB>(r0, c0);
    vkf_f4 acc[2][NB];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < NB; j++) acc[i][j] = vkf_f4{0, 0, 0, 0};
    const EpiPreN<NB> pre = epi_prefetch_n<NB>(a, r0, c0);
    gemm_mainloop_q4k_n<NB>(a, r0, c0, acc, smem);
    vkf_f4 mine[NB];
    gemm_group_exchange_n<NB>(acc, mine, smem);
    gemm_epilogue_n<2, NB>(a, r0, c0, mine, smem, pre);
}

// dynamic LDS: QnLayout<NB>::BYTES
#define VKF_GEMM_Q4K_N(NB)                                                              \
    VKF_KERNEL void __launch_bounds__(512) vkf_gemm_q4_k_f16_n##NB(VkfGemmArgs a) {    \
        extern __shared__ __attribute__((aligned(16))) uint8_t qn_smem[];             \
        gemm_q4k_n_body<NB>(a, qn_smem);                                                \
    }
VKF_GEMM_Q4K_N(4)
VKF_GEMM_Q4K_N(5)

// ---------------------------------------------------------------------------
// Dense GEMM on 256 x 256 tiles for grids of at least one such tile per CU
// (4096³: 256 tiles): half the tile bytes per MAC of the 128 x 128 kernel.
// 512 threads, eight waves of 128 x 64 (wave w: rows 128(w >> 2), columns
// 64(w & 3); 8 x 4 fragments of 16 x 16, two waves per SIMD), both operands
// K-contiguous by direct-to-LDS loads, two stages of 64 KiB (one step in
// flight while one is multiplied).  The epilogue stages the two 128-row
// halves one after the other through a 128 x 260 fp32 tile (epi_one's
// steps per value); D_I32 stores the int32 sums from the registers.
// ---------------------------------------------------------------------------
#define GEMM_B256_LDS (128 * 260 * 4)

// rows 128H .. 128H + 127 of the 256 x 256 tile: waves 4H .. 4H + 3 stage
// their values, all 512 threads store them
template <int H, class ACC>
__device__ __forceinline__ void b256_epilogue_half(const VkfGemmArgs &a, uint32_t r0, uint32_t c0,
                                                   const ACC acc[8][4], uint8_t *smem) {
    constexpr uint32_t TP = 260;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, wr = wave >> 2, wc = wave & 3;
    const int li = lane & 15, lg = lane >> 4;
    float *tile = (float *)smem;
    if (wr == H) {
#pragma unroll
        for (int i = 0; i < 8; i++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const uint32_t tr = 16 * i + 4 * lg + e, r = r0 + 128 * H + tr;
                const uint32_t rc = r < a.R ? r : a.R - 1;
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const uint32_t tc = wc * 64 + 16 * j + li, c = c0 + tc < a.Cn ? c0 + tc : a.Cn - 1;
                    tile[tr * TP + tc] = epi_one(a, rc, c, (float)acc[i][j][e]);
                }
            }
    }
    __syncthreads();
    const bool f32 = (a.flags & VKF_GF_D_F32) != 0;
    const uint32_t vec = f32 ? 4 : 8;  // elements per 16-byte store
    const bool vok = (a.ldd % vec) == 0 && (((uintptr_t)a.D & 15) == 0);
    const uint32_t per_row = 256 / vec;
    for (uint32_t q = threadIdx.x; q < 128 * per_row; q += 512) {
        const uint32_t tr = q / per_row, tc = (q % per_row) * vec;
        const uint32_t r = r0 + 128 * H + tr, c = c0 + tc;
        if (r >= a.R || c >= a.Cn) continue;
        const float *src = tile + tr * TP + tc;
        if (vok && c + vec <= a.Cn) {
            if (f32) {
                *(vkf_f4 *)((float *)a.D + (uint64_t)r * a.ldd + c) = *(const vkf_f4 *)src;
            } else {
                vkf_h8 hv;
#pragma unroll
                for (int k = 0; k < 8; k++) hv[k] = vkf_to_f16(src[k]);
                *(vkf_h8 *)((_Float16 *)a.D + (uint64_t)r * a.ldd + c) = hv;
            }
        } else {
            for (uint32_t k = 0; k < vec && c + k < a.Cn; k++) {
                if (f32) ((float *)a.D)[(uint64_t)r * a.ldd + c + k] = src[k];
                else ((_Float16 *)a.D)[(uint64_t)r * a.ldd + c + k] = vkf_to_f16(src[k]);
            }
        }
    }
    __syncthreads();
}

template <int ES, class ACC>
__device__ __forceinline__ void gemm_b256_body(const VkfGemmArgs &a0, uint8_t *smem) {
    const VkfGemmArgs a = gemm_batch(a0);
    uint32_t r0, c0;
    gemm_tile_of_n<256, 256>(r0, c0);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, wr = wave >> 2, wc = wave & 3;
    const int li = lane & 15, lg = lane >> 4, sw = li & 7;
    ACC acc[8][4];
#pragma unroll
    for (int i = 0; i < 8; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = ACC{0, 0, 0, 0};
    const uint32_t nk = (uint32_t)(((uint64_t)a.K * ES) / 128);
    const uint8_t *gx[4], *gy[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const uint32_t rr = (4 * wave + j) * 8 + (lane >> 3);  // 0..255
        const uint32_t ch = (lane & 7) ^ (rr & 7);
        const uint32_t rx = r0 + rr < a.R ? r0 + rr : a.R - 1;  // rows past the edge: any valid row
        const uint32_t ry = c0 + rr < a.Cn ? c0 + rr : a.Cn - 1;
        gx[j] = (const uint8_t *)a.X + (uint64_t)rx * a.ldx * ES + ch * 16;
        gy[j] = (const uint8_t *)a.Y + (uint64_t)ry * a.ldy * ES + ch * 16;
    }
    auto issue = [&](uint32_t kt, uint32_t st) {
        uint8_t *sx = smem + st * 65536, *sy = sx + 32768;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            vkf_load_lds16(gx[j] + (uint64_t)kt * 128, sx + (4 * wave + j) * 1024);
            vkf_load_lds16(gy[j] + (uint64_t)kt * 128, sy + (4 * wave + j) * 1024);
        }
    };
    if (nk > 0) issue(0, 0);
    for (uint32_t kt = 0; kt < nk; kt++) {
        wait_vm<0>();  // step kt's loads are the only ones in flight
        __syncthreads();
        if (kt + 1 < nk) issue(kt + 1, (kt + 1) & 1);
        const uint8_t *lx = smem + (kt & 1) * 65536, *ly = lx + 32768;
#pragma unroll
        for (int s = 0; s < 2; s++) {
            const int c = 4 * s + lg;
            vkf_i4 fa[8], fb[4];
#pragma unroll
            for (int i = 0; i < 8; i++) fa[i] = *(const vkf_i4 *)(lx + (wr * 128 + 16 * i + li) * 128 + ((c ^ sw) << 4));
#pragma unroll
            for (int j = 0; j < 4; j++) fb[j] = *(const vkf_i4 *)(ly + (wc * 64 + 16 * j + li) * 128 + ((c ^ sw) << 4));
#pragma unroll
            for (int i = 0; i < 8; i++)
#pragma unroll
                for (int j = 0; j < 4; j++) acc[i][j] = mfma_frag<ES>(fa[i], fb[j], acc[i][j]);
        }
    }
    __syncthreads();  // LDS free for the epilogue
    if constexpr (ES == 1) {
        if (a.flags & VKF_GF_D_I32) {
            const int32_t al = __builtin_bit_cast(int32_t, a.alpha), be = __builtin_bit_cast(int32_t, a.beta);
#pragma unroll
            for (int i = 0; i < 8; i++)
#pragma unroll
                for (int j = 0; j < 4; j++)
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        const uint32_t r = r0 + wr * 128 + 16 * i + 4 * lg + e, c = c0 + wc * 64 + 16 * j + li;
                        if (r < a.R && c < a.Cn) {
                            int32_t v = acc[i][j][e];
                            if (al != 1 || be != 0)
                                v = al * v + (be ? be * ((const int32_t *)a.Cin)[(uint64_t)r * a.ldc + c] : 0);
                            ((int32_t *)a.D)[(uint64_t)r * a.ldd + c] = v;
                        }
                    }
            return;
        }
    }
    b256_epilogue_half<0>(a, r0, c0, acc, smem);
    b256_epilogue_half<1>(a, r0, c0, acc, smem);
}

VKF_KERNEL void __launch_bounds__(512) vkf_gemm_f16_b256(VkfGemmArgs a) {
    __shared__ __attribute__((aligned(16))) uint8_t smem[GEMM_B256_LDS];
    gemm_b256_body<2, vkf_f4>(a, smem);
}
VKF_KERNEL void __launch_bounds__(512) vkf_gemm_i8_b256(VkfGemmArgs a) {
    __shared__ __attribute__((aligned(16))) uint8_t smem[GEMM_B256_LDS];
    gemm_b256_body<1, vkf_i4>(a, smem);
}
