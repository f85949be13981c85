// gemv_dot.hip — decode GEMV (M <= 4) for Q4_0, Q4_1, Q8_0 and Q4_K weights
// with fp16 or fp32 activations, on the VALU integer dot-product path.
//
// A weight stream at 8 TB/s is 14 G 4-bit weights per µs against ~39 G VALU
// lane-ops per µs, so what decides the speed is how few instructions each
// weight costs.  Decoding nibbles to floats costs ~2 per weight and row; here
// the activations are turned into integers once per workgroup instead, and
// each weight byte meets them in v_dot4_i32_i8 (4 MACs per instruction):
//
//   per 32-element group g of activation row m: E = exponent with
//   max|x| < 2^(E+13), v = rint(x * 2^-E) in [-8192, 8192]
//   (|x - v*2^E| <= 2^(E-1) <= max|x| / 16384), split exactly as
//   v = 128*h + l with h in [-64, 64], l in [0, 127] (both int8).
//
// For a 32-weight group with integer codes q (nibbles 0..15, or Q8_0's int8):
//   P = 128 * sum(q*h) + sum(q*l) = sum(q*v)      exact, |P| < 2^22
// and the group's output contribution is the format's affine map applied to
// P and S = sum(v) (stored as fs = 2^E * S):
//   Q4_0  d * (2^E*P - 8*fs)           (value (q - 8) * d)
//   Q4_1  d * 2^E*P + m * fs           (value q*d + m)
//   Q8_0  d * 2^E*P                    (value q*d)
//   Q4_K  dall * 2^E*(sc*P) - dmin * mn * fs   (value dall*sc*q - dmin*mn)
// The 14-bit activation grid is the only rounding besides fp32 accumulation:
// it bounds the output error by ~1e-4 of max|y| (1e-3 tolerance).
//
// Work split.  One 1024-thread workgroup per CU stages all M activation rows
// in LDS once, then its 16 waves walk row tiles (tile t -> wave t % (16*G)
// of workgroup ...).  Inside a wave, segments of S lanes (S = 8..64, host
// choice) own RPL rows each; lane p of a segment takes the 64-element chunks
// c = p, p + S, ... of its rows (two groups 2c, 2c+1 per chunk: a Q4_K
// sub-block pair, or two Q4_0/Q4_1/Q8_0 blocks), reads each chunk's bytes
// with 128-bit loads, and reuses the chunk's activations for its RPL rows.
// Partial sums are reduced across the segment with lane shuffles.
#include "vkf_device.h"

#define DOT_WAVES 16

typedef unsigned int vkf_u4 __attribute__((ext_vector_type(4)));
typedef unsigned int vkf_u2 __attribute__((ext_vector_type(2)));
// Vectors at 4- / 8-byte aligned addresses (Q4_0 / Q8_0 block pairs start on
// 4-byte boundaries, Q4_1 pairs on 8): still one global_load_dwordx4 each.
typedef unsigned int vkf_u4a4 __attribute__((ext_vector_type(4), aligned(4)));
typedef unsigned int vkf_u2a4 __attribute__((ext_vector_type(2), aligned(4)));

// ---------------------------------------------------------------------------
// LDS image of the activations.  G = K/32 groups per row, C = G/2 chunks.
//   xq: for row m, parity b (group 2c+b) and piece q, a plane of C 16-byte
//       entries; entry c holds piece q of group 2c+b:
//       q = 0: h[0..15], 1: h[16..31], 2: l[0..15], 3: l[16..31].
//       (Lanes of a segment read consecutive entries: no bank conflicts.)
//   xs: one float4 per (m, c): {2^E, fs} of group 2c, then of group 2c+1.
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t xq_entry(uint32_t m, uint32_t b, uint32_t q, uint32_t C, uint32_t c) {
    return ((m * 2 + b) * 4 + q) * C + c;
}

template <int XK>
__device__ __forceinline__ void dot_stage_x(const VkfGemvArgs &a, vkf_u4 *xq, vkf_f4 *xs, uint32_t G, uint32_t M) {
    const uint32_t C = G / 2;
    const uint32_t items = M * G * 4;  // item = 8 consecutive elements; 4 per group
    for (uint32_t i0 = 0; i0 < items; i0 += blockDim.x) {
        const uint32_t i = i0 + threadIdx.x;
        const bool live = i < items;
        const uint32_t m = live ? i / (G * 4) : 0;
        const uint32_t r = live ? i - m * G * 4 : 0;
        const uint32_t g = r >> 2, qq = r & 3;  // group, eighth of the group
        float v[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        if (live) {
            const uint64_t off = (uint64_t)m * a.ldx + 32ull * g + 8 * qq;
            if (XK == 1) {
                const vkf_f4 *p = (const vkf_f4 *)((const float *)a.x + off);
                const vkf_f4 p0 = p[0], p1 = p[1];
                v[0] = p0[0]; v[1] = p0[1]; v[2] = p0[2]; v[3] = p0[3];
                v[4] = p1[0]; v[5] = p1[1]; v[6] = p1[2]; v[7] = p1[3];
            } else {
                const vkf_h8 h = *(const vkf_h8 *)((const _Float16 *)a.x + off);
#pragma unroll
                for (int j = 0; j < 8; j++) v[j] = (float)h[j];
            }
        }
        // The 4 items of a group sit in 4 adjacent lanes (blockDim % 4 == 0).
        float amax = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; j++) amax = fmaxf(amax, fabsf(v[j]));
        amax = fmaxf(amax, __shfl_xor(amax, 1, 64));
        amax = fmaxf(amax, __shfl_xor(amax, 2, 64));
        int e2;
        (void)frexpf(amax, &e2);  // amax < 2^e2 (amax == 0: e2 = 0)
        const int E = e2 - 13;    // |x| * 2^-E < 2^13
        uint32_t hw[2] = {0, 0}, lw[2] = {0, 0};
        int sum = 0;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int vi = (int)rintf(ldexpf(v[j], -E));
            sum += vi;
            hw[j >> 2] |= ((uint32_t)(vi >> 7) & 0xffu) << (8 * (j & 3));
            lw[j >> 2] |= ((uint32_t)vi & 127u) << (8 * (j & 3));
        }
        sum += __shfl_xor(sum, 1, 64);
        sum += __shfl_xor(sum, 2, 64);
        if (live) {
            const uint32_t c = g >> 1, b = g & 1, q = qq >> 1, half = qq & 1;
            vkf_u2 *ph = (vkf_u2 *)(xq + xq_entry(m, b, q, C, c)) + half;
            vkf_u2 *pl = (vkf_u2 *)(xq + xq_entry(m, b, 2 + q, C, c)) + half;
            *ph = vkf_u2{hw[0], hw[1]};
            *pl = vkf_u2{lw[0], lw[1]};
            if (qq == 0) {
                const float fe = ldexpf(1.0f, E);
                float *s = (float *)(xs + (uint64_t)m * C + c) + 2 * b;
                s[0] = fe;
                s[1] = fe * (float)sum;  // |sum| <= 2^18: exact
            }
        }
    }
}

// sum over one 32-element group: w[i] holds codes of elements 4i..4i+3.
__device__ __forceinline__ int group_dot(const uint32_t w[8], const vkf_u4 *xq, uint32_t m, uint32_t b,
                                         uint32_t C, uint32_t c) {
    const vkf_u4 h0 = xq[xq_entry(m, b, 0, C, c)], h1 = xq[xq_entry(m, b, 1, C, c)];
    const vkf_u4 l0 = xq[xq_entry(m, b, 2, C, c)], l1 = xq[xq_entry(m, b, 3, C, c)];
    int ph = 0, pl = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        ph = __builtin_amdgcn_sdot4((int)w[i], (int)h0[i], ph, false);
        pl = __builtin_amdgcn_sdot4((int)w[i], (int)l0[i], pl, false);
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        ph = __builtin_amdgcn_sdot4((int)w[4 + i], (int)h1[i], ph, false);
        pl = __builtin_amdgcn_sdot4((int)w[4 + i], (int)l1[i], pl, false);
    }
    return ph * 128 + pl;
}

// ---------------------------------------------------------------------------
// Formats.  Each chunk (64 elements, groups 2c and 2c+1 of a row) is loaded
// as NW raw dwords, then decoded into integer codes w[2][8] plus per-group
// constants, and finished by `fold` given P and the group's {2^E, fs}.
// ---------------------------------------------------------------------------
template <int QT> struct DotFmt;

__device__ __forceinline__ float h_lo(uint32_t w) { return vkf_h2f(w & 0xffffu); }
__device__ __forceinline__ float h_hi(uint32_t w) { return vkf_h2f(w >> 16); }
__device__ __forceinline__ uint32_t nib_lo(uint32_t w) { return w & 0x0f0f0f0fu; }
__device__ __forceinline__ uint32_t nib_hi(uint32_t w) { return (w >> 4) & 0x0f0f0f0fu; }

// Q4_0: 18-byte blocks {fp16 d, qs[16]}; element i < 16 = low nibble of
// qs[i], i >= 16 = high nibble of qs[i-16] (kernels/dequant_q4_0.glsl:30-35).
// A chunk = blocks 2c, 2c+1 = 36 bytes at a 4-byte aligned offset.
template <> struct DotFmt<VKF_Q4_0> {
    static constexpr int NW = 9;
    struct Dec { uint32_t w[2][8]; float d[2]; };
    static __device__ __forceinline__ void load(const uint8_t *row, uint32_t c, uint32_t r[NW]) {
        const uint8_t *p = row + 36ull * c;
        const vkf_u4 a = *(const vkf_u4a4 *)p, b = *(const vkf_u4a4 *)(p + 16);
        r[0] = a[0]; r[1] = a[1]; r[2] = a[2]; r[3] = a[3];
        r[4] = b[0]; r[5] = b[1]; r[6] = b[2]; r[7] = b[3];
        r[8] = *(const uint32_t *)(p + 32);
    }
    static __device__ __forceinline__ void decode(const uint32_t r[NW], uint32_t il, Dec &o) {
        (void)il;
        o.d[0] = h_lo(r[0]);
        o.d[1] = h_hi(r[4]);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t q0 = __builtin_amdgcn_alignbyte(r[i + 1], r[i], 2);  // bytes 2 + 4i ..
            const uint32_t q1 = r[5 + i];                                         // bytes 20 + 4i ..
            o.w[0][i] = nib_lo(q0); o.w[0][4 + i] = nib_hi(q0);
            o.w[1][i] = nib_lo(q1); o.w[1][4 + i] = nib_hi(q1);
        }
    }
    static __device__ __forceinline__ float fold(const Dec &o, int b, int P, float fe, float fs, float acc) {
        return fmaf(o.d[b], fmaf(fe, (float)P, -8.0f * fs), acc);
    }
};

// Q4_1: 20-byte blocks {fp16 d, fp16 m, qs[16]} (dequant_q4_1.glsl); a chunk
// = 40 bytes at an 8-byte aligned offset.
template <> struct DotFmt<VKF_Q4_1> {
    static constexpr int NW = 10;
    struct Dec { uint32_t w[2][8]; float d[2], m[2]; };
    static __device__ __forceinline__ void load(const uint8_t *row, uint32_t c, uint32_t r[NW]) {
        const uint8_t *p = row + 40ull * c;
        const vkf_u4 a = *(const vkf_u4a4 *)p, b = *(const vkf_u4a4 *)(p + 16);
        const vkf_u2 e = *(const vkf_u2a4 *)(p + 32);
        r[0] = a[0]; r[1] = a[1]; r[2] = a[2]; r[3] = a[3];
        r[4] = b[0]; r[5] = b[1]; r[6] = b[2]; r[7] = b[3];
        r[8] = e[0]; r[9] = e[1];
    }
    static __device__ __forceinline__ void decode(const uint32_t r[NW], uint32_t il, Dec &o) {
        (void)il;
#pragma unroll
        for (int b = 0; b < 2; b++) {
            o.d[b] = h_lo(r[5 * b]);
            o.m[b] = h_hi(r[5 * b]);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t q = r[5 * b + 1 + i];
                o.w[b][i] = nib_lo(q);
                o.w[b][4 + i] = nib_hi(q);
            }
        }
    }
    static __device__ __forceinline__ float fold(const Dec &o, int b, int P, float fe, float fs, float acc) {
        return fmaf(o.m[b], fs, fmaf(o.d[b], fe * (float)P, acc));
    }
};

// Q8_0: 34-byte blocks {fp16 d, int8 qs[32]} (dequant_q8_0.glsl); a chunk =
// 68 bytes at a 4-byte aligned offset.
template <> struct DotFmt<VKF_Q8_0> {
    static constexpr int NW = 17;
    struct Dec { uint32_t w[2][8]; float d[2]; };
    static __device__ __forceinline__ void load(const uint8_t *row, uint32_t c, uint32_t r[NW]) {
        const uint8_t *p = row + 68ull * c;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const vkf_u4 a = *(const vkf_u4a4 *)(p + 16 * k);
            r[4 * k] = a[0]; r[4 * k + 1] = a[1]; r[4 * k + 2] = a[2]; r[4 * k + 3] = a[3];
        }
        r[16] = *(const uint32_t *)(p + 64);
    }
    static __device__ __forceinline__ void decode(const uint32_t r[NW], uint32_t il, Dec &o) {
        (void)il;
        o.d[0] = h_lo(r[0]);
        o.d[1] = h_hi(r[8]);
#pragma unroll
        for (int i = 0; i < 8; i++) {
            o.w[0][i] = __builtin_amdgcn_alignbyte(r[i + 1], r[i], 2);  // bytes 2 + 4i ..
            o.w[1][i] = r[9 + i];                                         // bytes 36 + 4i ..
        }
    }
    static __device__ __forceinline__ float fold(const Dec &o, int b, int P, float fe, float fs, float acc) {
        (void)fs;
        return fmaf(o.d[b], fe * (float)P, acc);
    }
};

// Q4_K: 144-byte super-blocks {fp16 dall, fp16 dmin, scales[12], qs[128]};
// chunk c = 4*sb + il covers qs[32il .. 32il+31] of super-block sb: low
// nibbles = sub-block 2il, high nibbles = sub-block 2il+1
// (kernels/dequant_q4_k.glsl:49-57).  6-bit scales and mins, 4 at a time
// (dequant_q4_k.glsl:16-24): sub-blocks 0..3: sc = s[j] & 63, mn = s[j+4] &
// 63; sub-blocks 4..7: sc = (s[j+4] & 15) | (s[j-4] >> 6) << 4,
// mn = (s[j+4] >> 4) | (s[j] >> 6) << 4.
template <> struct DotFmt<VKF_Q4_K> {
    static constexpr int NW = 12;
    struct Dec { uint32_t w[2][8]; float dall, dmin; int sc[2]; float mn[2]; };
    static __device__ __forceinline__ void load(const uint8_t *row, uint32_t c, uint32_t r[NW]) {
        const uint8_t *p = row + 144ull * (c >> 2);
        const vkf_u4 h = *(const vkf_u4 *)p;
        const vkf_u4 a = *(const vkf_u4 *)(p + 16 + 32 * (c & 3)), b = *(const vkf_u4 *)(p + 32 + 32 * (c & 3));
        r[0] = h[0]; r[1] = h[1]; r[2] = h[2]; r[3] = h[3];
        r[4] = a[0]; r[5] = a[1]; r[6] = a[2]; r[7] = a[3];
        r[8] = b[0]; r[9] = b[1]; r[10] = b[2]; r[11] = b[3];
    }
    static __device__ __forceinline__ void decode(const uint32_t r[NW], uint32_t il, Dec &o) {
        o.dall = h_lo(r[0]);
        o.dmin = h_hi(r[0]);
        const uint32_t s0 = r[1], s4 = r[2], s8 = r[3];
        // bytes k = 0..3 of scW / mnW: sc / mn of sub-block k (il < 2) or k + 4
        const uint32_t scW = il < 2 ? (s0 & 0x3f3f3f3fu) : ((s8 & 0x0f0f0f0fu) | ((s0 >> 2) & 0x30303030u));
        const uint32_t mnW = il < 2 ? (s4 & 0x3f3f3f3fu) : (((s8 >> 4) & 0x0f0f0f0fu) | ((s4 >> 2) & 0x30303030u));
        const uint32_t sh = 16 * (il & 1);
        o.sc[0] = (int)((scW >> sh) & 0xffu);
        o.sc[1] = (int)((scW >> (sh + 8)) & 0xffu);
        o.mn[0] = (float)((mnW >> sh) & 0xffu);
        o.mn[1] = (float)((mnW >> (sh + 8)) & 0xffu);
#pragma unroll
        for (int i = 0; i < 8; i++) {
            o.w[0][i] = nib_lo(r[4 + i]);
            o.w[1][i] = nib_hi(r[4 + i]);
        }
    }
    static __device__ __forceinline__ float fold(const Dec &o, int b, int P, float fe, float fs, float acc) {
        // sc * P: |P| < 2^22, sc < 64 -> exact in int32
        return fmaf(-o.dmin, o.mn[b] * fs, fmaf(o.dall, fe * (float)(o.sc[b] * P), acc));
    }
};

// ---------------------------------------------------------------------------
// The kernel.  flags bit 0: y += instead of y =; bits 8..15: S (lanes per
// row segment, a power of two 8..64).  Dynamic LDS: M*K*2 bytes of xq plus
// M*K/4 bytes of xs.
// ---------------------------------------------------------------------------
template <int QT, int XK, int MM, int RPL>
__device__ __forceinline__ void gemv_dot(const VkfGemvArgs &a) {
    using F = DotFmt<QT>;
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    const uint32_t G = a.K / 32, C = G / 2;
    const uint32_t M = a.M;
    vkf_u4 *xq = (vkf_u4 *)smem;
    vkf_f4 *xs = (vkf_f4 *)(smem + (uint64_t)M * G * 64);
    dot_stage_x<XK>(a, xq, xs, G, M);
    __syncthreads();

    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t S = (a.flags >> 8) & 0xffu;
    const uint32_t seg = lane / S, p = lane & (S - 1);
    const uint32_t TR = (64 / S) * RPL;  // rows per wave tile
    const uint32_t ntiles = (a.N + TR - 1) / TR;
    const uint32_t iters = (C + S - 1) / S;
    const uint32_t il = p & 3;  // Q4_K: chunk c = p + S*it has c & 3 == p & 3 (S % 4 == 0)

    for (uint32_t tile = wave * gridDim.x + blockIdx.x; tile < ntiles; tile += gridDim.x * DOT_WAVES) {
        uint32_t n[RPL];
        const uint8_t *row[RPL];
#pragma unroll
        for (int j = 0; j < RPL; j++) {
            n[j] = tile * TR + seg * RPL + j;
            row[j] = a.w + (uint64_t)(n[j] < a.N ? n[j] : 0) * a.row_bytes;
        }
        float acc[RPL][MM];
#pragma unroll
        for (int j = 0; j < RPL; j++)
#pragma unroll
            for (int m = 0; m < MM; m++) acc[j][m] = 0.0f;

        // Loads of chunk it+1 are issued before chunk it is consumed.
        uint32_t raw[RPL][F::NW];
        {
            const uint32_t c0 = p < C ? p : C - 1;
#pragma unroll
            for (int j = 0; j < RPL; j++) F::load(row[j], c0, raw[j]);
        }
        for (uint32_t it = 0; it < iters; it++) {
            const uint32_t c = p + it * S;
            typename F::Dec dec[RPL];
#pragma unroll
            for (int j = 0; j < RPL; j++) F::decode(raw[j], il, dec[j]);
            if (it + 1 < iters) {
                const uint32_t cn = c + S < C ? c + S : C - 1;
#pragma unroll
                for (int j = 0; j < RPL; j++) F::load(row[j], cn, raw[j]);
            }
            if (c < C) {
#pragma unroll
                for (int m = 0; m < MM; m++) {
                    if (m < (int)M) {
                        const vkf_f4 s = xs[(uint64_t)m * C + c];
#pragma unroll
                        for (int b = 0; b < 2; b++) {
#pragma unroll
                            for (int j = 0; j < RPL; j++) {
                                const int P = group_dot(dec[j].w[b], xq, m, b, C, c);
                                acc[j][m] = F::fold(dec[j], b, P, s[2 * b], s[2 * b + 1], acc[j][m]);
                            }
                        }
                    }
                }
            }
        }

        // segment reduction (segments are aligned groups of S lanes)
#pragma unroll
        for (int j = 0; j < RPL; j++) {
#pragma unroll
            for (int m = 0; m < MM; m++) {
                float v = acc[j][m];
                for (uint32_t o = S >> 1; o > 0; o >>= 1) v += __shfl_xor(v, (int)o, 64);
                if (p == 0 && m < (int)M && n[j] < a.N) {
                    float *yp = a.y + (uint64_t)m * a.ldy + n[j];
                    *yp = (a.flags & 1u) ? *yp + v : v;
                }
            }
        }
    }
}

// Kernel names: vkf_gemv_dot_{q4_0,q4_1,q8_0,q4_k}_{f16,f32}_m{1,4}.
#define VKF_GEMV_DOT(name, QT)                                                                          \
    VKF_KERNEL void __launch_bounds__(64 * DOT_WAVES) vkf_gemv_dot_##name##_f16_m1(VkfGemvArgs a) {     \
        gemv_dot<QT, 0, 1, 1>(a);                                                                       \
    }                                                                                                   \
    VKF_KERNEL void __launch_bounds__(64 * DOT_WAVES) vkf_gemv_dot_##name##_f32_m1(VkfGemvArgs a) {     \
        gemv_dot<QT, 1, 1, 1>(a);                                                                       \
    }                                                                                                   \
    VKF_KERNEL void __launch_bounds__(64 * DOT_WAVES) vkf_gemv_dot_##name##_f16_m4(VkfGemvArgs a) {     \
        gemv_dot<QT, 0, 4, 2>(a);                                                                       \
    }                                                                                                   \
    VKF_KERNEL void __launch_bounds__(64 * DOT_WAVES) vkf_gemv_dot_##name##_f32_m4(VkfGemvArgs a) {     \
        gemv_dot<QT, 1, 4, 2>(a);                                                                       \
    }

VKF_GEMV_DOT(q4_0, VKF_Q4_0)
VKF_GEMV_DOT(q4_1, VKF_Q4_1)
VKF_GEMV_DOT(q8_0, VKF_Q8_0)
VKF_GEMV_DOT(q4_k, VKF_Q4_K)
