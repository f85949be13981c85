// gemv_dot.hip — decode GEMV (M <= 4) for Q4_0, Q4_1, Q8_0 and Q4_K weights
// with fp16 or fp32 activations, on the VALU integer dot-product path.
//
// A weight stream at 8 TB/s is 14 G 4-bit weights per µs against ~39 G VALU
// lane-ops per µs, so what decides the speed is how few instructions each
// weight costs.  Decoding nibbles to floats costs ~2 per weight and row; here
// the activations are turned into integers once per workgroup instead, and
// each weight byte meets them in v_dot4_i32_i8 (4 MACs per instruction):
//
//   per 64-element chunk of activation row m (two 32-element groups):
//   E = exponent with max|x| < 2^(E+13), v = rint(x * 2^-E) in
//   [-8192, 8192] (|x - v*2^E| <= 2^(E-1) <= max|x| / 16384), split exactly
//   as v = 128*h + l with h in [-64, 64], l in [0, 127] (both int8).
//
// For a 32-weight group with integer codes q (nibbles 0..15, or Q8_0's int8):
//   P = 128 * sum(q*h) + sum(q*l) = sum(q*v)      exact, |P| < 2^22
// and the group's output contribution is the format's affine map applied to
// P and the group's activation sum S = sum(v):
//   Q4_0  2^E * d * (P - 8*S)          (value (q - 8) * d)
//   Q4_1  2^E * (d*P + m*S)            (value q*d + m)
//   Q8_0  2^E * d * P                  (value q*d)
//   Q4_K  2^E * (dall*(sc*P) - dmin*(mn*S))   (value dall*sc*q - dmin*mn;
//         the two groups of a chunk share E, so their integers add first)
// The 14-bit activation grid is the only rounding besides fp32 accumulation:
// it bounds the output error by ~1e-4 of max|y| (1e-3 tolerance).
//
// Work split.  One 1024-thread workgroup per CU stages all M activation rows
// in LDS once, then its 16 waves walk row tiles.  Inside a wave, segments of
// S lanes (S = 8..64, host choice) own RPL rows each; lane p of a segment
// takes the 64-element chunks c = p, p + S, ... of its rows (groups 2c and
// 2c+1: a Q4_K sub-block pair, or two Q4_0/Q4_1/Q8_0 blocks), reads each
// chunk's bytes with 128-bit loads and reuses the chunk's activations for
// its RPL rows.  Partial sums are reduced across the segment with shuffles.
#include "vkf_device.h"

#define DOT_WAVES 16
#define DOT_PLANE 4096  // bytes per LDS plane: chunks c < 256, K <= 16384

// Vectors at 4- / 8-byte aligned addresses (Q4_0 / Q8_0 block pairs start on
// 4-byte boundaries, Q4_1 pairs on 8): still one global_load_dwordx4 each.
typedef unsigned int vkf_u4a4 __attribute__((ext_vector_type(4), aligned(4)));
typedef unsigned int vkf_u2a4 __attribute__((ext_vector_type(2), aligned(4)));

// ---------------------------------------------------------------------------
// LDS image of the activations (MM rows reserved, M staged), one exponent E
// per 64-element chunk c (groups 2c, 2c+1):
//   xq: plane (m*8 + b*4 + q) of DOT_PLANE bytes, entry c (16 bytes) holds
//       piece q of group 2c+b: q = 0: h[0..15], 1: h[16..31], 2: l[0..15],
//       3: l[16..31].  Lanes of a segment read consecutive entries (no bank
//       conflicts) and the 8 pieces of a chunk sit at fixed offsets from one
//       address (immediate ds_read offsets).
//   xs: after the MM*8 planes, int4 per (m, c): {bits of 2^E, S0, S1, 0},
//       S_b = sum of v over group 2c+b (|S_b| <= 2^18).
// ---------------------------------------------------------------------------
template <int MM>
__device__ __forceinline__ uint32_t xs_offset(uint32_t m, uint32_t c) {
    return MM * 8 * DOT_PLANE + (m * 256 + c) * 16;
}
template <int MM>
constexpr uint32_t dot_lds_bytes() { return MM * 8 * DOT_PLANE + MM * 256 * 16; }

// Staging.  Item i = 8 consecutive elements of one row (8 items per chunk,
// K/8 per row, row m = i / (K/8) for M <= 4).  The 8 items of a chunk sit
// in 8 adjacent lanes (lane groups aligned to 8) and meet through DPP
// moves: quad_perm within 4 lanes (one group), row_half_mirror between the
// two quads of the 8.
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) { return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xf, 0xf, false); }
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) { return __int_as_float(dpp_i<CTRL>(__float_as_int(v))); }
#define DPP_XOR1 0xb1        // quad_perm [1,0,3,2]
#define DPP_XOR2 0x4e        // quad_perm [2,3,0,1]
#define DPP_HALF_MIRROR 0x141

template <int XK>
__device__ __forceinline__ void dot_load_x(const VkfGemvArgs &a, uint32_t i, uint32_t items, uint32_t K8, float v[8]) {
#pragma unroll
    for (int j = 0; j < 8; j++) v[j] = 0.0f;
    if (i >= items) return;
    const uint32_t m = (i >= K8) + (i >= 2 * K8) + (i >= 3 * K8), r = i - m * K8;
    const uint64_t off = (uint64_t)m * a.ldx + 8ull * r;
    if (XK == 2) {
        // Q8_1 (ldx in bytes, 36-byte blocks of 32): d*q, exact in fp32
        const uint8_t *b = (const uint8_t *)a.x + (uint64_t)m * a.ldx + 36ull * (r >> 2);
        const float d = vkf_h2f(*(const uint16_t *)b);
        const vkf_u2 q = *(const vkf_u2a4 *)(b + 4 + 8 * (r & 3));
#pragma unroll
        for (int j = 0; j < 8; j++) v[j] = d * (float)(int8_t)(q[j >> 2] >> (8 * (j & 3)));
    } else if (XK == 1) {
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

// Quantise item i and store it; every lane of the wave takes part.
template <int MM>
__device__ __forceinline__ void dot_store_x(unsigned char *lds, uint32_t i, uint32_t items, uint32_t K8,
                                            const float v[8]) {
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; j++) amax = fmaxf(amax, fabsf(v[j]));
    amax = fmaxf(amax, dpp_f<DPP_XOR1>(amax));
    amax = fmaxf(amax, dpp_f<DPP_XOR2>(amax));
    amax = fmaxf(amax, dpp_f<DPP_HALF_MIRROR>(amax));
    // amax < 2^e2 with e2 = biased exponent - 126 (amax == 0 or subnormal:
    // e2 = -126, still a bound), E = e2 - 13 so that |x| * 2^-E < 2^13.
    const int E = (int)((__float_as_uint(amax) >> 23) & 0xffu) - 139;
    uint32_t hw[2] = {0, 0}, lw[2] = {0, 0};
    int sum = 0;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const int vi = (int)__builtin_rintf(__builtin_amdgcn_ldexpf(v[j], -E));
        sum += vi;
        hw[j >> 2] |= ((uint32_t)(vi >> 7) & 0xffu) << (8 * (j & 3));
        lw[j >> 2] |= ((uint32_t)vi & 127u) << (8 * (j & 3));
    }
    sum += dpp_i<DPP_XOR1>(sum);  // group sums: the quad of items 4b .. 4b+3
    sum += dpp_i<DPP_XOR2>(sum);
    const int s1 = dpp_i<DPP_HALF_MIRROR>(sum);
    if (i < items) {
        const uint32_t m = (i >= K8) + (i >= 2 * K8) + (i >= 3 * K8), r = i - m * K8;
        const uint32_t c = r >> 3, e = r & 7;  // chunk, eighth of the chunk
        const uint32_t b = e >> 2, q = (e >> 1) & 1, half = e & 1;
        unsigned char *base = lds + (m * 8 + b * 4) * DOT_PLANE + c * 16 + half * 8;
        *(vkf_u2 *)(base + q * DOT_PLANE) = vkf_u2{hw[0], hw[1]};
        *(vkf_u2 *)(base + (2 + q) * DOT_PLANE) = vkf_u2{lw[0], lw[1]};
        if (e == 0)
            *(vkf_i4 *)(lds + xs_offset<MM>(m, c)) =
                vkf_i4{__float_as_int(__builtin_amdgcn_ldexpf(1.0f, E)), sum, s1, 0};
    }
}

// P of one 32-element group: w[i] holds the codes of elements 4i..4i+3,
// xb points at the chunk's entry in plane (m, b, 0).
__device__ __forceinline__ int group_dot(const uint32_t w[8], const unsigned char *xb) {
    const vkf_u4 h0 = *(const vkf_u4 *)xb, h1 = *(const vkf_u4 *)(xb + DOT_PLANE);
    const vkf_u4 l0 = *(const vkf_u4 *)(xb + 2 * DOT_PLANE), l1 = *(const vkf_u4 *)(xb + 3 * DOT_PLANE);
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
// as NW raw dwords; `consts` extracts its scalars, `codes(raw, b, w)` the
// integer codes of group b (w[i] = elements 4i..4i+3), and `fold` finishes
// a group given P and the group's {2^E, fs}.
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
    struct K { float d[2]; };
    static __device__ __forceinline__ void load(const uint8_t *row, uint32_t c, uint32_t r[NW]) {
        const uint8_t *p = row + 36ull * c;
        const vkf_u4 a = *(const vkf_u4a4 *)p, b = *(const vkf_u4a4 *)(p + 16);
        r[0] = a[0]; r[1] = a[1]; r[2] = a[2]; r[3] = a[3];
        r[4] = b[0]; r[5] = b[1]; r[6] = b[2]; r[7] = b[3];
        r[8] = *(const uint32_t *)(p + 32);
    }
    static __device__ __forceinline__ void consts(const uint32_t r[NW], uint32_t il, K &k) {
        (void)il;
        k.d[0] = h_lo(r[0]);
        k.d[1] = h_hi(r[4]);
    }
    static __device__ __forceinline__ void codes(const uint32_t r[NW], int b, uint32_t il, uint32_t w[8]) {
        (void)il;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            // block 0: qs at bytes 2..17, block 1: bytes 20..35
            const uint32_t q = b == 0 ? __builtin_amdgcn_alignbyte(r[i + 1], r[i], 2) : r[5 + i];
            w[i] = nib_lo(q);
            w[4 + i] = nib_hi(q);
        }
    }
    // values (q - 8) * d: sum = d * 2^E * (P - 8*S) per block
    static __device__ __forceinline__ float fold(const K &k, int P0, int P1, float fe, int S0, int S1, float acc) {
        const float t = fmaf(k.d[1], (float)(P1 - 8 * S1), k.d[0] * (float)(P0 - 8 * S0));
        return fmaf(fe, t, acc);
    }
};

// Q4_1: 20-byte blocks {fp16 d, fp16 m, qs[16]} (dequant_q4_1.glsl); a chunk
// = 40 bytes at an 8-byte aligned offset.
template <> struct DotFmt<VKF_Q4_1> {
    static constexpr int NW = 10;
    struct K { float d[2], m[2]; };
    static __device__ __forceinline__ void load(const uint8_t *row, uint32_t c, uint32_t r[NW]) {
        const uint8_t *p = row + 40ull * c;
        const vkf_u4 a = *(const vkf_u4a4 *)p, b = *(const vkf_u4a4 *)(p + 16);
        const vkf_u2 e = *(const vkf_u2a4 *)(p + 32);
        r[0] = a[0]; r[1] = a[1]; r[2] = a[2]; r[3] = a[3];
        r[4] = b[0]; r[5] = b[1]; r[6] = b[2]; r[7] = b[3];
        r[8] = e[0]; r[9] = e[1];
    }
    static __device__ __forceinline__ void consts(const uint32_t r[NW], uint32_t il, K &k) {
        (void)il;
#pragma unroll
        for (int b = 0; b < 2; b++) {
            k.d[b] = h_lo(r[5 * b]);
            k.m[b] = h_hi(r[5 * b]);
        }
    }
    static __device__ __forceinline__ void codes(const uint32_t r[NW], int b, uint32_t il, uint32_t w[8]) {
        (void)il;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t q = r[5 * b + 1 + i];
            w[i] = nib_lo(q);
            w[4 + i] = nib_hi(q);
        }
    }
    // values q*d + m: sum = 2^E * (d*P + m*S) per block
    static __device__ __forceinline__ float fold(const K &k, int P0, int P1, float fe, int S0, int S1, float acc) {
        float t = k.d[0] * (float)P0;
        t = fmaf(k.m[0], (float)S0, t);
        t = fmaf(k.d[1], (float)P1, t);
        t = fmaf(k.m[1], (float)S1, t);
        return fmaf(fe, t, acc);
    }
};

// Q8_0: 34-byte blocks {fp16 d, int8 qs[32]} (dequant_q8_0.glsl); a chunk =
// 68 bytes at a 4-byte aligned offset.
template <> struct DotFmt<VKF_Q8_0> {
    static constexpr int NW = 17;
    struct K { float d[2]; };
    static __device__ __forceinline__ void load(const uint8_t *row, uint32_t c, uint32_t r[NW]) {
        const uint8_t *p = row + 68ull * c;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const vkf_u4 a = *(const vkf_u4a4 *)(p + 16 * k);
            r[4 * k] = a[0]; r[4 * k + 1] = a[1]; r[4 * k + 2] = a[2]; r[4 * k + 3] = a[3];
        }
        r[16] = *(const uint32_t *)(p + 64);
    }
    static __device__ __forceinline__ void consts(const uint32_t r[NW], uint32_t il, K &k) {
        (void)il;
        k.d[0] = h_lo(r[0]);
        k.d[1] = h_hi(r[8]);
    }
    static __device__ __forceinline__ void codes(const uint32_t r[NW], int b, uint32_t il, uint32_t w[8]) {
        (void)il;
#pragma unroll
        for (int i = 0; i < 8; i++)  // block 0: qs at bytes 2..33, block 1: bytes 36..67
            w[i] = b == 0 ? __builtin_amdgcn_alignbyte(r[i + 1], r[i], 2) : r[9 + i];
    }
    // values q*d: sum = 2^E * d * P per block
    static __device__ __forceinline__ float fold(const K &k, int P0, int P1, float fe, int S0, int S1, float acc) {
        (void)S0;
        (void)S1;
        return fmaf(fe, fmaf(k.d[1], (float)P1, k.d[0] * (float)P0), acc);
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
    struct K { float dall, dmin; int sc[2], mn[2]; };
    static __device__ __forceinline__ void load(const uint8_t *row, uint32_t c, uint32_t r[NW]) {
        const uint8_t *p = row + (144u * (c >> 2) + 32u * (c & 3));
        const vkf_u4 h = *(const vkf_u4 *)(p - 32u * (c & 3));
        const vkf_u4 a = *(const vkf_u4 *)(p + 16), b = *(const vkf_u4 *)(p + 32);
        r[0] = h[0]; r[1] = h[1]; r[2] = h[2]; r[3] = h[3];
        r[4] = a[0]; r[5] = a[1]; r[6] = a[2]; r[7] = a[3];
        r[8] = b[0]; r[9] = b[1]; r[10] = b[2]; r[11] = b[3];
    }
    static __device__ __forceinline__ void consts(const uint32_t r[NW], uint32_t il, K &k) {
        k.dall = h_lo(r[0]);
        k.dmin = h_hi(r[0]);
        const uint32_t s0 = r[1], s4 = r[2], s8 = r[3];
        // bytes k = 0..3 of scW / mnW: sc / mn of sub-block k (il < 2) or k + 4
        const uint32_t scW = il < 2 ? (s0 & 0x3f3f3f3fu) : ((s8 & 0x0f0f0f0fu) | ((s0 >> 2) & 0x30303030u));
        const uint32_t mnW = il < 2 ? (s4 & 0x3f3f3f3fu) : (((s8 >> 4) & 0x0f0f0f0fu) | ((s4 >> 2) & 0x30303030u));
        const uint32_t sh = 16 * (il & 1);
        k.sc[0] = (int)((scW >> sh) & 0xffu);
        k.sc[1] = (int)((scW >> (sh + 8)) & 0xffu);
        k.mn[0] = (int)((mnW >> sh) & 0xffu);
        k.mn[1] = (int)((mnW >> (sh + 8)) & 0xffu);
    }
    static __device__ __forceinline__ void codes(const uint32_t r[NW], int b, uint32_t il, uint32_t w[8]) {
        (void)il;
#pragma unroll
        for (int i = 0; i < 8; i++) w[i] = b == 0 ? nib_lo(r[4 + i]) : nib_hi(r[4 + i]);
    }
    // values dall*sc*q - dmin*mn: sum = 2^E * (dall*Q - dmin*mS) with the
    // integers Q = sc0*P0 + sc1*P1 (|Q| < 2^29) and mS = mn0*S0 + mn1*S1
    // (|mS| < 2^25), all factors within the 24-bit multiplier's range.
    static __device__ __forceinline__ float fold(const K &k, int P0, int P1, float fe, int S0, int S1, float acc) {
        const int Q = __mul24(k.sc[0], P0) + __mul24(k.sc[1], P1);
        const int mS = __mul24(k.mn[0], S0) + __mul24(k.mn[1], S1);
        return fmaf(fe, fmaf(k.dall, (float)Q, -k.dmin * (float)mS), acc);
    }
};

// Q5_K: 176-byte super-blocks {fp16 dall, fp16 dmin, scales[12], qh[32],
// qs[128]} (kernels/dequant_q5_k.glsl:34-42, 51-73): as Q4_K, with the 5th
// bit of element l of chunk il in qh[l], bit 2il (low nibbles, sub-block 2il)
// or 2il+1 (high nibbles).  Codes 0..31; scales, mins and fold as Q4_K, the
// integer products in full 32-bit (|sc*P| < 2^31, beyond __mul24's range).
template <> struct DotFmt<VKF_Q5_K> {
    static constexpr int NW = 20;
    using K = DotFmt<VKF_Q4_K>::K;
    static __device__ __forceinline__ void load(const uint8_t *row, uint32_t c, uint32_t r[NW]) {
        const uint8_t *b = row + 176u * (c >> 2);
        const vkf_u4 h = *(const vkf_u4 *)b, q0 = *(const vkf_u4 *)(b + 16), q1 = *(const vkf_u4 *)(b + 32);
        const vkf_u4 s0 = *(const vkf_u4 *)(b + 48 + 32u * (c & 3)), s1 = *(const vkf_u4 *)(b + 64 + 32u * (c & 3));
        r[0] = h[0]; r[1] = h[1]; r[2] = h[2]; r[3] = h[3];
        r[4] = q0[0]; r[5] = q0[1]; r[6] = q0[2]; r[7] = q0[3];
        r[8] = q1[0]; r[9] = q1[1]; r[10] = q1[2]; r[11] = q1[3];
        r[12] = s0[0]; r[13] = s0[1]; r[14] = s0[2]; r[15] = s0[3];
        r[16] = s1[0]; r[17] = s1[1]; r[18] = s1[2]; r[19] = s1[3];
    }
    static __device__ __forceinline__ void consts(const uint32_t r[NW], uint32_t il, K &k) {
        DotFmt<VKF_Q4_K>::consts(r, il, k);  // header words r[0..3], same layout
    }
    static __device__ __forceinline__ void codes(const uint32_t r[NW], int b, uint32_t il, uint32_t w[8]) {
        const uint32_t hs = 2 * il + (uint32_t)b;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const uint32_t q = b == 0 ? nib_lo(r[12 + i]) : nib_hi(r[12 + i]);
            w[i] = q | (((r[4 + i] >> hs) & 0x01010101u) << 4);
        }
    }
    static __device__ __forceinline__ float fold(const K &k, int P0, int P1, float fe, int S0, int S1, float acc) {
        const int Q = k.sc[0] * P0 + k.sc[1] * P1;
        const int mS = __mul24(k.mn[0], S0) + __mul24(k.mn[1], S1);
        return fmaf(fe, fmaf(k.dall, (float)Q, -k.dmin * (float)mS), acc);
    }
};

// ---------------------------------------------------------------------------
// The kernel.  flags bit 0: y += instead of y =; bits 8..15: S (lanes per
// row segment, a power of two 8..64).  Dynamic LDS: dot_lds_bytes<MM>().
//
// Each lane keeps the loads of its next D chunks in flight (a register ring
// refilled as chunks are consumed); the first tile's loads are issued before
// the activations are staged and each next tile's before the reduction.
// ---------------------------------------------------------------------------
template <int QT, int XK, int MM, int RPL, int D>
__device__ __forceinline__ void gemv_dot(const VkfGemvArgs &a) {
    using F = DotFmt<QT>;
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    const uint32_t G = a.K / 32, C = G / 2;
    const uint32_t M = a.M;

    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t S = (a.flags >> 8) & 0xffu;
    const uint32_t seg = lane / S, p = lane & (S - 1);
    const uint32_t TR = (64 / S) * RPL;  // rows per wave tile
    const uint32_t ntiles = (a.N + TR - 1) / TR;
    const uint32_t iters = (C + S - 1) / S;
    const uint32_t il = p & 3;  // Q4_K: chunk c = p + S*it has c & 3 == p & 3 (S % 4 == 0)
    const uint32_t tstep = gridDim.x * DOT_WAVES;

    uint32_t n[RPL];
    const uint8_t *row[RPL];
    uint32_t raw[D][RPL][F::NW];
    auto start_tile = [&](uint32_t tile) {
#pragma unroll
        for (int j = 0; j < RPL; j++) {
            n[j] = tile * TR + seg * RPL + j;
            row[j] = a.w + (uint64_t)(n[j] < a.N ? n[j] : 0) * a.row_bytes;
        }
#pragma unroll
        for (int d = 0; d < D; d++) {
            const uint32_t c = p + d * S;
            const uint32_t cl = c < C ? c : C - 1;  // clamped: every load in bounds
#pragma unroll
            for (int j = 0; j < RPL; j++) F::load(row[j], cl, raw[d][j]);
        }
    };

    // Activations first: the first two staging rounds are loaded and
    // quantised before any weight load is issued (a weight flood from the
    // whole GPU ahead of them would delay every workgroup's staging), then
    // the first tile's weights are requested while the rest is staged.
    // (Waves whose first item of a round is past the end skip the round.)
    const uint32_t K8 = a.K / 8, items = M * K8, w0 = wave * 64;
    float xv[2][8];
    dot_load_x<XK>(a, threadIdx.x, items, K8, xv[0]);
    dot_load_x<XK>(a, blockDim.x + threadIdx.x, items, K8, xv[1]);
    if (w0 < items) dot_store_x<MM>(smem, threadIdx.x, items, K8, xv[0]);
    if (blockDim.x + w0 < items) dot_store_x<MM>(smem, blockDim.x + threadIdx.x, items, K8, xv[1]);
    asm volatile("" ::: "memory");  // keep the weight loads below
    uint32_t tile = wave * gridDim.x + blockIdx.x;
    if (tile < ntiles) start_tile(tile);
    for (uint32_t i0 = 2 * blockDim.x; i0 + w0 < items; i0 += blockDim.x) {
        dot_load_x<XK>(a, i0 + threadIdx.x, items, K8, xv[0]);
        dot_store_x<MM>(smem, i0 + threadIdx.x, items, K8, xv[0]);
    }
    __syncthreads();

    for (; tile < ntiles; tile += tstep) {
        float acc[RPL][MM];
#pragma unroll
        for (int j = 0; j < RPL; j++)
#pragma unroll
            for (int m = 0; m < MM; m++) acc[j][m] = 0.0f;

        for (uint32_t it0 = 0; it0 < iters; it0 += D) {
#pragma unroll
            for (int d = 0; d < D; d++) {
                const uint32_t it = it0 + d;
                if (it < iters) {
                    const uint32_t c = p + it * S;
                    if (c < C) {
                        typename F::K k[RPL];
#pragma unroll
                        for (int j = 0; j < RPL; j++) F::consts(raw[d][j], il, k[j]);
                        int P[2][RPL][MM];
#pragma unroll
                        for (int b = 0; b < 2; b++) {
                            uint32_t w[RPL][8];
#pragma unroll
                            for (int j = 0; j < RPL; j++) F::codes(raw[d][j], b, il, w[j]);
#pragma unroll
                            for (int m = 0; m < MM; m++) {
                                if (MM == 1 || m < (int)M) {
                                    const unsigned char *xb = smem + (m * 8 + b * 4) * DOT_PLANE + c * 16;
#pragma unroll
                                    for (int j = 0; j < RPL; j++) P[b][j][m] = group_dot(w[j], xb);
                                }
                            }
                        }
#pragma unroll
                        for (int m = 0; m < MM; m++) {
                            if (MM == 1 || m < (int)M) {
                                const vkf_i4 xs = *(const vkf_i4 *)(smem + xs_offset<MM>(m, c));
                                const float fe = __int_as_float(xs[0]);
#pragma unroll
                                for (int j = 0; j < RPL; j++)
                                    acc[j][m] = F::fold(k[j], P[0][j][m], P[1][j][m], fe, xs[1], xs[2], acc[j][m]);
                            }
                        }
                    }
                    if (it + D < iters) {  // refill this slot with chunk it + D
                        const uint32_t cn = c + D * S < C ? c + D * S : C - 1;
#pragma unroll
                        for (int j = 0; j < RPL; j++) F::load(row[j], cn, raw[d][j]);
                    }
                }
            }
        }

        uint32_t nout[RPL];
#pragma unroll
        for (int j = 0; j < RPL; j++) nout[j] = n[j];
        if (tile + tstep < ntiles) start_tile(tile + tstep);  // next tile's loads under the reduction

        // segment reduction (segments are aligned groups of S lanes)
#pragma unroll
        for (int j = 0; j < RPL; j++) {
#pragma unroll
            for (int m = 0; m < MM; m++) {
                float v = acc[j][m];
                for (uint32_t o = S >> 1; o > 0; o >>= 1) v += __shfl_xor(v, (int)o, 64);
                if (p == 0 && m < (int)M && nout[j] < a.N) {
                    float *yp = a.y + (uint64_t)m * a.ldy + nout[j];
                    *yp = (a.flags & 1u) ? *yp + v : v;
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// M = 1 with the weights through LDS (Q4_0, Q4_1, Q4_K, Q5_K, Q8_0: 36-,
// 40-, 44- or 68-byte chunks).  Per iteration a wave needs S consecutive chunks of each of its
// 64/S rows: CB*S contiguous bytes per row, 4*CB 16-byte pieces per wave.
// They are fetched with direct-to-LDS loads over consecutive addresses into
// one of the wave's two LDS buffers (each 128-byte line requested once; a
// CU keeps only ~64 line requests in flight, so fewer requests are more
// bandwidth), and each lane reads its chunk from there while the next
// iteration's loads fill the other buffer.  The last iteration's region may
// end 4, 8 or 12 bytes into a piece: that piece is fetched shifted and its
// valid bytes are loaded again into registers and written over it.
// NWV waves per workgroup, NLD direct loads per lane per iteration (NLD * 64
// >= 4 * CB pieces, more than 64 * (NLD - 1) so that every load instruction
// has active lanes and the vmcnt waits count NLD per iteration).
// Dynamic LDS: dot_lds_bytes<1>() + NWV * 2 * NLD * 1024.
// ---------------------------------------------------------------------------
template <int QT> constexpr uint32_t dot_cb() {
    return QT == VKF_Q4_1 ? 40 : QT == VKF_Q5_K ? 44 : QT == VKF_Q8_0 ? 68 : 36;
}
#define DOT_NLD 3  // direct loads per lane per iteration (3 x 64 >= 4 * 44, > 2 x 64 >= 4 * 36)

template <int QT, int XK, uint32_t S, int NWV, int NLD>
__device__ __forceinline__ void gemv_dot_lds(const VkfGemvArgs &a, unsigned char *smem) {
    using F = DotFmt<QT>;
    constexpr uint32_t CB = dot_cb<QT>(), TR = 64 / S, PR = CB * S / 16, NP = TR * PR;
    static_assert(NP <= 64 * NLD && NP > 64 * (NLD - 1), "every direct load instruction has active lanes");
    const uint32_t C = a.K / 64;
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t seg = lane / S, p = lane & (S - 1);
    const uint32_t ntiles = (a.N + TR - 1) / TR;
    const uint32_t iters = (C + S - 1) / S;
    const uint32_t il = p & 3;  // Q4_K: chunk c = p + S*it has c & 3 == p & 3 (S % 4 == 0)
    constexpr uint32_t WBUF = NLD * 64 * 16;
    const uint32_t tstep = gridDim.x * NWV;
    unsigned char *wb = smem + dot_lds_bytes<1>() + wave * 2 * WBUF;
    const uint32_t last = (uint32_t)a.row_bytes - 16;  // last 16-byte piece of a row (row_bytes % 4 == 0)
    const uint32_t rl = CB * S * (iters - 1), tl = (uint32_t)a.row_bytes - rl, rem = tl % 16;
    const bool straddle = rem != 0 && tl < 16 * PR;  // uniform

    uint32_t tile = wave * gridDim.x + blockIdx.x;
    uint32_t fixp = 0xffffffffu, fixv[3] = {0, 0, 0};
    auto issue = [&](uint32_t it) {
        const uint32_t r0 = CB * S * it;  // region start within the row
        unsigned char *buf = wb + (it & 1) * WBUF;
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // this wave's reads of the buffer are done
        // raised issue priority while the wave requests its next region: the
        // loads go out ahead of other waves' dot math (2 % at 13824x5120)
        __builtin_amdgcn_s_setprio(2);
#pragma unroll
        for (int j = 0; j < NLD; j++) {
            const uint32_t P = 64 * j + lane, pp = P < NP ? P : NP - 1, rr = pp / PR;
            const uint32_t nn = tile * TR + rr < a.N ? tile * TR + rr : a.N - 1;
            const uint32_t off = r0 + 16 * (pp - rr * PR);
            if (64 * j + 63 < NP || P < NP)  // lanes past the region's pieces issue nothing (fewer L1 accesses)
                vkf_load_lds16_nt(a.w + (uint64_t)nn * a.row_bytes + (off < last ? off : last), buf + 64 * j * 16);
        }
        __builtin_amdgcn_s_setprio(0);
        if (it == iters - 1 && straddle) {
            // piece tl/16 of each row: at most one per lane (PR < 64 or TR = 1)
            const uint8_t *fa = a.w;  // a valid address for lanes without one
            fixp = 0xffffffffu;
#pragma unroll
            for (int j = 0; j < NLD; j++) {
                const uint32_t P = 64 * j + lane, rr = P / PR;
                if (rr < TR && P - rr * PR == tl / 16) {
                    const uint32_t nn = tile * TR + rr < a.N ? tile * TR + rr : a.N - 1;
                    fa = a.w + (uint64_t)nn * a.row_bytes + rl + (tl & ~15u);
                    fixp = P;
                }
            }
#pragma unroll
            for (int d = 0; d < 3; d++) fixv[d] = *(const uint32_t *)(fa + (4 * d < rem ? 4 * d : 0));
        }
    };

    // activations first (see gemv_dot), then the first tile's weights while
    // the rest is staged
    const uint32_t K8 = a.K / 8, items = K8, w0 = wave * 64;
    float xv[2][8];
    dot_load_x<XK>(a, threadIdx.x, items, K8, xv[0]);
    dot_load_x<XK>(a, blockDim.x + threadIdx.x, items, K8, xv[1]);
    if (w0 < items) dot_store_x<1>(smem, threadIdx.x, items, K8, xv[0]);
    if (blockDim.x + w0 < items) dot_store_x<1>(smem, blockDim.x + threadIdx.x, items, K8, xv[1]);
    asm volatile("" ::: "memory");
    if (tile < ntiles) issue(0);
    for (uint32_t i0 = 2 * blockDim.x; i0 + w0 < items; i0 += blockDim.x) {
        dot_load_x<XK>(a, i0 + threadIdx.x, items, K8, xv[0]);
        dot_store_x<1>(smem, i0 + threadIdx.x, items, K8, xv[0]);
    }
    __syncthreads();

    for (; tile < ntiles; tile += tstep) {
        float acc = 0.0f;
        for (uint32_t it = 0; it < iters; it++) {
            if (it + 1 < iters) {  // wave-uniform
                issue(it + 1);
                if (it + 2 == iters && straddle) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(NLD + 3) : "memory");
                else asm volatile("s_waitcnt vmcnt(%0)" ::"n"(NLD) : "memory");
            } else {
                asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            }
            unsigned char *buf = wb + (it & 1) * WBUF;
            if (it == iters - 1 && straddle && fixp != 0xffffffffu) {
#pragma unroll
                for (int d = 0; d < 3; d++)
                    if (4 * d < rem) *(uint32_t *)(buf + 16 * fixp + 4 * d) = fixv[d];
            }
            const uint32_t c = p + it * S;
            if (c < C) {
                uint32_t raw[F::NW];
                F::load(buf + seg * PR * 16, p, raw);  // chunk p of the row's region
                typename F::K k;
                F::consts(raw, il, k);
                int P[2];
#pragma unroll
                for (int b = 0; b < 2; b++) {
                    uint32_t w[8];
                    F::codes(raw, b, il, w);
                    P[b] = group_dot(w, smem + (b * 4) * DOT_PLANE + c * 16);
                }
                const vkf_i4 xs = *(const vkf_i4 *)(smem + xs_offset<1>(0, c));
                acc = F::fold(k, P[0], P[1], __int_as_float(xs[0]), xs[1], xs[2], acc);
            }
        }
        const uint32_t nout = tile * TR + seg;
        if (tile + tstep < ntiles) {  // next tile's first loads under the reduction
            tile += tstep;
            issue(0);
            tile -= tstep;
        }
        for (uint32_t o = S >> 1; o > 0; o >>= 1) acc += __shfl_xor(acc, (int)o, 64);
        if (p == 0 && nout < a.N) {
            float *yp = a.y + nout;
            *yp = (a.flags & 1u) ? *yp + acc : acc;
        }
    }
}

template <int QT, int XK, int NWV = DOT_WAVES, int NLD = DOT_NLD>
__device__ __forceinline__ void gemv_dot_lds_entry(const VkfGemvArgs &a) {
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    switch ((a.flags >> 8) & 0xffu) {
    case 8: gemv_dot_lds<QT, XK, 8, NWV, NLD>(a, smem); break;
    case 16: gemv_dot_lds<QT, XK, 16, NWV, NLD>(a, smem); break;
    case 32: gemv_dot_lds<QT, XK, 32, NWV, NLD>(a, smem); break;
    default: gemv_dot_lds<QT, XK, 64, NWV, NLD>(a, smem); break;
    }
}

// Chunks kept in flight per lane: two (one consumed while the other loads)
// for one row per lane, one for two rows.
template <int QT> constexpr int dot_depth(int rpl) { return rpl == 1 ? 2 : 1; }

// Kernel names: vkf_gemv_dot_{q4_0,q4_1,q8_0,q4_k}_{f16,f32}_m{1,4}.
#define VKF_GEMV_DOT(name, QT)                                                                          \
    VKF_KERNEL void __launch_bounds__(64 * DOT_WAVES) vkf_gemv_dot_##name##_f16_m1(VkfGemvArgs a) {     \
        gemv_dot<QT, 0, 1, 1, dot_depth<QT>(1)>(a);                                                                       \
    }                                                                                                   \
    VKF_KERNEL void __launch_bounds__(64 * DOT_WAVES) vkf_gemv_dot_##name##_f32_m1(VkfGemvArgs a) {     \
        gemv_dot<QT, 1, 1, 1, dot_depth<QT>(1)>(a);                                                                       \
    }                                                                                                   \
    VKF_KERNEL void __launch_bounds__(64 * DOT_WAVES) vkf_gemv_dot_##name##_f16_m4(VkfGemvArgs a) {     \
        gemv_dot<QT, 0, 4, 2, dot_depth<QT>(2)>(a);                                                                       \
    }                                                                                                   \
    VKF_KERNEL void __launch_bounds__(64 * DOT_WAVES) vkf_gemv_dot_##name##_f32_m4(VkfGemvArgs a) {     \
        gemv_dot<QT, 1, 4, 2, dot_depth<QT>(2)>(a);                                                                       \
    }

VKF_GEMV_DOT(q4_0, VKF_Q4_0)
VKF_GEMV_DOT(q4_1, VKF_Q4_1)
VKF_GEMV_DOT(q8_0, VKF_Q8_0)
VKF_GEMV_DOT(q4_k, VKF_Q4_K)
VKF_GEMV_DOT(q5_k, VKF_Q5_K)
// Q8_1 activations, M = 1 (the other formats take them through LDS below)
VKF_KERNEL void __launch_bounds__(64 * DOT_WAVES) vkf_gemv_dot_q8_0_q8_1_m1(VkfGemvArgs a) {
    gemv_dot<VKF_Q8_0, 2, 1, 1, dot_depth<VKF_Q8_0>(1)>(a);
}

// M = 1 through LDS: vkf_gemv_dotl_{q4_0,q4_1,q4_k,q5_k}_{f16,f32,q8_1}
#define VKF_GEMV_DOTL(name, QT)                                                                         \
    VKF_KERNEL void __launch_bounds__(64 * DOT_WAVES) vkf_gemv_dotl_##name##_f16(VkfGemvArgs a) {       \
        gemv_dot_lds_entry<QT, 0>(a);                                                                   \
    }                                                                                                   \
    VKF_KERNEL void __launch_bounds__(64 * DOT_WAVES) vkf_gemv_dotl_##name##_f32(VkfGemvArgs a) {       \
        gemv_dot_lds_entry<QT, 1>(a);                                                                   \
    }                                                                                                   \
    VKF_KERNEL void __launch_bounds__(64 * DOT_WAVES) vkf_gemv_dotl_##name##_q8_1(VkfGemvArgs a) {      \
        gemv_dot_lds_entry<QT, 2>(a);                                                                   \
    }
VKF_GEMV_DOTL(q4_0, VKF_Q4_0)
VKF_GEMV_DOTL(q4_1, VKF_Q4_1)
VKF_GEMV_DOTL(q4_k, VKF_Q4_K)
VKF_GEMV_DOTL(q5_k, VKF_Q5_K)
// Q8_0 (68-byte chunks, 4352 bytes per wave and iteration: five direct loads
// per lane) on twelve waves, whose two buffers each fit LDS beside the
// activations (dot_lds_bytes<1>() + 12 * 2 * 5 KiB = 156 KiB):
// vkf_gemv_dotl_q8_0_{f16,f32}
#define DOT_Q8_WAVES 12
#define DOT_Q8_NLD 5
VKF_KERNEL void __launch_bounds__(64 * DOT_Q8_WAVES) vkf_gemv_dotl_q8_0_f16(VkfGemvArgs a) {
    gemv_dot_lds_entry<VKF_Q8_0, 0, DOT_Q8_WAVES, DOT_Q8_NLD>(a);
}
VKF_KERNEL void __launch_bounds__(64 * DOT_Q8_WAVES) vkf_gemv_dotl_q8_0_f32(VkfGemvArgs a) {
    gemv_dot_lds_entry<VKF_Q8_0, 1, DOT_Q8_WAVES, DOT_Q8_NLD>(a);
}
