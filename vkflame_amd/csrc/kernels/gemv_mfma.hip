// gemv_mfma.hip — small-batch GEMV (2 <= M <= 16) of Q4_K, Q5_K, Q4_0, Q4_1,
// Q5_0, Q8_0 and Q6_K weights on the matrix cores: y[M, N] = x[M, K] . Wdeq[N, K]^T,
// with fp16, fp32 or Q8_1 activations (the latter two staged in LDS as
// fp16: fp32 rounded once, Q8_1 as fp16(d*q), the value the prefill GEMM's
// activation decode produces).
//
// With 2..16 activation rows the VALU dot product costs M multiply-adds per
// weight; a 16x16x32 fp16 MFMA takes 16 weight rows x 32 k against up to 16
// activation rows at once, so the per-weight cost is the decode only.  Work
// is counted in groups of 256 k of a row: a Q4_K super-block (144 bytes), 8
// Q4_0 blocks (144 bytes) or 8 Q4_1 blocks (160 bytes); a group of a 16-row
// tile is 8 MFMA steps.
//
// Q4_K arithmetic.  A weight is dall*sc*q - dmin*mn (kernels/dequant_q4_k.glsl:
// 16-58; sc, mn 6-bit per 32-element sub-block, q a nibble).  Per super-block
// and output (m, n):
//   y += dall * sum_k x*(sc*q)  -  dmin * sum_j mn_j * xs_j
// with xs_j the sum of x over sub-block j.  sc*q <= 945 is an integer, exact
// in fp16, so the 8 MFMAs of a super-block see exact operands and accumulate
// in fp32; dall is applied once per super-block.  The min term is one more
// MFMA whose k runs over the 8 sub-blocks: A = xs/32 as two fp16 halves
// (hi + lo, ~22 bits) on k-slices 0 and 1, B = mn.
//
// Q5_K arithmetic: as Q4_K with q = nibble + 16 * (bit j of qh[e]) for
// element e of sub-block j (kernels/dequant_q5_k.glsl); sc*q <= 63*31 = 1953
// is still an exact fp16 integer.  The fifth bit goes into the fp16 pair at
// bit 4 (1024 + q) or bit 8 (1024 + 16q) by one more v_and_or_b32.
//
// Q6_K arithmetic.  A weight is d*sc*(q - 32) (kernels/dequant_q6_k.glsl;
// sc int8 per 16 elements, q 6 bits from a ql nibble and two qh bits).  The
// MFMA operand is sc*(q - 32) in fp16: an integer of magnitude <= 4096,
// exact up to 2048 and rounded once (relative 2^-12) above; d is applied
// once per super-block to the fp32 sum of its 8 MFMAs.
//
// Q4_0 / Q4_1 / Q8_0 arithmetic.  The MFMA operand is the dequantised weight
// in fp16, d*(q-8) (kernels/dequant_q4_0.glsl), d*q + m (dequant_q4_1.glsl)
// or d*q (dequant_q8_0.glsl), rounded once from the exact value; products
// and sums run in fp32.  Q8_0 codes become fp16 pairs as
// (1024 + (b ^ 0x80)) - 1152 = b.
//
// Decode.  A code dword holds bytes b0..b3.  (v & 0x000f000f) | 0x64006400 is
// the fp16 pair (1024 + b0.lo, 1024 + b2.lo); mask 0x00f000f0 gives
// (1024 + 16*b0.hi, 1024 + 16*b2.hi), and v >> 8 the b1, b3 pairs.  Q4_K:
// one packed fp16 FMA per pair, (1024 + q)*sc - 1024*sc or
// (1024 + 16q)*(sc/16) - 64*sc, yields sc*q exactly.  Q4_0 / Q4_1: one packed
// op makes q (or q - 8) exactly, a second applies d (and m).  A lane's 8 k of
// a step thus come in the order 0,2,1,3,4,6,5,7, and the activations are
// staged in that order.
//
// Loads and k order.  Lane l = 16g + i owns weight row i of the tile.
//   Q4_K: per super-block the 16-byte header and qs bytes 16g .. +15 and
//   64 + 16g .. +15 (64 contiguous bytes per row per load instruction): the
//   elements 16(g&1) .. +15 of sub-blocks j = 4L + 2(g>>1) + nib (L = which
//   load, nib = low / high nibbles).  Step t = 4L + 2nib + hf takes, in
//   k-slice g, elements 16(g&1) + 8hf .. +7 of that sub-block.
//   Q5_K: as Q4_K (header; qs bytes 48 + 16g .., 112 + 16g ..) plus qh bytes
//   16 + 16(g&1) .. +15, the fifth bits of the same elements.
//   Q6_K: ql bytes 16g .. +15 and 64 + 16g .. +15 (halves n = 0, 1), qh
//   bytes 128 + 16(g&1) .. and 160 + 16(g&1) .., the 16 scales, d.  Element
//   x of ql byte run n is k = 128n + 64h + 16g + x for nibble h, its two high
//   bits at 4h + 2(g>>1) of qh byte 32n + 16(g&1) + x, its scale byte
//   8n + 4h + g.  Step t = 4n + 2h + hf takes elements x = 8hf .. +7.  Super-
//   blocks (210 bytes) are 2-byte aligned: each run loads from the 4-byte
//   aligned address below it and is shifted into place (v_alignbyte).
//   Q5_0: the block pair 2g, 2g+1 (44 bytes: d, qh, qs of each), the same
//   steps as Q4_0; element e's fifth bit is bit e of the block's qh.
//   Q8_0: the block pair 2g, 2g+1 (68 bytes); step t = 4blk + s takes
//   elements 8s .. +7 of block 2g + blk (the same k as Q4_0's steps).
//   Q4_0 / Q4_1: the block pair 2g, 2g+1 of the group (36 or 40 contiguous
//   bytes, 4-byte aligned).  Step t = 4blk + 2nib + hf takes, in k-slice g,
//   elements 16nib + 8hf .. +7 of block 2g + blk (low nibbles of qs bytes
//   8hf .. +7, or their high nibbles).
//
// Work split.  One 1024-thread workgroup per CU stages the activation rows in
// LDS once, with the first weight loads already in flight.  Its 16 waves form
// 16/P groups; a group owns a 16-row tile of W per round and its P waves
// split the tile's 256-k groups P ways (P = 4, 8 or 16 from the host, larger
// for fewer rows, so that enough loads are in flight).  A wave issues the
// loads of up to gm_maxsb groups, then runs the MFMAs; the P partial 16x16
// results of a tile meet in LDS.  The host splits a K too long for LDS into
// launches over K slices, the later ones accumulating into y.  Accumulator:
// lane l holds y-tile element (activation row 4g + e, weight row i).
#include "vkf_device.h"

#define GM_WAVES 16
enum { GF_Q4_K = 0, GF_Q4_0 = 1, GF_Q4_1 = 2, GF_Q6_K = 3, GF_Q5_K = 4, GF_Q8_0 = 5, GF_Q5_0 = 6 };

// formats with a per-sub-block min term (dmin * mn), fed by the sub-block sums of x
template <int F> constexpr bool gm_kmin() { return F == GF_Q4_K || F == GF_Q5_K; }

// 256-k groups per wave held in registers at once (the most without spills)
template <int F> constexpr int gm_maxsb() {
    return F == GF_Q4_K ? 5 : F == GF_Q6_K ? 1 : (F == GF_Q5_K || F == GF_Q8_0) ? 3 : 4;
}

// Q4_K, Q4_0, Q4_1, Q8_0: two half-batches of gm_maxsb/2 groups alternate,
// one loading while the other is decoded (5-8 % faster on MI355X).  Q5_K and
// Q6_K hold too few groups for halves to pay (Q6_K 13824x5120 M=8 2.7 %
// slower) and load a batch of gm_maxsb, then decode it.
template <int F> constexpr bool gm_pingpong() { return F != GF_Q5_K && F != GF_Q6_K; }
template <int F> constexpr int gm_half() { return gm_pingpong<F>() ? gm_maxsb<F>() / 2 : gm_maxsb<F>(); }

template <int F> constexpr uint32_t gm_group_bytes() {
    return F == GF_Q4_1 ? 160 : F == GF_Q6_K ? 210 : (F == GF_Q5_K || F == GF_Q5_0) ? 176 : F == GF_Q8_0 ? 272 : 144;
}

// k offset, within its 256-k group, of the 8 elements of MFMA step t, k-slice g
template <int F>
__device__ __forceinline__ uint32_t gm_k0(uint32_t t, uint32_t g) {
    if constexpr (gm_kmin<F>()) {
        const uint32_t j = 4 * (t >> 2) + 2 * (g >> 1) + ((t >> 1) & 1), r = 2 * (g & 1) + (t & 1);
        return 32 * j + 8 * r;
    } else if constexpr (F == GF_Q6_K) {
        return 128 * (t >> 2) + 64 * ((t >> 1) & 1) + 16 * g + 8 * (t & 1);
    } else {
        return 64 * g + 32 * (t >> 2) + 16 * ((t >> 1) & 1) + 8 * (t & 1);
    }
}

// LDS image, MR = M rounded up to 8 or 16 (rows M .. MR-1 repeat row M-1
// and feed only discarded outputs):
//   x:  for MFMA step s = 8*group + t, k-slice g, row i: 8 fp16 at
//       ((s*4 + g)*MR + i)*16, the elements k0 = 256*group + gm_k0(t, g) ..
//       +7 in the decode's order 0,2,1,3,4,6,5,7;
//   xs (Q4_K only): at K*MR*2, for super-block sb, h = 0, 1 and row i: 16
//       bytes at ((sb*2 + h)*MR + i)*16 holding xs/32 of sub-blocks
//       J_h = {2h, 2h+1, 4+2h, 5+2h} as 4 fp16 hi parts, then 4 lo parts;
//   partials: 16 KiB after that.
// Staging: direct-to-LDS loads put each 16-byte piece of x in place (piece
// = lane of a 1 KiB load), then a pass reorders the halves of every piece
// (and, for Q4_K, writes the sub-block sums).
template <int F> constexpr uint32_t gm_xs_bytes_per_group(uint32_t MR) { return gm_kmin<F>() ? 32 * MR : 0; }

// fp32 or Q8_1 activations (XK = 1, 2) are staged per row scaled by a power
// of two that puts the row's largest magnitude in [2^14, 2^15): fp16 holds
// any fp32 row without overflow (nor, relative to the row's maximum, loss
// below 2^-24), and Q8_1 rows with d*127 past 65504 likewise.  The scaling
// is exact; y is unscaled per row in the epilogue.  Row maxima (fp32 bits,
// 16 words) sit after the K-split partials.
template <int F, uint32_t MR>
__device__ __forceinline__ uint32_t *gm_row_max(const VkfGemvArgs &a, unsigned char *lds) {
    return (uint32_t *)(lds + (uint64_t)a.K * MR * 2 + (uint64_t)(a.K / 256) * gm_xs_bytes_per_group<F>(MR) + 16384);
}

__device__ __forceinline__ float gm_row_scale(uint32_t mx_bits) {
    const float mx = __builtin_bit_cast(float, mx_bits);
    int e;
    (void)frexpf(mx, &e);
    return mx > 0.0f ? ldexpf(1.0f, 15 - e < 126 ? 15 - e : 126) : 1.0f;
}

// each 16-byte piece of the fp16 LDS image (8 consecutive k of one row, at
// the position the direct loads give it) converted by one thread
template <int F, uint32_t MR, int XK>
__device__ __forceinline__ void gm_convert_x(const VkfGemvArgs &a, unsigned char *lds) {
    uint32_t *rmax = gm_row_max<F, MR>(a, lds);
    if (threadIdx.x < MR) rmax[threadIdx.x] = 0;
    __syncthreads();
    {
        // blockDim.x / MR threads per row, one LDS atomic each
        const uint32_t row = threadIdx.x % MR, rr = row < a.M ? row : a.M - 1;
        float mx = 0.0f;
        if constexpr (XK == 1) {
            const float *src = (const float *)a.x + (uint64_t)rr * a.ldx;
            for (uint32_t c = threadIdx.x / MR; c < a.K / 4; c += blockDim.x / MR) {
                const vkf_f4 v = *(const vkf_f4 *)(src + 4 * c);
                mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3]))));
            }
        } else {
            const uint8_t *src = (const uint8_t *)a.x + (uint64_t)rr * a.ldx;
            for (uint32_t b = threadIdx.x / MR; b < a.K / 32; b += blockDim.x / MR)
                mx = fmaxf(mx, fabsf(vkf_h2f(*(const uint16_t *)(src + 36ull * b))));
            mx *= 127.0f;
        }
        atomicMax(&rmax[row], __builtin_bit_cast(uint32_t, mx));  // non-negative floats order as integers
    }
    __syncthreads();
    const uint32_t pieces = MR * a.K / 8;
    for (uint32_t P = threadIdx.x; P < pieces; P += blockDim.x) {
        const uint32_t i = P % MR, g = (P / MR) & 3, s = P / (4 * MR);
        const uint32_t row = i < a.M ? i : a.M - 1, k0 = (s >> 3) * 256 + gm_k0<F>(s & 7, g);
        const float sc = gm_row_scale(rmax[i]);
        vkf_h8 h;
        if constexpr (XK == 1) {
            const float *src = (const float *)a.x + (uint64_t)row * a.ldx + k0;
            const vkf_f4 v0 = *(const vkf_f4 *)src, v1 = *(const vkf_f4 *)(src + 4);
#pragma unroll
            for (int e = 0; e < 4; e++) {
                h[e] = (_Float16)(v0[e] * sc);
                h[4 + e] = (_Float16)(v1[e] * sc);
            }
        } else {
            // Q8_1 block k0/32: d (fp16) at byte 0, codes at 4 .. 35
            const uint8_t *blk = (const uint8_t *)a.x + (uint64_t)row * a.ldx + (uint64_t)(k0 / 32) * 36;
            const float d = vkf_h2f(*(const uint16_t *)blk) * sc;
            const uint32_t q0 = *(const uint32_t *)(blk + 4 + k0 % 32), q1 = *(const uint32_t *)(blk + 8 + k0 % 32);
#pragma unroll
            for (int e = 0; e < 4; e++) {
                h[e] = (_Float16)(d * (float)(int8_t)(q0 >> (8 * e)));
                h[4 + e] = (_Float16)(d * (float)(int8_t)(q1 >> (8 * e)));
            }
        }
        *(vkf_h8 *)(lds + (uint64_t)P * 16) = h;
    }
}

// the x pieces of the workgroup's 1 KiB direct load c
template <int F, uint32_t MR>
__device__ __forceinline__ void gm_dma_x(const VkfGemvArgs &a, unsigned char *lds, uint32_t c, int lane) {
    const uint32_t P = c * 64 + lane, i = P % MR, g = (P / MR) & 3, s = P / (4 * MR);
    const _Float16 *src =
        (const _Float16 *)a.x + (uint64_t)(i < a.M ? i : a.M - 1) * a.ldx + (s >> 3) * 256 + gm_k0<F>(s & 7, g);
    vkf_load_lds16(src, lds + c * 1024);
}

// halves 0,1,2,3 -> 0,2,1,3 (and 4..7 likewise)
__device__ __forceinline__ vkf_u4 gm_reorder(vkf_u4 v) {
    return vkf_u4{__builtin_amdgcn_perm(v[1], v[0], 0x05040100u), __builtin_amdgcn_perm(v[1], v[0], 0x07060302u),
                  __builtin_amdgcn_perm(v[3], v[2], 0x05040100u), __builtin_amdgcn_perm(v[3], v[2], 0x07060302u)};
}

// the reorder (and Q4_K's sub-block sums), after the direct loads have landed
template <int F, uint32_t MR>
__device__ __forceinline__ void gm_stage_pass(const VkfGemvArgs &a, unsigned char *lds) {
    if constexpr (!gm_kmin<F>()) {
        const uint32_t pieces = (a.K / 8) * MR;
        for (uint32_t p = threadIdx.x; p < pieces; p += blockDim.x) {
            vkf_u4 *pc = (vkf_u4 *)(lds + p * 16);
            *pc = gm_reorder(*pc);
        }
        return;
    }
    const uint32_t items = (a.K / 32) * MR;  // (super-block, sub-block, row)
    unsigned char *xs = lds + (uint64_t)a.K * MR * 2;
    const vkf_h2 ones = {(_Float16)1.0f, (_Float16)1.0f};
    for (uint32_t it = threadIdx.x; it < items; it += blockDim.x) {
        const uint32_t m = it % MR, sj = it / MR, sb = sj >> 3, j = sj & 7;
        vkf_u4 *pc[4];
        vkf_u4 v[4];
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const uint32_t t = 4 * (j >> 2) + 2 * (j & 1) + (r & 1), g = 2 * ((j >> 1) & 1) + (r >> 1);
            pc[r] = (vkf_u4 *)(lds + (((sb * 8 + t) * 4 + g) * MR + m) * 16);
            v[r] = *pc[r];
        }
        float f = 0.0f;
#pragma unroll
        for (int r = 0; r < 4; r++) {
#pragma unroll
            for (int d = 0; d < 4; d++) {
                // (a bit_cast of the vector element itself read element 0 for
                // every d with this compiler)
                const uint32_t w = v[r][d];
                f = __builtin_amdgcn_fdot2(__builtin_bit_cast(vkf_h2, w), ones, f, false);
            }
            *pc[r] = gm_reorder(v[r]);
        }
        const float fs = f * 0.03125f;
        const _Float16 hi = (_Float16)fs, lo = (_Float16)(fs - (float)hi);
        _Float16 *e = (_Float16 *)(xs + ((sb * 2 + ((j >> 1) & 1)) * MR + m) * 16);
        const uint32_t pos = (j & 1) + 2 * (j >> 2);
        e[pos] = hi;
        e[4 + pos] = lo;
    }
}

// One lane's share of a 256-k group: Q4_K header, qs 16g.. and 64+16g..;
// Q4_0 the 36 bytes of block pair g (v[2][0] last); Q4_1 its 40 bytes
// (v[2][0..1] last); Q6_K its four 16-byte runs and the scales, each as the
// 20 bytes from the 4-byte aligned address below it, and d.
template <int F>
struct GmSb {
    vkf_u4 v[3];
};
template <>
struct GmSb<GF_Q5_0> {
    vkf_u4 v[3];  // bytes 0 .. 15, 16 .. 31, 28 .. 43 of the block pair
};
template <>
struct GmSb<GF_Q8_0> {
    vkf_u4 v[4];  // bytes 0 .. 63 of the block pair
    uint32_t e;   // bytes 64 .. 67
};
template <>
struct GmSb<GF_Q5_K> {
    vkf_u4 v[4];  // header, qh run, qs runs
};
template <>
struct GmSb<GF_Q6_K> {
    vkf_u4 r[5];     // ql run 0, ql run 1, qh run 0, qh run 1, scales: first 16 bytes
    uint32_t e[5];   // the dword after each
    uint32_t d, sh;  // d (fp16 bits); byte offset of the super-block in its dword
};

template <int F>
__device__ __forceinline__ void gm_load(const uint8_t *row, uint32_t sb, int g, GmSb<F> &t) {
    typedef unsigned int u4a4 __attribute__((ext_vector_type(4), aligned(4)));
    typedef unsigned int u2a4 __attribute__((ext_vector_type(2), aligned(4)));
    const uint8_t *b = row + (uint64_t)gm_group_bytes<F>() * sb;
    if constexpr (F == GF_Q6_K) {
        // runs at 16g, 64 + 16g, 128 + 16(g&1), 160 + 16(g&1), 192; with
        // sh = 2 the aligned 20 bytes start 2 bytes before the run and end
        // at its byte 17, for the scales at byte 209 of the super-block (d);
        // with sh = 0 the scales' extra dword is re-read from byte 204 (not
        // used) so that no load passes byte 209
        t.sh = (uint32_t)(uintptr_t)b & 3u;
        const uint8_t *a = b - t.sh;
        const uint32_t off[5] = {16u * g, 64u + 16u * g, 128u + 16u * (g & 1), 160u + 16u * (g & 1), 192u};
#pragma unroll
        for (int k = 0; k < 5; k++) {
            t.r[k] = *(const u4a4 *)(a + off[k]);
            t.e[k] = *(const uint32_t *)(a + off[k] + (k < 4 || t.sh ? 16 : 12));
        }
        t.d = *(const uint16_t *)(b + 208);
    } else if constexpr (F == GF_Q5_0) {
        const uint8_t *p = b + 44 * g;
        t.v[0] = *(const u4a4 *)p;
        t.v[1] = *(const u4a4 *)(p + 16);
        t.v[2] = *(const u4a4 *)(p + 28);
    } else if constexpr (F == GF_Q8_0) {
        const uint8_t *p = b + 68 * g;
#pragma unroll
        for (int k = 0; k < 4; k++) t.v[k] = *(const u4a4 *)(p + 16 * k);
        t.e = *(const uint32_t *)(p + 64);
    } else if constexpr (F == GF_Q5_K) {
        t.v[0] = *(const vkf_u4 *)b;
        t.v[1] = *(const vkf_u4 *)(b + 16 + 16 * (g & 1));
        t.v[2] = *(const vkf_u4 *)(b + 48 + 16 * g);
        t.v[3] = *(const vkf_u4 *)(b + 112 + 16 * g);
    } else if constexpr (F == GF_Q4_K) {
        t.v[0] = *(const vkf_u4 *)b;
        t.v[1] = *(const vkf_u4 *)(b + 16 + 16 * g);
        t.v[2] = *(const vkf_u4 *)(b + 80 + 16 * g);
    } else if constexpr (F == GF_Q4_0) {
        const uint8_t *p = b + 36 * g;
        t.v[0] = *(const u4a4 *)p;
        t.v[1] = *(const u4a4 *)(p + 16);
        t.v[2][0] = *(const uint32_t *)(p + 32);
    } else {
        const uint8_t *p = b + 40 * g;
        t.v[0] = *(const u4a4 *)p;
        t.v[1] = *(const u4a4 *)(p + 16);
        const vkf_u2 c = *(const u2a4 *)(p + 32);
        t.v[2][0] = c[0];
        t.v[2][1] = c[1];
    }
}

// Loads of groups s0 .. s0 + gm_maxsb - 1, those at or past sb1 clamped to
// sb1 - 1 (loaded and not used), so that the loads form one straight
// sequence.  sb1 >= 1.
template <int F, int NB>
__device__ __forceinline__ void gm_load_batch(const uint8_t *row, uint32_t s0, uint32_t sb1, int g, GmSb<F> *t) {
#pragma unroll
    for (int u = 0; u < NB; u++) gm_load<F>(row, s0 + u < sb1 ? s0 + u : sb1 - 1, g, t[u]);
}

// load instructions gm_load issues
template <int F> constexpr int gm_loads_per_group() {
    return F == GF_Q6_K ? 11 : F == GF_Q8_0 ? 5 : F == GF_Q5_K ? 4 : 3;
}

__device__ __forceinline__ vkf_h2 gm_h2(uint32_t u) { return __builtin_bit_cast(vkf_h2, u); }
__device__ __forceinline__ uint32_t gm_u(vkf_h2 h) { return __builtin_bit_cast(uint32_t, h); }

// (v & mask) | c in one v_and_or_b32.  gfx9 VOP3 takes no literal and one
// scalar operand, so the mask comes in an SGPR and c in a VGPR.
__device__ __forceinline__ uint32_t gm_and_or(uint32_t v, uint32_t mask, uint32_t c) {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(v), "s"(mask), "v"(c));
    return r;
}

// (1024 + q) or (1024 + 16q) fp16 pairs of 8 elements held in the low (HI = 0)
// or high (HI = 1) nibbles of code dwords d0, d1 and their >> 8 shifts t0, t1;
// c64 = 0x64006400
template <int HI>
__device__ __forceinline__ void gm_nibbles(uint32_t d0, uint32_t t0, uint32_t d1, uint32_t t1, uint32_t c64,
                                           vkf_h2 h[4]) {
    const uint32_t mask = HI ? 0x00f000f0u : 0x000f000fu;
    h[0] = gm_h2(gm_and_or(d0, mask, c64));
    h[1] = gm_h2(gm_and_or(t0, mask, c64));
    h[2] = gm_h2(gm_and_or(d1, mask, c64));
    h[3] = gm_h2(gm_and_or(t1, mask, c64));
}

// Q4_K: sc*q; s, n = the sub-block's (sc, -1024*sc) or (sc/16, -64*sc)
template <int HI>
__device__ __forceinline__ vkf_h8 gm_decode(uint32_t d0, uint32_t t0, uint32_t d1, uint32_t t1, _Float16 s,
                                            _Float16 n, uint32_t c64) {
    vkf_h2 h[4];
    gm_nibbles<HI>(d0, t0, d1, t1, c64, h);
    const vkf_h2 s2 = {s, s}, n2 = {n, n};
    vkf_u4 r;
#pragma unroll
    for (int p = 0; p < 4; p++) r[p] = gm_u(__builtin_elementwise_fma(h[p], s2, n2));
    return __builtin_bit_cast(vkf_h8, r);
}

// Q5_K: gm_decode with the fifth bits; u0, u1 = the qh dwords of d0, d1
// shifted right by the sub-block index, so bit 0 of each byte is the bit
template <int HI>
__device__ __forceinline__ vkf_h8 gm_decode5(uint32_t d0, uint32_t t0, uint32_t d1, uint32_t t1, uint32_t u0,
                                             uint32_t u1, _Float16 s, _Float16 n, uint32_t c64) {
    vkf_h2 h[4];
    gm_nibbles<HI>(d0, t0, d1, t1, c64, h);
    const uint32_t m5 = HI ? 0x01000100u : 0x00100010u;
    const uint32_t f[4] = {HI ? u0 << 8 : u0 << 4, HI ? u0 : u0 >> 4, HI ? u1 << 8 : u1 << 4, HI ? u1 : u1 >> 4};
    const vkf_h2 s2 = {s, s}, n2 = {n, n};
    vkf_u4 r;
#pragma unroll
    for (int p = 0; p < 4; p++)
        r[p] = gm_u(__builtin_elementwise_fma(gm_h2(gm_and_or(f[p], m5, gm_u(h[p]))), s2, n2));
    return __builtin_bit_cast(vkf_h8, r);
}

// Q8_0: d*b of the 8 int8 codes in dwords d0, d1; d2 = {d, d}
__device__ __forceinline__ vkf_h8 gm_decode_q8(uint32_t d0, uint32_t d1, vkf_h2 d2, uint32_t c64) {
    const vkf_h2 m1152 = {(_Float16)-1152.0f, (_Float16)-1152.0f};
    const uint32_t u0 = d0 ^ 0x80808080u, u1 = d1 ^ 0x80808080u;
    const uint32_t p[4] = {gm_and_or(u0, 0x00ff00ffu, c64), gm_and_or(u0 >> 8, 0x00ff00ffu, c64),
                           gm_and_or(u1, 0x00ff00ffu, c64), gm_and_or(u1 >> 8, 0x00ff00ffu, c64)};
    vkf_u4 r;
#pragma unroll
    for (int k = 0; k < 4; k++) r[k] = gm_u((gm_h2(p[k]) + m1152) * d2);
    return __builtin_bit_cast(vkf_h8, r);
}

// Q5_0: d*(q - 16) of 8 elements: code dwords d0, d1 (nibble HI), fifth bits
// b0, b1 (bit 4k of byte... : bit k of the element's byte, one byte per
// element, as gm_decode5 takes them); d2 = {d, d}
template <int HI>
__device__ __forceinline__ vkf_h8 gm_decode_q50(uint32_t d0, uint32_t d1, uint32_t b0, uint32_t b1, vkf_h2 d2,
                                                uint32_t c64) {
    vkf_h2 h[4];
    gm_nibbles<HI>(d0, d0 >> 8, d1, d1 >> 8, c64, h);
    const uint32_t m5 = HI ? 0x01000100u : 0x00100010u;
    const uint32_t f[4] = {HI ? b0 << 8 : b0 << 4, HI ? b0 : b0 >> 4, HI ? b1 << 8 : b1 << 4, HI ? b1 : b1 >> 4};
    // (1024 + q) - 1040 or (1024 + 16q)/16 - 80: q - 16, exact; then d, one rounding
    const _Float16 sc = HI ? (_Float16)0.0625f : (_Float16)1.0f, of = HI ? (_Float16)-80.0f : (_Float16)-1040.0f;
    const vkf_h2 sc2 = {sc, sc}, of2 = {of, of};
    vkf_u4 r;
#pragma unroll
    for (int p = 0; p < 4; p++) {
        const vkf_h2 q = __builtin_elementwise_fma(gm_h2(gm_and_or(f[p], m5, gm_u(h[p]))), sc2, of2);
        r[p] = gm_u(q * d2);
    }
    return __builtin_bit_cast(vkf_h8, r);
}

// the four fifth bits of elements e .. e+3 (bits e.. of qh) one per byte, at bit 0
__device__ __forceinline__ uint32_t gm_spread4(uint32_t qh, uint32_t e) {
    return (((qh >> e) & 0xfu) * 0x00204081u) & 0x01010101u;
}

// Q4_0 (d*(q - 8)) or Q4_1 (d*q + m) weights of 8 elements; d, m fp16
template <int F, int HI>
__device__ __forceinline__ vkf_h8 gm_decode_w(uint32_t d0, uint32_t d1, _Float16 d, _Float16 m, uint32_t c64) {
    vkf_h2 h[4];
    gm_nibbles<HI>(d0, d0 >> 8, d1, d1 >> 8, c64, h);
    // (1024 + q) - off or (1024 + 16q)/16 - off: q - 8 (Q4_0) or q (Q4_1)
    const _Float16 sc = HI ? (_Float16)0.0625f : (_Float16)1.0f;
    const _Float16 of = F == GF_Q4_0 ? (HI ? (_Float16)-72.0f : (_Float16)-1032.0f)
                                     : (HI ? (_Float16)-64.0f : (_Float16)-1024.0f);
    const vkf_h2 sc2 = {sc, sc}, of2 = {of, of}, d2 = {d, d}, m2 = {m, m};
    vkf_u4 r;
#pragma unroll
    for (int p = 0; p < 4; p++) {
        const vkf_h2 q = __builtin_elementwise_fma(h[p], sc2, of2);
        r[p] = gm_u(F == GF_Q4_0 ? q * d2 : __builtin_elementwise_fma(q, d2, m2));
    }
    return __builtin_bit_cast(vkf_h8, r);
}

__device__ __forceinline__ _Float16 gm_f16(uint32_t bits) { return __builtin_bit_cast(_Float16, (uint16_t)bits); }

// Q6_K: sc*(q - 32) of 8 elements from ql dwords d0, d1 (nibble HI) and qh
// dwords e0, e1 (two bits at qs of each byte); sc2 = {sc, sc}
template <int HI>
__device__ __forceinline__ vkf_h8 gm_decode_q6(uint32_t d0, uint32_t d1, uint32_t e0, uint32_t e1, uint32_t qs,
                                               vkf_h2 sc2, uint32_t c64) {
    const vkf_h2 m1056 = {(_Float16)-1056.0f, (_Float16)-1056.0f};
    const uint32_t n0 = HI ? d0 >> 4 : d0, n1 = HI ? d1 >> 4 : d1;
    const uint32_t b0 = ((e0 >> qs) & 0x03030303u) << 4, b1 = ((e1 >> qs) & 0x03030303u) << 4;
    // (1024 + q) pairs (bytes 0,2 then 1,3 of each dword)
    const uint32_t p[4] = {gm_and_or(b0, 0x00300030u, gm_and_or(n0, 0x000f000fu, c64)),
                           gm_and_or(b0 >> 8, 0x00300030u, gm_and_or(n0 >> 8, 0x000f000fu, c64)),
                           gm_and_or(b1, 0x00300030u, gm_and_or(n1, 0x000f000fu, c64)),
                           gm_and_or(b1 >> 8, 0x00300030u, gm_and_or(n1 >> 8, 0x000f000fu, c64))};
    vkf_u4 r;
#pragma unroll
    for (int k = 0; k < 4; k++) r[k] = gm_u((gm_h2(p[k]) + m1056) * sc2);
    return __builtin_bit_cast(vkf_h8, r);
}

// One 256-k group of one 16-row tile: y4 += the group's products.  X(t)
// gives the activation operand of MFMA step t (8 fp16, the decode's k
// order) and XM() the min-term operand of Q4_K / Q5_K (the sub-block sums
// of x on even k-slices, zero on odd ones).
template <int F, class XF, class XMF>
__device__ __forceinline__ void gm_group(const GmSb<F> &T, XF X, XMF XM, int lg, uint32_t sel, uint32_t c64,
                                         vkf_f4 &y4) {
    const vkf_f4 zero = {0, 0, 0, 0};
    const vkf_h2 one16 = {(_Float16)1.0f, (_Float16)0.0625f}, off = {(_Float16)-1024.0f, (_Float16)-64.0f};
    const vkf_h2 m1024 = {(_Float16)-1024.0f, (_Float16)-1024.0f};
    (void)XM;
    (void)sel;
    (void)one16;
    (void)off;
    (void)m1024;
    if constexpr (F == GF_Q6_K) {
        uint32_t w[5][4];  // the runs, shifted into place
#pragma unroll
        for (int k = 0; k < 5; k++)
#pragma unroll
            for (int c = 0; c < 4; c++)
                w[k][c] = __builtin_amdgcn_alignbyte(c < 3 ? T.r[k][c + 1] : T.e[k], T.r[k][c], T.sh);
        const uint32_t qs = 2u * (lg >> 1);  // + 4h
        vkf_f4 acc = zero;
#pragma unroll
        for (int n = 0; n < 2; n++)
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const int8_t scb = (int8_t)(w[4][2 * n + h] >> (8 * lg));
                const _Float16 sc = (_Float16)(float)scb;
                const vkf_h2 sc2 = {sc, sc};
#pragma unroll
                for (int hf = 0; hf < 2; hf++) {
                    const vkf_h8 xv = X(4 * n + 2 * h + hf);
                    const uint32_t d0 = w[n][2 * hf], d1 = w[n][2 * hf + 1];
                    const uint32_t e0 = w[2 + n][2 * hf], e1 = w[2 + n][2 * hf + 1];
                    const vkf_h8 bv = h ? gm_decode_q6<1>(d0, d1, e0, e1, qs + 4, sc2, c64)
                                        : gm_decode_q6<0>(d0, d1, e0, e1, qs, sc2, c64);
                    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(xv, bv, acc, 0, 0, 0);
                }
            }
        const float d = vkf_h2f(T.d);
#pragma unroll
        for (int e = 0; e < 4; e++) y4[e] = fmaf(d, acc[e], y4[e]);
    } else if constexpr (F == GF_Q5_0) {
        // block 0: d at bytes 0-1, qh 2 .. 5, qs 6 .. 21; block 1: d at 22-23,
        // qh 24 .. 27, qs 28 .. 43 (dwords w[k] = bytes 4k .. 4k+3)
        
        const uint32_t w[11] = {T.v[0][0], T.v[0][1], T.v[0][2], T.v[0][3], T.v[1][0], T.v[1][1],
                                T.v[1][2], T.v[1][3], T.v[2][1], T.v[2][2], T.v[2][3]};
        uint32_t q[2][4], qh[2], dd[2];
        dd[0] = w[0] & 0xffffu;
        qh[0] = __builtin_amdgcn_alignbyte(w[1], w[0], 2);
#pragma unroll
        for (int k = 0; k < 4; k++) q[0][k] = __builtin_amdgcn_alignbyte(w[k + 2], w[k + 1], 2);
        dd[1] = w[5] >> 16;
        qh[1] = w[6];
        q[1][0] = w[7]; q[1][1] = w[8]; q[1][2] = w[9]; q[1][3] = w[10];
#pragma unroll
        for (int blk = 0; blk < 2; blk++) {
            const _Float16 d = gm_f16(dd[blk]);
            const vkf_h2 d2 = {d, d};
#pragma unroll
            for (int hf = 0; hf < 2; hf++) {
                const uint32_t c0 = q[blk][2 * hf], c1 = q[blk][2 * hf + 1];
                // steps 4blk + hf (elements 8hf .. +7, low nibbles) and 4blk + 2 + hf (16 + 8hf .., high)
                const vkf_h8 xl = X(4 * blk + hf);
                const vkf_h8 xh = X(4 * blk + hf + 2);
                const uint32_t el = 8 * hf, eh = 16 + 8 * hf;
                const vkf_h8 bl = gm_decode_q50<0>(c0, c1, gm_spread4(qh[blk], el), gm_spread4(qh[blk], el + 4), d2, c64);
                const vkf_h8 bh = gm_decode_q50<1>(c0, c1, gm_spread4(qh[blk], eh), gm_spread4(qh[blk], eh + 4), d2, c64);
                y4 = __builtin_amdgcn_mfma_f32_16x16x32_f16(xl, bl, y4, 0, 0, 0);
                y4 = __builtin_amdgcn_mfma_f32_16x16x32_f16(xh, bh, y4, 0, 0, 0);
            }
        }
    } else if constexpr (F == GF_Q8_0) {
        // block 0: d at bytes 0-1, codes 2 .. 33; block 1: d at 34-35, codes 36 .. 67
        
        const uint32_t w[17] = {T.v[0][0], T.v[0][1], T.v[0][2], T.v[0][3], T.v[1][0], T.v[1][1],
                                T.v[1][2], T.v[1][3], T.v[2][0], T.v[2][1], T.v[2][2], T.v[2][3],
                                T.v[3][0], T.v[3][1], T.v[3][2], T.v[3][3], T.e};
#pragma unroll
        for (int blk = 0; blk < 2; blk++) {
            const _Float16 d = gm_f16(blk ? w[8] >> 16 : w[0] & 0xffffu);
            const vkf_h2 d2 = {d, d};
#pragma unroll
            for (int st = 0; st < 4; st++) {
                uint32_t c0, c1;
                if (blk == 0) {
                    c0 = __builtin_amdgcn_alignbyte(w[2 * st + 1], w[2 * st], 2);
                    c1 = __builtin_amdgcn_alignbyte(w[2 * st + 2], w[2 * st + 1], 2);
                } else {
                    c0 = w[9 + 2 * st];
                    c1 = w[10 + 2 * st];
                }
                const vkf_h8 xv = X(4 * blk + st);
                y4 = __builtin_amdgcn_mfma_f32_16x16x32_f16(xv, gm_decode_q8(c0, c1, d2, c64), y4, 0, 0,
                                                            0);
            }
        }
    } else if constexpr (gm_kmin<F>()) {
        const vkf_u4 hdr = T.v[0];
        const float dall = vkf_h2f(hdr[0] & 0xffffu), dmin = vkf_h2f(hdr[0] >> 16);
        const uint32_t s0w = hdr[1], s4w = hdr[2], s8w = hdr[3];
        const uint32_t sc[2] = {s0w & 0x3f3f3f3fu, (s8w & 0x0f0f0f0fu) | ((s0w >> 2) & 0x30303030u)};
        const uint32_t mn[2] = {s4w & 0x3f3f3f3fu,
                                ((s8w >> 4) & 0x0f0f0f0fu) | ((s4w >> 2) & 0x30303030u)};
        // load L covers sub-blocks 4L + 2h (low nibbles) and 4L + 2h + 1
        // (high): scale pairs (sc, sc'/16), (-1024 sc, -64 sc'), and
        // the mins (mn, mn') of those sub-blocks
        vkf_h2 S[2], Nn[2];
        uint32_t bm[2];
#pragma unroll
        for (int L = 0; L < 2; L++) {
            S[L] = __builtin_elementwise_fma(gm_h2(__builtin_amdgcn_perm(0x64646464u, sc[L], sel)), one16,
                                             off);
            Nn[L] = S[L] * m1024;
            bm[L] = gm_u(gm_h2(__builtin_amdgcn_perm(0x64646464u, mn[L], sel)) + m1024);
        }
        vkf_f4 acc = zero;
#pragma unroll
        for (int L = 0; L < 2; L++)
#pragma unroll
            for (int hf = 0; hf < 2; hf++) {
                const vkf_u4 q = T.v[(F == GF_Q5_K ? 2 : 1) + L];
                const uint32_t d0 = q[2 * hf], d1 = q[2 * hf + 1], e0 = d0 >> 8, e1 = d1 >> 8;
                // MFMA steps 8sb + 4L + hf (low nibbles) and 8sb + 4L + 2 + hf (high)
                const vkf_h8 xl = X(4 * L + hf);
                const vkf_h8 xh = X(4 * L + hf + 2);
                vkf_h8 bl, bh;
                if constexpr (F == GF_Q5_K) {
                    // sub-blocks 4L + 2(g>>1) (low nibbles) and + 1 (high)
                    const uint32_t jl = 4 * L + 2 * (lg >> 1);
                    const uint32_t h0 = T.v[1][2 * hf], h1 = T.v[1][2 * hf + 1];
                    bl = gm_decode5<0>(d0, e0, d1, e1, h0 >> jl, h1 >> jl, S[L][0], Nn[L][0], c64);
                    bh = gm_decode5<1>(d0, e0, d1, e1, h0 >> (jl + 1), h1 >> (jl + 1), S[L][1], Nn[L][1],
                                       c64);
                } else {
                    bl = gm_decode<0>(d0, e0, d1, e1, S[L][0], Nn[L][0], c64);
                    bh = gm_decode<1>(d0, e0, d1, e1, S[L][1], Nn[L][1], c64);
                }
                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(xl, bl, acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(xh, bh, acc, 0, 0, 0);
            }
        // min term: even k-slices carry xs hi and lo of the lane pair's 4
        // sub-blocks, odd ones zero
        const vkf_h8 xm = XM();
        const vkf_u4 bmin = {bm[0], bm[1], bm[0], bm[1]};
        const vkf_f4 am =
            __builtin_amdgcn_mfma_f32_16x16x32_f16(xm, __builtin_bit_cast(vkf_h8, bmin), zero, 0, 0, 0);
        const float dm32 = -32.0f * dmin;
#pragma unroll
        for (int e = 0; e < 4; e++) y4[e] = fmaf(dm32, am[e], fmaf(dall, acc[e], y4[e]));
    } else {
        // block pair 2g, 2g+1: code dwords and (d, m) of each block
        const vkf_u4 w0 = T.v[0], w1 = T.v[1];
        uint32_t q[2][4], dm[2];
        if constexpr (F == GF_Q4_0) {
            // 18-byte blocks: block 0 = bytes 0..17 (qs from byte 2),
            // block 1 = bytes 18..35 (qs from byte 20, aligned)
            const uint32_t w[5] = {w0[0], w0[1], w0[2], w0[3], w1[0]};
#pragma unroll
            for (int j = 0; j < 4; j++) q[0][j] = __builtin_amdgcn_alignbyte(w[j + 1], w[j], 2);
            q[1][0] = w1[1]; q[1][1] = w1[2]; q[1][2] = w1[3]; q[1][3] = T.v[2][0];
            dm[0] = w0[0] & 0xffffu;
            dm[1] = w1[0] >> 16;
        } else {
            // 20-byte blocks: (d, m), 16 bytes of qs
            q[0][0] = w0[1]; q[0][1] = w0[2]; q[0][2] = w0[3]; q[0][3] = w1[0];
            q[1][0] = w1[2]; q[1][1] = w1[3]; q[1][2] = T.v[2][0]; q[1][3] = T.v[2][1];
            dm[0] = w0[0];
            dm[1] = w1[1];
        }
#pragma unroll
        for (int blk = 0; blk < 2; blk++) {
            const _Float16 d = gm_f16(dm[blk] & 0xffffu), m = gm_f16(dm[blk] >> 16);
#pragma unroll
            for (int hf = 0; hf < 2; hf++) {
                const uint32_t d0 = q[blk][2 * hf], d1 = q[blk][2 * hf + 1];
                // steps 4blk + hf (low nibbles) and 4blk + 2 + hf (high)
                const vkf_h8 xl = X(4 * blk + hf);
                const vkf_h8 xh = X(4 * blk + hf + 2);
                const vkf_h8 bl = gm_decode_w<F, 0>(d0, d1, d, m, c64);
                const vkf_h8 bh = gm_decode_w<F, 1>(d0, d1, d, m, c64);
                y4 = __builtin_amdgcn_mfma_f32_16x16x32_f16(xl, bl, y4, 0, 0, 0);
                y4 = __builtin_amdgcn_mfma_f32_16x16x32_f16(xh, bh, y4, 0, 0, 0);
            }
        }
    }
}

template <int F, uint32_t MR, int XK>
__device__ __forceinline__ void gemv_mfma(const VkfGemvArgs &a, unsigned char *smem) {
    const uint32_t nsb = a.K / 256;
    const uint32_t P = (a.flags >> 8) & 0xffu;  // waves per tile: 4, 8 or 16
    const uint32_t G = GM_WAVES / P;            // tiles per workgroup round
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: scalar loop bounds
    const int li = lane & 15, lg = lane >> 4;
    const uint32_t grp = wave / P, part = wave % P;
    const uint32_t ntiles = (a.N + 15) / 16;
    const uint32_t per = (nsb + P - 1) / P;  // groups per wave
    const uint32_t sb0 = part * per, sb1 = sb0 + per < nsb ? sb0 + per : nsb;  // sb1 >= 1

    // x goes to LDS by direct loads, the first batch of weight loads right
    // behind it; vmcnt counts in order, so waiting for x leaves the weights
    // in flight.  blockIdx.x * G < ntiles: the host launches at most
    // ceil(ntiles / G) workgroups.
    constexpr int H = gm_half<F>();
    GmSb<F> ta[H], tb[gm_pingpong<F>() ? H : 1];
    const uint32_t nc = MR * a.K * 2 / 1024;  // 1 KiB loads of x (MR * K * 2 is a multiple of 4096)
    if constexpr (XK == 0) {
        for (uint32_t c = wave; c < nc; c += GM_WAVES) gm_dma_x<F, MR>(a, smem, c, lane);
    } else {
        (void)nc;
        gm_convert_x<F, MR, XK>(a, smem);
    }
    asm volatile("" ::: "memory");
    {
        const uint32_t n = (blockIdx.x * G + grp) * 16 + li;
        gm_load_batch<F, H>(a.w + (uint64_t)(n < a.N ? n : a.N - 1) * a.row_bytes, sb0, sb1, lg, ta);
    }
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(gm_loads_per_group<F>() * H) : "memory");
    __syncthreads();
    gm_stage_pass<F, MR>(a, smem);
    __syncthreads();
    bool pre = true;
    const unsigned char *xs = smem + (uint64_t)a.K * MR * 2;
    float *red = (float *)(xs + nsb * gm_xs_bytes_per_group<F>(MR));  // [16 waves][64 lanes][4]

    const uint32_t arow = li < (int)MR ? li : li & 7;  // rows >= M feed discarded outputs
    const unsigned char *xw = smem + (lg * MR + arow) * 16;  // this lane's x pieces
    const unsigned char *xsw = xs + ((lg >> 1) * MR + arow) * 16;
    const uint32_t sel = (lg >> 1) ? 0x04030402u : 0x04010400u;  // bytes 2h, 2h+1 as (1024 + v) fp16
    const vkf_f4 zero = {0, 0, 0, 0};
    uint32_t c64 = 0x64006400u;
    asm volatile("" : "+v"(c64));  // held in a VGPR for gm_and_or

    for (uint32_t t0 = blockIdx.x * G; t0 < ntiles; t0 += gridDim.x * G) {  // workgroup-uniform loop
        const uint32_t tile = t0 + grp;
        const uint32_t n = tile * 16 + li;
        const uint8_t *row = a.w + (uint64_t)(n < a.N ? n : a.N - 1) * a.row_bytes;
        vkf_f4 y4 = zero;
        auto proc = [&](const GmSb<F> *tt, uint32_t s0) {
#pragma unroll
            for (int u = 0; u < H; u++) {
                const uint32_t sb = s0 + u;
                if (sb >= sb1) break;
                const unsigned char *xg = xw + sb * (32 * MR * 16);  // step 8sb
                const auto X = [&](int t) { return *(const vkf_h8 *)(xg + t * (4 * MR * 16)); };
                const auto XM = [&]() {
                    vkf_h8 xm = {};
                    if ((lg & 1) == 0) xm = *(const vkf_h8 *)(xsw + sb * (2 * MR * 16));
                    return xm;
                };
                gm_group<F>(tt[u], X, XM, lg, sel, c64, y4);
            }
        };
        if constexpr (gm_pingpong<F>()) {
            // two half-batches in turn: while one is decoded the other's loads
            // are in flight (the compiler's vmcnt waits keep the younger half
            // pending)
            if (!pre) gm_load_batch<F, H>(row, sb0, sb1, lg, ta);
            pre = false;
            for (uint32_t s0 = sb0; s0 < sb1; s0 += 2 * H) {
                if (s0 + H < sb1) gm_load_batch<F, H>(row, s0 + H, sb1, lg, tb);
                proc(ta, s0);
                if (s0 + 2 * H < sb1) gm_load_batch<F, H>(row, s0 + 2 * H, sb1, lg, ta);
                if (s0 + H < sb1) proc(tb, s0 + H);
            }
        } else {
            (void)tb;
            for (uint32_t s0 = sb0; s0 < sb1; s0 += H) {
                if (!pre) gm_load_batch<F, H>(row, s0, sb1, lg, ta);
                pre = false;
                proc(ta, s0);
            }
        }
        // K-split partials: waves of the group meet in LDS
        float *r = red + (wave * 64 + lane) * 4;
#pragma unroll
        for (int e = 0; e < 4; e++) r[e] = y4[e];
        __syncthreads();
        if (part == 0) {
            vkf_f4 s = y4;
            for (uint32_t p = 1; p < P; p++)
#pragma unroll
                for (int e = 0; e < 4; e++) s[e] += red[((wave + p) * 64 + lane) * 4 + e];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const uint32_t m = 4 * lg + e;
                if (m < a.M && n < a.N) {
                    float v = s[e];
                    if constexpr (XK != 0) v *= 1.0f / gm_row_scale(gm_row_max<F, MR>(a, smem)[m]);  // exact
                    float *yp = a.y + (uint64_t)m * a.ldy + n;
                    *yp = (a.flags & 1u) ? *yp + v : v;
                }
            }
        }
        __syncthreads();
    }
}

template <int F, int XK>
__device__ __forceinline__ void gemv_mfma_entry(const VkfGemvArgs &a) {
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    if (a.M <= 8) gemv_mfma<F, 8, XK>(a, smem);
    else gemv_mfma<F, 16, XK>(a, smem);
}

#define VKF_GEMV_MFMA(name, F)                                                                            \
    VKF_KERNEL void __launch_bounds__(64 * GM_WAVES) vkf_gemv_mfma_##name##_f16(VkfGemvArgs a) {           \
        gemv_mfma_entry<F, 0>(a);                                                                         \
    }                                                                                                     \
    VKF_KERNEL void __launch_bounds__(64 * GM_WAVES) vkf_gemv_mfma_##name##_f32(VkfGemvArgs a) {           \
        gemv_mfma_entry<F, 1>(a);                                                                         \
    }                                                                                                     \
    VKF_KERNEL void __launch_bounds__(64 * GM_WAVES) vkf_gemv_mfma_##name##_q8_1(VkfGemvArgs a) {          \
        gemv_mfma_entry<F, 2>(a);                                                                         \
    }
VKF_GEMV_MFMA(q4_k, GF_Q4_K)
VKF_GEMV_MFMA(q4_0, GF_Q4_0)
VKF_GEMV_MFMA(q4_1, GF_Q4_1)
VKF_GEMV_MFMA(q6_k, GF_Q6_K)
VKF_GEMV_MFMA(q5_k, GF_Q5_K)
VKF_GEMV_MFMA(q8_0, GF_Q8_0)
VKF_GEMV_MFMA(q5_0, GF_Q5_0)

// ---------------------------------------------------------------------------
// fp16 activations in registers (gemv_mfma_xr).  The P waves of a
// workgroup split K P ways: wave w owns the 256-k groups [w*G/P,
// (w+1)*G/P) (at most NG of them) of every tile and holds those groups'
// activation pieces in registers for the whole launch, in the decode's k
// order (no LDS image, no staging barrier; Q4_K / Q5_K also hold the
// sub-block sums of x for the min-term MFMA, added across the lane pair
// that shares each sub-block).  The workgroup walks its tiles one per
// round: a wave multiplies its groups of the round's tile, requests the
// next round's weights, and the P partial tiles meet in LDS, where waves
// 0..3 each add one of the four elements per lane in wave order.  Rows >= M of the MFMA operand repeat row M - 1
// (MR = M rounded up to 4, 8 or 16) and feed discarded outputs.
//
// K slices (KS, for K longer than P waves hold): the S = flags bits 8..15
// slices [s*G/S, (s+1)*G/S) of the groups go to different workgroups;
// workgroup b takes slice b % S of the tiles b / S, b / S + gridDim.x / S,
// ... (gridDim.x a multiple of S) and stores its partial tile to
// y[(s*M + m)*ldy + n] (y is then the caller's workspace), which
// vkf_gemv_split_sum adds up in slice order.
// ---------------------------------------------------------------------------
template <int F, uint32_t MR, int NG, int P, bool KS>
__device__ __forceinline__ void gemv_mfma_xr(const VkfGemvArgs &a, unsigned char *smem) {
    const uint32_t nsb = a.K / 256;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int li = lane & 15, lg = lane >> 4;
    const uint32_t ntiles = (a.N + 15) / 16;
    const uint32_t S = KS ? (a.flags >> 8) & 0xffu : 1u, slice = KS ? blockIdx.x % S : 0u;
    const auto tstep = [&]() { return KS ? gridDim.x / S : gridDim.x; };  // tiles between rounds
    // this wave's groups [g0, g0 + ng), ng <= NG (the host's choice of P and S)
    const uint32_t sg0 = slice * nsb / S, sgn = (slice + 1) * nsb / S - sg0;
    const uint32_t g0 = KS ? sg0 + wave * sgn / P : wave * nsb / P;
    const uint32_t ng = KS ? sg0 + (wave + 1) * sgn / P - g0 : (wave + 1) * nsb / P - g0;
    const uint32_t arow = li < (int)MR ? li : li & (MR - 1);
    const uint32_t xrow = arow < a.M ? arow : a.M - 1;
    const _Float16 *xp = (const _Float16 *)a.x + (uint64_t)xrow * a.ldx;
    vkf_h8 xr[NG][8];
#pragma unroll
    for (int u = 0; u < NG; u++)
#pragma unroll
        for (int t = 0; t < 8; t++) {
            const uint32_t g = g0 + (u < (int)ng ? u : 0);
            const vkf_u4 v = *(const vkf_u4 *)(xp + 256 * g + gm_k0<F>(t, lg));
            xr[u][t] = __builtin_bit_cast(vkf_h8, gm_reorder(v));
        }
    // Q4_K / Q5_K: lane (i, g) holds half of each of the sub-blocks
    // J = {2h, 2h+1, 4+2h, 5+2h}, h = g >> 1 (steps t = 4(j>>2) + 2(j&1)
    // and t + 1); the other half is in lane (i, g ^ 1).  Even k-slices
    // carry xs/32 of J as 4 fp16 hi parts, then 4 lo parts (order
    // (j & 1) + 2(j >> 2)); odd ones zero.
    vkf_h8 xmr[gm_kmin<F>() ? NG : 1];
    if constexpr (gm_kmin<F>()) {
        const vkf_h2 ones = {(_Float16)1.0f, (_Float16)1.0f};
#pragma unroll
        for (int u = 0; u < NG; u++) {
            vkf_h8 m = {};
#pragma unroll
            for (int pos = 0; pos < 4; pos++) {
                const int t0 = 4 * (pos >> 1) + 2 * (pos & 1);
                float f = 0.0f;
#pragma unroll
                for (int q = 0; q < 2; q++) {
                    const vkf_u4 v = __builtin_bit_cast(vkf_u4, xr[u][t0 + q]);
#pragma unroll
                    for (int d = 0; d < 4; d++) {
                        const uint32_t w = v[d];
                        f = __builtin_amdgcn_fdot2(__builtin_bit_cast(vkf_h2, w), ones, f, false);
                    }
                }
                f += __shfl_xor(f, 16, 64);
                const float fs = f * 0.03125f;
                const _Float16 hi = (_Float16)fs, lo = (_Float16)(fs - (float)hi);
                m[pos] = hi;
                m[4 + pos] = lo;
            }
            xmr[u] = (lg & 1) == 0 ? m : vkf_h8{};
        }
    }
    const uint32_t sel = (lg >> 1) ? 0x04030402u : 0x04010400u;  // bytes 2h, 2h+1 as (1024 + v) fp16
    GmSb<F> ta[NG];
    auto load_round = [&](uint32_t tile, GmSb<F> *t) {
        const uint32_t n = tile * 16 + li;
        const uint8_t *row = a.w + (uint64_t)(n < a.N ? n : a.N - 1) * a.row_bytes;
#pragma unroll
        for (int u = 0; u < NG; u++) gm_load<F>(row, g0 + (u < (int)ng ? u : 0), lg, t[u]);
    };
    uint32_t c64 = 0x64006400u;
    asm volatile("" : "+v"(c64));
    float *red = (float *)smem;  // [P waves][4 elements][64 lanes]
    const vkf_f4 zero = {0, 0, 0, 0};
    auto round = [&](uint32_t tile, GmSb<F> *cur) {
        vkf_f4 y4 = zero;
#pragma unroll
        for (int u = 0; u < NG; u++) {
            if (u < (int)ng) {
                const auto X = [&](int t) { return xr[u][t]; };
                const auto XM = [&]() {
                    if constexpr (gm_kmin<F>()) return xmr[u];
                    else return vkf_h8{};
                };
                gm_group<F>(cur[u], X, XM, lg, sel, c64, y4);
            }
        }
        // the next round's weights load under the reduction
        if (tile + tstep() < ntiles && ng > 0) load_round(tile + tstep(), cur);
#pragma unroll
        for (int e = 0; e < 4; e++) red[(wave * 4 + e) * 64 + lane] = y4[e];
        __syncthreads();
        if (wave < 4) {  // wave e adds element e of the P partial tiles, in wave order
            const int e = wave;
            float s = red[e * 64 + lane];
            for (int w = 1; w < P; w++) s += red[(w * 4 + e) * 64 + lane];
            const uint32_t n = tile * 16 + li, m = 4 * lg + e;
            if (m < a.M && n < a.N) {
                if constexpr (KS) {
                    a.y[((uint64_t)slice * a.M + m) * a.ldy + n] = s;
                } else {
                    float *yp = a.y + (uint64_t)m * a.ldy + n;
                    *yp = (a.flags & 1u) ? *yp + s : s;
                }
            }
        }
        __syncthreads();
    };
    uint32_t tile = KS ? blockIdx.x / S : blockIdx.x;
    if (tile < ntiles && ng > 0) load_round(tile, ta);
    for (; tile < ntiles; tile += tstep()) round(tile, ta);  // workgroup-uniform
}

template <int F, int NG, int P, bool KS>
__device__ __forceinline__ void gemv_mfma_xr_entry(const VkfGemvArgs &a) {
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    if (a.M <= 4) gemv_mfma_xr<F, 4, NG, P, KS>(a, smem);
    else if (a.M <= 8) gemv_mfma_xr<F, 8, NG, P, KS>(a, smem);
    else gemv_mfma_xr<F, 16, NG, P, KS>(a, smem);
}
// vkf_gemv_mfma_xr_<q>_f16_p<P>: P waves, up to NG = ceil(G / P) groups each;
// vkf_gemv_mfma_xr_<q>_f16_p<P>_ks: the same on K slices of up to NG*P groups
#define VKF_GEMV_MFMA_XR(name, F, NG, P)                                                                   \
    VKF_KERNEL void __launch_bounds__(64 * P) vkf_gemv_mfma_xr_##name##_f16_p##P(VkfGemvArgs a) {        \
        gemv_mfma_xr_entry<F, NG, P, false>(a);                                                          \
    }                                                                                                    \
    VKF_KERNEL void __launch_bounds__(64 * P) vkf_gemv_mfma_xr_##name##_f16_p##P##_ks(VkfGemvArgs a) {   \
        gemv_mfma_xr_entry<F, NG, P, true>(a);                                                           \
    }
VKF_GEMV_MFMA_XR(q4_0, GF_Q4_0, 1, 16)
VKF_GEMV_MFMA_XR(q4_1, GF_Q4_1, 1, 16)
VKF_GEMV_MFMA_XR(q4_k, GF_Q4_K, 2, 10)
VKF_GEMV_MFMA_XR(q8_0, GF_Q8_0, 2, 12)

// y[m, n] = sum over s = 0, 1, ..., S-1 (in that order) of
// part[(s*M + m)*N + n]: the K slices of vkf_gemv_mfma_xr_*_ks, S <= 8.  One
// thread per output, grid (ceil(N / 256), M); the S loads are issued
// together, then added in slice order.
VKF_KERNEL void __launch_bounds__(256) vkf_gemv_split_sum(VkfSplitSumArgs a) {
    const uint32_t n = blockIdx.x * 256 + threadIdx.x, m = blockIdx.y;
    if (n >= a.N || m >= a.M) return;
    const uint64_t plane = (uint64_t)a.M * a.N;
    const float *p = a.part + (uint64_t)m * a.N + n;
    float v[8];
#pragma unroll
    for (uint32_t k = 0; k < 8; k++) v[k] = k < a.S ? p[k * plane] : 0.0f;
    float s = v[0];
#pragma unroll
    for (uint32_t k = 1; k < 8; k++)
        if (k < a.S) s += v[k];
    a.y[(uint64_t)m * a.ldy + n] = s;
}
