// gemv_mfma.hip — small-batch GEMV (5 <= M <= 16) of Q4_K weights on the
// matrix cores: y[M, N] = x[M, K] . Wdeq[N, K]^T, fp16 activations.
//
// With 5..16 activation rows the VALU dot product costs M multiply-adds per
// weight; a 16x16x32 fp16 MFMA takes 16 weight rows x 32 k against up to 16
// activation rows at once, so the per-weight cost is the decode only.
//
// Arithmetic.  A Q4_K weight is dall*sc*q - dmin*mn (kernels/dequant_q4_k.glsl:
// 16-58; sc, mn 6-bit per 32-element sub-block, q a nibble).  Per super-block
// and output (m, n):
//   y += dall * sum_k x*(sc*q)  -  dmin * sum_j mn_j * xs_j
// with xs_j the sum of x over sub-block j.  sc*q <= 945 is an integer, exact
// in fp16, so the 8 MFMAs of a super-block see exact operands and accumulate
// in fp32; dall is applied once per super-block.  The min term is one more
// MFMA whose k runs over the 8 sub-blocks: A = xs/32 as two fp16 halves
// (hi + lo, ~22 bits) on k-slices 0 and 1, B = mn.
//
// Decode.  A code dword holds bytes b0..b3 (low nibble: sub-block 2il,
// high: 2il+1).  (v & 0x000f000f) | 0x64006400 is the fp16 pair
// (1024 + b0.lo, 1024 + b2.lo); the same with mask 0x00f000f0 gives
// (1024 + 16*b0.hi, 1024 + 16*b2.hi), and v >> 8 the b1, b3 pairs.  One
// packed fp16 FMA per pair, (1024 + q)*sc - 1024*sc or (1024 + 16q)*(sc/16)
// - 64*sc, yields sc*q exactly.
//
// Loads and k order.  Lane l = 16g + i (weight row i) loads, per
// super-block, the 16-byte header and qs bytes 16g .. +15 and 64 + 16g ..
// +15, so that each load instruction reads 64 contiguous bytes of each of
// the 16 rows.  Those are elements 16(g&1) .. +15 of sub-blocks
// j = 4L + 2(g>>1) + nib (L = which load, nib = low / high nibbles).  MFMA
// step t = 4L + 2nib + hf of the super-block takes, in k-slice g, elements
// 16(g&1) + 8hf + {0,2,1,3,4,6,5,7} of that sub-block (the decode's order),
// and the activations are staged to match.
//
// Work split.  One 1024-thread workgroup per CU stages the activation rows in
// LDS once, with the first weight loads already in flight.  Its 16 waves form
// 16/P groups; a group owns a 16-row tile of W per round and its P waves
// split the tile's super-blocks P ways (P = 4, 8 or 16 from the host, larger
// for fewer rows, so that enough loads are in flight).  A wave issues the
// loads of up to GM_MAXSB super-blocks, then runs 9 MFMAs per super-block;
// the P partial 16x16 results of a group meet in LDS.  The host splits a K
// too long for LDS into launches over K slices, the later ones accumulating
// into y.  Accumulator: lane l holds y-tile element (activation row 4g + e,
// weight row i).
#include "vkf_device.h"

#define GM_WAVES 16
#define GM_MAXSB 5   // super-blocks per wave held in registers at once

// LDS image, MR = M rounded up to 8 or 16 (rows M .. MR-1 repeat row M-1
// and feed only discarded outputs):
//   x:  for MFMA step s = 8sb + t, k-slice g, row i: 8 fp16 at
//       ((s*4 + g)*MR + i)*16, the elements 32j + 8r .. +7 of super-block sb
//       with j = 4(t>>2) + 2(g>>1) + ((t>>1)&1), r = 2(g&1) + (t&1), in the
//       decode's order 0,2,1,3,4,6,5,7;
//   xs: at K*MR*2, for super-block sb, h = 0, 1 and row i: 16 bytes at
//       ((sb*2 + h)*MR + i)*16 holding xs/32 of sub-blocks
//       J_h = {2h, 2h+1, 4+2h, 5+2h} as 4 fp16 hi parts, then 4 lo parts;
//   partials: 16 KiB after that.
// Staging: direct-to-LDS loads put each 16-byte piece of x in place (piece
// = lane of a 1 KiB load), then one pass per (row, sub-block) reorders the
// 4 pieces' halves and writes the sub-block sum.

// the x pieces of the workgroup's 1 KiB direct load c
template <uint32_t MR>
__device__ __forceinline__ void gm_dma_x(const VkfGemvArgs &a, unsigned char *lds, uint32_t c, int lane) {
    const uint32_t P = c * 64 + lane, i = P % MR, g = (P / MR) & 3, s = P / (4 * MR);
    const uint32_t sb = s >> 3, t = s & 7;
    const uint32_t j = 4 * (t >> 2) + 2 * (g >> 1) + ((t >> 1) & 1), r = 2 * (g & 1) + (t & 1);
    const _Float16 *src = (const _Float16 *)a.x + (uint64_t)(i < a.M ? i : a.M - 1) * a.ldx + sb * 256 + 32 * j + 8 * r;
    // Written out (M0 = LDS base, one wait state after the M0 write) so that
    // the compiler does not track it: its waits for direct-to-LDS loads are
    // vmcnt(0) before every later LDS access, weights included.  The caller
    // waits for it with s_waitcnt vmcnt.
    const uint32_t base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) unsigned char *)(lds + c * 1024);
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(base)
                 : "memory", "m0");
}

// the reorder and sub-block sums, after the direct loads have landed
template <uint32_t MR>
__device__ __forceinline__ void gm_stage_pass(const VkfGemvArgs &a, unsigned char *lds) {
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
                const uint32_t w = v[r][d];
                f = __builtin_amdgcn_fdot2(__builtin_bit_cast(vkf_h2, w), ones, f, false);
            }
            // halves 0,1,2,3 -> 0,2,1,3 (and 4..7 likewise)
            *pc[r] = vkf_u4{__builtin_amdgcn_perm(v[r][1], v[r][0], 0x05040100u),
                            __builtin_amdgcn_perm(v[r][1], v[r][0], 0x07060302u),
                            __builtin_amdgcn_perm(v[r][3], v[r][2], 0x05040100u),
                            __builtin_amdgcn_perm(v[r][3], v[r][2], 0x07060302u)};
        }
        const float fs = f * 0.03125f;
        const _Float16 hi = (_Float16)fs, lo = (_Float16)(fs - (float)hi);
        _Float16 *e = (_Float16 *)(xs + ((sb * 2 + ((j >> 1) & 1)) * MR + m) * 16);
        const uint32_t pos = (j & 1) + 2 * (j >> 2);
        e[pos] = hi;
        e[4 + pos] = lo;
    }
}

struct GmSb {          // one lane's share of a Q4_K super-block
    vkf_u4 hdr;        // dall, dmin, scales[12]
    vkf_u4 q[2];       // qs bytes 16g .. +15 and 64 + 16g .. +15
};

__device__ __forceinline__ void gm_load(const uint8_t *row, uint32_t sb, int g, GmSb &t) {
    const uint8_t *b = row + 144ull * sb;
    t.hdr = *(const vkf_u4 *)b;
    t.q[0] = *(const vkf_u4 *)(b + 16 + 16 * g);
    t.q[1] = *(const vkf_u4 *)(b + 80 + 16 * g);
}

// Loads of super-blocks s0 .. s0 + GM_MAXSB - 1, those at or past sb1
// clamped to sb1 - 1 (loaded and not used), so that the loads form one
// straight sequence.  sb1 >= 1.
__device__ __forceinline__ void gm_load_batch(const uint8_t *row, uint32_t s0, uint32_t sb1, int g, GmSb *t) {
#pragma unroll
    for (int u = 0; u < GM_MAXSB; u++) gm_load(row, s0 + u < sb1 ? s0 + u : sb1 - 1, g, t[u]);
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

// sc*q for 8 elements of a sub-block held in low nibbles (HI = 0) or high
// nibbles (HI = 1) of a lane's code dwords d0, d1 and their >> 8 shifts
// t0, t1; s, n = the sub-block's (sc, -1024*sc) or (sc/16, -64*sc);
// c64 = 0x64006400
template <int HI>
__device__ __forceinline__ vkf_h8 gm_decode(uint32_t d0, uint32_t t0, uint32_t d1, uint32_t t1, _Float16 s,
                                            _Float16 n, uint32_t c64) {
    const uint32_t mask = HI ? 0x00f000f0u : 0x000f000fu;
    const vkf_h2 s2 = {s, s}, n2 = {n, n};
    vkf_u4 r;
    r[0] = gm_u(__builtin_elementwise_fma(gm_h2(gm_and_or(d0, mask, c64)), s2, n2));
    r[1] = gm_u(__builtin_elementwise_fma(gm_h2(gm_and_or(t0, mask, c64)), s2, n2));
    r[2] = gm_u(__builtin_elementwise_fma(gm_h2(gm_and_or(d1, mask, c64)), s2, n2));
    r[3] = gm_u(__builtin_elementwise_fma(gm_h2(gm_and_or(t1, mask, c64)), s2, n2));
    return __builtin_bit_cast(vkf_h8, r);
}

template <uint32_t MR>
__device__ __forceinline__ void gemv_mfma_q4k(const VkfGemvArgs &a, unsigned char *smem) {
    const uint32_t nsb = a.K / 256;
    const uint32_t P = (a.flags >> 8) & 0xffu;  // waves per tile: 4, 8 or 16
    const uint32_t G = GM_WAVES / P;            // tiles per workgroup round
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: scalar loop bounds
    const int li = lane & 15, lg = lane >> 4;
    const uint32_t grp = wave / P, part = wave % P;
    const uint32_t ntiles = (a.N + 15) / 16;
    const uint32_t per = (nsb + P - 1) / P;  // super-blocks per wave
    const uint32_t sb0 = part * per, sb1 = sb0 + per < nsb ? sb0 + per : nsb;  // sb1 >= 1

    // x goes to LDS by direct loads, the first batch of weight loads right
    // behind it; vmcnt counts in order, so waiting for x leaves the weights
    // in flight.  blockIdx.x * G < ntiles: the host launches at most
    // ceil(ntiles / G) workgroups.
    GmSb t[GM_MAXSB];
    const uint32_t nc = MR * a.K * 2 / 1024;  // 1 KiB loads of x (MR * K * 2 is a multiple of 4096)
    for (uint32_t c = wave; c < nc; c += GM_WAVES) gm_dma_x<MR>(a, smem, c, lane);
    asm volatile("" ::: "memory");
    {
        const uint32_t n = (blockIdx.x * G + grp) * 16 + li;
        gm_load_batch(a.w + (uint64_t)(n < a.N ? n : a.N - 1) * a.row_bytes, sb0, sb1, lg, t);
    }
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(3 * GM_MAXSB) : "memory");
    __syncthreads();
    gm_stage_pass<MR>(a, smem);
    __syncthreads();
    bool pre = true;
    const unsigned char *xs = smem + (uint64_t)a.K * MR * 2;
    float *red = (float *)(xs + nsb * MR * 32);  // [16 waves][64 lanes][4]

    const uint32_t arow = li < (int)MR ? li : li & 7;  // rows >= M feed discarded outputs
    const unsigned char *xw = smem + (lg * MR + arow) * 16;  // this lane's x pieces
    const unsigned char *xsw = xs + ((lg >> 1) * MR + arow) * 16;
    const uint32_t sel = (lg >> 1) ? 0x04030402u : 0x04010400u;  // bytes 2h, 2h+1 as (1024 + v) fp16
    const vkf_f4 zero = {0, 0, 0, 0};
    const vkf_h2 one16 = {(_Float16)1.0f, (_Float16)0.0625f}, off = {(_Float16)-1024.0f, (_Float16)-64.0f};
    const vkf_h2 m1024 = {(_Float16)-1024.0f, (_Float16)-1024.0f};
    uint32_t c64 = 0x64006400u;
    asm volatile("" : "+v"(c64));  // held in a VGPR for gm_and_or

    for (uint32_t t0 = blockIdx.x * G; t0 < ntiles; t0 += gridDim.x * G) {  // workgroup-uniform loop
        const uint32_t tile = t0 + grp;
        const uint32_t n = tile * 16 + li;
        const uint8_t *row = a.w + (uint64_t)(n < a.N ? n : a.N - 1) * a.row_bytes;
        vkf_f4 y4 = zero;
        for (uint32_t s0 = sb0; s0 < sb1; s0 += GM_MAXSB) {
            if (!pre) gm_load_batch(row, s0, sb1, lg, t);
            pre = false;
#pragma unroll
            for (int u = 0; u < GM_MAXSB; u++) {
                const uint32_t sb = s0 + u;
                if (sb >= sb1) break;
                const float dall = vkf_h2f(t[u].hdr[0] & 0xffffu), dmin = vkf_h2f(t[u].hdr[0] >> 16);
                const uint32_t s0w = t[u].hdr[1], s4w = t[u].hdr[2], s8w = t[u].hdr[3];
                const uint32_t sc[2] = {s0w & 0x3f3f3f3fu, (s8w & 0x0f0f0f0fu) | ((s0w >> 2) & 0x30303030u)};
                const uint32_t mn[2] = {s4w & 0x3f3f3f3fu, ((s8w >> 4) & 0x0f0f0f0fu) | ((s4w >> 2) & 0x30303030u)};
                // load L covers sub-blocks 4L + 2h (low nibbles) and 4L + 2h + 1
                // (high): scale pairs (sc, sc'/16), (-1024 sc, -64 sc'), and
                // the mins (mn, mn') of those sub-blocks
                vkf_h2 S[2], Nn[2];
                uint32_t bm[2];
#pragma unroll
                for (int L = 0; L < 2; L++) {
                    S[L] = __builtin_elementwise_fma(gm_h2(__builtin_amdgcn_perm(0x64646464u, sc[L], sel)), one16, off);
                    Nn[L] = S[L] * m1024;
                    bm[L] = gm_u(gm_h2(__builtin_amdgcn_perm(0x64646464u, mn[L], sel)) + m1024);
                }
                vkf_f4 acc = zero;
#pragma unroll
                for (int L = 0; L < 2; L++)
#pragma unroll
                    for (int hf = 0; hf < 2; hf++) {
                        const uint32_t d0 = t[u].q[L][2 * hf], d1 = t[u].q[L][2 * hf + 1], e0 = d0 >> 8, e1 = d1 >> 8;
                        // MFMA steps 8sb + 4L + hf (low nibbles) and 8sb + 4L + 2 + hf (high)
                        const unsigned char *xp = xw + sb * (32 * MR * 16) + (4 * L + hf) * (4 * MR * 16);
                        const vkf_h8 xl = *(const vkf_h8 *)xp;
                        const vkf_h8 xh = *(const vkf_h8 *)(xp + 2 * (4 * MR * 16));
                        const vkf_h8 bl = gm_decode<0>(d0, e0, d1, e1, S[L][0], Nn[L][0], c64);
                        const vkf_h8 bh = gm_decode<1>(d0, e0, d1, e1, S[L][1], Nn[L][1], c64);
                        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(xl, bl, acc, 0, 0, 0);
                        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(xh, bh, acc, 0, 0, 0);
                    }
                // min term: even k-slices carry xs hi and lo of the lane pair's 4
                // sub-blocks, odd ones zero
                vkf_h8 xm = {};
                if ((lg & 1) == 0) xm = *(const vkf_h8 *)(xsw + sb * (2 * MR * 16));
                const vkf_u4 bmin = {bm[0], bm[1], bm[0], bm[1]};
                const vkf_f4 am = __builtin_amdgcn_mfma_f32_16x16x32_f16(xm, __builtin_bit_cast(vkf_h8, bmin), zero,
                                                                          0, 0, 0);
                const float dm32 = -32.0f * dmin;
#pragma unroll
                for (int e = 0; e < 4; e++) y4[e] = fmaf(dm32, am[e], fmaf(dall, acc[e], y4[e]));
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
                    float *yp = a.y + (uint64_t)m * a.ldy + n;
                    *yp = (a.flags & 1u) ? *yp + s[e] : s[e];
                }
            }
        }
        __syncthreads();
    }
}

VKF_KERNEL void __launch_bounds__(64 * GM_WAVES) vkf_gemv_mfma_q4_k_f16(VkfGemvArgs a) {
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    if (a.M <= 8) gemv_mfma_q4k<8>(a, smem);
    else gemv_mfma_q4k<16>(a, smem);
}
