// gemv_q6k.hip — decode GEMV of Q6_K weights x Q8_1 activations (a
// vocabulary projection at decode), M = 1, integer dot products.
//
// y[m, n] = sum over 32-element blocks kb of dw(n, sb) * dx(m, kb) * Q,
//   Q = sum_l sc * (u_l - 32) * q_l          (exact int32)
// with u the 6-bit code (low nibble from ql, two high bits from qh), sc the
// int8 sub-block scale (one per 16 elements) and q the Q8_1 activation
// (kernels/dequant_q6_k.glsl:34-58 for the element order; the arithmetic is
// ggml's vec_dot_q6_K_q8_1).  u*q runs in v_dot4_i32_i8; the -32 offset
// is applied to the integer activation sums X = sum q of each 16-element half.
//
// Layout.  A chunk is one 128-element half of a super-block (ip = c & 1 of
// super-block c >> 1): ql[64ip .. +63], qh[32ip .. +31], sc[8ip .. +7] and d,
// 106 bytes for 128 weights.  Super-blocks are 210 bytes, so a chunk's
// fields sit at a 2-byte (odd super-block) or 4-byte (even) offset from the
// 4-byte aligned row start; each field is loaded as the aligned dwords that
// cover it and realigned with v_alignbyte.
//
// Work split as in gemv_dot.hip: one 1024-thread workgroup per CU stages the
// activations in LDS, segments of S lanes own rows, lane p takes chunks p,
// p+S, ..., and the segment reduces with lane shuffles.
//
// Loads.  Per iteration a wave needs, for each of its 64/S rows, the S/2
// consecutive super-blocks its lanes decode: 105*S contiguous bytes per
// row.  The wave fetches them with direct-to-LDS 16-byte loads over
// consecutive addresses into one of its two LDS buffers (each 128-byte line
// requested once: a CU keeps only about 64 line requests in flight, and
// loading each lane's chunk fields straight from memory requested ~1.45
// lines per line of weights), then every lane reads its chunk's fields from
// there while the next iteration's loads fill the other buffer.  Two
// buffers per wave fit LDS for 8 waves per CU (512-thread workgroups).
#include "vkf_device.h"

#define Q6_WAVES 8
// bytes per LDS plane: 16 per chunk; MM = 1 up to 256 chunks (K <= 32768),
// MM = 4 up to 128 (K <= 16384)
template <int MM> constexpr uint32_t q6_plane_bytes() { return MM == 1 ? 4096 : 2048; }

typedef unsigned int vkf_u4a4 __attribute__((ext_vector_type(4), aligned(4)));

// LDS image of MM activation rows, per chunk c (4 Q8_1 blocks t = 0..3):
//   planes m*11 + j, j = 0..7: bytes 16j .. 16j+15 of the chunk's 128 q;
//   plane m*11 + 8: {dx(t)} as 4 floats; planes 9, 10: {X0(t)}, {X1(t)}
//   (sums of q over elements 0..15 and 16..31 of block t).
template <int MM>
__device__ __forceinline__ unsigned char *q6_plane(unsigned char *lds, uint32_t m, uint32_t j, uint32_t c) {
    return lds + (m * 11 + j) * q6_plane_bytes<MM>() + c * 16;
}

// One thread per Q8_1 block: row m, block kb (36 bytes: fp16 d, fp16 s,
// int8 q[32]; the s field is not used).
template <int MM>
__device__ __forceinline__ void q6_stage_block(const VkfGemvArgs &a, unsigned char *lds, uint32_t m, uint32_t kb) {
    const uint32_t *b = (const uint32_t *)((const uint8_t *)a.x + (uint64_t)m * a.ldx + 36ull * kb);
    uint32_t q[8];
#pragma unroll
    for (int i = 0; i < 8; i++) q[i] = b[1 + i];
    const float dx = vkf_h2f(b[0] & 0xffffu);
    int x0 = 0, x1 = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        x0 = __builtin_amdgcn_sdot4((int)q[i], 0x01010101, x0, false);
        x1 = __builtin_amdgcn_sdot4((int)q[4 + i], 0x01010101, x1, false);
    }
    const uint32_t c = kb >> 2, t = kb & 3;
    *(vkf_u4 *)q6_plane<MM>(lds, m, 2 * t, c) = vkf_u4{q[0], q[1], q[2], q[3]};
    *(vkf_u4 *)q6_plane<MM>(lds, m, 2 * t + 1, c) = vkf_u4{q[4], q[5], q[6], q[7]};
    ((float *)q6_plane<MM>(lds, m, 8, c))[t] = dx;
    ((int *)q6_plane<MM>(lds, m, 9, c))[t] = x0;
    ((int *)q6_plane<MM>(lds, m, 10, c))[t] = x1;
}

// fp16 / fp32 activations at M = 1 (XK 0 / 1): block kb of x (32 values)
// as two int8 rows with fp32 scales, x ~ dh*qh + dl*ql: rows 0 and 1 of the
// LDS image.  qh = round(x/dh) with dh = max|x|/127, ql the same of the
// residual x - dh*qh (|x - dh*qh - dl*ql| <= dl/2 <= max|x|/(4*127*127)),
// so the integer dot products of the two rows, summed, carry x to ~16 bits.
template <int XK>
__device__ __forceinline__ void q6_stage_split(const VkfGemvArgs &a, unsigned char *lds, uint32_t kb) {
    float x[32];
    if (XK == 1) {
        const vkf_f4 *p = (const vkf_f4 *)((const float *)a.x + 32ull * kb);
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const vkf_f4 v = p[i];
            x[4 * i] = v[0]; x[4 * i + 1] = v[1]; x[4 * i + 2] = v[2]; x[4 * i + 3] = v[3];
        }
    } else {
        const vkf_h8 *p = (const vkf_h8 *)((const _Float16 *)a.x + 32ull * kb);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const vkf_h8 v = p[i];
#pragma unroll
            for (int j = 0; j < 8; j++) x[8 * i + j] = (float)v[j];
        }
    }
    const uint32_t c = kb >> 2, t = kb & 3;
#pragma unroll
    for (int m = 0; m < 2; m++) {
        float amax = 0.0f;
#pragma unroll
        for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(x[i]));
        const float d = amax / 127.0f, id = d != 0.0f ? 1.0f / d : 0.0f;
        uint32_t q[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        int x0 = 0, x1 = 0;
#pragma unroll
        for (int i = 0; i < 32; i++) {
            const int v = (int)rintf(x[i] * id);  // |v| <= 127
            x[i] = fmaf(-d, (float)v, x[i]);       // residual for the next row
            q[i >> 2] |= ((uint32_t)v & 0xffu) << (8 * (i & 3));
            if (i < 16) x0 += v; else x1 += v;
        }
        *(vkf_u4 *)q6_plane<2>(lds, m, 2 * t, c) = vkf_u4{q[0], q[1], q[2], q[3]};
        *(vkf_u4 *)q6_plane<2>(lds, m, 2 * t + 1, c) = vkf_u4{q[4], q[5], q[6], q[7]};
        ((float *)q6_plane<2>(lds, m, 8, c))[t] = d;
        ((int *)q6_plane<2>(lds, m, 9, c))[t] = x0;
        ((int *)q6_plane<2>(lds, m, 10, c))[t] = x1;
    }
}

// Raw dwords of one chunk: ql 17, qh 9, sc 3 (one extra dword each for the
// realignment), and the fp16 d.  Every load stays inside the chunk's
// super-block: the dwords beyond byte 209 that an even super-block would
// need for sc are never needed (no realignment there) and d is a 2-byte load.
struct Q6Raw {
    uint32_t ql[17], qh[9], sc[3], d;
};

// fields of chunk (local super-block lsb, half ip) from a row region that
// starts 4-byte aligned
__device__ __forceinline__ void q6_load(const uint8_t *region, uint32_t lsb, uint32_t ip, Q6Raw &r) {
    const uint32_t base = 210u * lsb - 2u * (lsb & 1);  // 4-byte aligned
    const uint8_t *p = region + base;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const vkf_u4 v = *(const vkf_u4a4 *)(p + 64 * ip + 16 * k);
        r.ql[4 * k] = v[0]; r.ql[4 * k + 1] = v[1]; r.ql[4 * k + 2] = v[2]; r.ql[4 * k + 3] = v[3];
    }
    r.ql[16] = *(const uint32_t *)(p + 64 * ip + 64);
#pragma unroll
    for (int k = 0; k < 2; k++) {
        const vkf_u4 v = *(const vkf_u4a4 *)(p + 128 + 32 * ip + 16 * k);
        r.qh[4 * k] = v[0]; r.qh[4 * k + 1] = v[1]; r.qh[4 * k + 2] = v[2]; r.qh[4 * k + 3] = v[3];
    }
    r.qh[8] = *(const uint32_t *)(p + 128 + 32 * ip + 32);
    r.sc[0] = *(const uint32_t *)(p + 192 + 8 * ip);
    r.sc[1] = *(const uint32_t *)(p + 196 + 8 * ip);
    r.sc[2] = *(const uint32_t *)(p + ((lsb & 1) ? 200 + 8 * ip : 196 + 8 * ip));
    r.d = *(const uint16_t *)(region + 210u * lsb + 208);
}

// sum over the chunk for activation row m: d_w * sum_t dx(t) * Q_t
template <int MM>
__device__ __forceinline__ float q6_chunk(const Q6Raw &r, uint32_t sh, const unsigned char *lds, uint32_t m,
                                          uint32_t c) {
    // realigned fields (sh = 0 or 2 bytes); ql words are realigned where they
    // are used (each serves two blocks), qh once
    uint32_t qh[8];
#pragma unroll
    for (int i = 0; i < 8; i++) qh[i] = __builtin_amdgcn_alignbyte(r.qh[i + 1], r.qh[i], sh);
    const uint32_t s0 = __builtin_amdgcn_alignbyte(r.sc[1], r.sc[0], sh);
    const uint32_t s1 = __builtin_amdgcn_alignbyte(r.sc[2], r.sc[1], sh);
    const float dw = vkf_h2f(r.d);
    const vkf_f4 dx = *(const vkf_f4 *)q6_plane<MM>((unsigned char *)lds, m, 8, c);
    const vkf_i4 X0 = *(const vkf_i4 *)q6_plane<MM>((unsigned char *)lds, m, 9, c);
    const vkf_i4 X1 = *(const vkf_i4 *)q6_plane<MM>((unsigned char *)lds, m, 10, c);
    float acc = 0.0f;
#pragma unroll
    for (int t = 0; t < 4; t++) {
        const vkf_u4 xa = *(const vkf_u4 *)q6_plane<MM>((unsigned char *)lds, m, 2 * t, c);
        const vkf_u4 xb = *(const vkf_u4 *)q6_plane<MM>((unsigned char *)lds, m, 2 * t + 1, c);
        int p0 = 0, p1 = 0;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            // element 4i..4i+3 of block t: low nibble (t < 2) or high nibble
            // of ql[32(t&1) + 4i ..], bits 2t, 2t+1 of qh[4i ..]
            const int w = 8 * (t & 1) + i;
            const uint32_t l = __builtin_amdgcn_alignbyte(r.ql[w + 1], r.ql[w], sh);
            const uint32_t lo = (t >> 1) ? ((l >> 4) & 0x0f0f0f0fu) : (l & 0x0f0f0f0fu);
            const uint32_t hs = t == 0 ? (qh[i] << 4) : t == 1 ? (qh[i] << 2) : t == 2 ? qh[i] : (qh[i] >> 2);
            const uint32_t u = (hs & 0x30303030u) | lo;
            if (i < 4) p0 = __builtin_amdgcn_sdot4((int)u, (int)xa[i], p0, false);
            else p1 = __builtin_amdgcn_sdot4((int)u, (int)xb[i - 4], p1, false);
        }
        // int8 scales of the two 16-element halves: bytes 2t, 2t+1
        const uint32_t sw = t < 2 ? s0 : s1;
        const int sc0 = (int)(int8_t)(sw >> (16 * (t & 1))), sc1 = (int)(int8_t)(sw >> (16 * (t & 1) + 8));
        const int Q = sc0 * (p0 - 32 * X0[t]) + sc1 * (p1 - 32 * X1[t]);
        acc = fmaf(dx[t], (float)Q, acc);
    }
    return dw * acc;
}

// Per-wave LDS buffers: two of 64/S rows x PR 16-byte pieces each, PR =
// ceil(105*S/16) (at most 424 pieces, S = 8), room for all 7 x 64 slots.
#define Q6_NLD 7  // direct loads per lane per iteration (7 x 64 >= 424)
#define Q6_WBUF (Q6_NLD * 64 * 16)

// flags bit 0: y += instead of y =; bits 8..15: S (lanes per row segment,
// a power of two 8..64).  Dynamic LDS: MM * 11 * q6_plane_bytes<MM>() +
// Q6_WAVES * 2 * Q6_WBUF.  row_bytes % 4 == 0 and K >= 256 (host).
template <int MM, uint32_t S, int XS = -1>
__device__ __forceinline__ void gemv_q6k_q81(const VkfGemvArgs &a, unsigned char *smem) {
    const uint32_t C = a.K / 128, M = XS >= 0 ? 2 : a.M, nkb = a.K / 32;
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t seg = lane / S, p = lane & (S - 1);
    constexpr uint32_t TR = 64 / S;  // rows per wave tile
    constexpr uint32_t PR = (105 * S + 15) / 16, NP = TR * PR;
    const uint32_t ntiles = (a.N + TR - 1) / TR;
    const uint32_t iters = (C + S - 1) / S;
    const uint32_t tstep = gridDim.x * Q6_WAVES;
    unsigned char *wb = smem + MM * 11 * q6_plane_bytes<MM>() + wave * 2 * Q6_WBUF;
    const uint32_t last = (uint32_t)a.row_bytes - 16;  // last 16-byte piece of a row (row_bytes % 4 == 0)

    if constexpr (XS >= 0) {
        for (uint32_t i = threadIdx.x; i < nkb; i += blockDim.x) q6_stage_split<XS>(a, smem, i);
    } else {
        for (uint32_t i = threadIdx.x; i < M * nkb; i += blockDim.x) {
            const uint32_t m = i / nkb;
            q6_stage_block<MM>(a, smem, m, i - m * nkb);
        }
    }
    __syncthreads();

    for (uint32_t tile = wave * gridDim.x + blockIdx.x; tile < ntiles; tile += tstep) {
        // piece P = 64j + lane of an iteration: row P / PR of the tile, bytes
        // 16 * (P % PR) of that row's region, to LDS byte 16P of the buffer
        // (slots past NP fetch a valid piece into the unused buffer tail)
        // The last iteration's region may end inside a 16-byte piece (rows are
        // 210*K/256 bytes, a multiple of 4): that piece is fetched from the
        // row's last 16 bytes (shifted), and its rem = 4, 8 or 12 valid bytes
        // are loaded again into registers (3 dword loads, unused ones from a
        // valid dummy address), to be written over it once the direct loads
        // have landed.
        const uint32_t rl = 105u * S * (iters - 1), tl = (uint32_t)a.row_bytes - rl, rem = tl % 16;
        const bool straddle = rem != 0 && tl < 16 * PR;  // uniform
        uint32_t fixp = 0xffffffffu, fixv[3] = {0, 0, 0};
        auto issue = [&](uint32_t it) {
            const uint32_t r0 = 105u * S * it;  // region start within the row
            unsigned char *buf = wb + (it & 1) * Q6_WBUF;
            // this wave's reads of the buffer (two iterations ago) are done
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
            for (int j = 0; j < Q6_NLD; j++) {
                const uint32_t P = 64 * j + lane, pp = P < NP ? P : NP - 1, rr = pp / PR;
                const uint32_t nn = tile * TR + rr < a.N ? tile * TR + rr : a.N - 1;
                const uint32_t off = r0 + 16 * (pp - rr * PR);
                vkf_load_lds16_nt(a.w + (uint64_t)nn * a.row_bytes + (off < last ? off : last), buf + 64 * j * 16);
            }
            if (it == iters - 1 && straddle) {
                // piece tl/16 of each row: at most one per lane (PR is not a
                // multiple of 64 and a tile has fewer than 64 rows)
                const uint8_t *fa = a.w;  // a valid address for lanes without one
                fixp = 0xffffffffu;
#pragma unroll
                for (int j = 0; j < Q6_NLD; j++) {
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
        float acc[MM];
#pragma unroll
        for (int m = 0; m < MM; m++) acc[m] = 0.0f;
        issue(0);
        for (uint32_t it = 0; it < iters; it++) {
            if (it + 1 < iters) {  // wave-uniform
                issue(it + 1);
                if (it + 2 == iters && straddle) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(Q6_NLD + 3) : "memory");
                else asm volatile("s_waitcnt vmcnt(%0)" ::"n"(Q6_NLD) : "memory");
            } else {
                asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            }
            unsigned char *buf = wb + (it & 1) * Q6_WBUF;
            if (it == iters - 1 && straddle && fixp != 0xffffffffu) {
#pragma unroll
                for (int d = 0; d < 3; d++)
                    if (4 * d < rem) *(uint32_t *)(buf + 16 * fixp + 4 * d) = fixv[d];
            }
            const uint32_t c = p + it * S;
            if (c < C) {
                Q6Raw r;
                q6_load(buf + seg * PR * 16, p >> 1, p & 1, r);
                const uint32_t sh = 2u * ((p >> 1) & 1u);  // super-block c/2 = S*it/2 + p/2, S*it/2 even
#pragma unroll
                for (int m = 0; m < MM; m++)
                    if (MM == 1 || m < (int)M) acc[m] += q6_chunk<MM>(r, sh, smem, m, c);
            }
        }
        if constexpr (XS >= 0) acc[0] += acc[1];  // the two rows of x sum to x
#pragma unroll
        for (int m = 0; m < (XS >= 0 ? 1 : MM); m++) {
            float v = acc[m];
            for (uint32_t o = S >> 1; o > 0; o >>= 1) v += __shfl_xor(v, (int)o, 64);
            if (p == 0 && m < (int)M && tile * TR + seg < a.N) {
                float *yp = a.y + (uint64_t)m * a.ldy + tile * TR + seg;
                *yp = (a.flags & 1u) ? *yp + v : v;
            }
        }
    }
}

VKF_KERNEL void __launch_bounds__(64 * Q6_WAVES) vkf_gemv_q6k_q81_dot_m1(VkfGemvArgs a) {
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    switch ((a.flags >> 8) & 0xffu) {
    case 8: gemv_q6k_q81<1, 8>(a, smem); break;
    case 16: gemv_q6k_q81<1, 16>(a, smem); break;
    case 32: gemv_q6k_q81<1, 32>(a, smem); break;
    default: gemv_q6k_q81<1, 64>(a, smem); break;
    }
}

// Q6_K x fp16 / fp32 activations at M = 1: x split into two int8 rows in LDS
// (q6_stage_split), dynamic LDS 2 * 11 * q6_plane_bytes<2>() + Q6_WAVES * 2 *
// Q6_WBUF, K <= 16384.
template <int XK>
__device__ __forceinline__ void gemv_q6k_x_entry(const VkfGemvArgs &a) {
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    switch ((a.flags >> 8) & 0xffu) {
    case 8: gemv_q6k_q81<2, 8, XK>(a, smem); break;
    case 16: gemv_q6k_q81<2, 16, XK>(a, smem); break;
    case 32: gemv_q6k_q81<2, 32, XK>(a, smem); break;
    default: gemv_q6k_q81<2, 64, XK>(a, smem); break;
    }
}
VKF_KERNEL void __launch_bounds__(64 * Q6_WAVES) vkf_gemv_q6k_f16_dot_m1(VkfGemvArgs a) { gemv_q6k_x_entry<0>(a); }
VKF_KERNEL void __launch_bounds__(64 * Q6_WAVES) vkf_gemv_q6k_f32_dot_m1(VkfGemvArgs a) { gemv_q6k_x_entry<1>(a); }
