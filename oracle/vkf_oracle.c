/*
 * vkf_oracle.c — CPU restatement of vkflame's quantized-linear arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY (see vkf_oracle.h).  Built with
 * -O2 -ffp-contract=off -fno-fast-math so every fp32 expression rounds exactly
 * where the reference's GLSL writes it.
 *
 * Reference files restated (paths in the vkflame tree):
 *   kernels/dequant_q4_0.glsl:16-37   kernels/dequant_q4_1.glsl:16-37
 *   kernels/dequant_q5_0.glsl:18-47   kernels/dequant_q8_0.glsl:18-28
 *   kernels/dequant_q8_1.glsl:21-32   kernels/dequant_q4_k.glsl:16-58
 *   kernels/dequant_q5_k.glsl:16-75   kernels/dequant_q6_k.glsl:17-59
 *   kernels/linear_int8.glsl:54-100   kernels/linear_fp16.glsl:22-50
 * and ggml's quantize_row_q8_1_ref (third party, not vendored in the
 * reference; no version pinned there).
 */
#include "vkf_oracle.h"

#include <math.h>
#include <string.h>

/* ------------------------------------------------------------------ */
/* fp16                                                                */
/* ------------------------------------------------------------------ */

static uint32_t f_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float    bits_f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

float vkfo_h2f(uint16_t h)
{
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    if (e == 0) {
        /* zero or subnormal: m * 2^-24, exact in fp32 */
        float v = (float)m * 5.9604644775390625e-08f;
        return sign ? -v : v;
    }
    if (e == 31)
        return bits_f(sign | 0x7f800000u | (m << 13));
    return bits_f(sign | ((e - 15u + 127u) << 23) | (m << 13));
}

uint16_t vkfo_f2h(float f)
{
    uint32_t x = f_bits(f);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    x &= 0x7fffffffu;
    if (x >= 0x7f800000u) {                     /* inf / nan */
        if (x == 0x7f800000u) return sign | 0x7c00u;
        return sign | 0x7e00u | (uint16_t)((x >> 13) & 0x3ffu);
    }
    if (x >= 0x477ff000u)                       /* >= 65520 rounds to inf */
        return sign | 0x7c00u;
    int e = (int)(x >> 23) - 127;
    uint32_t mant = x & 0x7fffffu;
    if (e < -25)                                /* < 2^-25: rounds to zero */
        return sign;
    if (e < -14) {                              /* fp16 subnormal */
        uint32_t m24 = mant | 0x800000u;
        int s = -e - 1;                         /* 14 .. 24 */
        uint32_t r = m24 >> s;
        uint32_t rem = m24 & ((1u << s) - 1u);
        uint32_t half = 1u << (s - 1);
        if (rem > half || (rem == half && (r & 1u))) r++;
        return sign | (uint16_t)r;
    }
    uint32_t h = ((uint32_t)(e + 15) << 10) | (mant >> 13);
    uint32_t rem = mant & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return sign | (uint16_t)h;
}

/* ------------------------------------------------------------------ */
/* block geometry                                                      */
/* ------------------------------------------------------------------ */

int vkfo_block_bytes(int qtype)
{
    switch (qtype) {
    case VKFO_Q4_0: return 18;   /* kernels/dequant_q4_0.glsl:2 */
    case VKFO_Q4_1: return 20;   /* kernels/dequant_q4_1.glsl:2 */
    case VKFO_Q8_0: return 34;   /* kernels/dequant_q8_0.glsl:2 */
    case VKFO_Q5_0: return 22;   /* kernels/dequant_q5_0.glsl:2 */
    case VKFO_Q4_K: return 144;  /* kernels/dequant_q4_k.glsl:2 */
    case VKFO_Q5_K: return 176;  /* kernels/dequant_q5_k.glsl:2 */
    case VKFO_Q6_K: return 210;  /* kernels/dequant_q6_k.glsl:2 */
    case VKFO_Q8_1: return 36;   /* kernels/dequant_q8_1.glsl:2 */
    default: return -1;
    }
}

int vkfo_block_elems(int qtype)
{
    switch (qtype) {
    case VKFO_Q4_0: case VKFO_Q4_1: case VKFO_Q8_0:
    case VKFO_Q5_0: case VKFO_Q8_1: return 32;
    case VKFO_Q4_K: case VKFO_Q5_K: case VKFO_Q6_K: return 256;
    default: return -1;
    }
}

static uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static uint32_t rd32(const uint8_t *p)
{
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

/* ------------------------------------------------------------------ */
/* per-block dequantisers (fp32), one function per GLSL shader         */
/* ------------------------------------------------------------------ */

/* kernels/dequant_q4_0.glsl:24-36: y = d*q + (-8d), q = low nibble of
 * qs[i] for element i < 16 and high nibble of qs[i-16] for i >= 16. */
static void dq_q4_0(const uint8_t *b, float *y)
{
    float d = vkfo_h2f(rd16(b));
    float dm = -8.0f * d;
    const uint8_t *qs = b + 2;
    for (int l = 0; l < 16; l++) {
        uint32_t q = qs[l];
        y[l]      = d * (float)(q & 0xfu) + dm;
        y[l + 16] = d * (float)(q >> 4)   + dm;
    }
}

/* kernels/dequant_q4_1.glsl:24-35: y = d*q + m. */
static void dq_q4_1(const uint8_t *b, float *y)
{
    float d = vkfo_h2f(rd16(b));
    float m = vkfo_h2f(rd16(b + 2));
    const uint8_t *qs = b + 4;
    for (int l = 0; l < 16; l++) {
        uint32_t q = qs[l];
        y[l]      = d * (float)(q & 0xfu) + m;
        y[l + 16] = d * (float)(q >> 4)   + m;
    }
}

/* kernels/dequant_q5_0.glsl:26-45: x = nibble | (qh bit i) << 4 for
 * element i (bit i for i < 16, bit i for the high half too: the GLSL's
 * (qh >> (iqs+12)) & 0x10 is bit iqs+16); y = x*d + (-16d). */
static void dq_q5_0(const uint8_t *b, float *y)
{
    float d = vkfo_h2f(rd16(b));
    float dm = -16.0f * d;
    uint32_t qh = rd32(b + 2);
    const uint8_t *qs = b + 6;
    for (int l = 0; l < 16; l++) {
        uint32_t q = qs[l];
        uint32_t xh0 = ((qh >> (l + 0)) << 4) & 0x10u;
        uint32_t xh1 = ((qh >> (l + 12))) & 0x10u;
        float x0 = (float)((q & 0xfu) | xh0);
        float x1 = (float)((q >> 4) | xh1);
        y[l]      = x0 * d + dm;
        y[l + 16] = x1 * d + dm;
    }
}

/* kernels/dequant_q8_0.glsl:23-27: y = d*q. */
static void dq_q8_0(const uint8_t *b, float *y)
{
    float d = vkfo_h2f(rd16(b));
    for (int i = 0; i < 32; i++) y[i] = d * (float)(int8_t)b[2 + i];
}

/* kernels/dequant_q8_1.glsl:26-31: y = d*q, s (at +2) unused. */
static void dq_q8_1(const uint8_t *b, float *y)
{
    float d = vkfo_h2f(rd16(b));
    for (int i = 0; i < 32; i++) y[i] = d * (float)(int8_t)b[4 + i];
}

/* kernels/dequant_q4_k.glsl:16-24 (get_scale_min_k4). */
static void scale_min_k4(int j, const uint8_t *s, uint32_t *sc, uint32_t *mn)
{
    if (j < 4) {
        *sc = s[j] & 63u;
        *mn = s[j + 4] & 63u;
    } else {
        *sc = (s[j + 4] & 0xfu) | ((uint32_t)(s[j - 4] >> 6) << 4);
        *mn = (uint32_t)(s[j + 4] >> 4) | ((uint32_t)(s[j] >> 6) << 4);
    }
}

/* kernels/dequant_q4_k.glsl:35-57: chunk il (0..3) holds qs[32il .. 32il+31];
 * low nibble of qs[32il+l] -> element 64il+l with sub-block 2il, high
 * nibble -> element 64il+32+l with sub-block 2il+1; y = (dall*sc)*q - dmin*m. */
static void dq_q4_k(const uint8_t *b, float *y)
{
    float dall = vkfo_h2f(rd16(b));
    float dmin = vkfo_h2f(rd16(b + 2));
    const uint8_t *sc = b + 4;
    const uint8_t *qs = b + 16;
    for (int il = 0; il < 4; il++) {
        uint32_t s0, m0, s1, m1;
        scale_min_k4(2 * il, sc, &s0, &m0);
        scale_min_k4(2 * il + 1, sc, &s1, &m1);
        float d0 = dall * (float)s0, min0 = dmin * (float)m0;
        float d1 = dall * (float)s1, min1 = dmin * (float)m1;
        for (int l = 0; l < 32; l++) {
            uint32_t q = qs[32 * il + l];
            y[64 * il + l]      = d0 * (float)(q & 0xfu) - min0;
            y[64 * il + l + 32] = d1 * (float)(q >> 4)   - min1;
        }
    }
}

/* kernels/dequant_q5_k.glsl:37-73: as Q4_K, plus 16 when bit 2il (low) or
 * 2il+1 (high) of qh[l] is set; qh at +16, qs at +48. */
static void dq_q5_k(const uint8_t *b, float *y)
{
    float dall = vkfo_h2f(rd16(b));
    float dmin = vkfo_h2f(rd16(b + 2));
    const uint8_t *sc = b + 4;
    const uint8_t *qh = b + 16;
    const uint8_t *qs = b + 48;
    for (int il = 0; il < 4; il++) {
        uint32_t s0, m0, s1, m1;
        scale_min_k4(2 * il, sc, &s0, &m0);
        scale_min_k4(2 * il + 1, sc, &s1, &m1);
        float d0 = dall * (float)s0, min0 = dmin * (float)m0;
        float d1 = dall * (float)s1, min1 = dmin * (float)m1;
        uint32_t hm0 = 1u << (2 * il), hm1 = hm0 << 1;
        for (int l = 0; l < 32; l++) {
            uint32_t q = qs[32 * il + l];
            uint32_t h = qh[l];
            y[64 * il + l]      = d0 * (float)((q & 0xfu) + ((h & hm0) ? 16u : 0u)) - min0;
            y[64 * il + l + 32] = d1 * (float)((q >> 4)   + ((h & hm1) ? 16u : 0u)) - min1;
        }
    }
}

/* Q6_K element e of a 210-B block as (v - 32, scale index):
 * kernels/dequant_q6_k.glsl:19-58.  Half ip = e/128; within it quarter
 * t = (e%128)/32 and l = e%32; ql0 = ql[64ip+l], ql32 = ql[64ip+l+32],
 * h = qh[32ip+l]; scale index 8ip + l/16 + 2t. */
static void q6k_unpack(const uint8_t *b, int v[256], int sci[256])
{
    const uint8_t *ql = b, *qh = b + 128;
    for (int ip = 0; ip < 2; ip++)
        for (int l = 0; l < 32; l++) {
            uint32_t q0 = ql[64 * ip + l], q32 = ql[64 * ip + l + 32];
            uint32_t h = qh[32 * ip + l];
            int base = 128 * ip + l;
            v[base + 0]  = (int)((q0 & 0xfu)  | (((h >> 0) & 3u) << 4)) - 32;
            v[base + 32] = (int)((q32 & 0xfu) | (((h >> 2) & 3u) << 4)) - 32;
            v[base + 64] = (int)((q0 >> 4)    | (((h >> 4) & 3u) << 4)) - 32;
            v[base + 96] = (int)((q32 >> 4)   | (((h >> 6) & 3u) << 4)) - 32;
            int is = 8 * ip + l / 16;
            sci[base + 0] = is + 0; sci[base + 32] = is + 2;
            sci[base + 64] = is + 4; sci[base + 96] = is + 6;
        }
}

/* kernels/dequant_q6_k.glsl:55-58: y = d * float(sc * v). */
static void dq_q6_k(const uint8_t *b, float *y)
{
    int v[256], sci[256];
    q6k_unpack(b, v, sci);
    const int8_t *sc = (const int8_t *)(b + 192);
    float d = vkfo_h2f(rd16(b + 208));
    for (int e = 0; e < 256; e++) y[e] = d * (float)(sc[sci[e]] * v[e]);
}

int vkfo_dequant_f32(int qtype, const uint8_t *src, size_t n_blocks, float *dst)
{
    int bb = vkfo_block_bytes(qtype), be = vkfo_block_elems(qtype);
    if (bb < 0) return -1;
    for (size_t i = 0; i < n_blocks; i++) {
        const uint8_t *b = src + i * (size_t)bb;
        float *y = dst + i * (size_t)be;
        switch (qtype) {
        case VKFO_Q4_0: dq_q4_0(b, y); break;
        case VKFO_Q4_1: dq_q4_1(b, y); break;
        case VKFO_Q8_0: dq_q8_0(b, y); break;
        case VKFO_Q5_0: dq_q5_0(b, y); break;
        case VKFO_Q4_K: dq_q4_k(b, y); break;
        case VKFO_Q5_K: dq_q5_k(b, y); break;
        case VKFO_Q6_K: dq_q6_k(b, y); break;
        case VKFO_Q8_1: dq_q8_1(b, y); break;
        }
    }
    return 0;
}

int vkfo_dequant_f16(int qtype, const uint8_t *src, size_t n_blocks, uint16_t *dst)
{
    int be = vkfo_block_elems(qtype);
    if (be < 0) return -1;
    float tmp[256];
    int bb = vkfo_block_bytes(qtype);
    for (size_t i = 0; i < n_blocks; i++) {
        vkfo_dequant_f32(qtype, src + i * (size_t)bb, 1, tmp);
        for (int e = 0; e < be; e++) dst[i * (size_t)be + e] = vkfo_f2h(tmp[e]);
    }
    return 0;
}

/* ------------------------------------------------------------------ */
/* Symmetric per-row int8 quantiser, the rule of the reference's weight */
/* quantiser (tools/quantise.py:35-41): scale = max|row|/127 clamped to */
/* >= 1e-8, q = round-half-even(x/scale) clamped to +-127.              */
/* ------------------------------------------------------------------ */

void vkfo_quantize_rows_i8(const float *x, int M, int K, int8_t *q, float *scale)
{
    for (int m = 0; m < M; m++) {
        const float *xr = x + (size_t)m * K;
        float amax = 0.0f;
        for (int k = 0; k < K; k++) {
            float a = fabsf(xr[k]);
            amax = amax > a ? amax : a;
        }
        float s = amax / 127.0f;
        if (s < 1e-8f) s = 1e-8f;
        scale[m] = s;
        for (int k = 0; k < K; k++) {
            float v = rintf(xr[k] / s);
            if (v > 127.0f) v = 127.0f;
            if (v < -127.0f) v = -127.0f;
            q[(size_t)m * K + k] = (int8_t)v;
        }
    }
}

/* ------------------------------------------------------------------ */
/* Q8_1 quantizer (ggml quantize_row_q8_1_ref)                         */
/* ------------------------------------------------------------------ */

void vkfo_quantize_q8_1(const float *x, size_t n, uint8_t *dst)
{
    size_t nb = n / 32;
    for (size_t i = 0; i < nb; i++) {
        const float *xb = x + 32 * i;
        uint8_t *yb = dst + 36 * i;
        float amax = 0.0f;
        for (int j = 0; j < 32; j++) {
            float a = fabsf(xb[j]);
            amax = amax > a ? amax : a;
        }
        float d = amax / 127.0f;
        float id = d != 0.0f ? 1.0f / d : 0.0f;
        int sum = 0;
        for (int j = 0; j < 32; j++) {
            float v = xb[j] * id;
            int q = (int)roundf(v);
            yb[4 + j] = (uint8_t)(int8_t)q;
            sum += q;
        }
        uint16_t hd = vkfo_f2h(d);
        uint16_t hs = vkfo_f2h((float)sum * d);
        yb[0] = (uint8_t)hd; yb[1] = (uint8_t)(hd >> 8);
        yb[2] = (uint8_t)hs; yb[3] = (uint8_t)(hs >> 8);
    }
}

/* ------------------------------------------------------------------ */
/* integer products                                                    */
/* ------------------------------------------------------------------ */

int vkfo_gemm_i8_nt(const int8_t *A, const int8_t *B, int32_t *C,
                    int M, int N, int K)
{
    int ok = 0;
    for (int m = 0; m < M; m++)
        for (int n = 0; n < N; n++) {
            int64_t acc = 0;
            const int8_t *a = A + (size_t)m * K, *b = B + (size_t)n * K;
            for (int k = 0; k < K; k++) acc += (int64_t)a[k] * (int64_t)b[k];
            if (acc > INT32_MAX || acc < INT32_MIN) ok = -1;
            C[(size_t)m * N + n] = (int32_t)acc;
        }
    return ok;
}

void vkfo_q6k_q8_1_partials(const uint8_t *w, const uint8_t *xq, int32_t *P,
                            int M, int N, int K)
{
    int nsb = K / 256, nkb = K / 32;
    int v[256], sci[256];
    for (int n = 0; n < N; n++) {
        for (int sb = 0; sb < nsb; sb++) {
            const uint8_t *b = w + ((size_t)n * nsb + sb) * 210;
            const int8_t *sc = (const int8_t *)(b + 192);
            q6k_unpack(b, v, sci);
            for (int m = 0; m < M; m++) {
                for (int j = 0; j < 8; j++) {
                    int kb = sb * 8 + j;
                    const int8_t *qx = (const int8_t *)(xq + ((size_t)m * nkb + kb) * 36 + 4);
                    int32_t acc = 0;
                    for (int i = 0; i < 32; i++) {
                        int e = 32 * j + i;
                        acc += (int32_t)qx[i] * (int32_t)sc[sci[e]] * v[e];
                    }
                    P[((size_t)m * N + n) * nkb + kb] = acc;
                }
            }
        }
    }
}

/* ------------------------------------------------------------------ */
/* activation epilogue                                                 */
/* ------------------------------------------------------------------ */

/* kernels/linear_fp16.glsl:23-28: erf by Abramowitz & Stegun 7.1.26. */
static float erf_as(float x)
{
    float t = 1.0f / (1.0f + 0.3275911f * fabsf(x));
    float y = 1.0f - ((((1.061405429f * t - 1.453152027f) * t + 1.421413741f) * t
                       - 0.284496736f) * t + 0.254829592f) * t * expf(-x * x);
    return x >= 0.0f ? y : -y;
}

/* kernels/linear_fp16.glsl:31-36 */
float vkfo_act(int act, float x)
{
    switch (act) {
    case 1: return x * (1.0f / (1.0f + expf(-x)));
    case 2: return x > 0.0f ? x : 0.0f;
    case 3: return 0.5f * x * (1.0f + erf_as(x * 0.70710678118654f));
    default: return x;
    }
}
