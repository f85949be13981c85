// vkf_device.h — device-side helpers shared by the gfx950 kernels:
// fp16 conversion, little-endian field loads from byte-aligned ggml blocks,
// and per-format element decoders that reproduce the reference's fp32
// dequantisation bit for bit (kernels/dequant_*.glsl).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include "../include/vkf_kernargs.h"

#define VKF_KERNEL extern "C" __global__

typedef _Float16 vkf_h2 __attribute__((ext_vector_type(2)));
typedef _Float16 vkf_h8 __attribute__((ext_vector_type(8)));
typedef float vkf_f4 __attribute__((ext_vector_type(4)));
typedef float vkf_f16v __attribute__((ext_vector_type(16)));
typedef int vkf_i4 __attribute__((ext_vector_type(4)));
typedef int vkf_i2 __attribute__((ext_vector_type(2)));
typedef unsigned int vkf_u4 __attribute__((ext_vector_type(4)));
typedef unsigned int vkf_u2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float vkf_h2f(uint16_t h) {
    return (float)__builtin_bit_cast(_Float16, h);
}
// fp32 -> fp16 of a value that was itself rounded to fp32 first (round to
// nearest even, subnormals kept: v_cvt_f16_f32 in the default mode).  The
// empty asm pins the fp32 value in a VGPR: without it the compiler folds
// fptrunc(fmul a, b) into one v_fma_mixlo_f16, rounding the exact product to
// fp16 once, which differs from the reference's fp32-then-fp16 rounding.
__device__ __forceinline__ _Float16 vkf_to_f16(float f) {
    asm volatile("" : "+v"(f));
    return (_Float16)f;
}
__device__ __forceinline__ uint16_t vkf_f2h(float f) {
    return __builtin_bit_cast(uint16_t, vkf_to_f16(f));
}

// Block geometry (bytes, elements) per quant type.
template <int QT> struct QTraits;
template <> struct QTraits<VKF_Q4_0> { static constexpr int BB = 18,  BE = 32; };
template <> struct QTraits<VKF_Q4_1> { static constexpr int BB = 20,  BE = 32; };
template <> struct QTraits<VKF_Q8_0> { static constexpr int BB = 34,  BE = 32; };
template <> struct QTraits<VKF_Q5_0> { static constexpr int BB = 22,  BE = 32; };
template <> struct QTraits<VKF_Q4_K> { static constexpr int BB = 144, BE = 256; };
template <> struct QTraits<VKF_Q5_K> { static constexpr int BB = 176, BE = 256; };
template <> struct QTraits<VKF_Q6_K> { static constexpr int BB = 210, BE = 256; };
template <> struct QTraits<VKF_Q8_1> { static constexpr int BB = 36,  BE = 32; };

// ---- byte-aligned little-endian loads (blocks are only 2-byte aligned) ----
__device__ __forceinline__ uint32_t ld_u16(const uint8_t *p) {
    return *(const uint16_t *)p;
}
// 4 bytes at a 2-byte aligned address.
__device__ __forceinline__ uint32_t ld_u32_a2(const uint8_t *p) {
    const uint16_t *q = (const uint16_t *)p;
    return (uint32_t)q[0] | ((uint32_t)q[1] << 16);
}
__device__ __forceinline__ uint32_t ld_u32(const uint8_t *p) {
    return *(const uint32_t *)p;
}

// ---- Q4_K / Q5_K 6-bit scale unpack: kernels/dequant_q4_k.glsl:16-24 ----
__device__ __forceinline__ void scale_min_k4(int j, const uint8_t *s, uint32_t &sc, uint32_t &mn) {
    if (j < 4) {
        sc = s[j] & 63u;
        mn = s[j + 4] & 63u;
    } else {
        sc = (s[j + 4] & 0xfu) | ((uint32_t)(s[j - 4] >> 6) << 4);
        mn = (uint32_t)(s[j + 4] >> 4) | ((uint32_t)(s[j] >> 6) << 4);
    }
}

// ---------------------------------------------------------------------------
// decode8<QT>(block, g, y): elements 8g .. 8g+7 of one block as the exact fp32
// values the reference shaders write.  Element order per format:
//   Q4_0/Q4_1/Q5_0: element i < 16 is the low nibble of qs[i], i >= 16 the
//     high nibble of qs[i-16] (dequant_q4_0.glsl:30-35);
//   Q4_K/Q5_K: element 64il+l (l<32) is the low nibble of qs[32il+l] with
//     sub-block 2il, element 64il+32+l the high nibble with sub-block 2il+1
//     (dequant_q4_k.glsl:49-57);
//   Q6_K: dequant_q6_k.glsl:34-58.
// ---------------------------------------------------------------------------
template <int QT> __device__ __forceinline__ void decode8(const uint8_t *b, int g, float y[8]);

template <> __device__ __forceinline__ void decode8<VKF_Q8_0>(const uint8_t *b, int g, float y[8]) {
    float d = vkf_h2f(ld_u16(b));
    uint32_t w0 = ld_u32_a2(b + 2 + 8 * g), w1 = ld_u32_a2(b + 6 + 8 * g);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        y[i] = d * (float)(int8_t)(w0 >> (8 * i));
        y[4 + i] = d * (float)(int8_t)(w1 >> (8 * i));
    }
}

template <> __device__ __forceinline__ void decode8<VKF_Q8_1>(const uint8_t *b, int g, float y[8]) {
    float d = vkf_h2f(ld_u16(b));
    uint32_t w0 = ld_u32(b + 4 + 8 * g), w1 = ld_u32(b + 8 + 8 * g);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        y[i] = d * (float)(int8_t)(w0 >> (8 * i));
        y[4 + i] = d * (float)(int8_t)(w1 >> (8 * i));
    }
}

// 8 nibbles for elements 8g..8g+7 of a 32-element nibble block with qs at q.
__device__ __forceinline__ void nib8(const uint8_t *qs, int g, uint32_t q[8], bool aligned4) {
    int off = 8 * (g & 1);
    uint32_t w0 = aligned4 ? ld_u32(qs + off) : ld_u32_a2(qs + off);
    uint32_t w1 = aligned4 ? ld_u32(qs + off + 4) : ld_u32_a2(qs + off + 4);
    int sh = (g >> 1) * 4;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        q[i] = (w0 >> (8 * i + sh)) & 0xfu;
        q[4 + i] = (w1 >> (8 * i + sh)) & 0xfu;
    }
}

template <> __device__ __forceinline__ void decode8<VKF_Q4_0>(const uint8_t *b, int g, float y[8]) {
    float d = vkf_h2f(ld_u16(b));
    float dm = -8.0f * d;
    uint32_t q[8];
    nib8(b + 2, g, q, false);
#pragma unroll
    for (int i = 0; i < 8; i++) y[i] = d * (float)q[i] + dm;
}

template <> __device__ __forceinline__ void decode8<VKF_Q4_1>(const uint8_t *b, int g, float y[8]) {
    float d = vkf_h2f(ld_u16(b));
    float m = vkf_h2f(ld_u16(b + 2));
    uint32_t q[8];
    nib8(b + 4, g, q, true);
#pragma unroll
    for (int i = 0; i < 8; i++) y[i] = d * (float)q[i] + m;
}

template <> __device__ __forceinline__ void decode8<VKF_Q5_0>(const uint8_t *b, int g, float y[8]) {
    float d = vkf_h2f(ld_u16(b));
    float dm = -16.0f * d;
    uint32_t qh = ld_u32_a2(b + 2);
    uint32_t q[8];
    nib8(b + 6, g, q, false);
#pragma unroll
    for (int i = 0; i < 8; i++) {
        int e = 8 * g + i;  // element e uses bit e of qh (dequant_q5_0.glsl:40-41)
        float x = (float)(q[i] | (((qh >> e) & 1u) << 4));
        y[i] = x * d + dm;
    }
}

template <> __device__ __forceinline__ void decode8<VKF_Q4_K>(const uint8_t *b, int g, float y[8]) {
    float dall = vkf_h2f(ld_u16(b)), dmin = vkf_h2f(ld_u16(b + 2));
    int il = g >> 3, w = (g & 7) * 8;   // element 64il + w
    int hi = w >= 32;
    uint32_t sc, mn;
    scale_min_k4(2 * il + hi, b + 4, sc, mn);
    float dj = dall * (float)sc, mj = dmin * (float)mn;
    const uint8_t *qs = b + 16 + 32 * il + (w & 31);
    uint32_t w0 = ld_u32(qs), w1 = ld_u32(qs + 4);
    int sh = hi * 4;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        y[i] = dj * (float)((w0 >> (8 * i + sh)) & 0xfu) - mj;
        y[4 + i] = dj * (float)((w1 >> (8 * i + sh)) & 0xfu) - mj;
    }
}

template <> __device__ __forceinline__ void decode8<VKF_Q5_K>(const uint8_t *b, int g, float y[8]) {
    float dall = vkf_h2f(ld_u16(b)), dmin = vkf_h2f(ld_u16(b + 2));
    int il = g >> 3, w = (g & 7) * 8;
    int hi = w >= 32;
    uint32_t sc, mn;
    scale_min_k4(2 * il + hi, b + 4, sc, mn);
    float dj = dall * (float)sc, mj = dmin * (float)mn;
    int l = w & 31;
    const uint8_t *qs = b + 48 + 32 * il + l;
    const uint8_t *qh = b + 16 + l;
    uint32_t w0 = ld_u32(qs), w1 = ld_u32(qs + 4);
    uint32_t h0 = ld_u32(qh), h1 = ld_u32(qh + 4);
    int sh = hi * 4, hb = 2 * il + hi;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        uint32_t q0 = ((w0 >> (8 * i + sh)) & 0xfu) + (((h0 >> (8 * i + hb)) & 1u) << 4);
        uint32_t q1 = ((w1 >> (8 * i + sh)) & 0xfu) + (((h1 >> (8 * i + hb)) & 1u) << 4);
        y[i] = dj * (float)q0 - mj;
        y[4 + i] = dj * (float)q1 - mj;
    }
}

template <> __device__ __forceinline__ void decode8<VKF_Q6_K>(const uint8_t *b, int g, float y[8]) {
    int e = 8 * g;
    int ip = e >> 7, t = (e >> 5) & 3, l = e & 31;
    const uint8_t *ql = b + 64 * ip + 32 * (t & 1) + l;
    const uint8_t *qh = b + 128 + 32 * ip + l;
    int sc = (int)(int8_t)b[192 + 8 * ip + (l >> 4) + 2 * t];
    float d = vkf_h2f(ld_u16(b + 208));
    uint32_t w0 = ld_u32_a2(ql), w1 = ld_u32_a2(ql + 4);
    uint32_t h0 = ld_u32_a2(qh), h1 = ld_u32_a2(qh + 4);
    int sh = (t >> 1) * 4, hs = 2 * t;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        int v0 = (int)(((w0 >> (8 * i + sh)) & 0xfu) | (((h0 >> (8 * i + hs)) & 3u) << 4)) - 32;
        int v1 = (int)(((w1 >> (8 * i + sh)) & 0xfu) | (((h1 >> (8 * i + hs)) & 3u) << 4)) - 32;
        y[i] = d * (float)(sc * v0);
        y[4 + i] = d * (float)(sc * v1);
    }
}

// ---- direct-to-LDS load: each lane's 16 bytes at src go to LDS byte
// lds + 16 * lane (lds wave-uniform) ----
// Written out (M0 = LDS base, one wait state after the M0 write) so that the
// compiler does not track it: its own waits for direct-to-LDS loads are
// vmcnt(0) before every later LDS access and barrier, which would also wait
// for every later global load.  The caller waits with s_waitcnt vmcnt(N).
// M0 is named as clobbered; the kernels that use this hold nothing else in
// M0 (checked in their ISA: every M0 write is this one).
__device__ __forceinline__ void vkf_load_lds16(const void *src, const void *lds) {
    const uint32_t base = __builtin_amdgcn_readfirstlane(
        (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const unsigned char *)lds);
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(base)
                 : "memory", "m0");
}

// ---- streamed weights: loads with the non-temporal cache policy (nt) ----
// Contiguous runs read exactly once (the GEMV weight regions fetched into
// LDS) are loaded with nt set.  A plain read of 39.8 MB (640 MB) on MI355X
// takes 7.60 (102.3) us with default-policy loads and 7.02 (92.7) us with nt
// loads, the same gain with direct-to-LDS loads (7.89 -> 7.37 us); sc0 / sc1
// add nothing to nt.  Register loads of 16-byte pieces that neighbouring
// lanes' pieces share lines with measured slower with nt (Q8_0 4096x4096
// GEMV 6.7 -> 9.7 us): the policy drops a line before its other pieces are
// read.
__device__ __forceinline__ void vkf_load_lds16_nt(const void *src, const void *lds) {
    const uint32_t base = __builtin_amdgcn_readfirstlane(
        (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const unsigned char *)lds);
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off nt" ::"v"(src), "s"(base)
                 : "memory", "m0");
}
template <class T>
__device__ __forceinline__ T vkf_ld_nt(const void *p) {
    return __builtin_nontemporal_load((const T *)p);
}

// ---- wavefront reductions (64 lanes) ----
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// ---- activation epilogue: kernels/linear_fp16.glsl:22-36 ----
__device__ __forceinline__ float vkf_erf_as(float x) {
    float t = 1.0f / (1.0f + 0.3275911f * fabsf(x));
    float y = 1.0f - ((((1.061405429f * t - 1.453152027f) * t + 1.421413741f) * t
                       - 0.284496736f) * t + 0.254829592f) * t * __expf(-x * x);
    return x >= 0.0f ? y : -y;
}
__device__ __forceinline__ float vkf_act(uint32_t act, float x) {
    if (act == VKF_ACT_SILU) return x * (1.0f / (1.0f + __expf(-x)));
    if (act == VKF_ACT_RELU) return fmaxf(x, 0.0f);
    if (act == VKF_ACT_GELU_ERF) return 0.5f * x * (1.0f + vkf_erf_as(x * 0.70710678118654f));
    return x;
}
