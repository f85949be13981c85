// dequant.hip — ggml block dequantisers and the Q8_1 activation quantizer.
//
// Replaces kernels/dequant_{q4_0,q4_1,q5_0,q8_0,q8_1,q4_k,q5_k,q6_k}.glsl.
// The reference launches 32 or 64 lanes per block and fetches every byte with
// a 32-bit load plus shift (kernels/dequant_q4_0.glsl:13, 32-36).  Here one
// lane produces 8 consecutive outputs, so a wave writes 2 KiB (fp32) or 1 KiB
// (fp16) of contiguous output per pass; the kernel is bound by HBM writes.
//
// Output values are the reference's exact fp32 values (the per-format
// decoders in vkf_device.h follow the GLSL expressions); the fp16 variants
// round those values to nearest even, which ggml's fp16 dequant path expects.
#include "vkf_device.h"

template <int QT, bool F16>
__device__ __forceinline__ void dequant_body(const VkfDequantArgs &a) {
    constexpr int BB = QTraits<QT>::BB, GPB = QTraits<QT>::BE / 8;
    uint64_t g = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= a.n_blocks * GPB) return;
    uint64_t ib = g / GPB;
    int sub = (int)(g - ib * GPB);
    float y[8];
    decode8<QT>(a.src + ib * BB, sub, y);
    if (F16) {
        vkf_h8 h;
#pragma unroll
        for (int i = 0; i < 8; i++) h[i] = vkf_to_f16(y[i]);
        ((vkf_h8 *)a.dst)[g] = h;
    } else {
        vkf_f4 *o = (vkf_f4 *)a.dst + 2 * g;
        o[0] = vkf_f4{y[0], y[1], y[2], y[3]};
        o[1] = vkf_f4{y[4], y[5], y[6], y[7]};
    }
}

#define VKF_DEQUANT_KERNELS(name, QT)                                                        \
    VKF_KERNEL void __launch_bounds__(256) vkf_dequant_##name##_f32(VkfDequantArgs a) {      \
        dequant_body<QT, false>(a);                                                          \
    }                                                                                        \
    VKF_KERNEL void __launch_bounds__(256) vkf_dequant_##name##_f16(VkfDequantArgs a) {      \
        dequant_body<QT, true>(a);                                                           \
    }

VKF_DEQUANT_KERNELS(q4_0, VKF_Q4_0)
VKF_DEQUANT_KERNELS(q4_1, VKF_Q4_1)
VKF_DEQUANT_KERNELS(q8_0, VKF_Q8_0)
VKF_DEQUANT_KERNELS(q5_0, VKF_Q5_0)
VKF_DEQUANT_KERNELS(q4_k, VKF_Q4_K)
VKF_DEQUANT_KERNELS(q5_k, VKF_Q5_K)
VKF_DEQUANT_KERNELS(q6_k, VKF_Q6_K)
VKF_DEQUANT_KERNELS(q8_1, VKF_Q8_1)

// ---------------------------------------------------------------------------
// fp32 -> Q8_1.  The reference has no quantizer (it only decodes Q8_1,
// kernels/dequant_q8_1.glsl); this follows ggml's quantize_row_q8_1_ref:
//   amax = max|x|, d = amax/127, id = d ? 1/d : 0, q = roundf(x*id),
//   block = {fp16(d), fp16(sum(q)*d), q[32]}.
// 32 lanes per block; max and the integer sum are order-independent, so the
// butterfly reduction gives the sequential reference's bits exactly.  The
// divisions are IEEE correctly rounded (hipcc's default for fp32 divide).
// ---------------------------------------------------------------------------
VKF_KERNEL void __launch_bounds__(256) vkf_quantize_q8_1(VkfQuantizeArgs a) {
    const uint32_t nbk = a.K / 32;
    uint64_t gid = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    uint64_t blk = gid >> 5;
    int lane = (int)(gid & 31);
    if (blk >= (uint64_t)a.M * nbk) return;  // whole 32-lane groups exit together
    uint64_t m = blk / nbk, kb = blk - m * nbk;
    float x = a.x[m * a.ldx + kb * 32 + lane];
    float amax = fabsf(x);
#pragma unroll
    for (int o = 16; o > 0; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 32));
    float d = amax / 127.0f;
    float id = d != 0.0f ? 1.0f / d : 0.0f;
    int q = (int)roundf(x * id);
    int sum = q;
#pragma unroll
    for (int o = 16; o > 0; o >>= 1) sum += __shfl_xor(sum, o, 32);
    uint8_t *blkp = a.dst + blk * 36;
    blkp[4 + lane] = (uint8_t)(int8_t)q;
    if (lane == 0) {
        uint32_t hd = vkf_f2h(d), hs = vkf_f2h((float)sum * d);
        *(uint32_t *)blkp = hd | (hs << 16);
    }
}

// ---------------------------------------------------------------------------
// Symmetric per-row int8 quantisation, the input step of the int8 linear:
// the rule of the reference's weight quantiser (tools/quantise.py:35-41,
// scale = max|row|/127 clamped to >= 1e-8, q = round(x/scale) clamped to
// +-127, round half to even as torch.round) applied per output channel of a
// weight or per token of an activation matrix.  One 256-thread workgroup per
// row: a max reduction, then one rounding division per element (IEEE
// correctly rounded, hipcc's default for fp32 divide), so the result is the
// same bits as the sequential rule.
// ---------------------------------------------------------------------------
VKF_KERNEL void __launch_bounds__(256) vkf_quantize_rows_i8(VkfQuantRowsArgs a) {
    __shared__ float red[4];
    const uint64_t m = blockIdx.x;
    const _Float16 *xh = (const _Float16 *)a.x + m * a.ldx;
    const float *xf = (const float *)a.x + m * a.ldx;
    auto ld = [&](uint32_t k) { return a.x_f16 ? (float)xh[k] : xf[k]; };
    float amax = 0.0f;
    for (uint32_t k = threadIdx.x; k < a.K; k += 256) amax = fmaxf(amax, fabsf(ld(k)));
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 64));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const float scale = fmaxf(amax / 127.0f, 1e-8f);
    int8_t *q = a.q + m * a.K;
    for (uint32_t k = threadIdx.x; k < a.K; k += 256) {
        const float v = rintf(ld(k) / scale);
        q[k] = (int8_t)(int)fminf(fmaxf(v, -127.0f), 127.0f);
    }
    if (threadIdx.x == 0) a.scale[m] = scale;
}
