// vkf_launch_table.cpp — kernel-name dispatch table.
//
// The reference's amdhip64 shim maps every hipLaunchKernel to a Vulkan
// dispatch by substring tests on the registered device-function name and
// decodes the kernel's arguments by ggml's calling convention
// (shim/hip_runtime_shim.cpp:833-1213).  This file keeps that table as a pure
// function (vkflame_resolve_launch, unit-testable on the CPU with synthetic
// names and argument arrays) plus an executor (vkflame_execute_launch) that
// runs the plan on the gfx950 kernels.  The LD_PRELOAD interposer
// (vkf_preload.cpp) calls both and falls through to the real hipLaunchKernel
// for every name that resolves to VKF_LAUNCH_NONE.
//
// Deliberate differences from the reference, each fixing a defect:
//  * mul_mat is tested before the dequant substrings, so the quantised mul_mat
//    branch (shim/hip_runtime_shim.cpp:1102-1172) is reachable;
//  * the dequant branch also requires "dequant" in the name, so other kernels
//    that carry a type substring (get_rows_q4_0, cpy_f32_q8_0, ...) are not
//    mistaken for dequantisers;
//  * dequant output dtype follows the kernel's destination type (fp16 for a
//    __half/_Float16 instantiation) instead of always fp32;
//  * unknown and unsupported names (IQ formats) run the original kernel
//    instead of returning hipSuccess without doing the work;
//  * a bf16 mul_mat (whose name also contains "f16") is not taken for fp16;
//  * a quantised mul_mat is routed only when its name also names the Q8_1
//    activations its argument layout assumes;
//  * fp16 mul_mat computes D[M,N] = vy[M,K] . vx[N,K]^T into the fp32 ggml
//    destination (the reference passed vx as the M-row operand and wrote fp16).
#include <cstdint>
#include <cstring>

#include "../../../include/vkflame_amd.h"
#include "vkf_runtime.h"

namespace {

struct Name {
    const char *s;
    bool has(const char *sub) const { return std::strstr(s, sub) != nullptr; }
};

void *arg_ptr(void **args, int i) { return *reinterpret_cast<void **>(args[i]); }
int32_t arg_i32(void **args, int i) { return *reinterpret_cast<int32_t *>(args[i]); }
int64_t arg_i64(void **args, int i) { return *reinterpret_cast<int64_t *>(args[i]); }

// Weight type named in a mul_mat kernel (reference order, 1132-1143).
int mul_mat_qtype(const Name &n) {
    if (n.has("q4_1")) return VKF_DEQUANT_Q4_1;
    if (n.has("q8_0")) return VKF_DEQUANT_Q8_0;
    if (n.has("q5_0")) return VKF_DEQUANT_Q5_0;
    if (n.has("q4_K")) return VKF_DEQUANT_Q4_K;
    if (n.has("q5_K")) return VKF_DEQUANT_Q5_K;
    if (n.has("q6_K")) return VKF_DEQUANT_Q6_K;
    return VKF_DEQUANT_Q4_0;
}

}  // namespace

extern "C" {

int vkflame_resolve_launch(const char *name, unsigned grid_x, unsigned grid_y, unsigned grid_z, unsigned block_x,
                           unsigned block_y, unsigned block_z, void **args, VkflameLaunchPlan *plan) {
    (void)grid_y;
    (void)grid_z;
    (void)block_y;
    (void)block_z;
    if (!plan) return VKF_LAUNCH_NONE;
    std::memset(plan, 0, sizeof(*plan));
    plan->kind = VKF_LAUNCH_NONE;
    if (!name || !args) return VKF_LAUNCH_NONE;
    Name n{name};

    if (n.has("mul_mat")) {
        if (n.has("iq2") || n.has("iq3") || n.has("iq4")) return VKF_LAUNCH_NONE;
        bool quant = n.has("q4_0") || n.has("q4_1") || n.has("q4_K") || n.has("q5_0") || n.has("q5_K") ||
                     n.has("q6_K") || n.has("q8_0");
        // Only the quantised-weight x Q8_1-activation kernels the reference
        // describes (mul_mat_q*_q8_1, shim/hip_runtime_shim.cpp:1097-1099)
        // take this argument layout; other mul_mat kernels that name a weight
        // type (ggml's dequantize_mul_mat_vec: 5 arguments, fp32 y) run as
        // launched.
        if (quant && n.has("q8_1")) {
            // (vx, vy, dst, ncols_x, nrows_x, ncols_y, nrows_y, ...) (1123-1125)
            plan->kind = VKF_LAUNCH_MUL_MAT_Q;
            plan->quant_type = mul_mat_qtype(n);
            plan->src = arg_ptr(args, 0);
            plan->src1 = arg_ptr(args, 1);
            plan->dst = arg_ptr(args, 2);
            plan->K = arg_i32(args, 3);
            plan->N = arg_i32(args, 4);
            plan->M = arg_i32(args, 6);
            if (plan->K < 1 || plan->N < 1 || plan->M < 1) plan->kind = VKF_LAUNCH_NONE;
            return plan->kind;
        }
        if ((n.has("f16") || n.has("fp16")) && !n.has("bf16")) {  // (1174-1188)
            plan->kind = VKF_LAUNCH_MUL_MAT_F16;
            plan->src = arg_ptr(args, 0);
            plan->src1 = arg_ptr(args, 1);
            plan->dst = arg_ptr(args, 2);
            plan->K = arg_i32(args, 3);
            plan->N = arg_i32(args, 4);
            plan->M = arg_i32(args, 6);
            if (plan->K < 1 || plan->N < 1 || plan->M < 1) plan->kind = VKF_LAUNCH_NONE;
            return plan->kind;
        }
        return VKF_LAUNCH_NONE;
    }

    if (!n.has("dequant")) return VKF_LAUNCH_NONE;
    int qt = -1;
    uint64_t nb = 0;
    // Substring order and nb rules: shim/hip_runtime_shim.cpp:896-952.
    if (n.has("q4_0") || n.has("q4K_0")) {
        qt = VKF_DEQUANT_Q4_0;
        nb = (uint64_t)(uint32_t)arg_i32(args, 2);
    } else if (n.has("q4_1")) {
        qt = VKF_DEQUANT_Q4_1;
        nb = (uint64_t)(uint32_t)arg_i32(args, 2);
    } else if (n.has("q5_0") || n.has("q5K_0")) {
        qt = VKF_DEQUANT_Q5_0;
        nb = (uint64_t)(uint32_t)arg_i32(args, 2);
    } else if (n.has("q8_0")) {
        qt = VKF_DEQUANT_Q8_0;
        nb = (block_x == 32) ? (uint64_t)(uint32_t)arg_i32(args, 2) : (uint64_t)(arg_i64(args, 2) / 32);
    } else if (n.has("q4_K") || n.has("q4K")) {
        qt = VKF_DEQUANT_Q4_K;
        nb = grid_x;
    } else if (n.has("q5_K") || n.has("q5K")) {
        qt = VKF_DEQUANT_Q5_K;
        nb = grid_x;
    } else if (n.has("q6_K") || n.has("q6K")) {
        qt = VKF_DEQUANT_Q6_K;
        nb = grid_x;
    } else {
        return VKF_LAUNCH_NONE;
    }
    plan->kind = VKF_LAUNCH_DEQUANT;
    plan->quant_type = qt;
    plan->out_dtype = (n.has("__half") || n.has("DF16_")) ? VKF_DTYPE_FP16 : VKF_DTYPE_FP32;
    plan->src = arg_ptr(args, 0);
    plan->dst = arg_ptr(args, 1);
    plan->n_blocks = nb;
    return plan->kind;
}

int vkflame_execute_launch(const VkflameLaunchPlan *plan, void *stream) {
    if (!plan) return hipErrorInvalidValue;
    switch (plan->kind) {
    case VKF_LAUNCH_DEQUANT:
        return vkflame_dispatch_dequant(plan->src, plan->dst, plan->n_blocks, plan->quant_type, plan->out_dtype,
                                        stream);
    case VKF_LAUNCH_MUL_MAT_Q:
        // dst[M, N] = deq(vy: Q8_1)[M, K] . deq(vx)[N, K]^T  (1161-1166)
        return vkflame_dispatch_gemm_q(plan->src, plan->quant_type, 0, plan->src1, VKF_DTYPE_Q8_1, 0,
                                       (float *)plan->dst, 0, plan->M, plan->N, plan->K, stream);
    case VKF_LAUNCH_MUL_MAT_F16:
        return vkflame_dispatch_linear(plan->src1, plan->src, nullptr, plan->dst, plan->M, plan->N, plan->K,
                                       VKF_DTYPE_FP16_FP32OUT, 0, 1, 0, nullptr, nullptr, stream);
    default:
        return hipErrorInvalidValue;
    }
}

}  // extern "C"
