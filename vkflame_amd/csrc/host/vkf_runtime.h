// vkf_runtime.h — internal host runtime: gfx950 code-object loader, kernel
// table and launcher.  Replaces the reference's Vulkan pipeline table
// (runtime/pipeline.h:10-44 VKFKernelID, runtime/pipeline.cpp:143-251) and
// do_dispatch (runtime/dispatch.cpp:105-227): code objects are embedded in the
// library at build time, loaded once per device with hipModuleLoadData, and
// every launch is one hipModuleLaunchKernel with a packed kernarg struct on the
// caller's stream (no descriptor sets, no fence wait).
#pragma once
#include <hip/hip_runtime_api.h>
#include <stddef.h>
#include <stdint.h>
#include "../include/vkf_kernargs.h"

// Kernel ids.  X-macro: (id, symbol in the code object).
#define VKF_KERNEL_LIST(X)                                  \
    X(DEQ_Q4_0_F32, "vkf_dequant_q4_0_f32")                 \
    X(DEQ_Q4_0_F16, "vkf_dequant_q4_0_f16")                 \
    X(DEQ_Q4_1_F32, "vkf_dequant_q4_1_f32")                 \
    X(DEQ_Q4_1_F16, "vkf_dequant_q4_1_f16")                 \
    X(DEQ_Q8_0_F32, "vkf_dequant_q8_0_f32")                 \
    X(DEQ_Q8_0_F16, "vkf_dequant_q8_0_f16")                 \
    X(DEQ_Q5_0_F32, "vkf_dequant_q5_0_f32")                 \
    X(DEQ_Q5_0_F16, "vkf_dequant_q5_0_f16")                 \
    X(DEQ_Q4_K_F32, "vkf_dequant_q4_k_f32")                 \
    X(DEQ_Q4_K_F16, "vkf_dequant_q4_k_f16")                 \
    X(DEQ_Q5_K_F32, "vkf_dequant_q5_k_f32")                 \
    X(DEQ_Q5_K_F16, "vkf_dequant_q5_k_f16")                 \
    X(DEQ_Q6_K_F32, "vkf_dequant_q6_k_f32")                 \
    X(DEQ_Q6_K_F16, "vkf_dequant_q6_k_f16")                 \
    X(DEQ_Q8_1_F32, "vkf_dequant_q8_1_f32")                 \
    X(DEQ_Q8_1_F16, "vkf_dequant_q8_1_f16")                 \
    X(QUANT_Q8_1, "vkf_quantize_q8_1")                      \
    X(STREAM_READ, "vkf_stream_read")                       \
    X(QUANT_ROWS_I8, "vkf_quantize_rows_i8")                \
    /* GEMV: 3 activation kinds per weight type, VKF_Q* order */ \
    X(GEMV_Q4_0_F16, "vkf_gemv_q4_0_f16")                   \
    X(GEMV_Q4_0_F32, "vkf_gemv_q4_0_f32")                   \
    X(GEMV_Q4_0_Q81, "vkf_gemv_q4_0_q8_1")                  \
    X(GEMV_Q4_1_F16, "vkf_gemv_q4_1_f16")                   \
    X(GEMV_Q4_1_F32, "vkf_gemv_q4_1_f32")                   \
    X(GEMV_Q4_1_Q81, "vkf_gemv_q4_1_q8_1")                  \
    X(GEMV_Q8_0_F16, "vkf_gemv_q8_0_f16")                   \
    X(GEMV_Q8_0_F32, "vkf_gemv_q8_0_f32")                   \
    X(GEMV_Q8_0_Q81, "vkf_gemv_q8_0_q8_1")                  \
    X(GEMV_Q5_0_F16, "vkf_gemv_q5_0_f16")                   \
    X(GEMV_Q5_0_F32, "vkf_gemv_q5_0_f32")                   \
    X(GEMV_Q5_0_Q81, "vkf_gemv_q5_0_q8_1")                  \
    X(GEMV_Q4_K_F16, "vkf_gemv_q4_k_f16")                   \
    X(GEMV_Q4_K_F32, "vkf_gemv_q4_k_f32")                   \
    X(GEMV_Q4_K_Q81, "vkf_gemv_q4_k_q8_1")                  \
    X(GEMV_Q5_K_F16, "vkf_gemv_q5_k_f16")                   \
    X(GEMV_Q5_K_F32, "vkf_gemv_q5_k_f32")                   \
    X(GEMV_Q5_K_Q81, "vkf_gemv_q5_k_q8_1")                  \
    X(GEMV_Q6_K_F16, "vkf_gemv_q6_k_f16")                   \
    X(GEMV_Q6_K_F32, "vkf_gemv_q6_k_f32")                   \
    X(GEMV_Q6_K_Q81, "vkf_gemv_q6_k_q8_1_int")              \
    X(Q6_K_Q8_1_PARTIALS, "vkf_q6_k_q8_1_partials")         \
    X(GEMV_Q6K_Q81_DOT_M1, "vkf_gemv_q6k_q81_dot_m1")      \
    X(GEMV_Q6K_F16_DOT_M1, "vkf_gemv_q6k_f16_dot_m1")      \
    X(GEMV_Q6K_F32_DOT_M1, "vkf_gemv_q6k_f32_dot_m1")      \
    X(GEMV_DOTL_Q4_0_F16, "vkf_gemv_dotl_q4_0_f16")        \
    X(GEMV_DOTL_Q4_0_F32, "vkf_gemv_dotl_q4_0_f32")        \
    X(GEMV_DOTL_Q4_0_Q81, "vkf_gemv_dotl_q4_0_q8_1")       \
    X(GEMV_DOTL_Q4_1_F16, "vkf_gemv_dotl_q4_1_f16")        \
    X(GEMV_DOTL_Q4_1_F32, "vkf_gemv_dotl_q4_1_f32")        \
    X(GEMV_DOTL_Q4_1_Q81, "vkf_gemv_dotl_q4_1_q8_1")       \
    X(GEMV_DOTL_Q4_K_F16, "vkf_gemv_dotl_q4_k_f16")        \
    X(GEMV_DOTL_Q4_K_F32, "vkf_gemv_dotl_q4_k_f32")        \
    X(GEMV_DOTL_Q4_K_Q81, "vkf_gemv_dotl_q4_k_q8_1")       \
    X(GEMV_DOTL_Q5_K_F16, "vkf_gemv_dotl_q5_k_f16")        \
    X(GEMV_DOTL_Q5_K_F32, "vkf_gemv_dotl_q5_k_f32")        \
    X(GEMV_DOTL_Q5_K_Q81, "vkf_gemv_dotl_q5_k_q8_1")       \
    X(GEMV_DOTL_Q8_0_F16, "vkf_gemv_dotl_q8_0_f16")        \
    X(GEMV_DOTL_Q8_0_F32, "vkf_gemv_dotl_q8_0_f32")        \
    X(GEMV_MFMA_Q4_K_F16, "vkf_gemv_mfma_q4_k_f16")        \
    X(GEMV_MFMA_Q4_0_F16, "vkf_gemv_mfma_q4_0_f16")        \
    X(GEMV_MFMA_Q4_1_F16, "vkf_gemv_mfma_q4_1_f16")        \
    X(GEMV_MFMA_Q6_K_F16, "vkf_gemv_mfma_q6_k_f16")        \
    X(GEMV_MFMA_Q5_K_F16, "vkf_gemv_mfma_q5_k_f16")        \
    X(GEMV_MFMA_Q8_0_F16, "vkf_gemv_mfma_q8_0_f16")        \
    X(GEMV_MFMA_Q5_0_F16, "vkf_gemv_mfma_q5_0_f16")         \
    X(GEMV_MFMA_Q4_K_F32, "vkf_gemv_mfma_q4_k_f32")         \
    X(GEMV_MFMA_Q4_0_F32, "vkf_gemv_mfma_q4_0_f32")         \
    X(GEMV_MFMA_Q4_1_F32, "vkf_gemv_mfma_q4_1_f32")         \
    X(GEMV_MFMA_Q6_K_F32, "vkf_gemv_mfma_q6_k_f32")         \
    X(GEMV_MFMA_Q5_K_F32, "vkf_gemv_mfma_q5_k_f32")         \
    X(GEMV_MFMA_Q8_0_F32, "vkf_gemv_mfma_q8_0_f32")         \
    X(GEMV_MFMA_Q5_0_F32, "vkf_gemv_mfma_q5_0_f32")         \
    X(GEMV_MFMA_Q4_K_Q81, "vkf_gemv_mfma_q4_k_q8_1")        \
    X(GEMV_MFMA_Q4_0_Q81, "vkf_gemv_mfma_q4_0_q8_1")        \
    X(GEMV_MFMA_Q4_1_Q81, "vkf_gemv_mfma_q4_1_q8_1")        \
    X(GEMV_MFMA_Q6_K_Q81, "vkf_gemv_mfma_q6_k_q8_1")        \
    X(GEMV_MFMA_Q5_K_Q81, "vkf_gemv_mfma_q5_k_q8_1")        \
    X(GEMV_MFMA_Q8_0_Q81, "vkf_gemv_mfma_q8_0_q8_1")        \
    X(GEMV_MFMA_Q5_0_Q81, "vkf_gemv_mfma_q5_0_q8_1")        \
    /* dot-product GEMV: per format {f16, f32} x {m1, m4} */ \
    X(GEMV_DOT_Q4_0_F16_M1, "vkf_gemv_dot_q4_0_f16_m1") \
    X(GEMV_DOT_Q4_0_F32_M1, "vkf_gemv_dot_q4_0_f32_m1") \
    X(GEMV_DOT_Q4_0_F16_M4, "vkf_gemv_dot_q4_0_f16_m4") \
    X(GEMV_DOT_Q4_0_F32_M4, "vkf_gemv_dot_q4_0_f32_m4") \
    X(GEMV_DOT_Q4_1_F16_M1, "vkf_gemv_dot_q4_1_f16_m1") \
    X(GEMV_DOT_Q4_1_F32_M1, "vkf_gemv_dot_q4_1_f32_m1") \
    X(GEMV_DOT_Q4_1_F16_M4, "vkf_gemv_dot_q4_1_f16_m4") \
    X(GEMV_DOT_Q4_1_F32_M4, "vkf_gemv_dot_q4_1_f32_m4") \
    X(GEMV_DOT_Q8_0_F16_M1, "vkf_gemv_dot_q8_0_f16_m1") \
    X(GEMV_DOT_Q8_0_F32_M1, "vkf_gemv_dot_q8_0_f32_m1") \
    X(GEMV_DOT_Q8_0_F16_M4, "vkf_gemv_dot_q8_0_f16_m4") \
    X(GEMV_DOT_Q8_0_F32_M4, "vkf_gemv_dot_q8_0_f32_m4") \
    X(GEMV_DOT_Q4_K_F16_M1, "vkf_gemv_dot_q4_k_f16_m1") \
    X(GEMV_DOT_Q4_K_F32_M1, "vkf_gemv_dot_q4_k_f32_m1") \
    X(GEMV_DOT_Q4_K_F16_M4, "vkf_gemv_dot_q4_k_f16_m4") \
    X(GEMV_DOT_Q4_K_F32_M4, "vkf_gemv_dot_q4_k_f32_m4") \
    X(GEMV_DOT_Q5_K_F16_M1, "vkf_gemv_dot_q5_k_f16_m1") \
    X(GEMV_DOT_Q5_K_F32_M1, "vkf_gemv_dot_q5_k_f32_m1") \
    X(GEMV_DOT_Q5_K_F16_M4, "vkf_gemv_dot_q5_k_f16_m4") \
    X(GEMV_DOT_Q5_K_F32_M4, "vkf_gemv_dot_q5_k_f32_m4") \
    X(GEMV_DOT_Q8_0_Q81_M1, "vkf_gemv_dot_q8_0_q8_1_m1") \
    X(GEMM_F16, "vkf_gemm_f16")                             \
    X(GEMM_F32, "vkf_gemm_f32")                             \
    X(GEMM_I8, "vkf_gemm_i8")                               \
    X(GEMM_F16_K2, "vkf_gemm_f16_k2")                       \
    X(GEMM_I8_K2, "vkf_gemm_i8_k2")                         \
    X(GEMM_F16_N4, "vkf_gemm_f16_n4")                       \
    X(GEMM_F16_N5, "vkf_gemm_f16_n5")                       \
    X(GEMM_I8_N4, "vkf_gemm_i8_n4")                         \
    X(GEMM_I8_N5, "vkf_gemm_i8_n5")                         \
    X(GEMM_F16_N4T, "vkf_gemm_f16_n4t")                     \
    X(GEMM_F16_N2, "vkf_gemm_f16_n2")                       \
    X(GEMM_I8_N2, "vkf_gemm_i8_n2")                         \
    X(GEMM_F16_N2T, "vkf_gemm_f16_n2t")                     \
    X(GEMM_F16_N1, "vkf_gemm_f16_n1")                       \
    X(GEMM_I8_N1, "vkf_gemm_i8_n1")                         \
    X(GEMM_F16_N1T, "vkf_gemm_f16_n1t")                     \
    X(GEMM_F16_N3, "vkf_gemm_f16_n3")                       \
    X(GEMM_I8_N3, "vkf_gemm_i8_n3")                         \
    X(GEMM_F16_N5T, "vkf_gemm_f16_n5t")                     \
    X(GEMM_F16_B256, "vkf_gemm_f16_b256")                   \
    X(GEMM_I8_B256, "vkf_gemm_i8_b256")                     \
    X(GEMM_Q4_K_F16_N4, "vkf_gemm_q4_k_f16_n4")             \
    X(GEMM_Q4_K_F16_N5, "vkf_gemm_q4_k_f16_n5")             \
    X(GEMV_MFMA_XR_Q4_0_F16, "vkf_gemv_mfma_xr_q4_0_f16_p16") \
    X(GEMV_MFMA_XR_Q4_1_F16, "vkf_gemv_mfma_xr_q4_1_f16_p16") \
    X(GEMV_MFMA_XR_Q4_K_F16_P10, "vkf_gemv_mfma_xr_q4_k_f16_p10") \
    X(GEMV_MFMA_XR_Q4_0_F16_KS, "vkf_gemv_mfma_xr_q4_0_f16_p16_ks") \
    X(GEMV_MFMA_XR_Q4_1_F16_KS, "vkf_gemv_mfma_xr_q4_1_f16_p16_ks") \
    X(GEMV_MFMA_XR_Q4_K_F16_P10_KS, "vkf_gemv_mfma_xr_q4_k_f16_p10_ks") \
    X(GEMV_SPLIT_SUM, "vkf_gemv_split_sum")                 \
    X(GEMV_MFMA_XR_Q8_0_F16_P12, "vkf_gemv_mfma_xr_q8_0_f16_p12") \
    X(GEMV_MFMA_XR_Q8_0_F16_P12_KS, "vkf_gemv_mfma_xr_q8_0_f16_p12_ks") \
    X(GEMM_F16_SKINNY, "vkf_gemm_f16_skinny")               \
    /* GEMM: fp16 and Q8_1 activations per weight type */   \
    X(GEMM_Q4_0_F16, "vkf_gemm_q4_0_f16")                   \
    X(GEMM_Q4_0_Q81, "vkf_gemm_q4_0_q8_1")                  \
    X(GEMM_Q4_1_F16, "vkf_gemm_q4_1_f16")                   \
    X(GEMM_Q4_1_Q81, "vkf_gemm_q4_1_q8_1")                  \
    X(GEMM_Q8_0_F16, "vkf_gemm_q8_0_f16")                   \
    X(GEMM_Q8_0_Q81, "vkf_gemm_q8_0_q8_1")                  \
    X(GEMM_Q5_0_F16, "vkf_gemm_q5_0_f16")                   \
    X(GEMM_Q5_0_Q81, "vkf_gemm_q5_0_q8_1")                  \
    X(GEMM_Q4_K_F16, "vkf_gemm_q4_k_f16")                   \
    X(GEMM_Q4_K_Q81, "vkf_gemm_q4_k_q8_1")                  \
    X(GEMM_Q5_K_F16, "vkf_gemm_q5_k_f16")                   \
    X(GEMM_Q5_K_Q81, "vkf_gemm_q5_k_q8_1")                  \
    X(GEMM_Q6_K_F16, "vkf_gemm_q6_k_f16")                   \
    X(GEMM_Q6_K_Q81, "vkf_gemm_q6_k_q8_1")                  \
    /* wide (256 x 128 tile, 512 threads) GEMM, fp16 activations */ \
    X(GEMM_W_Q4_0_F16, "vkf_gemm_q4_0_f16_w")               \
    X(GEMM_W_Q4_1_F16, "vkf_gemm_q4_1_f16_w")               \
    X(GEMM_W_Q8_0_F16, "vkf_gemm_q8_0_f16_w")               \
    X(GEMM_W_Q5_0_F16, "vkf_gemm_q5_0_f16_w")               \
    X(GEMM_W_Q4_K_F16, "vkf_gemm_q4_k_f16_w")               \
    X(GEMM_W_Q5_K_F16, "vkf_gemm_q5_k_f16_w")               \
    X(GEMM_W_Q6_K_F16, "vkf_gemm_q6_k_f16_w")             \
    X(GEMM_K2_Q4_0_F16, "vkf_gemm_q4_0_f16_k2")             \
    X(GEMM_K2_Q4_1_F16, "vkf_gemm_q4_1_f16_k2")             \
    X(GEMM_K2_Q8_0_F16, "vkf_gemm_q8_0_f16_k2")             \
    X(GEMM_K2_Q5_0_F16, "vkf_gemm_q5_0_f16_k2")             \
    X(GEMM_K2_Q4_K_F16, "vkf_gemm_q4_k_f16_k2")             \
    X(GEMM_K2_Q5_K_F16, "vkf_gemm_q5_k_f16_k2")             \
    X(GEMM_K2_Q6_K_F16, "vkf_gemm_q6_k_f16_k2")             \
    X(GEMM_Q8_0_Q81_I8, "vkf_gemm_q8_0_q8_1_i8")            \
    X(Q8_0_Q8_1_PARTIALS, "vkf_q8_0_q8_1_partials_mfma")

enum VkfKernelId {
#define VKF_X(id, sym) VKF_K_##id,
    VKF_KERNEL_LIST(VKF_X)
#undef VKF_X
    VKF_K_COUNT
};

namespace vkf {

// Loads the code objects on the current device (once) and returns the kernel.
hipError_t get_kernel(VkfKernelId id, hipFunction_t *out);
const char *kernel_name(VkfKernelId id);

// One launch of kernel `id` with a single by-value kernarg struct.
hipError_t launch(VkfKernelId id, dim3 grid, dim3 block, const void *args, size_t args_size,
                  hipStream_t stream, size_t shmem = 0);

template <class T>
inline hipError_t launch(VkfKernelId id, dim3 grid, dim3 block, const T &args, hipStream_t stream,
                         size_t shmem = 0) {
    return launch(id, grid, block, &args, sizeof(T), stream, shmem);
}

// A VkfGemmArgs launch: 128x128 output tile per 256-thread workgroup, `batch`
// matrices along grid z (g's batch strides or pointer arrays).  For
// GEMM_F16 / GEMM_I8 with no more tiles than CUs and operands the
// direct-to-LDS loads take, the 512-thread split-K kernel (_K2) instead.
hipError_t launch_gemm(VkfKernelId id, const VkfGemmArgs &g, hipStream_t stream, uint32_t batch = 1);

// VKFLAME_DEBUG=1: one stderr line per dispatch (reference: torch_backend/mode.py:13).
bool debug_enabled();
void debug_log(const char *fmt, ...);

// The HIP runtime's own definition of entry point `name` (looked up in the
// shared object that defines hipGetDevice), never an interposer of the same
// name: the library's own launches go straight to the runtime even when
// libvkflame_preload.so, which interposes hipModuleLaunchKernel, is loaded.
void *real_hip_symbol(const char *name);

// The vendor library's (ROCm's) own definition of `name` in `lib`
// ("libhipblas.so", "libhipblaslt.so"): the process's copy of that library
// (dlopen'ed if it is not loaded yet) searched with dlsym on its handle, so
// never this library's export of the same name.  nullptr when no GPU is
// visible (the vendor libraries may end the process when they find none), or
// the library or symbol is absent.
void *vendor_symbol(const char *lib, const char *name);

// Tile width (16·nb columns) of the narrow-tile GEMMs for this grid: the
// narrowest of those allowed (bit nb of nbs) whose grid fits one tile per
// CU, 0 if none does or they do not apply (es: bytes per X element).
constexpr uint32_t kNarrowAll = 0x3e;                 // nb = 1 .. 5 (dense kernels)
constexpr uint32_t kNarrowQ4K = (1u << 4) | (1u << 5);  // the Q4_K kernel's two widths
uint32_t narrow_nb(const VkfGemmArgs &g, uint32_t batch, uint32_t es, uint32_t nbs);

// Number of compute units of the current device (cached per device).
int cu_count();
// LDS bytes one workgroup may use on the current device.
size_t max_lds();

}  // namespace vkf
