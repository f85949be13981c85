// module_kernels.hip — TEST HELPER for tests/test_gpu_preload.py, not part of
// the library.  Built with hipcc --genco into module_kernels.co, a code object
// that tests/native/module_probe loads with hipModuleLoad and launches through
// hipModuleLaunchKernel / hipExtModuleLaunchKernel, the way AOT-compiled
// kernels are launched.  The names are ones the launch table routes
// (dequantize_block_q4_K_f32, mul_mat_vec_q4_K_q8_1) plus one it does not
// know (scale_f32); the routed kernels' own bodies only write a marker
// (-7.0), so the output shows which code ran.
#include <hip/hip_runtime.h>

extern "C" __global__ void dequantize_block_q4_K_f32(const void *vx, float *y) {
    for (int i = threadIdx.x; i < 256; i += blockDim.x) y[(size_t)blockIdx.x * 256 + i] = -7.0f;
}

extern "C" __global__ void mul_mat_vec_q4_K_q8_1(const void *vx, const void *vy, float *dst, int ncols_x,
                                                 int nrows_x, int ncols_y, int nrows_y) {
    const long n = (long)nrows_x * nrows_y;
    for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x)
        dst[i] = -7.0f;
}

extern "C" __global__ void scale_f32(float *x, float s, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) x[i] *= s;
}
