// vkf_noalloc.hip — vkflame_dispatch_gemm_q_noalloc: the quantised GEMV/GEMM
// entry point for callers that cannot allocate device memory (code under HIP
// graph capture, tight serving loops, harnesses that forbid hipMalloc).
//
// vkflame_dispatch_gemm_q allocates one scratch buffer, stream-ordered: the
// fp16 copy of Q8_1 activations at M > 16 (M*K*2 bytes), or the K-slice
// partials of the register-activation GEMV (S*M*N*4 bytes).  Here that buffer
// is a file-scope device array, `scratch`, of kScratchBytes; each GPU the
// library runs on holds its own copy until the process ends.  Host code
// never passes the array's name to a kernel (on the host it is only a
// stand-in symbol): the first call on a device, with that device current,
// looks up the array's device address with hipGetSymbolAddress and keeps it
// per device, and every launch gets that address.
//
// Built by hipcc (host + gfx950 device code) and linked into
// libvkflame_amd.so; the kernels that use the buffer are the library's own
// (vkflame_dispatch_gemm_q_ws with the buffer as its workspace).
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <mutex>

#include "../../../include/vkflame_amd.h"

namespace {

constexpr size_t kScratchBytes = (size_t)VKFLAME_NOALLOC_SCRATCH_BYTES;
constexpr int kMaxDevices = 64;

static __device__ __align__(256) uint8_t scratch[kScratchBytes];

struct DeviceScratch {
    std::once_flag once;
    hipError_t status = hipSuccess;
    void *ptr = nullptr;  // device address of `scratch` on this device
};
DeviceScratch g_scratch[kMaxDevices];

// Device address of this device's `scratch`, looked up once per device with
// that device current.  Returns nullptr (and *err) on failure.
void *scratch_ptr(hipError_t *err) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        *err = e != hipSuccess ? e : hipErrorInvalidDevice;
        return nullptr;
    }
    DeviceScratch &s = g_scratch[dev];
    std::call_once(s.once, [&s] {
        void *p = nullptr;
        const hipError_t r = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (r != hipSuccess || p == nullptr) {
            std::fprintf(stderr, "[vkflame] hipGetSymbolAddress(scratch) failed: %s\n", hipGetErrorString(r));
            s.status = r != hipSuccess ? r : hipErrorInvalidSymbol;
            (void)hipGetLastError();
            return;
        }
        s.ptr = p;
    });
    *err = s.status;
    return s.ptr;
}

}  // namespace

extern "C" {

size_t vkflame_noalloc_scratch_bytes(void) { return kScratchBytes; }

int vkflame_dispatch_gemm_q_noalloc(const void *w, int quant_type, uint64_t row_bytes, const void *x, int x_dtype,
                                    int64_t ldx, float *y, int64_t ldy, int M, int N, int K, void *stream) {
    const size_t need = vkflame_gemm_q_workspace_bytes(quant_type, x_dtype, M, N, K);
    // no scratch on this route, or GEMV K-slice partials beyond the array (the
    // GEMV then runs its slices one launch after another, as with no workspace)
    if (need == 0 || (M <= 16 && need > kScratchBytes))
        return vkflame_dispatch_gemm_q_ws(w, quant_type, row_bytes, x, x_dtype, ldx, y, ldy, M, N, K, nullptr, 0,
                                          stream);
    if (need > kScratchBytes) {
        std::fprintf(stderr,
                     "[vkflame] vkflame_dispatch_gemm_q_noalloc: M=%d K=%d needs %zu bytes of scratch, more than "
                     "its fixed %zu; use vkflame_dispatch_gemm_q_ws with a workspace\n",
                     M, K, need, kScratchBytes);
        return hipErrorInvalidValue;
    }
    hipError_t e = hipSuccess;
    void *p = scratch_ptr(&e);
    if (!p) return e;
    return vkflame_dispatch_gemm_q_ws(w, quant_type, row_bytes, x, x_dtype, ldx, y, ldy, M, N, K, p, kScratchBytes,
                                      stream);
}

}  // extern "C"
