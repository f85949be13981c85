// vkf_runtime.cpp — gfx950 code-object loader and launcher.
//
// The reference turns SPIR-V blobs into VkPipelines at init
// (runtime/pipeline.cpp:100-251) and records/submits/waits a command buffer
// per dispatch (runtime/dispatch.cpp:105-227).  Here the gfx950 code objects
// built from vkflame_amd/csrc/kernels/*.hip are linked into this library's
// .rodata (build step: .incbin), loaded with hipModuleLoadData the first time
// a device needs them, and launched asynchronously on the caller's stream.
#include "vkf_runtime.h"

#include <dlfcn.h>

#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <mutex>

// Generated at build time (vkflame_amd/build.py): one entry per code object.
struct VkfCodeObject {
    const char *name;
    const unsigned char *begin;
    const unsigned char *end;
};
extern "C" const VkfCodeObject vkf_code_objects[];
extern "C" const int vkf_n_code_objects;

namespace vkf {
namespace {

const char *const k_names[VKF_K_COUNT] = {
#define VKF_X(id, sym) sym,
    VKF_KERNEL_LIST(VKF_X)
#undef VKF_X
};

constexpr int kMaxDevices = 64;

using ModuleLaunchFn = hipError_t (*)(hipFunction_t, unsigned, unsigned, unsigned, unsigned, unsigned, unsigned,
                                      unsigned, hipStream_t, void **, void **);
using ModuleGetFunctionFn = hipError_t (*)(hipFunction_t *, hipModule_t, const char *);

ModuleLaunchFn real_module_launch() {
    static const ModuleLaunchFn fn = reinterpret_cast<ModuleLaunchFn>(real_hip_symbol("hipModuleLaunchKernel"));
    return fn;
}

ModuleGetFunctionFn real_module_get_function() {
    static const ModuleGetFunctionFn fn =
        reinterpret_cast<ModuleGetFunctionFn>(real_hip_symbol("hipModuleGetFunction"));
    return fn;
}

struct DeviceTable {
    std::once_flag once;
    hipError_t status = hipSuccess;
    hipFunction_t fn[VKF_K_COUNT] = {};
    int cus = 0;
    size_t max_lds = 65536;  // dynamic + static LDS one workgroup may use
};

DeviceTable g_dev[kMaxDevices];

void load_device(DeviceTable &t, int dev) {
    hipDeviceProp_t prop;
    hipError_t e = hipGetDeviceProperties(&prop, dev);
    if (e != hipSuccess) { t.status = e; return; }
    t.cus = prop.multiProcessorCount;
    t.max_lds = prop.sharedMemPerBlock;
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        std::fprintf(stderr, "[vkflame] device %d is %s; this library is built for gfx950 only\n", dev,
                     prop.gcnArchName);
        t.status = hipErrorInvalidDeviceFunction;
        return;
    }
    hipModule_t mods[16];
    int nm = vkf_n_code_objects;
    for (int i = 0; i < nm; i++) {
        e = hipModuleLoadData(&mods[i], vkf_code_objects[i].begin);
        if (e != hipSuccess) {
            std::fprintf(stderr, "[vkflame] hipModuleLoadData(%s) failed: %s\n", vkf_code_objects[i].name,
                         hipGetErrorString(e));
            t.status = e;
            return;
        }
    }
    for (int k = 0; k < VKF_K_COUNT; k++) {
        hipFunction_t f = nullptr;
        for (int i = 0; i < nm && !f; i++) {
            if (real_module_get_function()(&f, mods[i], k_names[k]) != hipSuccess) f = nullptr;
        }
        if (!f) {
            std::fprintf(stderr, "[vkflame] kernel %s missing from the code objects\n", k_names[k]);
            (void)hipGetLastError();
            t.status = hipErrorNotFound;
            return;
        }
        t.fn[k] = f;
    }
    (void)hipGetLastError();
}

DeviceTable *table_for_current(hipError_t *err) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        *err = e != hipSuccess ? e : hipErrorInvalidDevice;
        return nullptr;
    }
    DeviceTable &t = g_dev[dev];
    std::call_once(t.once, load_device, std::ref(t), dev);
    *err = t.status;
    return t.status == hipSuccess ? &t : nullptr;
}

}  // namespace

void *real_hip_symbol(const char *name) {
    static void *const runtime = [] () -> void * {
        Dl_info info{};
        if (!dladdr(reinterpret_cast<void *>(&hipGetDevice), &info) || !info.dli_fname) return nullptr;
        return dlopen(info.dli_fname, RTLD_NOW | RTLD_NOLOAD);
    }();
    return runtime ? dlsym(runtime, name) : nullptr;
}

const char *kernel_name(VkfKernelId id) { return (id >= 0 && id < VKF_K_COUNT) ? k_names[id] : "?"; }

hipError_t get_kernel(VkfKernelId id, hipFunction_t *out) {
    hipError_t e;
    DeviceTable *t = table_for_current(&e);
    if (!t) return e;
    *out = t->fn[id];
    return hipSuccess;
}

int cu_count() {
    hipError_t e;
    DeviceTable *t = table_for_current(&e);
    return t ? t->cus : 256;
}

size_t max_lds() {
    hipError_t e;
    DeviceTable *t = table_for_current(&e);
    return t ? t->max_lds : 65536;
}

hipError_t launch(VkfKernelId id, dim3 grid, dim3 block, const void *args, size_t args_size, hipStream_t stream,
                  size_t shmem) {
    (void)args_size;
    hipFunction_t f;
    hipError_t e = get_kernel(id, &f);
    if (e != hipSuccess) return e;
    if (grid.x == 0 || grid.y == 0 || grid.z == 0) return hipSuccess;  // empty problem
    if (debug_enabled())
        debug_log("launch %s grid=(%u,%u,%u) block=(%u,%u,%u) lds=%zu stream=%p", k_names[id], grid.x, grid.y,
                  grid.z, block.x, block.y, block.z, shmem, (void *)stream);
    void *params[1] = {const_cast<void *>(args)};
    const ModuleLaunchFn real = real_module_launch();
    if (!real) return hipErrorNotInitialized;
    return real(f, grid.x, grid.y, grid.z, block.x, block.y, block.z, (unsigned)shmem, stream, params, nullptr);
}

// The condition under which the dense GEMM kernels take their direct-to-LDS
// main loop (dma_ok in kernels/gemm.hip): K-contiguous rows, 16-byte aligned
// base and row pitch, K*es a multiple of 128 bytes.
static bool dma_operand(const void *p, uint64_t ld, bool trans, uint32_t K, uint32_t es) {
    return !trans && (ld * es) % 16 == 0 && ((uintptr_t)p & 15) == 0 && ((uint64_t)K * es) % 128 == 0;
}

// The skinny fp16 kernel's conditions (gemm_skinny in kernels/gemm.hip):
// X K-contiguous with 16-byte rows, K % 32 == 0, Y 16-byte aligned with
// 16-byte rows (NT) or rows of C % 8 == 0 columns (NN).
static bool skinny_ok(const VkfGemmArgs &g, uint32_t batch) {
    if (g.R > 64 || (g.flags & (VKF_GF_X_TRANS | VKF_GF_X_F16Q)) || g.bpx) return false;
    if (batch > 1 && ((g.bsx | g.bsy) & 15) != 0) return false;
    if ((g.ldx * 2) % 16 != 0 || ((uintptr_t)g.X & 15) != 0 || g.K % 32 != 0) return false;
    if ((g.ldy * 2) % 16 != 0 || ((uintptr_t)g.Y & 15) != 0) return false;
    return !(g.flags & VKF_GF_Y_TRANS) || g.Cn % 8 == 0;
}

// The narrow-tile kernels (vkf_gemm_{f16,i8}_n{1..5}, vkf_gemm_q4_k_f16_n{4,5},
// kernels/gemm.hip): 128 x 16·nb tiles, three stages of both K groups'
// steps, whole pairs of 128-byte K steps.  The narrowest allowed tile whose
// grid fits one tile per CU (the most CUs busy); 0 when none fits or the
// 128 x 128 grid already fills the CUs.
constexpr uint32_t kNarrowStages = 3;
uint32_t narrow_nb(const VkfGemmArgs &g, uint32_t batch, uint32_t es, uint32_t nbs) {
    if (g.K == 0 || ((uint64_t)g.K * es) % 256 != 0) return 0;
    const uint64_t cus = (uint64_t)cu_count(), rows = ((uint64_t)g.R + 127) / 128 * batch;
    if (rows * (((uint64_t)g.Cn + 127) / 128) >= cus) return 0;
    for (uint32_t nb = 1; nb <= 5; nb++)
        if (((nbs >> nb) & 1u) && rows * (((uint64_t)g.Cn + 16 * nb - 1) / (16 * nb)) <= cus) return nb;
    return 0;
}

// The narrow-tile kernel for this product (nb set), VKF_K_COUNT if none: a
// grid of fewer 128 x 128 tiles than CUs, operands the direct-to-LDS loads
// take (checked here on the host: not for per-batch pointer arrays, which
// live on the device), whole pairs of 128-byte K steps.  NN (fp16 Y stored
// [K, C]) stages Y's k-rows as they lie and reads them back transposed, and
// skips the 48-column tiles (512x3072x1024 NN 12.9 us on 128 x 64, 13.6 on
// 128 x 48).
static VkfKernelId narrow_kernel(const VkfGemmArgs &g, uint32_t batch, VkfKernelId id, uint32_t &nb) {
    nb = 0;
    const uint64_t tiles = (uint64_t)((g.Cn + 127) / 128) * ((g.R + 127) / 128) * batch;
    if ((id != VKF_K_GEMM_F16 && id != VKF_K_GEMM_I8) || (g.flags & VKF_GF_X_F16Q) || g.bpx ||
        tiles > (uint64_t)cu_count() || (batch > 1 && ((g.bsx | g.bsy) & 15) != 0))
        return VKF_K_COUNT;
    const uint32_t es = id == VKF_K_GEMM_F16 ? 2 : 1;
    const bool xd = dma_operand(g.X, g.ldx, (g.flags & VKF_GF_X_TRANS) != 0, g.K, es);
    if (xd && dma_operand(g.Y, g.ldy, (g.flags & VKF_GF_Y_TRANS) != 0, g.K, es)) {
        static const VkfKernelId nk[2][5] = {
            {VKF_K_GEMM_I8_N1, VKF_K_GEMM_I8_N2, VKF_K_GEMM_I8_N3, VKF_K_GEMM_I8_N4, VKF_K_GEMM_I8_N5},
            {VKF_K_GEMM_F16_N1, VKF_K_GEMM_F16_N2, VKF_K_GEMM_F16_N3, VKF_K_GEMM_F16_N4, VKF_K_GEMM_F16_N5}};
        nb = narrow_nb(g, batch, es, kNarrowAll);
        return nb ? nk[es - 1][nb - 1] : VKF_K_COUNT;
    }
    if (id == VKF_K_GEMM_F16 && (g.flags & VKF_GF_Y_TRANS) && xd && (g.ldy * 2) % 16 == 0 &&
        ((uintptr_t)g.Y & 15) == 0 && g.Cn % 8 == 0) {
        static const VkfKernelId nt[5] = {VKF_K_GEMM_F16_N1T, VKF_K_GEMM_F16_N2T, VKF_K_GEMM_F16_N4T,
                                          VKF_K_GEMM_F16_N4T, VKF_K_GEMM_F16_N5T};  // nb = 3 not taken
        nb = narrow_nb(g, batch, 2, kNarrowAll & ~(1u << 3));
        return nb ? nt[nb - 1] : VKF_K_COUNT;
    }
    return VKF_K_COUNT;
}

hipError_t launch_gemm(VkfKernelId id, const VkfGemmArgs &g, hipStream_t stream, uint32_t batch) {
    if (g.R == 0 || g.Cn == 0 || batch == 0) return hipSuccess;
    dim3 grid((g.Cn + 127) / 128, (g.R + 127) / 128, batch);
    if (grid.y > 65535 || grid.z > 65535) return hipErrorInvalidValue;
    uint32_t nb = 0;
    const VkfKernelId nk = narrow_kernel(g, batch, id, nb);
    // at most 64 rows: Y streamed once by 16-column workgroups where no
    // narrow tiles apply, else up to 8 rows, and up to 32 while those
    // workgroups fit one per CU (same-process A/B, fp16 cold B, streamed
    // against narrow tiles: 4096x4096 NT M = 8 / 16 / 48 / 64 10.8 / 12.4 /
    // 22.2 / 25.5 against 19.1 / 19.0 / 19.0 / 18.9 us, NN M = 32 24.7
    // against 26.6; 11008x4096 NT M = 1 / 16 / 32 21.6 / 32.3 / 46.1
    // against 25.9 / 26.0 / 26.3 us, 688 streaming workgroups)
    const bool sk_fits = (uint64_t)((g.Cn + 15) / 16) * batch <= (uint64_t)cu_count();
    if (id == VKF_K_GEMM_F16 && skinny_ok(g, batch) &&
        (nk == VKF_K_COUNT || g.R <= 8 || (g.R <= 32 && sk_fits)))
        return launch(VKF_K_GEMM_F16_SKINNY, dim3((g.Cn + 15) / 16, 1, batch), dim3(1024), &g, sizeof(g), stream,
                      131072);
    // narrow tiles (128 x 16·nb) where they give the CUs more of the grid:
    // the narrowest whose grid still fits one tile per CU
    if (nk != VKF_K_COUNT)
        return launch(nk, dim3((g.Cn + 16 * nb - 1) / (16 * nb), grid.y, batch), dim3(512), &g, sizeof(g), stream,
                      kNarrowStages * 2 * (16384 + nb * 16 * 128));
    // otherwise on such grids with K-contiguous operands: the split-K kernels
    if ((id == VKF_K_GEMM_F16 || id == VKF_K_GEMM_I8) && !(g.flags & VKF_GF_X_F16Q) && !g.bpx &&
        (uint64_t)grid.x * grid.y * batch <= (uint64_t)cu_count() &&
        (batch == 1 || ((g.bsx | g.bsy) & 15) == 0)) {
        const uint32_t es = id == VKF_K_GEMM_F16 ? 2 : 1;
        if (dma_operand(g.X, g.ldx, (g.flags & VKF_GF_X_TRANS) != 0, g.K, es) &&
            dma_operand(g.Y, g.ldy, (g.flags & VKF_GF_Y_TRANS) != 0, g.K, es))
            return launch(id == VKF_K_GEMM_F16 ? VKF_K_GEMM_F16_K2 : VKF_K_GEMM_I8_K2, grid, dim3(512), &g,
                          sizeof(g), stream);
    }
    // grids of at least one 256 x 256 tile per CU, both operands K-contiguous:
    // the 256 x 256 kernel (half the tile bytes per MAC).  int8 gains on every
    // such grid measured (4096³ 101 -> 68 us); fp16 from K = 8192 on (4-8 %;
    // level or slower at K = 4096)
    if ((id == VKF_K_GEMM_I8 || (id == VKF_K_GEMM_F16 && g.K >= 8192)) && !(g.flags & VKF_GF_X_F16Q) && !g.bpx &&
        (batch == 1 || ((g.bsx | g.bsy) & 15) == 0)) {
        const uint32_t es = id == VKF_K_GEMM_F16 ? 2 : 1;
        const uint64_t t256 = ((uint64_t)g.R + 255) / 256 * (((uint64_t)g.Cn + 255) / 256) * batch;
        if (t256 >= (uint64_t)cu_count() && dma_operand(g.X, g.ldx, (g.flags & VKF_GF_X_TRANS) != 0, g.K, es) &&
            dma_operand(g.Y, g.ldy, (g.flags & VKF_GF_Y_TRANS) != 0, g.K, es))
            return launch(id == VKF_K_GEMM_F16 ? VKF_K_GEMM_F16_B256 : VKF_K_GEMM_I8_B256,
                          dim3((g.Cn + 255) / 256, (g.R + 255) / 256, batch), dim3(512), &g, sizeof(g), stream);
    }
    return launch(id, grid, dim3(256), &g, sizeof(g), stream);
}

bool debug_enabled() {
    static const bool on = [] {
        const char *v = std::getenv("VKFLAME_DEBUG");
        return v && *v && std::strcmp(v, "0") != 0;
    }();
    return on;
}

void debug_log(const char *fmt, ...) {
    std::va_list ap;
    va_start(ap, fmt);
    std::fputs("[vkflame] ", stderr);
    std::vfprintf(stderr, fmt, ap);
    std::fputc('\n', stderr);
    va_end(ap);
}

}  // namespace vkf
