// vkf_preload.cpp — libvkflame_preload.so, an LD_PRELOAD interposer for the
// HIP launch entry points: hipLaunchKernel (the <<<>>> launch of compiled-in
// kernels), hipModuleLaunchKernel and hipExtModuleLaunchKernel (kernels of
// loaded code objects: AOT-compiled HSACO, AOTriton), plus
// hipModuleGetFunction, whose kernel names it records.
//
// The reference replaces all of amdhip64 and routes every launch through its
// name table (shim/hip_runtime_shim.cpp:833-1213, 1298-1336), silently
// skipping kernels it does not know (849-850).  This interposer sits in front
// of the real ROCm runtime instead: it names the launched kernel (the
// runtime's hipKernelNameRefByPtr / hipKernelNameRef, or the name a
// hipModuleGetFunction call returned it for), asks the table
// (vkflame_resolve_launch) for a plan, runs the plan on the gfx950 kernels
// when there is one, and otherwise calls the real entry point unchanged.
// The library's own kernels are launched with the runtime's functions
// directly (vkf::real_hip_symbol), never through these, and names starting
// with "vkf_" are never routed.  Names are cached per function.
// VKFLAME_DEBUG=1 logs every decision.
#include <dlfcn.h>
#include <hip/hip_runtime_api.h>

#include <cstring>
#include <mutex>
#include <string>
#include <unordered_map>

#include "../../../include/vkflame_amd.h"
#include "vkf_runtime.h"

namespace {

using LaunchFn = hipError_t (*)(const void *, dim3, dim3, void **, size_t, hipStream_t);
using ModuleLaunchFn = hipError_t (*)(hipFunction_t, unsigned, unsigned, unsigned, unsigned, unsigned, unsigned,
                                      unsigned, hipStream_t, void **, void **);
using ExtModuleLaunchFn = hipError_t (*)(hipFunction_t, uint32_t, uint32_t, uint32_t, uint32_t, uint32_t, uint32_t,
                                         size_t, hipStream_t, void **, void **, hipEvent_t, hipEvent_t, uint32_t);
using GetFunctionFn = hipError_t (*)(hipFunction_t *, hipModule_t, const char *);

template <class F>
F real(const char *name) {
    return reinterpret_cast<F>(vkf::real_hip_symbol(name));
}

std::mutex g_mu;
std::unordered_map<const void *, std::string> g_names;  // host stub or hipFunction_t -> name

const std::string &cached_name(const void *key, const char *(*lookup)(const void *, hipStream_t), hipStream_t s) {
    std::lock_guard<std::mutex> lk(g_mu);
    auto it = g_names.find(key);
    if (it != g_names.end()) return it->second;
    const char *n = lookup(key, s);
    return g_names.emplace(key, n ? n : "").first->second;
}

const char *stub_name(const void *f, hipStream_t s) { return hipKernelNameRefByPtr(f, s); }
const char *function_name(const void *f, hipStream_t) {
    return hipKernelNameRef(reinterpret_cast<hipFunction_t>(const_cast<void *>(f)));
}

// The table's plan for a launch, or VKF_LAUNCH_NONE (then the caller runs the
// original kernel).  Only launches with per-argument kernelParams can be
// decoded; the library's own kernels (vkf_*) are never routed.
int plan_for(const std::string &name, dim3 grid, dim3 block, void **args, VkflameLaunchPlan *plan,
             const char *via) {
    int kind = VKF_LAUNCH_NONE;
    if (args && name.compare(0, 4, "vkf_") != 0)
        kind = vkflame_resolve_launch(name.c_str(), grid.x, grid.y, grid.z, block.x, block.y, block.z, args, plan);
    if (vkf::debug_enabled())
        vkf::debug_log("%s %s grid=(%u,%u,%u) block=(%u,%u,%u) -> plan %d", via, name.c_str(), grid.x, grid.y,
                       grid.z, block.x, block.y, block.z, kind);
    return kind;
}

}  // namespace

extern "C" {

__attribute__((visibility("default"))) hipError_t hipLaunchKernel(const void *function_address, dim3 numBlocks,
                                                                   dim3 dimBlocks, void **args,
                                                                   size_t sharedMemBytes, hipStream_t stream) {
    static const LaunchFn next = real<LaunchFn>("hipLaunchKernel");
    if (function_address && args) {
        VkflameLaunchPlan plan;
        const std::string &name = cached_name(function_address, stub_name, stream);
        if (plan_for(name, numBlocks, dimBlocks, args, &plan, "hipLaunchKernel") != VKF_LAUNCH_NONE)
            return (hipError_t)vkflame_execute_launch(&plan, stream);
    }
    if (!next) return hipErrorNotInitialized;
    return next(function_address, numBlocks, dimBlocks, args, sharedMemBytes, stream);
}

// Records the name each function handle was looked up by.
__attribute__((visibility("default"))) hipError_t hipModuleGetFunction(hipFunction_t *function, hipModule_t module,
                                                                        const char *kname) {
    static const GetFunctionFn next = real<GetFunctionFn>("hipModuleGetFunction");
    if (!next) return hipErrorNotInitialized;
    const hipError_t e = next(function, module, kname);
    if (e == hipSuccess && function && *function && kname) {
        std::lock_guard<std::mutex> lk(g_mu);
        g_names[*function] = kname;
    }
    return e;
}

// shim/hip_runtime_shim.cpp:1309-1316
__attribute__((visibility("default"))) hipError_t hipModuleLaunchKernel(hipFunction_t f, unsigned int gridDimX,
                                                                         unsigned int gridDimY, unsigned int gridDimZ,
                                                                         unsigned int blockDimX, unsigned int blockDimY,
                                                                         unsigned int blockDimZ,
                                                                         unsigned int sharedMemBytes,
                                                                         hipStream_t stream, void **kernelParams,
                                                                         void **extra) {
    static const ModuleLaunchFn next = real<ModuleLaunchFn>("hipModuleLaunchKernel");
    if (f && kernelParams) {
        VkflameLaunchPlan plan;
        const std::string &name = cached_name(f, function_name, stream);
        if (plan_for(name, dim3(gridDimX, gridDimY, gridDimZ), dim3(blockDimX, blockDimY, blockDimZ), kernelParams,
                     &plan, "hipModuleLaunchKernel") != VKF_LAUNCH_NONE)
            return (hipError_t)vkflame_execute_launch(&plan, stream);
    }
    if (!next) return hipErrorNotInitialized;
    return next(f, gridDimX, gridDimY, gridDimZ, blockDimX, blockDimY, blockDimZ, sharedMemBytes, stream,
                kernelParams, extra);
}

// ROCm's signature (hip/hip_ext.h:71-78, a header only hipcc compiles).
// shim/hip_runtime_shim.cpp:1321-1336: work sizes are threads, so the grid
// is ceil(global / local) per dimension; the start / stop events, when given,
// are recorded around the routed work as the runtime records them around the
// kernel.
__attribute__((visibility("default"))) hipError_t hipExtModuleLaunchKernel(
    hipFunction_t f, uint32_t globalWorkSizeX, uint32_t globalWorkSizeY, uint32_t globalWorkSizeZ,
    uint32_t localWorkSizeX, uint32_t localWorkSizeY, uint32_t localWorkSizeZ, size_t sharedMemBytes,
    hipStream_t hStream, void **kernelParams, void **extra, hipEvent_t startEvent, hipEvent_t stopEvent,
    uint32_t flags) {
    static const ExtModuleLaunchFn next = real<ExtModuleLaunchFn>("hipExtModuleLaunchKernel");
    if (f && kernelParams && localWorkSizeX && localWorkSizeY && localWorkSizeZ) {
        const dim3 grid((globalWorkSizeX + localWorkSizeX - 1) / localWorkSizeX,
                        (globalWorkSizeY + localWorkSizeY - 1) / localWorkSizeY,
                        (globalWorkSizeZ + localWorkSizeZ - 1) / localWorkSizeZ);
        VkflameLaunchPlan plan;
        const std::string &name = cached_name(f, function_name, hStream);
        if (plan_for(name, grid, dim3(localWorkSizeX, localWorkSizeY, localWorkSizeZ), kernelParams, &plan,
                     "hipExtModuleLaunchKernel") != VKF_LAUNCH_NONE) {
            if (startEvent) {
                const hipError_t e = hipEventRecord(startEvent, hStream);
                if (e != hipSuccess) return e;
            }
            const hipError_t e = (hipError_t)vkflame_execute_launch(&plan, hStream);
            if (e != hipSuccess || !stopEvent) return e;
            return hipEventRecord(stopEvent, hStream);
        }
    }
    if (!next) return hipErrorNotInitialized;
    return next(f, globalWorkSizeX, globalWorkSizeY, globalWorkSizeZ, localWorkSizeX, localWorkSizeY, localWorkSizeZ,
                sharedMemBytes, hStream, kernelParams, extra, startEvent, stopEvent, flags);
}

}  // extern "C"
