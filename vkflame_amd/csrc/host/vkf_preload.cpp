// vkf_preload.cpp — libvkflame_preload.so, an LD_PRELOAD interposer for
// hipLaunchKernel.
//
// The reference replaces all of amdhip64 and routes every launch through its
// name table (shim/hip_runtime_shim.cpp:833-1213), silently skipping kernels
// it does not know (849-850).  This interposer sits in front of the real ROCm
// runtime instead: it names the launched kernel with the runtime's own
// hipKernelNameRefByPtr, asks the table (vkflame_resolve_launch) for a plan,
// runs the plan on the gfx950 kernels when there is one, and otherwise calls
// the next hipLaunchKernel in the link chain (the real one) unchanged.
// Names are cached per host function pointer.  VKFLAME_DEBUG=1 logs every
// decision.
#include <dlfcn.h>
#include <hip/hip_runtime_api.h>

#include <mutex>
#include <string>
#include <unordered_map>

#include "../../../include/vkflame_amd.h"
#include "vkf_runtime.h"

namespace {

using LaunchFn = hipError_t (*)(const void *, dim3, dim3, void **, size_t, hipStream_t);

LaunchFn real_launch() {
    static LaunchFn fn = reinterpret_cast<LaunchFn>(dlsym(RTLD_NEXT, "hipLaunchKernel"));
    return fn;
}

std::mutex g_mu;
std::unordered_map<const void *, std::string> g_names;

const std::string &name_of(const void *f, hipStream_t s) {
    std::lock_guard<std::mutex> lk(g_mu);
    auto it = g_names.find(f);
    if (it != g_names.end()) return it->second;
    const char *n = hipKernelNameRefByPtr(f, s);
    return g_names.emplace(f, n ? n : "").first->second;
}

}  // namespace

extern "C" __attribute__((visibility("default"))) hipError_t hipLaunchKernel(const void *function_address,
                                                                              dim3 numBlocks, dim3 dimBlocks,
                                                                              void **args, size_t sharedMemBytes,
                                                                              hipStream_t stream) {
    LaunchFn next = real_launch();
    if (function_address && args) {
        const std::string &name = name_of(function_address, stream);
        VkflameLaunchPlan plan;
        int kind = vkflame_resolve_launch(name.c_str(), numBlocks.x, numBlocks.y, numBlocks.z, dimBlocks.x,
                                          dimBlocks.y, dimBlocks.z, args, &plan);
        if (vkf::debug_enabled())
            vkf::debug_log("hipLaunchKernel %s grid=(%u,%u,%u) block=(%u,%u,%u) -> plan %d", name.c_str(),
                           numBlocks.x, numBlocks.y, numBlocks.z, dimBlocks.x, dimBlocks.y, dimBlocks.z, kind);
        if (kind != VKF_LAUNCH_NONE) return (hipError_t)vkflame_execute_launch(&plan, stream);
    }
    if (!next) return hipErrorNotInitialized;
    return next(function_address, numBlocks, dimBlocks, args, sharedMemBytes, stream);
}
