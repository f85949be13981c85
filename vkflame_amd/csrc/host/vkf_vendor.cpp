// vkf_vendor.cpp — lookup of ROCm's own hipBLAS / hipBLASLt functions.
//
// libvkflame_amd.so exports hipBLAS / hipBLASLt entry points under ROCm's
// names.  When it is linked or preloaded ahead of ROCm's libraries, the
// handles and descriptors it hands out are ROCm's own objects (created by the
// vendor functions found here), so every function the library does not
// export reaches ROCm with objects ROCm created, and the calls the library
// does not run on its own kernels are forwarded to the vendor function.
#include <dlfcn.h>

#include <cstdlib>
#include <mutex>
#include <string>
#include <unordered_map>

#include "vkf_runtime.h"

namespace vkf {

void *vendor_symbol(const char *lib, const char *name) {
    static const bool gpu = [] {
        int n = 0;
        const bool ok = hipGetDeviceCount(&n) == hipSuccess && n > 0;
        (void)hipGetLastError();
        return ok;
    }();
    if (!gpu) return nullptr;
    static std::mutex mu;
    static std::unordered_map<std::string, void *> libs;
    void *h;
    {
        std::lock_guard<std::mutex> lk(mu);
        auto it = libs.find(lib);
        if (it == libs.end()) {
            h = dlopen(lib, RTLD_NOW | RTLD_LOCAL);
            if (!h) {
                const std::string rocm = std::string(std::getenv("ROCM_PATH") ? std::getenv("ROCM_PATH") : "/opt/rocm") +
                                         "/lib/" + lib;
                h = dlopen(rocm.c_str(), RTLD_NOW | RTLD_LOCAL);
            }
            it = libs.emplace(lib, h).first;
        }
        h = it->second;
    }
    return h ? dlsym(h, name) : nullptr;
}

}  // namespace vkf
