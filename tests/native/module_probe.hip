// module_probe.hip — TEST HELPER for tests/test_gpu_preload.py, not part of
// the library.  Loads module_kernels.co (hipModuleLoad), looks its kernels up
// by name (hipModuleGetFunction) and launches them with the driver-style
// entry points, as programs with AOT-compiled kernels do.  Under
// LD_PRELOAD=libvkflame_preload.so the table-named launches run the
// library's kernels; scale_f32 must always run its own body.
//
// usage: module_probe <mode> <code object> <in.bin> <out.bin> <a> [<b> <c>]
//   mod_dq4k  a = blocks: hipModuleLaunchKernel, grid a x 32 threads
//   ext_dq4k  a = blocks: hipExtModuleLaunchKernel with global work size
//             a*32 threads (grid a) and start / stop events, which must time
//   mod_mmq   a = N, b = K, c = M: in = Q4_K weights then Q8_1 activations
//   mod_scale a = n: in = n fp32, out = 3 * in
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>

#define CK(x)                                                                               \
    do {                                                                                    \
        hipError_t e_ = (x);                                                                \
        if (e_ != hipSuccess) {                                                             \
            std::fprintf(stderr, "%s failed: %s\n", #x, hipGetErrorString(e_));             \
            std::exit(2);                                                                   \
        }                                                                                   \
    } while (0)

static std::vector<char> read_file(const char *p) {
    FILE *f = std::fopen(p, "rb");
    if (!f) { std::fprintf(stderr, "cannot open %s\n", p); std::exit(2); }
    std::fseek(f, 0, SEEK_END);
    long n = std::ftell(f);
    std::fseek(f, 0, SEEK_SET);
    std::vector<char> b(n);
    if (n && std::fread(b.data(), 1, n, f) != (size_t)n) { std::fprintf(stderr, "short read\n"); std::exit(2); }
    std::fclose(f);
    return b;
}

static void write_file(const char *p, const void *d, size_t n) {
    FILE *f = std::fopen(p, "wb");
    if (!f || std::fwrite(d, 1, n, f) != n) { std::fprintf(stderr, "cannot write %s\n", p); std::exit(2); }
    std::fclose(f);
}

int main(int argc, char **argv) {
    if (argc < 6) { std::fprintf(stderr, "usage: module_probe mode co in out a [b c]\n"); return 2; }
    const std::string mode = argv[1];
    std::vector<char> in = read_file(argv[3]);
    const long a = std::atol(argv[5]), b = argc > 6 ? std::atol(argv[6]) : 0, c = argc > 7 ? std::atol(argv[7]) : 0;
    hipModule_t mod;
    CK(hipModuleLoad(&mod, argv[2]));
    void *din = nullptr, *dout = nullptr;
    CK(hipMalloc(&din, in.size() + 16));
    CK(hipMemcpy(din, in.data(), in.size(), hipMemcpyHostToDevice));
    size_t out_bytes = 0;
    hipFunction_t f;
    if (mode == "mod_dq4k" || mode == "ext_dq4k") {
        if ((long)in.size() != a * 144) return 3;
        out_bytes = (size_t)a * 256 * 4;
        CK(hipMalloc(&dout, out_bytes));
        CK(hipModuleGetFunction(&f, mod, "dequantize_block_q4_K_f32"));
        void *params[] = {&din, &dout};
        if (mode == "mod_dq4k") {
            CK(hipModuleLaunchKernel(f, (unsigned)a, 1, 1, 32, 1, 1, 0, nullptr, params, nullptr));
        } else {
            hipEvent_t e0, e1;
            CK(hipEventCreate(&e0));
            CK(hipEventCreate(&e1));
            CK(hipExtModuleLaunchKernel(f, (uint32_t)a * 32, 1, 1, 32, 1, 1, 0, nullptr, params, nullptr, e0, e1, 0));
            CK(hipEventSynchronize(e1));
            float ms = -1.0f;
            CK(hipEventElapsedTime(&ms, e0, e1));
            if (!(ms >= 0.0f)) { std::fprintf(stderr, "bad event time %f\n", ms); return 4; }
        }
    } else if (mode == "mod_mmq") {
        const long wb = a * (b / 256) * 144, xb = c * (b / 32) * 36;
        if ((long)in.size() != wb + xb) return 3;
        out_bytes = (size_t)a * c * 4;
        CK(hipMalloc(&dout, out_bytes));
        CK(hipModuleGetFunction(&f, mod, "mul_mat_vec_q4_K_q8_1"));
        void *vy = (char *)din + wb;
        int ncols_x = (int)b, nrows_x = (int)a, ncols_y = (int)b, nrows_y = (int)c;
        void *params[] = {&din, &vy, &dout, &ncols_x, &nrows_x, &ncols_y, &nrows_y};
        CK(hipModuleLaunchKernel(f, 64, 1, 1, 256, 1, 1, 0, nullptr, params, nullptr));
    } else if (mode == "mod_scale") {
        if ((long)in.size() != a * 4) return 3;
        out_bytes = (size_t)a * 4;
        dout = din;
        CK(hipModuleGetFunction(&f, mod, "scale_f32"));
        float s = 3.0f;
        int n = (int)a;
        void *params[] = {&din, &s, &n};
        CK(hipModuleLaunchKernel(f, (unsigned)((a + 255) / 256), 1, 1, 256, 1, 1, 0, nullptr, params, nullptr));
    } else {
        return 2;
    }
    CK(hipGetLastError());
    CK(hipDeviceSynchronize());
    std::vector<char> out(out_bytes);
    CK(hipMemcpy(out.data(), dout, out_bytes, hipMemcpyDeviceToHost));
    write_file(argv[4], out.data(), out_bytes);
    std::printf("module_probe %s ok\n", mode.c_str());
    return 0;
}
