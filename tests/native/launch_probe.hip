// launch_probe.hip — TEST HELPER for tests/test_gpu_preload.py, not part of
// the library.  A stand-alone HIP program whose kernels carry the names the
// launch table routes (ggml-style dequantize_block_q4_K<__half>, a reference
// style mul_mat_vec_q4_K_q8_1 and mul_mat_f16) plus one it does not know
// (scale_f32), each launched with <<<>>>, i.e. through hipLaunchKernel.  Under
// LD_PRELOAD=libvkflame_preload.so the routed launches run the library's
// kernels; the probe's own bodies only write a marker (0x7777 / -7.0), so the
// output shows which ran.  scale_f32 must always run its own body.
//
// usage: launch_probe <mode> <in.bin> <out.bin> <a> [<b> <c>]
//   dq4k  a = blocks:  in = a*144 bytes of Q4_K          out = a*256 fp16
//   mmq   a = N, b = K, c = M: in = N*(K/256)*144 bytes of Q4_K then M*(K/32)*36
//         bytes of Q8_1; out = M*N fp32
//   mmf16 a = N, b = K, c = M: in = N*K fp16 then M*K fp16; out = M*N fp32
//   scale a = n:       in = n fp32;  out = 3 * in
#include <hip/hip_fp16.h>
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

template <typename dst_t>
__global__ void dequantize_block_q4_K(const void *vx, dst_t *y) {
    // marker body: 256 outputs per block, one block per workgroup
    for (int i = threadIdx.x; i < 256; i += blockDim.x) {
        unsigned short m = 0x7777;
        y[(size_t)blockIdx.x * 256 + i] = *reinterpret_cast<dst_t *>(&m);
    }
}

__global__ void mul_mat_vec_q4_K_q8_1(const void *vx, const void *vy, float *dst, int ncols_x, int nrows_x,
                                      int ncols_y, int nrows_y) {
    const long n = (long)nrows_x * nrows_y;
    for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x)
        dst[i] = -7.0f;
}

__global__ void mul_mat_f16(const void *vx, const void *vy, float *dst, int ncols_x, int nrows_x, int ncols_y,
                            int nrows_y) {
    const long n = (long)nrows_x * nrows_y;
    for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x)
        dst[i] = -7.0f;
}

__global__ void scale_f32(float *x, float s, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) x[i] *= s;
}

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
    if (argc < 5) { std::fprintf(stderr, "usage: launch_probe mode in out a [b c]\n"); return 2; }
    const std::string mode = argv[1];
    std::vector<char> in = read_file(argv[2]);
    const long a = std::atol(argv[4]), b = argc > 5 ? std::atol(argv[5]) : 0, c = argc > 6 ? std::atol(argv[6]) : 0;
    void *din = nullptr, *dout = nullptr;
    CK(hipMalloc(&din, in.size() + 16));
    CK(hipMemcpy(din, in.data(), in.size(), hipMemcpyHostToDevice));
    size_t out_bytes = 0;
    if (mode == "dq4k") {
        if ((long)in.size() != a * 144) return 3;
        out_bytes = (size_t)a * 256 * 2;
        CK(hipMalloc(&dout, out_bytes));
        dequantize_block_q4_K<__half><<<(unsigned)a, 32>>>(din, (__half *)dout);
    } else if (mode == "mmq") {
        const long wb = a * (b / 256) * 144, xb = c * (b / 32) * 36;
        if ((long)in.size() != wb + xb) return 3;
        out_bytes = (size_t)a * c * 4;
        CK(hipMalloc(&dout, out_bytes));
        mul_mat_vec_q4_K_q8_1<<<64, 256>>>(din, (const char *)din + wb, (float *)dout, (int)b, (int)a, (int)b,
                                           (int)c);
    } else if (mode == "mmf16") {
        const long wb = a * b * 2, xb = c * b * 2;
        if ((long)in.size() != wb + xb) return 3;
        out_bytes = (size_t)a * c * 4;
        CK(hipMalloc(&dout, out_bytes));
        mul_mat_f16<<<64, 256>>>(din, (const char *)din + wb, (float *)dout, (int)b, (int)a, (int)b, (int)c);
    } else if (mode == "scale") {
        if ((long)in.size() != a * 4) return 3;
        out_bytes = (size_t)a * 4;
        dout = din;
        scale_f32<<<(unsigned)((a + 255) / 256), 256>>>((float *)din, 3.0f, (int)a);
    } else {
        return 2;
    }
    CK(hipGetLastError());
    CK(hipDeviceSynchronize());
    std::vector<char> out(out_bytes);
    CK(hipMemcpy(out.data(), dout, out_bytes, hipMemcpyDeviceToHost));
    write_file(argv[3], out.data(), out_bytes);
    std::printf("launch_probe %s ok\n", mode.c_str());
    return 0;
}
