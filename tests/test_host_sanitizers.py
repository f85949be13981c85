"""CPU: the library's host code and the oracle built with AddressSanitizer and
UndefinedBehaviorSanitizer (g++ / gcc, no GPU code) and run through
tests/native/host_sanity.cpp: the kernel-name table, the C-ABI argument
checks, the hipBLAS / hipBLASLt handle and descriptor handling and the
oracle's dequantisers, quantisers and integer GEMM, with every sanitizer
report fatal."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HOST = ["vkf_runtime", "vkf_dispatch", "vkf_launch_table", "vkf_vendor", "vkf_hipblas", "vkf_hipblaslt"]
SAN = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer", "-g", "-O1"]


@pytest.fixture(scope="module")
def sanity_binary(tmp_path_factory):
    if not shutil.which("g++") or not os.path.exists(os.path.join(ROCM, "lib", "libamdhip64.so")):
        pytest.skip("needs g++ and the ROCm host libraries")
    out = tmp_path_factory.mktemp("san")
    objs = []
    cxx = ["g++", "-std=c++17", "-fPIC", "-D__HIP_PLATFORM_AMD__", f"-I{ROCM}/include", *SAN]
    for h in HOST:
        o = str(out / (h + ".o"))
        subprocess.run([*cxx, "-c", os.path.join(ROOT, "vkflame_amd", "csrc", "host", h + ".cpp"), "-o", o],
                       check=True, capture_output=True)
        objs.append(o)
    o = str(out / "vkf_oracle.o")
    subprocess.run(["gcc", "-std=c11", "-fPIC", "-ffp-contract=off", *SAN, "-c",
                    os.path.join(ROOT, "oracle", "vkf_oracle.c"), "-o", o], check=True, capture_output=True)
    objs.append(o)
    # the library's no-allocation entry point and code-object table are
    # device-side or generated; stand-ins that carry no device code
    stub = out / "stubs.cpp"
    stub.write_text(
        '#include <cstddef>\n#include <cstdint>\n#include "vkflame_amd.h"\n'
        'struct VkfCodeObject { const char *name; const unsigned char *begin; const unsigned char *end; };\n'
        'extern "C" const VkfCodeObject vkf_code_objects[1] = {{"none", nullptr, nullptr}};\n'
        'extern "C" const int vkf_n_code_objects = 0;\n'
        'extern "C" size_t vkflame_noalloc_scratch_bytes(void) { return VKFLAME_NOALLOC_SCRATCH_BYTES; }\n'
        'extern "C" int vkflame_dispatch_gemm_q_noalloc(const void *w, int qt, uint64_t rb, const void *x, int xd,\n'
        '    int64_t ldx, float *y, int64_t ldy, int M, int N, int K, void *s) {\n'
        '  size_t need = vkflame_gemm_q_workspace_bytes(qt, xd, M, N, K);\n'
        '  if (M > 16 && need > VKFLAME_NOALLOC_SCRATCH_BYTES) return 1;\n'
        '  return vkflame_dispatch_gemm_q_ws(w, qt, rb, x, xd, ldx, y, ldy, M, N, K, nullptr, 0, s); }\n')
    so = str(out / "stubs.o")
    subprocess.run([*cxx, f"-I{ROOT}/include", "-c", str(stub), "-o", so], check=True, capture_output=True)
    objs.append(so)
    exe = str(out / "host_sanity")
    r = subprocess.run([*cxx, os.path.join(ROOT, "tests", "native", "host_sanity.cpp"), *objs, "-o", exe,
                        f"-L{ROCM}/lib", "-lamdhip64", "-ldl", "-lm", f"-Wl,-rpath,{ROCM}/lib"],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-3000:]
    return exe


def test_host_code_and_oracle_under_asan_ubsan(sanity_binary):
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=0", UBSAN_OPTIONS="print_stacktrace=1",
               HIP_VISIBLE_DEVICES="")
    r = subprocess.run([sanity_binary], capture_output=True, text=True, timeout=300, env=env)
    assert r.returncode == 0 and "host_sanity ok" in r.stdout, (r.stdout + r.stderr)[-4000:]
