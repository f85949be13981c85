"""ctypes binding of libvkflame_amd.so (the C ABI in include/vkflame_amd.h).

The library is the product; this module only declares argument types so the
tests, the smoke check and the benchmark can call it.  Loading fails loudly
when the library has not been built: there is no Python or CPU fallback for
any entry point.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libvkflame_amd.so")
PRELOAD_PATH = os.path.join(HERE, "libvkflame_preload.so")

# codes (include/vkflame_amd.h)
DTYPE_FP32, DTYPE_FP16, DTYPE_INT8, DTYPE_BF16, DTYPE_FP16_FP32OUT = 0, 1, 2, 3, 4
DTYPE_INT32, DTYPE_Q8_1, DTYPE_INT8_INT32OUT = 10, 11, 12
Q4_0, Q4_1, Q8_0, Q5_0, Q4_K, Q5_K, Q6_K, Q8_1 = range(8)
ACT_NONE, ACT_SILU, ACT_RELU, ACT_GELU_ERF = range(4)
LAUNCH_NONE, LAUNCH_DEQUANT, LAUNCH_MUL_MAT_Q, LAUNCH_MUL_MAT_F16 = range(4)

P = ctypes.c_void_p
I = ctypes.c_int
U64 = ctypes.c_uint64
I64 = ctypes.c_int64


class LaunchPlan(ctypes.Structure):
    _fields_ = [("kind", I), ("quant_type", I), ("out_dtype", I), ("pad", I),
                ("src", P), ("src1", P), ("dst", P), ("n_blocks", U64),
                ("M", I), ("N", I), ("K", I), ("pad2", I)]


class VkflameError(RuntimeError):
    pass


_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise VkflameError(f"{LIB_PATH} is not built; run `python -m vkflame_amd.build`")
    L = ctypes.CDLL(LIB_PATH)
    L.vkflame_version.restype = ctypes.c_char_p
    L.vkflame_version.argtypes = []
    L.vkflame_init.argtypes = []
    L.vkflame_block_bytes.argtypes = [I]
    L.vkflame_block_elems.argtypes = [I]
    L.vkflame_dispatch_dequant.argtypes = [P, P, U64, I, I, P]
    L.vkflame_quantize_q8_1.argtypes = [P, P, I, I, I64, P]
    L.vkflame_dispatch_gemm_q.argtypes = [P, I, U64, P, I, I64, P, I64, I, I, I, P]
    L.vkflame_dispatch_gemm_q_ws.argtypes = [P, I, U64, P, I, I64, P, I64, I, I, I, P, ctypes.c_size_t, P]
    L.vkflame_gemm_q_workspace_bytes.argtypes = [I, I, I, I, I]
    L.vkflame_gemm_q_workspace_bytes.restype = ctypes.c_size_t
    L.vkflame_dispatch_gemm_q_noalloc.argtypes = [P, I, U64, P, I, I64, P, I64, I, I, I, P]
    L.vkflame_noalloc_scratch_bytes.argtypes = []
    L.vkflame_noalloc_scratch_bytes.restype = ctypes.c_size_t
    L.vkflame_q6_k_q8_1_partials.argtypes = [P, P, P, I, I, I, P]
    L.vkflame_q8_0_q8_1_partials.argtypes = [P, P, P, I, I, I, P]
    L.vkflame_stream_read.argtypes = [P, U64, P, P]
    L.vkflame_quantize_rows_i8.argtypes = [P, I, I, I, I64, P, P, P]
    L.vkflame_dispatch_linear.argtypes = [P, P, P, P, I, I, I, I, I, I, I, P, P, P]
    L.vkflame_dispatch_linear_int8.argtypes = [P, P, P, P, P, I, P, I, I, I, I, I, P]
    L.vkflame_resolve_launch.argtypes = [ctypes.c_char_p, ctypes.c_uint, ctypes.c_uint, ctypes.c_uint,
                                         ctypes.c_uint, ctypes.c_uint, ctypes.c_uint,
                                         ctypes.POINTER(P), ctypes.POINTER(LaunchPlan)]
    L.vkflame_execute_launch.argtypes = [ctypes.POINTER(LaunchPlan), P]
    for f in ("vkflame_dispatch_dequant", "vkflame_quantize_q8_1", "vkflame_dispatch_gemm_q",
              "vkflame_dispatch_gemm_q_ws", "vkflame_dispatch_gemm_q_noalloc",
              "vkflame_q6_k_q8_1_partials", "vkflame_q8_0_q8_1_partials", "vkflame_dispatch_linear", "vkflame_dispatch_linear_int8",
              "vkflame_stream_read", "vkflame_quantize_rows_i8",
              "vkflame_resolve_launch", "vkflame_execute_launch", "vkflame_init",
              "vkflame_block_bytes", "vkflame_block_elems"):
        getattr(L, f).restype = I
    _lib = L
    return L


def check(rc: int, what: str = "vkflame call") -> None:
    if rc != 0:
        raise VkflameError(f"{what} failed with status {rc}")


def resolve_launch(name: str, grid, block, args: list) -> LaunchPlan:
    """Run the kernel-name table on a synthetic launch.  ``args`` holds ctypes
    objects (c_void_p, c_int32, c_int64 ...); their addresses form the HIP
    ``void** args`` array."""
    arr = (P * len(args))(*[ctypes.cast(ctypes.pointer(a), P) for a in args])
    plan = LaunchPlan()
    lib().vkflame_resolve_launch(name.encode(), grid[0], grid[1], grid[2], block[0], block[1], block[2],
                                 arr, ctypes.byref(plan))
    return plan
