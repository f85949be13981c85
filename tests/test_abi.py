"""CPU: the C-ABI library loads, exports every symbol the public header
declares plus the hipBLAS / hipBLASLt entry points, and its host-side logic
(kernel-name table, BLAS descriptors, argument checks) behaves as specified.
No call here reaches a GPU: every checked path returns before a launch."""
import ctypes
import os
import re
import subprocess

import pytest

from vkflame_amd import _lib as VL
from vkflame_amd import lib
import blas_abi as B

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

HIPBLAS = ["hipblasCreate", "hipblasDestroy", "hipblasSetStream", "hipblasGetStream", "hipblasSetPointerMode",
           "hipblasGetPointerMode", "hipblasGemmEx", "hipblasGemmBatchedEx", "hipblasGemmStridedBatchedEx",
           "hipblasHgemm", "hipblasHgemmBatched", "hipblasHgemmStridedBatched", "hipblasSgemm",
           "hipblasSgemmBatched", "hipblasSgemmStridedBatched"]
HIPBLASLT = ["hipblasLtCreate", "hipblasLtDestroy", "hipblasLtMatrixLayoutCreate", "hipblasLtMatrixLayoutDestroy",
             "hipblasLtMatrixLayoutSetAttribute", "hipblasLtMatrixLayoutGetAttribute", "hipblasLtMatmulDescCreate",
             "hipblasLtMatmulDescDestroy", "hipblasLtMatmulDescSetAttribute", "hipblasLtMatmulDescGetAttribute",
             "hipblasLtMatmulPreferenceCreate", "hipblasLtMatmulPreferenceDestroy",
             "hipblasLtMatmulPreferenceSetAttribute", "hipblasLtMatmulAlgoGetHeuristic", "hipblasLtMatmul"]


def _declared():
    txt = open(os.path.join(ROOT, "include", "vkflame_amd.h")).read()
    return sorted(set(re.findall(r"\b(vkflame_\w+)\s*\(", txt)))


def _declared_blas():
    txt = open(os.path.join(ROOT, "include", "vkflame_amd_blas.h")).read()
    return sorted(set(re.findall(r"\bX\((hipblas\w+),", txt)))


def test_blas_header_lists_the_exports():
    assert _declared_blas() == sorted(HIPBLAS + HIPBLASLT)


def _exported(path):
    out = subprocess.run(["nm", "-D", "--defined-only", path], capture_output=True, text=True, check=True).stdout
    return {l.split()[-1] for l in out.splitlines() if " T " in l}


def test_header_symbols_exported():
    decl = _declared()
    assert len(decl) >= 10
    exp = _exported(VL.LIB_PATH)
    missing = [s for s in decl + HIPBLAS + HIPBLASLT if s not in exp]
    assert not missing, missing
    L = lib()
    for s in decl + HIPBLAS + HIPBLASLT:
        assert getattr(L, s) is not None


def test_library_does_not_interpose_hip_runtime():
    exp = _exported(VL.LIB_PATH)
    assert not any(s.startswith("hipLaunch") or s.startswith("hipMalloc") for s in exp)


def test_preload_exports_only_the_launch_entry_points():
    assert _exported(VL.PRELOAD_PATH) == {"hipLaunchKernel", "hipModuleLaunchKernel", "hipExtModuleLaunchKernel",
                                          "hipModuleGetFunction"}


def test_version_and_block_geometry():
    L = lib()
    assert b"gfx950" in L.vkflame_version()
    assert [L.vkflame_block_bytes(q) for q in range(8)] == [18, 20, 34, 22, 144, 176, 210, 36]
    assert [L.vkflame_block_elems(q) for q in range(8)] == [32, 32, 32, 32, 256, 256, 256, 32]
    assert L.vkflame_block_bytes(8) == -1 and L.vkflame_block_elems(-1) == -1


# ---------------------------------------------------------------------------
# kernel-name table (shim/hip_runtime_shim.cpp:896-952, 1096-1188)
# ---------------------------------------------------------------------------

def P(v):
    return ctypes.c_void_p(v)


def _dq(name, grid=(5, 1, 1), block=(32, 1, 1), nb=7, i64=False):
    a2 = ctypes.c_int64(nb) if i64 else ctypes.c_int32(nb)
    return VL.resolve_launch(name, grid, block, [P(0x1000), P(0x2000), a2])


@pytest.mark.parametrize("name,qt", [
    ("_Z21dequantize_block_q4_0PKvPfi", 0), ("dequantize_block_q4K_0", 0), ("dequantize_block_q4_1<float>", 1),
    ("dequantize_block_q5_0", 3), ("dequantize_block_q5K_0", 3)])
def test_table_dequant_nb32_rule(name, qt):
    p = _dq(name, nb=123)
    assert (p.kind, p.quant_type, p.n_blocks, p.src, p.dst) == (VL.LAUNCH_DEQUANT, qt, 123, 0x1000, 0x2000)


def test_table_q8_0_nb_rule():
    assert _dq("dequantize_block_q8_0", block=(32, 1, 1), nb=77).n_blocks == 77
    assert _dq("dequantize_block_q8_0", block=(256, 1, 1), nb=32 * 1000, i64=True).n_blocks == 1000


@pytest.mark.parametrize("name,qt", [("dequantize_block_q4_K", 4), ("dequantize_block_q4K", 4),
                                     ("dequantize_block_q5_K", 5), ("dequantize_block_q5K", 5),
                                     ("dequantize_block_q6_K", 6), ("dequantize_block_q6K", 6)])
def test_table_k_quants_take_nb_from_grid(name, qt):
    p = _dq(name, grid=(4242, 1, 1))
    assert (p.kind, p.quant_type, p.n_blocks) == (VL.LAUNCH_DEQUANT, qt, 4242)


def test_table_output_dtype_from_name():
    assert _dq("_Z21dequantize_block_q4_KI6__halfEvPKvPT_").out_dtype == VL.DTYPE_FP16
    assert _dq("_Z21dequantize_block_q4_KIDF16_EvPKvPT_").out_dtype == VL.DTYPE_FP16
    assert _dq("_Z21dequantize_block_q4_KIfEvPKvPT_").out_dtype == VL.DTYPE_FP32


def test_table_mul_mat_before_dequant_substrings():
    args = [P(0x10), P(0x20), P(0x30), ctypes.c_int32(4096), ctypes.c_int32(11008), ctypes.c_int32(4096),
            ctypes.c_int32(7)]
    p = VL.resolve_launch("mul_mat_q4_0_q8_1", (1, 1, 1), (64, 1, 1), args)
    assert (p.kind, p.quant_type, p.K, p.N, p.M) == (VL.LAUNCH_MUL_MAT_Q, 0, 4096, 11008, 7)
    assert (p.src, p.src1, p.dst) == (0x10, 0x20, 0x30)
    for nm, qt in [("mul_mat_q4_1_q8_1", 1), ("mul_mat_vec_q8_0_q8_1", 2), ("mul_mat_q5_0_q8_1", 3),
                   ("mul_mat_q4_K_q8_1", 4), ("mul_mat_q5_K_q8_1", 5), ("mul_mat_q6_K_q8_1", 6)]:
        assert VL.resolve_launch(nm, (1, 1, 1), (64, 1, 1), args).quant_type == qt
    pf = VL.resolve_launch("mul_mat_f16", (1, 1, 1), (64, 1, 1), args)
    assert (pf.kind, pf.M, pf.N, pf.K) == (VL.LAUNCH_MUL_MAT_F16, 7, 11008, 4096)


def test_table_falls_through():
    args = [P(1), P(2), ctypes.c_int32(3), ctypes.c_int32(4), ctypes.c_int32(5), ctypes.c_int32(6),
            ctypes.c_int32(7)]
    for nm in ["mul_mat_iq2_xxs_q8_1", "mul_mat_iq4_nl", "get_rows_q4_0", "cpy_f32_q8_0", "softmax_f32",
               "some_other_kernel", "mul_mat_bf16"]:
        assert VL.resolve_launch(nm, (1, 1, 1), (64, 1, 1), args).kind == VL.LAUNCH_NONE, nm
    bad = [P(1), P(2), P(3), ctypes.c_int32(0), ctypes.c_int32(5), ctypes.c_int32(6), ctypes.c_int32(7)]
    assert VL.resolve_launch("mul_mat_q4_0_q8_1", (1, 1, 1), (64, 1, 1), bad).kind == VL.LAUNCH_NONE


def test_table_mul_mat_without_q8_1_falls_through():
    """Quantised mul_mat kernels that do not take Q8_1 activations (ggml's
    dequantize_mul_mat_vec: 5 arguments, fp32 y, the weight type in its
    template arguments) keep their own kernel: the table does not read a
    7-argument layout they do not have."""
    args = [P(1), P(2), P(3), ctypes.c_int32(4096), ctypes.c_int32(4096)]
    for nm in ["_Z22dequantize_mul_mat_vecILi32ELi2EXadL_ZL15dequantize_q4_0PKvllR6float2EEEvS1_PKfPfii",
               "dequantize_mul_mat_vec_q4_K", "mul_mat_q4_0", "mul_mat_vec_q6_K_f32"]:
        assert VL.resolve_launch(nm, (1, 1, 1), (64, 1, 1), args).kind == VL.LAUNCH_NONE, nm


# ---------------------------------------------------------------------------
# argument checks that return before any launch
# ---------------------------------------------------------------------------

def test_c_abi_rejects_bad_arguments():
    L = lib()
    s = None
    assert L.vkflame_dispatch_dequant(None, None, 1, 9, 0, s) == 1
    assert L.vkflame_dispatch_dequant(P(16), P(32), 1, 4, 5, s) == 1         # bad out dtype
    assert L.vkflame_dispatch_dequant(P(18), P(32), 1, 4, 0, s) == 1         # Q4_K source not 4-aligned
    assert L.vkflame_dispatch_dequant(P(16), P(40), 1, 0, 0, s) == 1         # dst not 16-aligned
    assert L.vkflame_dispatch_dequant(None, None, 0, 0, 0, s) == 0           # empty: no-op
    assert L.vkflame_quantize_q8_1(P(16), P(16), 4, 48, 0, s) == 1            # K % 32
    assert L.vkflame_quantize_q8_1(P(16), P(16), 4, 64, 32, s) == 1           # ldx < K
    assert L.vkflame_dispatch_gemm_q(P(16), 4, 0, P(16), 1, 0, P(16), 0, 1, 8, 300, s) == 1   # K % 256
    assert L.vkflame_dispatch_gemm_q(P(16), 7, 0, P(16), 1, 0, P(16), 0, 1, 8, 256, s) == 1   # Q8_1 weights
    assert L.vkflame_dispatch_gemm_q(P(16), 4, 0, P(16), 9, 0, P(16), 0, 1, 8, 256, s) == 1   # x dtype
    assert L.vkflame_dispatch_gemm_q(P(16), 4, 100, P(16), 1, 0, P(16), 0, 1, 8, 256, s) == 1  # row_bytes < packed
    assert L.vkflame_dispatch_gemm_q(P(16), 4, 0, P(18), 1, 0, P(16), 0, 1, 8, 256, s) == 1   # x misaligned
    assert L.vkflame_dispatch_gemm_q(P(16), 4, 0, P(16), 1, 0, P(16), 0, 0, 8, 256, s) == 0   # M = 0: no-op
    assert L.vkflame_dispatch_gemm_q(P(16), 4, 0, P(16), 0, 0, P(16), 0, 32, 8, 256, s) == 801  # fp32 prefill
    assert L.vkflame_dispatch_linear(P(16), P(16), None, P(16), 4, 4, 4, 1, 0, 0, 7, None, None, s) == 1
    assert L.vkflame_dispatch_linear(P(16), P(16), None, P(16), 4, 4, 4, 3, 0, 0, 0, None, None, s) == 801  # bf16
    half = ctypes.c_float(0.5)
    assert L.vkflame_dispatch_linear(P(16), P(16), None, P(16), 4, 4, 4, 0, 0, 0, 0, None, ctypes.byref(half),
                                     s) == 1  # fp32 with beta != 0 and no C
    assert L.vkflame_dispatch_linear(P(16), P(16), None, P(16), 4, 4, 4, 12, 0, 1, 1, None, None, s) == 1
    # the reference int8 contract: act_scale (alpha) must be finite and > 0, beta 0
    for bad_scale in (0.0, -1.0, float("inf"), float("nan")):
        f = ctypes.c_float(bad_scale)
        assert L.vkflame_dispatch_linear(P(16), P(16), None, P(16), 4, 4, 4, 2, 0, 1, 0, ctypes.byref(f), None,
                                         s) == 1
    one, half = ctypes.c_float(1.0), ctypes.c_float(0.5)
    assert L.vkflame_dispatch_linear(P(16), P(16), None, P(16), 4, 4, 4, 2, 0, 1, 0, ctypes.byref(one),
                                     ctypes.byref(half), s) == 1
    assert L.vkflame_dispatch_linear_int8(P(16), None, P(16), None, None, 1, P(16), 2, 4, 4, 4, 0, s) == 1
    assert L.vkflame_q6_k_q8_1_partials(P(16), P(16), P(16), 1, 1, 100, s) == 1
    assert L.vkflame_stream_read(P(16), 17, P(16), s) == 1                    # bytes % 16
    assert L.vkflame_stream_read(P(8), 32, P(16), s) == 1                     # src not 16-aligned
    assert L.vkflame_stream_read(P(16), 32, None, s) == 1                     # no sink
    assert L.vkflame_stream_read(None, 0, None, s) == 0                       # empty: no-op
    ws = L.vkflame_gemm_q_workspace_bytes
    q4_0, q4k, q6k = 0, 4, 6  # VKF_DEQUANT_*
    assert ws(q6k, VL.DTYPE_Q8_1, 512, 4096, 5120) == 512 * 5120 * 2
    assert ws(q6k, VL.DTYPE_Q8_1, 16, 4096, 5120) == 0 and ws(q6k, VL.DTYPE_FP16, 512, 4096, 5120) == 0
    assert ws(q6k, VL.DTYPE_Q8_1, 64, 4096, 100) == 0
    # K-slice partials of the matrix-core GEMV: S = ceil(K/256 / 20) (Q4_K), ceil(K/256 / 16) (Q4_0 / Q4_1)
    assert ws(q4k, VL.DTYPE_FP16, 8, 5120, 13824) == 3 * 8 * 5120 * 4
    assert ws(q4k, VL.DTYPE_FP16, 16, 5120, 5376) == 2 * 16 * 5120 * 4
    assert ws(q4_0, VL.DTYPE_FP16, 4, 4096, 11008) == 3 * 4 * 4096 * 4
    assert ws(q4_0, VL.DTYPE_FP16, 16, 4096, 4608) == 2 * 16 * 4096 * 4
    assert ws(q4k, VL.DTYPE_FP16, 8, 13824, 5120) == 0      # one workgroup's waves hold K = 5120
    assert ws(q4_0, VL.DTYPE_FP16, 4, 11008, 4096) == 0
    # one LDS-image launch holds 33 (Q4_K) / 35 (Q4_0) groups of 8 rows, 16 / 17 of 16 rows
    assert ws(q4k, VL.DTYPE_FP16, 8, 5120, 256 * 33) == 0 and ws(q4k, VL.DTYPE_FP16, 8, 5120, 256 * 34) > 0
    assert ws(q4_0, VL.DTYPE_FP16, 8, 4096, 256 * 35) == 0 and ws(q4_0, VL.DTYPE_FP16, 8, 4096, 256 * 36) > 0
    assert ws(q4_0, VL.DTYPE_FP16, 16, 4096, 256 * 17) == 0
    assert ws(q4k, VL.DTYPE_FP16, 1, 5120, 13824) == 0      # M = 1: the dot GEMV
    assert ws(q4k, VL.DTYPE_FP16, 17, 5120, 13824) == 0     # M > 16: the GEMM
    assert ws(q4k, VL.DTYPE_FP32, 8, 5120, 13824) == 0      # fp16 activations only
    assert ws(q6k, VL.DTYPE_FP16, 8, 5120, 13824) == 0
    assert ws(q4k, VL.DTYPE_FP16, 8, 5120, 256 * 161) == 0  # more than 8 slices
    assert ws(q4k, VL.DTYPE_FP16, 8, 5120, 256 * 160) == 8 * 8 * 5120 * 4
    q8_0 = 2  # VKF_DEQUANT_Q8_0
    assert ws(q8_0, VL.DTYPE_FP16, 16, 5120, 13824) == 3 * 16 * 5120 * 4  # Q8_0: 24-group slices at M > 8
    assert ws(q8_0, VL.DTYPE_FP16, 8, 5120, 13824) == 0 and ws(q8_0, VL.DTYPE_FP16, 16, 5120, 6144) == 0
    qws = L.vkflame_dispatch_gemm_q_ws
    assert qws(P(16), 4, 0, P(16), 1, 0, P(16), 0, 1, 8, 300, None, 0, s) == 1     # K % 256
    assert qws(P(16), 6, 0, P(18), 11, 0, P(16), 0, 64, 8, 256, P(16), 1 << 20, s) == 1  # Q8_1 x not 4-aligned
    assert qws(P(16), 6, 0, P(16), 11, 0, P(16), 0, 0, 8, 256, P(16), 1 << 20, s) == 0   # M = 0: no-op
    assert L.vkflame_execute_launch(ctypes.byref(VL.LaunchPlan()), s) == 1


# ---------------------------------------------------------------------------
# hipBLAS / hipBLASLt host objects
# ---------------------------------------------------------------------------

def test_hipblas_handles_and_errors():
    L = B.blas()
    h = ctypes.c_void_p()
    assert L.hipblasCreate(None) == B.ST_HANDLE_NULL
    assert L.hipblasCreate(ctypes.byref(h)) == 0
    assert L.hipblasSetStream(h, P(0x1234)) == 0
    st = ctypes.c_void_p()
    assert L.hipblasGetStream(h, ctypes.byref(st)) == 0 and st.value == 0x1234
    one = ctypes.c_float(1.0)
    # NULL handle, bad op, bad ld, unsupported type pair: all rejected before a launch
    args = (B.OP_T, B.OP_N, 8, 8, 8, ctypes.byref(one), P(16), B.R_16F, 8, P(16), B.R_16F, 8, ctypes.byref(one),
            P(16), B.R_32F, 8, B.COMPUTE_32F, B.GEMM_DEFAULT)
    assert L.hipblasGemmEx(None, *args) == B.ST_NOT_INIT
    assert L.hipblasGemmEx(h, 7, *args[1:]) == 10                                  # INVALID_ENUM
    bad_ld = list(args); bad_ld[8] = 4
    assert L.hipblasGemmEx(h, *bad_ld) == B.ST_INVALID_VALUE
    bf16 = list(args); bf16[7] = 14; bf16[10] = 14                                # HIP_R_16BF
    assert L.hipblasGemmEx(h, *bf16) == B.ST_NOT_SUPPORTED  # no vendor hipBLAS to forward to without a GPU
    empty = list(args); empty[2] = 0
    assert L.hipblasGemmEx(h, *empty) == B.ST_SUCCESS
    assert L.hipblasDestroy(h) == 0


def test_hipblaslt_descriptors_round_trip():
    L = B.blas()
    lay = B.layout(L, B.R_8I, 5120, 512, 5120)
    buf = ctypes.c_uint64()
    n = ctypes.c_size_t()
    assert L.hipblasLtMatrixLayoutGetAttribute(lay, B.LAYOUT_ROWS, ctypes.byref(buf), 8, ctypes.byref(n)) == 0
    assert buf.value == 5120 and n.value == 8
    ld = ctypes.c_int64(6000)
    assert L.hipblasLtMatrixLayoutSetAttribute(lay, B.LAYOUT_LD, ctypes.byref(ld), 8) == 0
    ld2 = ctypes.c_int64()
    assert L.hipblasLtMatrixLayoutGetAttribute(lay, B.LAYOUT_LD, ctypes.byref(ld2), 8, None) == 0 and ld2.value == 6000
    assert L.hipblasLtMatrixLayoutSetAttribute(lay, B.LAYOUT_LD, ctypes.byref(ld), 4) == B.ST_INVALID_VALUE
    t = ctypes.c_uint32()
    assert L.hipblasLtMatrixLayoutGetAttribute(lay, B.LAYOUT_TYPE, ctypes.byref(t), 4, None) == 0 and t.value == B.R_8I
    d = ctypes.c_void_p()
    assert L.hipblasLtMatmulDescCreate(ctypes.byref(d), B.COMPUTE_32I, B.R_32F) == 0
    assert B.set_desc(L, d, B.DESC_EPILOGUE, ctypes.c_uint32(B.EPI_GELU_BIAS)) == 0
    e = ctypes.c_uint32()
    assert L.hipblasLtMatmulDescGetAttribute(d, B.DESC_EPILOGUE, ctypes.byref(e), 4, None) == 0
    assert e.value == B.EPI_GELU_BIAS
    assert B.set_desc(L, d, B.DESC_BIAS_POINTER, P(0xABC0)) == 0
    bp = ctypes.c_void_p()
    assert L.hipblasLtMatmulDescGetAttribute(d, B.DESC_BIAS_POINTER, ctypes.byref(bp), 8, None) == 0
    assert bp.value == 0xABC0
    h = ctypes.c_void_p()
    assert L.hipblasLtCreate(ctypes.byref(h)) == 0
    pref = ctypes.c_void_p()
    assert L.hipblasLtMatmulPreferenceCreate(ctypes.byref(pref)) == 0
    ws = ctypes.c_uint64(1 << 20)
    assert L.hipblasLtMatmulPreferenceSetAttribute(pref, B.PREF_MAX_WORKSPACE, ctypes.byref(ws), 8) == 0
    res = (B.HeuristicResult * 2)()
    cnt = ctypes.c_int()
    assert L.hipblasLtMatmulAlgoGetHeuristic(h, d, lay, lay, lay, lay, pref, 2, res, ctypes.byref(cnt)) == 0
    assert cnt.value == 1 and res[0].state == 0 and res[0].workspaceSize == 0
    assert L.hipblasLtMatmulAlgoGetHeuristic(h, d, lay, lay, lay, lay, pref, 0, res, ctypes.byref(cnt)) == 3
    # shape mismatch and unsupported epilogue are rejected before any launch
    a = B.layout(L, B.R_8I, 64, 32, 64)
    b = B.layout(L, B.R_8I, 64, 16, 64)
    dd = B.layout(L, B.R_16F, 33, 16, 33)
    one = ctypes.c_float(1.0)
    assert B.set_desc(L, d, B.DESC_TRANSA, B.OP_T) == 0
    assert L.hipblasLtMatmul(h, d, ctypes.byref(one), P(16), a, P(16), b, ctypes.byref(one), P(16), dd, P(16), dd,
                             None, None, 0, None) == B.ST_INVALID_VALUE
    dd2 = B.layout(L, B.R_16F, 32, 16, 32)
    assert B.set_desc(L, d, B.DESC_EPILOGUE, ctypes.c_uint32(192)) == 0               # DGELU
    assert L.hipblasLtMatmul(h, d, ctypes.byref(one), P(16), a, P(16), b, ctypes.byref(one), P(16), dd2, P(16),
                             dd2, None, None, 0, None) == B.ST_NOT_SUPPORTED
    for x in (lay, a, b, dd, dd2):
        assert L.hipblasLtMatrixLayoutDestroy(x) == 0
    assert L.hipblasLtMatmulDescDestroy(d) == 0
    assert L.hipblasLtMatmulPreferenceDestroy(pref) == 0
    assert L.hipblasLtDestroy(h) == 0


def test_hipblaslt_int32_out_needs_integral_scalars():
    """int8 x int8 -> int32 scales by integers: a float alpha or beta that is
    not an exact int32 (0.5, 1.5, 2^31) is refused before any launch (without
    ROCm's hipBLASLt to forward to, as here); integral ones pass the check."""
    L = B.blas()
    h = ctypes.c_void_p()
    assert L.hipblasLtCreate(ctypes.byref(h)) == 0
    a = B.layout(L, B.R_8I, 64, 32, 64)
    b = B.layout(L, B.R_8I, 64, 16, 64)
    dd = B.layout(L, B.R_32I, 32, 16, 32)
    d = ctypes.c_void_p()
    assert L.hipblasLtMatmulDescCreate(ctypes.byref(d), B.COMPUTE_32I, B.R_32F) == 0
    assert B.set_desc(L, d, B.DESC_TRANSA, B.OP_T) == 0
    zero = ctypes.c_float(0.0)
    for bad in (0.5, 1.5, -2.25, 2.0 ** 31):
        al = ctypes.c_float(bad)
        assert L.hipblasLtMatmul(h, d, ctypes.byref(al), P(16), a, P(16), b, ctypes.byref(zero), P(16), dd, P(16),
                                 dd, None, None, 0, None) == B.ST_NOT_SUPPORTED, bad
        assert L.hipblasLtMatmul(h, d, ctypes.byref(zero), P(16), a, P(16), b, ctypes.byref(al), P(16), dd, P(16),
                                 dd, None, None, 0, None) == B.ST_NOT_SUPPORTED, bad
    for x in (a, b, dd):
        assert L.hipblasLtMatrixLayoutDestroy(x) == 0
    assert L.hipblasLtMatmulDescDestroy(d) == 0
    assert L.hipblasLtDestroy(h) == 0
