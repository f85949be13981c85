"""torch-tensor wrappers over the C ABI (for tests, smoke and the benchmark).

Each function checks that its tensors live on the GPU, calls exactly one
C-ABI entry point on torch's current stream and returns the output tensor.
There is no fallback: a missing library or a CPU tensor raises.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib as L
from ._lib import check, lib

BLOCK_BYTES = {L.Q4_0: 18, L.Q4_1: 20, L.Q8_0: 34, L.Q5_0: 22, L.Q4_K: 144, L.Q5_K: 176, L.Q6_K: 210, L.Q8_1: 36}
BLOCK_ELEMS = {L.Q4_0: 32, L.Q4_1: 32, L.Q8_0: 32, L.Q5_0: 32, L.Q4_K: 256, L.Q5_K: 256, L.Q6_K: 256, L.Q8_1: 32}


def _stream(stream=None) -> ctypes.c_void_p:
    s = stream if stream is not None else torch.cuda.current_stream()
    return ctypes.c_void_p(s.cuda_stream)


def _p(t: torch.Tensor | None) -> ctypes.c_void_p:
    if t is None:
        return ctypes.c_void_p(0)
    if not t.is_cuda:
        raise L.VkflameError("vkflame_amd ops take GPU tensors only")
    return ctypes.c_void_p(t.data_ptr())


def dequant(blocks: torch.Tensor, qtype: int, out_dtype=torch.float32, n_blocks: int | None = None) -> torch.Tensor:
    """Dequantise whole blocks (uint8 tensor) -> flat fp32 / fp16 tensor."""
    nb = blocks.numel() // BLOCK_BYTES[qtype] if n_blocks is None else n_blocks
    out = torch.empty(nb * BLOCK_ELEMS[qtype], dtype=out_dtype, device=blocks.device)
    code = L.DTYPE_FP16 if out_dtype == torch.float16 else L.DTYPE_FP32
    check(lib().vkflame_dispatch_dequant(_p(blocks), _p(out), nb, qtype, code, _stream()), "dequant")
    return out


def quantize_q8_1(x: torch.Tensor) -> torch.Tensor:
    """fp32 [M, K] -> uint8 [M, K/32*36] Q8_1 blocks."""
    assert x.dtype == torch.float32 and x.dim() == 2
    M, K = x.shape
    out = torch.empty((M, K // 32 * 36), dtype=torch.uint8, device=x.device)
    check(lib().vkflame_quantize_q8_1(_p(x), _p(out), M, K, x.stride(0), _stream()), "quantize_q8_1")
    return out


def gemm_q(w: torch.Tensor, qtype: int, x: torch.Tensor, N: int, K: int, M: int | None = None,
           out: torch.Tensor | None = None, workspace: bool = True) -> torch.Tensor:
    """y[M, N] fp32 = x[M, K] @ deq(w)[N, K]^T.  x: fp16 / fp32 [M, K] or
    uint8 Q8_1 rows [M, K/32*36].  The routes that take a workspace get a
    torch one (vkflame_dispatch_gemm_q_ws): Q8_1 activations at M > 16 for
    their one-time fp16 decode, and the long-K matrix-core GEMV (Q4_K, Q4_0,
    Q4_1 at 2 <= M <= 16, Q8_0 at 9 <= M <= 16) for its K-slice partials;
    workspace=False runs their no-workspace forms (activation tiles decoded
    per GEMM tile, K slices one launch after another)."""
    if x.dtype == torch.float16:
        xd, ldx = L.DTYPE_FP16, x.stride(0)
    elif x.dtype == torch.float32:
        xd, ldx = L.DTYPE_FP32, x.stride(0)
    elif x.dtype == torch.uint8:
        xd, ldx = L.DTYPE_Q8_1, x.stride(0)
    else:
        raise TypeError(x.dtype)
    M = x.shape[0] if M is None else M
    y = torch.empty((M, N), dtype=torch.float32, device=x.device) if out is None else out
    row_bytes = w.stride(0) if w.dim() == 2 else 0
    nws = lib().vkflame_gemm_q_workspace_bytes(qtype, xd, M, N, K) if workspace else 0
    ws = torch.empty(nws, dtype=torch.uint8, device=x.device) if nws else None
    check(lib().vkflame_dispatch_gemm_q_ws(_p(w), qtype, row_bytes, _p(x), xd, ldx, _p(y), y.stride(0), M, N, K,
                                           _p(ws), nws, _stream()), "gemm_q")
    return y


def q6k_q81_partials(w: torch.Tensor, xq: torch.Tensor, M: int, N: int, K: int) -> torch.Tensor:
    P = torch.empty((M, N, K // 32), dtype=torch.int32, device=w.device)
    check(lib().vkflame_q6_k_q8_1_partials(_p(w), _p(xq), _p(P), M, N, K, _stream()), "q6k_q81_partials")
    return P


def q8_0_q81_partials(w: torch.Tensor, xq: torch.Tensor, M: int, N: int, K: int) -> torch.Tensor:
    """Exact int32 block dots of Q8_0 weights x Q8_1 activations, [M, N, K/32]."""
    P = torch.empty((M, N, K // 32), dtype=torch.int32, device=w.device)
    check(lib().vkflame_q8_0_q8_1_partials(_p(w), _p(xq), _p(P), M, N, K, _stream()), "q8_0_q81_partials")
    return P


def quantize_rows_i8(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """fp16 / fp32 [M, K] -> (int8 [M, K], fp32 scale [M]): symmetric per-row
    quantisation (vkflame_quantize_rows_i8)."""
    assert x.dim() == 2 and x.dtype in (torch.float16, torch.float32) and x.stride(1) == 1
    M, K = x.shape
    q = torch.empty((M, K), dtype=torch.int8, device=x.device)
    scale = torch.empty(M, dtype=torch.float32, device=x.device)
    xd = L.DTYPE_FP16 if x.dtype == torch.float16 else L.DTYPE_FP32
    check(lib().vkflame_quantize_rows_i8(_p(x), xd, M, K, x.stride(0), _p(q), _p(scale), _stream()),
          "quantize_rows_i8")
    return q, scale


def stream_read(src: torch.Tensor, sink: torch.Tensor) -> None:
    """Read all of src once (the HBM read-bandwidth reference); sink: a
    device int32 tensor the kernel may write one word of."""
    check(lib().vkflame_stream_read(_p(src), src.numel() * src.element_size(), _p(sink), _stream()), "stream_read")


def linear(A, B, M, N, K, dtype_code, transA=0, transB=1, act=0, C=None, alpha=None, beta=None, out=None):
    """vkflame_dispatch_linear (row-major D[M,N] = act(alpha op(A) op(B) + beta C)).
    DTYPE_INT8 is the reference's int8 linear: fp16 A quantised by
    act_scale = alpha, int8 B, C = per-channel w_scale (fp32 [N]), fp16 D.
    DTYPE_INT8_INT32OUT: int8 A and B, exact int32 D, integer alpha / beta."""
    if out is None:
        odt = {L.DTYPE_FP16: torch.float16, L.DTYPE_FP16_FP32OUT: torch.float32, L.DTYPE_INT8: torch.float16,
               L.DTYPE_INT8_INT32OUT: torch.int32, L.DTYPE_FP32: torch.float32}[dtype_code]
        out = torch.empty((M, N), dtype=odt, device=A.device)
    if dtype_code == L.DTYPE_INT8_INT32OUT:
        al = ctypes.c_int32(1 if alpha is None else int(alpha))
        be = ctypes.c_int32(0 if beta is None else int(beta))
    else:
        al = ctypes.c_float(1.0 if alpha is None else float(alpha))
        be = ctypes.c_float(0.0 if beta is None else float(beta))
    check(lib().vkflame_dispatch_linear(_p(A), _p(B), _p(C), _p(out), M, N, K, dtype_code, transA, transB, act,
                                        ctypes.byref(al), ctypes.byref(be), _stream()), "dispatch_linear")
    return out


def linear_int8(A, a_scale, W, w_scale, bias=None, out_dtype=torch.float16, act=0, out=None):
    M, K = A.shape
    N = W.shape[0]
    if out is None:
        out = torch.empty((M, N), dtype=out_dtype, device=A.device)
    bd = L.DTYPE_FP32 if (bias is not None and bias.dtype == torch.float32) else L.DTYPE_FP16
    od = L.DTYPE_FP32 if out.dtype == torch.float32 else L.DTYPE_FP16
    check(lib().vkflame_dispatch_linear_int8(_p(A), _p(a_scale), _p(W), _p(w_scale), _p(bias), bd, _p(out), od,
                                             M, N, K, act, _stream()), "linear_int8")
    return out
