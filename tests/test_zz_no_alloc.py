"""GPU parity of vkflame_dispatch_gemm_q_noalloc (the entry point that
allocates nothing) against vkflame_dispatch_gemm_q, through the C ABI.

Both entry points run the same kernels on the same route (Q8_1 activations
at M > 16 decoded once to fp16 into a scratch buffer, then the fp16-activation
GEMM; the long-K matrix-core GEMV's K-slice partials); the no-allocation one
uses the library's fixed per-GPU scratch array instead of a stream-ordered
allocation, so the outputs agree bit for bit.
Two calls in a row, the second smaller, check that the second result does not
depend on what the first left in the shared array."""

import numpy as np
import pytest

import oracle as O
from _util import TOL_F32, bits_equal, first_mismatch, rel_err, seed_for, to_dev

pytestmark = pytest.mark.gpu


def _call(fn, w, qt, x, xd, y, M, N, K):
    from vkflame_amd import ops
    return fn(ops._p(w), qt, 0, ops._p(x), xd, x.stride(0), ops._p(y), y.stride(0), M, N, K, ops._stream())


def _case(dev, qt, M, N, K, seed, kind="q8_1"):
    import torch
    from vkflame_amd import _lib as L
    w = O.gen_weight(qt, N, K, seed)
    x = np.random.default_rng(seed + 1).normal(0, 1, (M, K)).astype(np.float32)
    if kind == "q8_1":
        xq = O.np_quantize_q8_1(x).reshape(M, -1)
        xdt, x64 = L.DTYPE_Q8_1, O.np_dequant(O.Q8_1, xq).reshape(M, K).astype(np.float64)
    else:
        xq = x.astype(np.float16)
        xdt, x64 = L.DTYPE_FP16, xq.astype(np.float64)
    wd, xd = to_dev(w, dev), to_dev(xq, dev)
    y_ref = torch.full((M, N), float("nan"), dtype=torch.float32, device=dev)
    y_na = torch.full((M, N), float("nan"), dtype=torch.float32, device=dev)
    lib = L.lib()
    L.check(_call(lib.vkflame_dispatch_gemm_q, wd, qt, xd, xdt, y_ref, M, N, K), "gemm_q")
    L.check(_call(lib.vkflame_dispatch_gemm_q_noalloc, wd, qt, xd, xdt, y_na, M, N, K), "gemm_q_noalloc")
    torch.cuda.synchronize()
    a, b = y_na.cpu().numpy(), y_ref.cpu().numpy()
    assert bits_equal(a, b), (O.QNAMES[qt], M, N, K, first_mismatch(a, b))
    rows = np.arange(0, N, max(1, N // 64))
    ref = O.ref_gemv(x64, O.np_dequant(qt, w[rows]).reshape(len(rows), K))
    assert rel_err(a[:, rows], ref) <= TOL_F32


def test_noalloc_matches_gemm_q_two_calls(dev):
    from vkflame_amd import _lib as L
    assert L.lib().vkflame_noalloc_scratch_bytes() == 16 << 20
    print("noalloc: Q6_K x Q8_1 512x1000x5120", flush=True)
    _case(dev, O.Q6_K, 512, 1000, 5120, seed_for(5, 200))
    print("noalloc: Q4_K x Q8_1 64x300x1024 (smaller, second call)", flush=True)
    _case(dev, O.Q4_K, 64, 300, 1024, seed_for(3, 200))


def test_noalloc_k_slice_gemv_two_calls(dev):
    """The long-K matrix-core GEMV keeps its K-slice partials in the array:
    two calls in a row, the second with fewer slices, rows and outputs."""
    from vkflame_amd import _lib as L
    assert L.lib().vkflame_gemm_q_workspace_bytes(O.Q4_K, L.DTYPE_FP16, 8, 5120, 13824) == 3 * 8 * 5120 * 4
    print("noalloc: Q4_K x fp16 8x5120x13824 (three K slices)", flush=True)
    _case(dev, O.Q4_K, 8, 5120, 13824, seed_for(3, 210), kind="f16")
    print("noalloc: Q4_K x fp16 3x700x8704 (two K slices, second call)", flush=True)
    _case(dev, O.Q4_K, 3, 700, 8704, seed_for(3, 220), kind="f16")


def test_noalloc_without_scratch_route(dev):
    """A GEMV that takes no workspace needs no scratch: the same call as
    vkflame_dispatch_gemm_q."""
    _case(dev, O.Q4_K, 8, 512, 2048, seed_for(3, 201))


def test_noalloc_rejects_oversize(dev):
    """M*K*2 beyond the fixed array is refused before any launch."""
    import torch
    from vkflame_amd import _lib as L
    M, N, K = 2048, 64, 8192  # 32 MiB of fp16 activations
    assert L.lib().vkflame_gemm_q_workspace_bytes(O.Q6_K, L.DTYPE_Q8_1, M, N, K) > L.lib().vkflame_noalloc_scratch_bytes()
    w = torch.zeros((N, K // 256 * 210), dtype=torch.uint8, device=dev)
    x = torch.zeros((M, K // 32 * 36), dtype=torch.uint8, device=dev)
    y = torch.zeros((M, N), dtype=torch.float32, device=dev)
    rc = _call(L.lib().vkflame_dispatch_gemm_q_noalloc, w, O.Q6_K, x, L.DTYPE_Q8_1, y, M, N, K)
    assert rc == 1  # hipErrorInvalidValue
    torch.cuda.synchronize()
    assert int(torch.count_nonzero(y)) == 0
