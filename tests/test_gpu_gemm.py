"""GPU parity: prefill GEMMs on the matrix cores (fp16 MFMA, int8 MFMA,
dequant-fused quantised GEMM, integer-exact Q6_K x Q8_1) through the C ABI."""
import numpy as np
import pytest

import oracle as O
from _util import TOL_F16, TOL_F32, bits_equal, first_mismatch, rel_err, seed_for, to_dev

pytestmark = pytest.mark.gpu


def _f16(rng, *shape):
    return rng.normal(0, 1, shape).astype(np.float16)


@pytest.mark.parametrize("M,N,K", [(128, 128, 32), (200, 72, 40), (17, 300, 1000), (256, 384, 4096)])
@pytest.mark.parametrize("transA,transB", [(0, 1), (0, 0), (1, 1), (1, 0)])
def test_linear_fp16_fp32out(dev, M, N, K, transA, transB):
    import torch
    from vkflame_amd import ops
    from vkflame_amd._lib import DTYPE_FP16_FP32OUT
    rng = np.random.default_rng(seed_for(4, 40) + M + N + K)
    A = _f16(rng, M, K)
    B = _f16(rng, N, K) if transB else _f16(rng, K, N)
    Am = A.T.copy() if transA else A
    D = ops.linear(to_dev(Am, dev), to_dev(B, dev), M, N, K, DTYPE_FP16_FP32OUT, transA=transA, transB=transB)
    torch.cuda.synchronize()
    Bm = B.T if transB else B
    ref = A.astype(np.float64) @ Bm.astype(np.float64)
    assert rel_err(D.cpu().numpy(), ref) <= TOL_F32


@pytest.mark.parametrize("M,N,K", [(128, 128, 64), (200, 136, 192), (17, 520, 1024), (300, 1000, 128),
                                   (1, 4096, 4096), (33, 8, 64)])
def test_linear_fp16_nn_transposed_reads(dev, M, N, K):
    """B stored [K, N] (NN, torch.mm(a, b)) with N % 8 == 0 and K % 64 == 0:
    the B tile is copied to LDS as it lies and read back transposed
    (ds_read_b64_tr_b16); ragged M and N, one K step, N below one tile."""
    import torch
    from vkflame_amd import ops
    from vkflame_amd._lib import DTYPE_FP16_FP32OUT
    rng = np.random.default_rng(seed_for(4, 45) + M + N + K)
    A, B = _f16(rng, M, K), _f16(rng, K, N)
    D = ops.linear(to_dev(A, dev), to_dev(B, dev), M, N, K, DTYPE_FP16_FP32OUT, transA=0, transB=0)
    torch.cuda.synchronize()
    ref = A.astype(np.float64) @ B.astype(np.float64)
    assert rel_err(D.cpu().numpy(), ref) <= TOL_F32


@pytest.mark.parametrize("M,N,K", [(1, 4096, 4096), (5, 136, 96), (16, 8, 32), (17, 520, 1024), (32, 4096, 4096),
                                   (33, 200, 4128), (64, 1000, 288), (48, 4096, 4096), (64, 1000, 256),
                                   (1, 11008, 1024), (16, 11008, 1024)])
@pytest.mark.parametrize("transB", [1, 0])
def test_linear_fp16_skinny(dev, M, N, K, transB):
    """Few rows of A: the skinny kernel (B streamed once by 16-column
    workgroups, K split over 16 waves, partial tiles summed in wave order)
    up to 64 rows where the narrow-tile kernels do not apply (K not whole
    pairs of 128-byte steps), else up to 8 rows, and up to 32 while its
    workgroups fit one per CU; the narrow tiles otherwise (48 x 4096 x
    4096, 64 x 1000 x 256, 16 x 11008 x 1024).  B [N, K] or [K, N]; fp32
    out, then fp16 out with alpha, beta*C and an activation, checked
    against the same float64 product."""
    import torch
    from vkflame_amd import ops
    from vkflame_amd._lib import DTYPE_FP16, DTYPE_FP16_FP32OUT
    rng = np.random.default_rng(seed_for(4, 47) + M + N + K + transB)
    A = _f16(rng, M, K)
    B = _f16(rng, N, K) if transB else _f16(rng, K, N)
    Bm = B.T if transB else B
    ref = A.astype(np.float64) @ Bm.astype(np.float64)
    D = ops.linear(to_dev(A, dev), to_dev(B, dev), M, N, K, DTYPE_FP16_FP32OUT, transB=transB)
    torch.cuda.synchronize()
    assert rel_err(D.cpu().numpy(), ref) <= TOL_F32
    D2 = ops.linear(to_dev(A, dev), to_dev(B, dev), M, N, K, DTYPE_FP16_FP32OUT, transB=transB)
    torch.cuda.synchronize()
    assert bits_equal(D.cpu().numpy(), D2.cpu().numpy())  # fixed summation order
    C = _f16(rng, M, N)
    E = ops.linear(to_dev(A, dev), to_dev(B, dev), M, N, K, DTYPE_FP16, transB=transB, act=1,
                   C=to_dev(C, dev), alpha=0.5, beta=0.25)
    torch.cuda.synchronize()
    pre = (0.5 * ref + 0.25 * C.astype(np.float64)).astype(np.float32)
    assert rel_err(E.cpu().numpy().astype(np.float32), O.np_act(1, pre)) <= TOL_F16


@pytest.mark.parametrize("act", [0, 1, 2, 3])
def test_linear_fp16_epilogue(dev, act):
    """fp16 out with alpha, beta*C and every activation."""
    import torch
    from vkflame_amd import ops
    from vkflame_amd._lib import DTYPE_FP16
    M, N, K = 96, 160, 256
    rng = np.random.default_rng(seed_for(4, 50 + act))
    A, B, C = _f16(rng, M, K), _f16(rng, N, K), _f16(rng, M, N)
    D = ops.linear(to_dev(A, dev), to_dev(B, dev), M, N, K, DTYPE_FP16, transB=1, act=act,
                   C=to_dev(C, dev), alpha=0.5, beta=0.25)
    torch.cuda.synchronize()
    pre = (0.5 * (A.astype(np.float64) @ B.astype(np.float64).T) + 0.25 * C.astype(np.float64)).astype(np.float32)
    ref = O.np_act(act, pre)
    assert rel_err(D.cpu().numpy().astype(np.float32), ref) <= TOL_F16


@pytest.mark.parametrize("M,N,K", [(64, 64, 64), (130, 70, 100), (512, 640, 5120)])
def test_linear_int8_int32_exact(dev, M, N, K):
    import torch
    from vkflame_amd import ops
    from vkflame_amd._lib import DTYPE_INT8_INT32OUT
    rng = np.random.default_rng(seed_for(4, 60) + M)
    A = rng.integers(-127, 128, (M, K)).astype(np.int8)
    W = rng.integers(-127, 128, (N, K)).astype(np.int8)
    D = ops.linear(to_dev(A, dev), to_dev(W, dev), M, N, K, DTYPE_INT8_INT32OUT, transB=1)
    torch.cuda.synchronize()
    ref = (A.astype(np.float64) @ W.astype(np.float64).T).astype(np.int64)  # exact: |sum| < 2^53
    assert np.array_equal(D.cpu().numpy().astype(np.int64), ref)


@pytest.mark.parametrize("M,N,K,transA,transB,act", [(64, 96, 256, 0, 1, 0), (130, 70, 200, 0, 1, 1),
                                                     (512, 640, 5120, 0, 1, 2), (100, 72, 384, 1, 0, 3),
                                                     (33, 300, 1000, 1, 1, 0), (300, 128, 640, 0, 0, 2)])
def test_linear_int8_reference_contract(dev, M, N, K, transA, transB, act):
    """vkflame_dispatch_linear(VKF_DTYPE_INT8) as kernels/linear_int8.glsl
    defines it: fp16 A quantised in the kernel by act_scale (alpha), int8
    weights, per-channel w_scale (C), activation, fp16 D -- against the
    oracle's exact int32 core and float64 epilogue."""
    import ctypes
    import torch
    from vkflame_amd import ops
    from vkflame_amd._lib import DTYPE_INT8
    rng = np.random.default_rng(seed_for(4, 90) + M + K + act)
    act_scale = 0.0371
    A = (rng.normal(0, 1.5, (M, K))).astype(np.float16)
    W = rng.integers(-127, 128, (N, K)).astype(np.int8)
    ws = np.abs(rng.normal(0, 0.01, N)).astype(np.float32)
    Am = A.T.copy() if transA else A
    Wm = W if transB else W.T.copy()
    D = ops.linear(to_dev(Am, dev), to_dev(Wm, dev), M, N, K, DTYPE_INT8, transA=transA, transB=transB, act=act,
                   C=to_dev(ws, dev), alpha=act_scale)
    torch.cuda.synchronize()
    assert D.dtype == torch.float16
    acc, y = O.ref_linear_int8_fp16a(A, W, act_scale, ws, act)
    assert rel_err(D.cpu().numpy().astype(np.float32), y) <= TOL_F16
    # act_scale 1 and integer-valued fp16 A: the int8 product itself, scaled
    Ai = rng.integers(-127, 128, (M, K)).astype(np.float16)
    Aim = Ai.T.copy() if transA else Ai
    D1 = ops.linear(to_dev(Aim, dev), to_dev(Wm, dev), M, N, K, DTYPE_INT8, transA=transA, transB=transB,
                    C=to_dev(ws, dev))
    torch.cuda.synchronize()
    ref = (Ai.astype(np.float64) @ W.astype(np.float64).T) * ws.astype(np.float64)[None, :]
    assert rel_err(D1.cpu().numpy().astype(np.float32), ref) <= TOL_F16


def _dense_shapes():
    """(M, N, K) cases on both sides of the split-K switch: grids of at most
    one 128x128 tile per CU take the 512-thread kernel that splits K between
    two wave groups (odd and even step counts, one step, ragged edges),
    larger grids the 256-thread kernel."""
    import torch
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    # K*bytes a multiple of 128 takes the direct-to-LDS kernels: int8 K = 128,
    # 384, 640 (1, 3, 5 steps); fp16 K = 192, 1088 (3, 17 steps) and the rest
    small = [(128, 128, 128), (130, 250, 384), (512, 640, 640), (200, 200, 192), (300, 1000, 1088)]
    big_m = 128 * (cus // 16 + 1)  # (cus/16 + 1) x 16 tiles > cus
    big = [(big_m, 2048, 256), (big_m - 37, 2000, 192)]
    return small, big, cus


def test_linear_dense_split_k_and_plain(dev):
    import torch
    from vkflame_amd import ops
    from vkflame_amd._lib import DTYPE_FP16_FP32OUT, DTYPE_INT8_INT32OUT
    small, big, cus = _dense_shapes()
    for (M, N, K) in small + big:
        tiles = -(-M // 128) * -(-N // 128)
        assert (tiles <= cus) == ((M, N, K) in small)
        rng = np.random.default_rng(seed_for(4, 80) + M + N + K)
        A = rng.integers(-127, 128, (M, K)).astype(np.int8)
        W = rng.integers(-127, 128, (N, K)).astype(np.int8)
        D = ops.linear(to_dev(A, dev), to_dev(W, dev), M, N, K, DTYPE_INT8_INT32OUT, transB=1)
        torch.cuda.synchronize()
        ref = A.astype(np.int64) @ W.astype(np.int64).T
        got = D.cpu().numpy().astype(np.int64)
        assert np.array_equal(got, ref), (M, N, K, int((got != ref).sum()))
        Af, Bf = _f16(rng, M, K), _f16(rng, N, K)
        D = ops.linear(to_dev(Af, dev), to_dev(Bf, dev), M, N, K, DTYPE_FP16_FP32OUT, transB=1)
        torch.cuda.synchronize()
        ref = Af.astype(np.float64) @ Bf.astype(np.float64).T
        assert rel_err(D.cpu().numpy(), ref) <= TOL_F32, (M, N, K)


def _narrow_nb(M, N, K, es, cus, batch=1, nbs=(4, 5)):
    """The tile width the host picks for the narrow-tile kernels (16*nb
    columns; the dense NT kernels nb = 1..5, NN 1, 2, 4, 5, the Q4_K one 4
    and 5), 0 if it takes another kernel (mirrors narrow_nb in
    csrc/host/vkf_runtime.cpp)."""
    rows = -(-M // 128) * batch
    if K == 0 or (K * es) % 256 or rows * -(-N // 128) >= cus:
        return 0
    for nb in nbs:
        if rows * -(-N // (16 * nb)) <= cus:
            return nb
    return 0


@pytest.mark.parametrize("M,N,K", [(512, 5120, 5120), (512, 4096, 1024), (500, 5000, 768), (128, 8192, 2048),
                                   (77, 200, 256), (384, 3000, 512), (1024, 1024, 1024), (300, 1000, 512), (128, 4096, 512),
                                   (256, 5120, 512), (512, 3000, 256)])
def test_linear_dense_narrow_tiles(dev, M, N, K):
    """Grids of fewer 128x128 tiles than CUs with whole pairs of K steps:
    the narrow-tile kernels (128 x 16 to 128 x 80 tiles, three stages, K
    split between two wave groups).  int8 -> exact int32 (also
    with integer alpha / beta), fp16 -> fp32 and fp16 with alpha, beta*C,
    bias-free activation; repeated calls give the same bits."""
    import torch
    from vkflame_amd import ops
    from vkflame_amd._lib import DTYPE_FP16, DTYPE_FP16_FP32OUT, DTYPE_INT8_INT32OUT
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    assert _narrow_nb(M, N, K, 1, cus, nbs=(1, 2, 3, 4, 5)) and _narrow_nb(M, N, K, 2, cus, nbs=(1, 2, 3, 4, 5))
    rng = np.random.default_rng(seed_for(4, 82) + M + N + K)
    A = rng.integers(-127, 128, (M, K)).astype(np.int8)
    W = rng.integers(-127, 128, (N, K)).astype(np.int8)
    Ci = rng.integers(-1000, 1000, (M, N)).astype(np.int32)
    ref = (A.astype(np.float64) @ W.astype(np.float64).T).astype(np.int64)  # exact: |sum| < 2^53, through BLAS
    D = ops.linear(to_dev(A, dev), to_dev(W, dev), M, N, K, DTYPE_INT8_INT32OUT, transB=1)
    D2 = ops.linear(to_dev(A, dev), to_dev(W, dev), M, N, K, DTYPE_INT8_INT32OUT, transB=1,
                    C=to_dev(Ci, dev), alpha=3, beta=-2)
    torch.cuda.synchronize()
    got = D.cpu().numpy().astype(np.int64)
    assert np.array_equal(got, ref), (M, N, K, int((got != ref).sum()))
    want2 = (3 * ref - 2 * Ci.astype(np.int64)).astype(np.int32)  # int32 wrap-around, as the kernel
    assert np.array_equal(D2.cpu().numpy(), want2)
    Af, Bf, C = _f16(rng, M, K), _f16(rng, N, K), _f16(rng, M, N)
    reff = Af.astype(np.float64) @ Bf.astype(np.float64).T
    outs = [ops.linear(to_dev(Af, dev), to_dev(Bf, dev), M, N, K, DTYPE_FP16_FP32OUT, transB=1) for _ in range(2)]
    E = ops.linear(to_dev(Af, dev), to_dev(Bf, dev), M, N, K, DTYPE_FP16, transB=1, act=2,
                   C=to_dev(C, dev), alpha=0.5, beta=0.25)
    torch.cuda.synchronize()
    assert rel_err(outs[0].cpu().numpy(), reff) <= TOL_F32, (M, N, K)
    assert torch.equal(outs[0].view(torch.int32), outs[1].view(torch.int32))
    pre = (0.5 * reff + 0.25 * C.astype(np.float64)).astype(np.float32)
    assert rel_err(E.cpu().numpy().astype(np.float32), O.np_act(2, pre)) <= TOL_F16


@pytest.mark.parametrize("M,N,K", [(128, 8192, 2048), (512, 4096, 1024), (300, 1000, 512), (77, 200, 256),
                                   (512, 5120, 5120), (500, 5000, 768), (1024, 1024, 1024), (256, 256, 256), (128, 4096, 512),
                                   (256, 5120, 512), (512, 3000, 256)])
def test_linear_fp16_nn_narrow_tiles(dev, M, N, K):
    """fp16 with B stored [K, N] (NN) on grids of fewer 128x128 tiles than
    CUs: the narrow kernel's 128 x 16 to 128 x 80 tiles with B's k-rows
    staged as they lie and read back transposed.  fp32 out against
    the float64 product, repeatable bits, and fp16 out with alpha, beta*C
    and an activation."""
    import torch
    from vkflame_amd import ops
    from vkflame_amd._lib import DTYPE_FP16, DTYPE_FP16_FP32OUT
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    assert M > 64 and N % 8 == 0 and _narrow_nb(M, N, K, 2, cus, nbs=(1, 2, 4, 5))
    rng = np.random.default_rng(seed_for(4, 83) + M + N + K)
    A, B, C = _f16(rng, M, K), _f16(rng, K, N), _f16(rng, M, N)
    ref = A.astype(np.float64) @ B.astype(np.float64)
    Ad, Bd = to_dev(A, dev), to_dev(B, dev)
    D = [ops.linear(Ad, Bd, M, N, K, DTYPE_FP16_FP32OUT, transB=0) for _ in range(2)]
    E = ops.linear(Ad, Bd, M, N, K, DTYPE_FP16, transB=0, act=3, C=to_dev(C, dev), alpha=0.5, beta=0.25)
    torch.cuda.synchronize()
    assert rel_err(D[0].cpu().numpy(), ref) <= TOL_F32
    assert torch.equal(D[0].view(torch.int32), D[1].view(torch.int32))
    pre = (0.5 * ref + 0.25 * C.astype(np.float64)).astype(np.float32)
    assert rel_err(E.cpu().numpy().astype(np.float32), O.np_act(3, pre)) <= TOL_F16


@pytest.mark.parametrize("M,N,K", [(4096, 4096, 128), (4100, 4104, 192), (4224, 4352, 256), (4100, 4104, 8192)])
def test_linear_dense_256_tiles(dev, M, N, K):
    """Grids of at least one 256x256 tile per CU with K-contiguous operands:
    the 256 x 256 kernel (eight waves of 128 x 64), ragged rows and columns;
    int8 always, fp16 from K = 8192 (below, the 128 x 128 kernel).  int8 ->
    exact int32 (also with integer alpha / beta), fp16 -> fp32 against the
    float64 product, fp16 out with alpha, beta*C and an activation."""
    import torch
    from vkflame_amd import ops
    from vkflame_amd._lib import DTYPE_FP16, DTYPE_FP16_FP32OUT, DTYPE_INT8_INT32OUT
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    assert -(-M // 256) * -(-N // 256) >= cus
    rng = np.random.default_rng(seed_for(4, 84) + M + N + K)
    A = rng.integers(-127, 128, (M, K)).astype(np.int8)
    W = rng.integers(-127, 128, (N, K)).astype(np.int8)
    Ci = rng.integers(-1000, 1000, (M, N)).astype(np.int32)
    ref = (A.astype(np.float64) @ W.astype(np.float64).T).astype(np.int64)  # exact: |sum| < 2^53, through BLAS
    D = ops.linear(to_dev(A, dev), to_dev(W, dev), M, N, K, DTYPE_INT8_INT32OUT, transB=1)
    D2 = ops.linear(to_dev(A, dev), to_dev(W, dev), M, N, K, DTYPE_INT8_INT32OUT, transB=1,
                    C=to_dev(Ci, dev), alpha=3, beta=-2)
    torch.cuda.synchronize()
    got = D.cpu().numpy().astype(np.int64)
    assert np.array_equal(got, ref), (M, N, K, int((got != ref).sum()))
    assert np.array_equal(D2.cpu().numpy(), (3 * ref - 2 * Ci.astype(np.int64)).astype(np.int32))
    del D, D2
    Af, Bf, C = _f16(rng, M, K), _f16(rng, N, K), _f16(rng, M, N)
    reff = Af.astype(np.float64) @ Bf.astype(np.float64).T
    F = ops.linear(to_dev(Af, dev), to_dev(Bf, dev), M, N, K, DTYPE_FP16_FP32OUT, transB=1)
    E = ops.linear(to_dev(Af, dev), to_dev(Bf, dev), M, N, K, DTYPE_FP16, transB=1, act=1,
                   C=to_dev(C, dev), alpha=0.5, beta=0.25)
    torch.cuda.synchronize()
    assert rel_err(F.cpu().numpy(), reff) <= TOL_F32
    pre = (0.5 * reff + 0.25 * C.astype(np.float64)).astype(np.float32)
    assert rel_err(E.cpu().numpy().astype(np.float32), O.np_act(1, pre)) <= TOL_F16


def test_linear_dense_split_k_repeatable(dev):
    """The split-K kernel adds the two groups' fp32 sums in one fixed order:
    the same inputs give the same bits on every call."""
    import torch
    from vkflame_amd import ops
    from vkflame_amd._lib import DTYPE_FP16
    M, N, K = 512, 1024, 2048
    rng = np.random.default_rng(seed_for(4, 81))
    A, B = to_dev(_f16(rng, M, K), dev), to_dev(_f16(rng, N, K), dev)
    outs = [ops.linear(A, B, M, N, K, DTYPE_FP16, transB=1) for _ in range(3)]
    torch.cuda.synchronize()
    for o in outs[1:]:
        assert torch.equal(o.view(torch.int16), outs[0].view(torch.int16))


def test_config4_linear_int8(dev):
    """C4: int8 [512,5120] x int8 [5120,5120]^T, per-token and per-channel
    scales, fp16 bias, fp16 out."""
    import torch
    from vkflame_amd import ops
    from vkflame_amd._lib import DTYPE_INT8_INT32OUT
    M = 512
    N = K = 5120
    inp = O.gen_int8_linear(M, N, K, seed_for(4))
    A, W = to_dev(inp.A, dev), to_dev(inp.W, dev)
    acc = ops.linear(A, W, M, N, K, DTYPE_INT8_INT32OUT, transB=1)
    D = ops.linear_int8(A, to_dev(inp.a_scale, dev), W, to_dev(inp.w_scale, dev), to_dev(inp.bias, dev))
    torch.cuda.synchronize()
    ref_acc = (inp.A.astype(np.float64) @ inp.W.astype(np.float64).T)
    assert np.array_equal(acc.cpu().numpy().astype(np.float64), ref_acc)
    ref = ref_acc * inp.a_scale[:, None].astype(np.float64) * inp.w_scale[None, :].astype(np.float64) \
        + inp.bias.astype(np.float64)[None, :]
    assert rel_err(D.cpu().numpy().astype(np.float32), ref) <= TOL_F16


@pytest.mark.parametrize("act", [1, 2, 3])
def test_linear_int8_activation_fp32_out(dev, act):
    import torch
    from vkflame_amd import ops
    M, N, K = 40, 72, 320
    inp = O.gen_int8_linear(M, N, K, seed_for(4, 70 + act))
    D = ops.linear_int8(to_dev(inp.A, dev), to_dev(inp.a_scale, dev), to_dev(inp.W, dev),
                        to_dev(inp.w_scale, dev), to_dev(inp.bias, dev), out_dtype=torch.float32, act=act)
    torch.cuda.synchronize()
    _, yref, _ = O.ref_linear_int8(inp, act=act)
    assert rel_err(D.cpu().numpy(), yref) <= TOL_F32


WTYPES = [O.Q4_0, O.Q4_1, O.Q8_0, O.Q5_0, O.Q4_K, O.Q5_K, O.Q6_K]


@pytest.mark.parametrize("qt", WTYPES, ids=[O.QNAMES[q] for q in WTYPES])
def test_gemm_q_fp16_prefill(dev, qt):
    """M > 16: weight tiles dequantised to fp16 in LDS, fp16 MFMA."""
    import torch
    from vkflame_amd import ops
    M, N, K = 200, 150, 1024
    w = O.gen_weight(qt, N, K, seed_for(3, 30 + qt))
    x = _f16(np.random.default_rng(seed_for(3, 40 + qt)), M, K)
    y = ops.gemm_q(to_dev(w, dev), qt, to_dev(x, dev), N, K)
    torch.cuda.synchronize()
    ref = O.ref_gemv(x.astype(np.float64), O.np_dequant(qt, w).reshape(N, K))
    assert rel_err(y.cpu().numpy(), ref) <= TOL_F32


@pytest.mark.parametrize("qt,K", [(O.Q4_0, 64), (O.Q4_0, 1088), (O.Q8_0, 192), (O.Q5_0, 1088), (O.Q4_1, 320),
                                  (O.Q4_K, 256), (O.Q4_K, 768), (O.Q5_K, 1280), (O.Q6_K, 512)],
                         ids=["q4_0-k64", "q4_0-k1088", "q8_0-k192", "q5_0-k1088", "q4_1-k320", "q4_k-k256",
                              "q4_k-k768", "q5_k-k1280", "q6_k-k512"])
def test_gemm_q_split_k_edges(dev, qt, K):
    """Grids of at most one 128 x 128 tile per CU take the split-K kernel
    (two wave groups on alternate 64-k steps): one step (K = 64), odd step
    counts (group 1 idle on the last pair), ragged M and N, against the
    oracle."""
    import torch
    from vkflame_amd import ops
    M, N = 100, 203
    w = O.gen_weight(qt, N, K, seed_for(3, 110 + qt) + K)
    x = _f16(np.random.default_rng(seed_for(3, 120 + qt) + K), M, K)
    y = ops.gemm_q(to_dev(w, dev), qt, to_dev(x, dev), N, K)
    torch.cuda.synchronize()
    ref = O.ref_gemv(x.astype(np.float64), O.np_dequant(qt, w).reshape(N, K))
    assert rel_err(y.cpu().numpy(), ref) <= TOL_F32


@pytest.mark.parametrize("qt", [O.Q4_0, O.Q4_K, O.Q8_0], ids=["q4_0", "q4_k", "q8_0"])
def test_gemm_q_q8_1_activations_prefill(dev, qt):
    import torch
    from vkflame_amd import ops
    M, N, K = 64, 96, 512
    w = O.gen_weight(qt, N, K, seed_for(3, 50 + qt))
    x = np.random.default_rng(seed_for(3, 60 + qt)).normal(0, 1, (M, K)).astype(np.float32)
    xq = O.np_quantize_q8_1(x).reshape(M, -1)
    y = ops.gemm_q(to_dev(w, dev), qt, to_dev(xq, dev), N, K)
    torch.cuda.synchronize()
    x64 = O.np_dequant(O.Q8_1, xq).reshape(M, K).astype(np.float64)
    assert rel_err(y.cpu().numpy(), O.ref_gemv(x64, O.np_dequant(qt, w).reshape(N, K))) <= TOL_F32


def test_config3_q4_k_prefill(dev):
    """C3 at M=512: 13824x5120 Q4_K, fp16 activations."""
    import torch
    from vkflame_amd import ops
    N, K, M = 13824, 5120, 512
    w = O.gen_weight(O.Q4_K, N, K, seed_for(3))
    x = _f16(np.random.default_rng(seed_for(3, 512)), M, K)
    y = ops.gemm_q(to_dev(w, dev), O.Q4_K, to_dev(x, dev), N, K).cpu().numpy()
    torch.cuda.synchronize()
    rows = np.concatenate([[0, N - 1], np.random.default_rng(3).choice(N, 512, replace=False)])
    wd = O.np_dequant(O.Q4_K, w[rows]).reshape(len(rows), K)
    assert rel_err(y[:, rows], O.ref_gemv(x.astype(np.float64), wd)) <= TOL_F32


def test_config5_q6_k_q8_1_prefill(dev):
    """C5's activations (M = 512, K = 5120, Q8_1) on a 4096-row slice of the
    vocab projection.  The slice is 128 tiles of 128 x 128, at most one per
    CU, so it runs the split-K kernel (vkf_gemm_q6_k_f16_k2) after the
    one-time activation decode; the full 152064 rows run the 256-row wide
    kernel (test_config5_q6_k_q8_1_prefill_full)."""
    import torch
    from vkflame_amd import ops
    N, K, M = 4096, 5120, 512
    w = O.gen_weight(O.Q6_K, N, K, seed_for(5, 8))
    x = np.random.default_rng(seed_for(5, 9)).normal(0, 1, (M, K)).astype(np.float32)
    xq = ops.quantize_q8_1(to_dev(x, dev))
    y = ops.gemm_q(to_dev(w, dev), O.Q6_K, xq, N, K).cpu().numpy()
    torch.cuda.synchronize()
    xq_ref = O.np_quantize_q8_1(x).reshape(M, -1)
    x64 = O.np_dequant(O.Q8_1, xq_ref).reshape(M, K).astype(np.float64)
    rows = np.concatenate([[0, N - 1], np.random.default_rng(4).choice(N, 512, replace=False)])
    wd = O.np_dequant(O.Q6_K, w[rows]).reshape(len(rows), K)
    assert rel_err(y[:, rows], O.ref_gemv(x64, wd)) <= TOL_F32


@pytest.mark.parametrize("qt", WTYPES, ids=[O.QNAMES[q] for q in WTYPES])
def test_gemm_q_fp16_wide_tiles(dev, qt):
    """M >= 256 takes 256-row tiles (512 threads, weight tile decoded once per
    256 rows) when they fill at least half the CUs; M < 256 the 128-row
    tiles.  Both multiply the same fp16 operand values in the same MFMA
    order, so the first 255 rows of an M = 300 product equal the M = 255
    product bit for bit; both match the oracle.  N = 16600: 2 x 130 wide
    tiles, enough for the wide kernel on a 256-CU MI355X, and 2 x 130
    128-row tiles at M = 255, more than one per CU (fewer would take the
    split-K kernel, whose two partial sums round differently)."""
    import torch
    from vkflame_amd import ops
    N, K = 16600, 1024
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    assert 2 * 2 * -(-N // 128) >= cus and 2 * -(-N // 128) > cus
    w = O.gen_weight(qt, N, K, seed_for(3, 90 + qt))
    x = _f16(np.random.default_rng(seed_for(3, 100 + qt)), 300, K)
    wd, xd = to_dev(w, dev), to_dev(x, dev)
    y_wide = ops.gemm_q(wd, qt, xd, N, K).cpu().numpy()
    y_narrow = ops.gemm_q(wd, qt, xd[:255], N, K).cpu().numpy()
    torch.cuda.synchronize()
    assert bits_equal(y_wide[:255], y_narrow), first_mismatch(y_wide[:255], y_narrow)
    ref = O.ref_gemv(x.astype(np.float64), O.np_dequant(qt, w).reshape(N, K))
    assert rel_err(y_wide, ref) <= TOL_F32


@pytest.mark.parametrize("qt,M,K", [(O.Q4_0, 200, 1024), (O.Q4_0, 64, 96), (O.Q4_K, 300, 1024), (O.Q8_0, 200, 512),
                                    (O.Q6_K, 300, 2048), (O.Q5_K, 256, 768)],
                         ids=["q4_0", "q4_0-k96", "q4_k-m300", "q8_0", "q6_k-m300", "q5_k-m256"])
def test_gemm_q_q8_1_workspace_paths(dev, qt, M, K):
    """Q8_1 activations at M > 16 take three routes: decoded once into a
    caller workspace (vkflame_dispatch_gemm_q_ws, then the fp16-activation
    GEMM), into a stream-ordered allocation of the library's
    (vkflame_dispatch_gemm_q), or per tile inside the Q8_1 GEMM (no
    workspace).  Every route multiplies the same fp16 operand values in the
    same MFMA order: the two workspace routes agree bit for bit, and all
    match the oracle.  The per-tile route adds K in one sequence; on these
    small grids (at most one 128 x 128 tile per CU) the fp16-activation
    route splits K between two wave groups, so those two agree to rounding
    (bit for bit on larger grids)."""
    import torch
    from vkflame_amd import ops
    from vkflame_amd import _lib as L
    N = 300
    w = O.gen_weight(qt, N, K, seed_for(3, 70 + qt))
    x = np.random.default_rng(seed_for(3, 80 + qt)).normal(0, 1, (M, K)).astype(np.float32)
    xq = O.np_quantize_q8_1(x).reshape(M, -1)
    wd, xd = to_dev(w, dev), to_dev(xq, dev)
    assert L.lib().vkflame_gemm_q_workspace_bytes(qt, L.DTYPE_Q8_1, M, N, K) == M * K * 2
    assert L.lib().vkflame_gemm_q_workspace_bytes(qt, L.DTYPE_Q8_1, 16, N, K) == 0
    assert L.lib().vkflame_gemm_q_workspace_bytes(qt, L.DTYPE_FP16, M, N, K) == 0
    y_ws = ops.gemm_q(wd, qt, xd, N, K)
    y_tile = ops.gemm_q(wd, qt, xd, N, K, workspace=False)
    y_lib = torch.empty((M, N), dtype=torch.float32, device=dev)
    L.check(L.lib().vkflame_dispatch_gemm_q(ops._p(wd), qt, 0, ops._p(xd), L.DTYPE_Q8_1, xd.stride(0),
                                            ops._p(y_lib), N, M, N, K, ops._stream()), "gemm_q")
    torch.cuda.synchronize()
    a, b, c = y_ws.cpu().numpy(), y_tile.cpu().numpy(), y_lib.cpu().numpy()
    assert bits_equal(a, c), first_mismatch(a, c)
    assert rel_err(a, b) <= 1e-5
    x64 = O.np_dequant(O.Q8_1, xq).reshape(M, K).astype(np.float64)
    ref = O.ref_gemv(x64, O.np_dequant(qt, w).reshape(N, K))
    for y in (a, b, c):
        assert rel_err(y, ref) <= TOL_F32


def _wide_route(M, N, cus):
    """The dispatcher's condition for the 256-row wide kernel
    (vkf_gemm_<q>_f16_w): fp16 (or workspace-decoded Q8_1) activations,
    M >= 256, the wide grid filling at least half the CUs and the 128-row grid
    more than one tile per CU."""
    t = -(-N // 128)
    return M >= 256 and 2 * t * -(-M // 256) >= cus and t * -(-M // 128) > cus


def _split_k_route(M, N, cus):
    """The condition for the split-K kernel (vkf_gemm_<q>_f16_k2): not wide
    and the 128-row grid at most one tile per CU."""
    return not _wide_route(M, N, cus) and -(-N // 128) * -(-M // 128) <= cus


def test_config5_q6_k_q8_1_prefill_full(dev):
    """C5 at its full size: Q6_K 152064 x 5120 weights x Q8_1 activations
    [512, 5120] quantised on the GPU, through the route bench.py times: the
    activations decoded once into a workspace, then the wide 256-row kernel
    (vkf_gemm_q6_k_f16_w).  All 512 activation rows against the oracle's
    float64 product on 1026 weight rows (first, last and a random sample)."""
    import torch
    from vkflame_amd import ops
    N, K, M = 152064, 5120, 512
    assert _wide_route(M, N, torch.cuda.get_device_properties(0).multi_processor_count)
    w = O.gen_weight(O.Q6_K, N, K, seed_for(5))
    x = np.random.default_rng(seed_for(5, 1)).normal(0, 1, (M, K)).astype(np.float32)
    wd = to_dev(w, dev)
    xq = ops.quantize_q8_1(to_dev(x, dev))
    rows = np.concatenate([[0, N - 1], np.random.default_rng(5).choice(N, 1024, replace=False)])
    y = ops.gemm_q(wd, O.Q6_K, xq, N, K)
    torch.cuda.synchronize()
    ys = y[:, torch.from_numpy(rows).to(dev)].cpu().numpy()
    del y, wd
    torch.cuda.empty_cache()
    xq_ref = O.np_quantize_q8_1(x).reshape(M, -1)
    assert np.array_equal(xq.cpu().numpy(), xq_ref)
    x64 = O.np_dequant(O.Q8_1, xq_ref).reshape(M, K).astype(np.float64)
    wdq = O.np_dequant(O.Q6_K, w[rows]).reshape(len(rows), K)
    assert rel_err(ys, O.ref_gemv(x64, wdq)) <= TOL_F32


def test_wide_q6_k_q8_1_k5120(dev):
    """The wide kernel at C5's K with Q8_1 activations decoded into the
    workspace, every output checked: N = 8448 (66 tiles of 128 rows) is the
    smallest multiple of 128 that takes the wide route at M = 512 on a
    256-CU MI355X."""
    import torch
    from vkflame_amd import ops
    N, K, M = 8448, 5120, 512
    assert _wide_route(M, N, torch.cuda.get_device_properties(0).multi_processor_count)
    w = O.gen_weight(O.Q6_K, N, K, seed_for(5, 30))
    x = np.random.default_rng(seed_for(5, 31)).normal(0, 1, (M, K)).astype(np.float32)
    xq = O.np_quantize_q8_1(x).reshape(M, -1)
    y = ops.gemm_q(to_dev(w, dev), O.Q6_K, to_dev(xq, dev), N, K)
    torch.cuda.synchronize()
    x64 = O.np_dequant(O.Q8_1, xq).reshape(M, K).astype(np.float64)
    assert rel_err(y.cpu().numpy(), O.ref_gemv(x64, O.np_dequant(O.Q6_K, w).reshape(N, K))) <= TOL_F32


@pytest.mark.parametrize("M,N,K", [(512, 4096, 1024), (512, 5120, 2304), (300, 5000, 1280), (128, 8200, 512),
                                   (17, 100, 256), (200, 77, 768)])
def test_gemm_q4_k_narrow_tiles(dev, M, N, K):
    """Q4_K x fp16 on 128-row grids of fewer tiles than CUs: the narrow-tile
    kernel with raw Q4_K pieces staged three steps ahead (128 x 64 or
    128 x 80 tiles, ragged rows and columns, K from one super-block), fp32
    out against the oracle's float64 product; repeated calls give the same
    bits."""
    import torch
    from vkflame_amd import ops
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    assert _narrow_nb(M, N, K, 2, cus) in (4, 5)
    w = O.gen_weight(O.Q4_K, N, K, seed_for(3, 600 + M + N))
    x = _f16(np.random.default_rng(seed_for(3, 700 + K)), M, K)
    wd, xd = to_dev(w, dev), to_dev(x, dev)
    y = ops.gemm_q(wd, O.Q4_K, xd, N, K)
    y2 = ops.gemm_q(wd, O.Q4_K, xd, N, K)
    torch.cuda.synchronize()
    ref = O.ref_gemv(x.astype(np.float64), O.np_dequant(O.Q4_K, w).reshape(N, K))
    assert rel_err(y.cpu().numpy(), ref) <= TOL_F32
    assert torch.equal(y.view(torch.int32), y2.view(torch.int32))


def test_config3_q4_k_prefill_5120x13824(dev):
    """C3's second shape at M = 512: Q4_K 5120 x 13824 (the down projection),
    fp16 activations.  40 x 4 = 160 tiles of 128 x 128 on a 256-CU MI355X,
    so the narrow-tile kernel (vkf_gemm_q4_k_f16_n5, 256 tiles of 128 x 80),
    the route bench.py times.  All 512 activation rows against the oracle on
    514 weight rows."""
    import torch
    from vkflame_amd import ops
    N, K, M = 5120, 13824, 512
    assert _split_k_route(M, N, torch.cuda.get_device_properties(0).multi_processor_count)
    w = O.gen_weight(O.Q4_K, N, K, seed_for(3, 5))
    x = _f16(np.random.default_rng(seed_for(3, 517)), M, K)
    y = ops.gemm_q(to_dev(w, dev), O.Q4_K, to_dev(x, dev), N, K).cpu().numpy()
    torch.cuda.synchronize()
    rows = np.concatenate([[0, N - 1], np.random.default_rng(6).choice(N, 512, replace=False)])
    wd = O.np_dequant(O.Q4_K, w[rows]).reshape(len(rows), K)
    assert rel_err(y[:, rows], O.ref_gemv(x.astype(np.float64), wd)) <= TOL_F32


@pytest.mark.parametrize("M,N,K", [(64, 300, 5120), (100, 203, 1056), (17, 130, 32)])
def test_q8_0_q8_1_int8_partials_exact(dev, M, N, K):
    """The integer core of the Q8_0 x Q8_1 prefill on the int8 matrix cores
    (the GEMM's own MFMA code path): every block dot bit-exact against the
    oracle, including K not a multiple of the 4-block step (K = 1056: rows of
    33 blocks, so Q8_0 rows start 2 bytes off 4-byte alignment every other
    row) and a single block."""
    import torch
    from vkflame_amd import ops
    w = O.gen_weight(O.Q8_0, N, K, seed_for(3, 130) + K)
    x = np.random.default_rng(seed_for(3, 131) + K).normal(0, 1, (M, K)).astype(np.float32)
    xq = O.np_quantize_q8_1(x).reshape(M, -1)
    P = ops.q8_0_q81_partials(to_dev(w, dev), to_dev(xq, dev), M, N, K)
    torch.cuda.synchronize()
    ref = O.np_q8_0_q8_1_partials(w, xq, M, N, K)
    got = P.cpu().numpy()
    assert np.array_equal(got, ref), int((got != ref).sum())


@pytest.mark.parametrize("M,N,K", [(512, 5120, 5120), (100, 203, 1056), (300, 1000, 4096)])
def test_q8_0_q8_1_int8_prefill(dev, M, N, K):
    """Q8_0 weights x Q8_1 activations at M > 16: exact block dots scaled by
    dx*dw in fp32, against the float64 product of the dequantised operands
    (which the exact dots reproduce up to the fp32 scaling and sum)."""
    import torch
    from vkflame_amd import ops
    w = O.gen_weight(O.Q8_0, N, K, seed_for(3, 132) + K)
    x = np.random.default_rng(seed_for(3, 133) + K).normal(0, 1, (M, K)).astype(np.float32)
    xq = O.np_quantize_q8_1(x).reshape(M, -1)
    y = ops.gemm_q(to_dev(w, dev), O.Q8_0, to_dev(xq, dev), N, K)
    torch.cuda.synchronize()
    rows = np.arange(N) if N <= 1000 else np.concatenate([[0, N - 1], np.random.default_rng(9).choice(N, 510, False)])
    x64 = O.np_dequant(O.Q8_1, xq).reshape(M, K).astype(np.float64)
    ref = O.ref_gemv(x64, O.np_dequant(O.Q8_0, w[rows]).reshape(len(rows), K))
    err = rel_err(y.cpu().numpy()[:, rows], ref)
    assert err <= 1e-5, err  # fp32 rounding of the scaled sums only
