"""GPU parity: dequantisers and the Q8_1 quantizer, bit-exact against the
oracle (vkflame_dispatch_dequant / vkflame_quantize_q8_1 through the C ABI)."""
import numpy as np
import pytest

import oracle as O
from _util import bits_equal, first_mismatch, seed_for, to_dev

pytestmark = pytest.mark.gpu

ALL = [O.Q4_0, O.Q4_1, O.Q8_0, O.Q5_0, O.Q4_K, O.Q5_K, O.Q6_K, O.Q8_1]


def _blocks(qt, n, seed):
    rng = np.random.default_rng(seed)
    return np.concatenate([O.gen_blocks(qt, n, rng), O.special_blocks(qt)])


@pytest.mark.parametrize("qt", ALL, ids=[O.QNAMES[q] for q in ALL])
@pytest.mark.parametrize("f16", [False, True], ids=["f32", "f16"])
def test_dequant_bit_exact(dev, qt, f16):
    import torch
    from vkflame_amd import ops
    b = _blocks(qt, 3001, seed_for(0, qt))
    out = ops.dequant(to_dev(b, dev), qt, torch.float16 if f16 else torch.float32)
    torch.cuda.synchronize()
    ref = O.c_dequant(qt, b, out_f16=f16)
    got = out.cpu().numpy()
    assert bits_equal(got, ref), first_mismatch(got, ref)


@pytest.mark.parametrize("qt", [O.Q4_0, O.Q8_0, O.Q5_0, O.Q6_K], ids=["q4_0", "q8_0", "q5_0", "q6_k"])
def test_dequant_suballocated_source(dev, qt):
    """Sources at a 2-byte offset inside a larger allocation (the reference
    needs exact VkBuffer base pointers, shim/hip_runtime_shim.cpp:875-881)."""
    import torch
    from vkflame_amd import ops
    b = _blocks(qt, 257, seed_for(0, 20 + qt))
    buf = np.zeros(b.size + 2, np.uint8)
    buf[2:] = b.reshape(-1)
    d = to_dev(buf, dev)
    out = ops.dequant(d[2:], qt, torch.float32, n_blocks=b.shape[0])
    torch.cuda.synchronize()
    assert bits_equal(out.cpu().numpy(), O.c_dequant(qt, b))


def test_dequant_full_q8_0_config(dev):
    """C1 weights (4096x4096 Q8_0), every element."""
    import torch
    from vkflame_amd import ops
    w = O.gen_weight(O.Q8_0, 4096, 4096, seed_for(1))
    out = ops.dequant(to_dev(w, dev), O.Q8_0, torch.float32)
    torch.cuda.synchronize()
    assert bits_equal(out.cpu().numpy(), O.np_dequant(O.Q8_0, w))


def test_dequant_rejects_bad_arguments(dev):
    import ctypes
    from vkflame_amd import lib
    L = lib()
    assert L.vkflame_dispatch_dequant(None, None, 1, 99, 0, None) == 1
    assert L.vkflame_dispatch_dequant(None, None, 1, 0, 7, None) == 1
    assert L.vkflame_dispatch_dequant(ctypes.c_void_p(16), ctypes.c_void_p(17), 1, 0, 0, None) == 1  # dst misaligned
    assert L.vkflame_dispatch_dequant(None, None, 0, 0, 0, None) == 0  # empty is a no-op


def _q81_inputs(seed):
    rng = np.random.default_rng(seed)
    x = rng.normal(0, 1, (37, 512)).astype(np.float32)
    x[0] = 0.0                                      # amax == 0 -> d == 0, q == 0
    x[1] = rng.normal(0, 1e-6, 512)                 # tiny values (d far below fp16 normal)
    x[2] = rng.normal(0, 3e4, 512)                  # large values
    x[3, :32] = np.arange(32, dtype=np.float32) - 15.5  # exact .5 multiples
    x[4, :32] = 127.0 * (np.arange(32, dtype=np.float32) - 16) / 16.0
    x[5] = -x[5]
    x[6, ::2] = 0.0
    return x


def test_quantize_q8_1_bit_exact(dev):
    from vkflame_amd import ops
    import torch
    x = _q81_inputs(seed_for(5, 1))
    q = ops.quantize_q8_1(to_dev(x, dev))
    torch.cuda.synchronize()
    ref = O.c_quantize_q8_1(x).reshape(x.shape[0], -1)
    assert bits_equal(q.cpu().numpy(), ref), first_mismatch(q.cpu().numpy(), ref)


def test_quantize_q8_1_strided_rows(dev):
    from vkflame_amd import ops
    import torch
    x = np.random.default_rng(seed_for(5, 2)).normal(0, 1, (9, 320)).astype(np.float32)
    xd = to_dev(x, dev)[:, :256]               # row stride 320 elements
    q = ops.quantize_q8_1(xd)
    torch.cuda.synchronize()
    ref = O.c_quantize_q8_1(np.ascontiguousarray(x[:, :256])).reshape(9, -1)
    assert bits_equal(q.cpu().numpy(), ref)


def test_quantize_q8_1_full_config(dev):
    """C5 activations fp32 [512, 5120] ~ N(0,1)."""
    from vkflame_amd import ops
    import torch
    x = np.random.default_rng(seed_for(5)).normal(0, 1, (512, 5120)).astype(np.float32)
    q = ops.quantize_q8_1(to_dev(x, dev))
    torch.cuda.synchronize()
    assert bits_equal(q.cpu().numpy().reshape(-1), O.np_quantize_q8_1(x))
