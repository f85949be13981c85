"""GPU: the HIP library reproduces the committed golden fixtures bit for bit."""
import os

import numpy as np
import pytest

import oracle as O
from _util import to_dev

pytestmark = pytest.mark.gpu
FIX = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "fixtures.npz")


@pytest.fixture(scope="module")
def fx():
    return np.load(FIX, allow_pickle=False)


@pytest.mark.parametrize("qt", range(8), ids=[O.QNAMES[q] for q in range(8)])
def test_dequant_fixtures(dev, fx, qt):
    import torch
    from vkflame_amd import ops
    n = O.QNAMES[qt]
    b = to_dev(fx[f"{n}_blocks"], dev)
    y32 = ops.dequant(b, qt, torch.float32)
    y16 = ops.dequant(b, qt, torch.float16)
    torch.cuda.synchronize()
    assert np.array_equal(y32.cpu().numpy().view(np.uint32), fx[f"{n}_f32"].view(np.uint32))
    assert np.array_equal(y16.cpu().numpy().view(np.uint16), fx[f"{n}_f16"].view(np.uint16))


def test_q8_1_and_int_fixtures(dev, fx):
    import torch
    from vkflame_amd import ops
    from vkflame_amd._lib import DTYPE_INT8_INT32OUT
    q = ops.quantize_q8_1(to_dev(fx["quant_x"], dev))
    A, B = fx["i8_A"], fx["i8_B"]
    C = ops.linear(to_dev(A, dev), to_dev(B, dev), A.shape[0], B.shape[0], A.shape[1], DTYPE_INT8_INT32OUT, transB=1)
    P = ops.q6k_q81_partials(to_dev(fx["q6k_w"], dev), to_dev(fx["q6k_xq"], dev), 3, 6, 512)
    torch.cuda.synchronize()
    assert np.array_equal(q.cpu().numpy(), fx["quant_blocks"])
    assert np.array_equal(C.cpu().numpy(), fx["i8_C"])
    assert np.array_equal(P.cpu().numpy(), fx["q6k_P"])
