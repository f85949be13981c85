"""CPU: the oracle reproduces the committed golden fixtures bit for bit."""
import os

import numpy as np
import pytest

import oracle as O

FIX = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "fixtures.npz")


@pytest.fixture(scope="module")
def fx():
    return np.load(FIX, allow_pickle=False)


@pytest.mark.parametrize("qt", range(8), ids=[O.QNAMES[q] for q in range(8)])
def test_dequant_fixtures(fx, qt):
    n = O.QNAMES[qt]
    b = fx[f"{n}_blocks"]
    assert np.array_equal(O.c_dequant(qt, b).view(np.uint32), fx[f"{n}_f32"].view(np.uint32))
    assert np.array_equal(O.c_dequant(qt, b, True).view(np.uint16), fx[f"{n}_f16"].view(np.uint16))
    assert np.array_equal(O.np_dequant(qt, b).view(np.uint32), fx[f"{n}_f32"].view(np.uint32))


def test_q8_1_fixture(fx):
    assert np.array_equal(O.c_quantize_q8_1(fx["quant_x"]).reshape(fx["quant_x"].shape[0], -1), fx["quant_blocks"])


def test_int_fixtures(fx):
    assert np.array_equal(O.c_gemm_i8_nt(fx["i8_A"], fx["i8_B"]), fx["i8_C"])
    assert np.array_equal(O.c_q6k_q8_1_partials(fx["q6k_w"], fx["q6k_xq"], 3, 6, 512), fx["q6k_P"])
