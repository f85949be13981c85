"""CPU: the PyTorch front end (vkflame_amd.torch_mode) leaves CPU tensors to
PyTorch, and its CPU weight quantiser follows the reference's rule
(tools/quantise.py:35-41) bit for bit (checked against the oracle)."""
import numpy as np
import torch

import oracle as O
from vkflame_amd import torch_mode as TM


def test_cpu_tensors_fall_through():
    a = torch.randn(8, 16).half()
    b = torch.randn(16, 4).half()
    lin = torch.nn.Linear(16, 4).half()
    with TM.install() as mode:
        y = a.float() @ b.float()
        z = lin(a)
        w = torch.mm(a, b)
    assert mode.calls == {}
    assert torch.equal(y, a.float() @ b.float())
    assert z.shape == (8, 4) and w.shape == (8, 4)


def test_handler_table_names_aten_matmuls():
    names = sorted(op.overloadpacket.__name__ for op in TM._HANDLERS)
    assert names == ["_int_mm", "addmm", "linear", "mm"]


def test_quantise_weight_cpu_matches_oracle():
    rng = np.random.default_rng(11)
    w = (rng.normal(0, 0.02, (48, 96)) * rng.uniform(0.1, 3, (48, 1))).astype(np.float32)
    w[3] = 0.0
    q, s = TM.quantise_weight(torch.from_numpy(w).half())
    qo, so = O.np_quantize_rows_i8(torch.from_numpy(w).half().float().numpy())
    assert np.array_equal(q.numpy(), qo)
    assert np.array_equal(s.numpy(), so.astype(np.float16))


def test_quantise_linears_replaces_every_linear():
    m = torch.nn.Sequential(torch.nn.Linear(32, 64), torch.nn.ReLU(),
                            torch.nn.Sequential(torch.nn.Linear(64, 16, bias=False)))
    assert TM.quantise_linears_(m) == 2
    kinds = [type(x).__name__ for x in m.modules()]
    assert kinds.count("Int8Linear") == 2 and "Linear" not in kinds
    l0 = m[0]
    assert l0.weight_int8.dtype == torch.int8 and l0.weight_scale.dtype == torch.float16
    assert l0.weight_int8.shape == (64, 32) and l0.bias.dtype == torch.float16
