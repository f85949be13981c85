"""GPU parity: the PyTorch front end (vkflame_amd.torch_mode) routes aten
matmuls and int8 layers to the library, and the per-row int8 quantiser
(vkflame_quantize_rows_i8) matches the oracle bit for bit."""
import numpy as np
import pytest

import oracle as O
from _util import TOL_F16, bits_equal, first_mismatch, rel_err, seed_for, to_dev

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("M,K,dt,ldpad", [(1, 5120, "f16", 0), (37, 301, "f32", 0), (64, 4096, "f16", 24),
                                          (300, 1000, "f32", 8)])
def test_quantize_rows_i8(dev, M, K, dt, ldpad):
    import torch
    from vkflame_amd import ops
    rng = np.random.default_rng(seed_for(6, M))
    x = (rng.normal(0, 1, (M, K + ldpad)) * rng.uniform(1e-3, 20, (M, 1))).astype(np.float32)
    if M > 2:
        x[2] = 0.0
    x[0, 3] = 127.0 * 3.5 / max(np.abs(x[0]).max(), 1.0)  # a value that often lands on a .5 tie
    if dt == "f16":
        x = x.astype(np.float16)
    xd = to_dev(x, dev)[:, :K]
    q, s = ops.quantize_rows_i8(xd)
    torch.cuda.synchronize()
    qo, so = O.np_quantize_rows_i8(x[:, :K].astype(np.float32))
    assert bits_equal(s.cpu().numpy(), so), first_mismatch(s.cpu().numpy(), so)
    assert np.array_equal(q.cpu().numpy(), qo)


def test_mode_linear_and_mm(dev):
    import torch
    import torch.nn.functional as F
    from vkflame_amd import torch_mode as TM
    g = torch.Generator().manual_seed(seed_for(6, 1))
    x = torch.randn(4, 50, 640, generator=g).half().to(dev)
    w = (torch.randn(1000, 640, generator=g) * 0.05).half().to(dev)
    b = torch.randn(1000, generator=g).half().to(dev)
    a2 = torch.randn(200, 640, generator=g).half().to(dev)
    u = torch.randn(640, 333, generator=g).half().to(dev)
    with TM.install() as mode:
        y = F.linear(x, w, b)               # decomposes to addmm(b, x2, w.t()): transB, no copy
        z = torch.mm(a2, w.t())             # transposed view -> transB
        v = torch.mm(u.t(), w[:, :640][:1000].t())   # u.t(): transA
    torch.cuda.synchronize()
    assert sum(mode.calls.values()) >= 3, mode.calls
    ref_y = (x.float() @ w.float().t() + b.float())
    assert y.dtype == torch.float16 and rel_err(y.float().cpu().numpy(), ref_y.cpu().numpy()) <= TOL_F16
    ref_z = a2.float() @ w.float().t()
    assert rel_err(z.float().cpu().numpy(), ref_z.cpu().numpy()) <= TOL_F16
    ref_v = u.t().float() @ w.float().t()
    assert rel_err(v.float().cpu().numpy(), ref_v.cpu().numpy()) <= TOL_F16


def test_mode_addmm_full_c_and_scalars(dev):
    import torch
    from vkflame_amd import torch_mode as TM
    g = torch.Generator().manual_seed(seed_for(6, 2))
    a = torch.randn(130, 256, generator=g).half().to(dev)
    bt = torch.randn(96, 256, generator=g).half().to(dev)   # b = bt.t(): transB
    c = torch.randn(130, 96, generator=g).half().to(dev)
    at = torch.randn(256, 130, generator=g).half().to(dev)  # a2 = at.t(): transA
    with TM.install() as mode:
        y = torch.addmm(c, a, bt.t(), beta=0.5, alpha=2.0)
        y2 = torch.addmm(c[0], at.t(), bt.t())
    torch.cuda.synchronize()
    assert mode.calls.get("addmm") == 2
    ref = 0.5 * c.float() + 2.0 * (a.float() @ bt.float().t())
    assert rel_err(y.float().cpu().numpy(), ref.cpu().numpy()) <= TOL_F16
    ref2 = c[0].float() + at.t().float() @ bt.float().t()
    assert rel_err(y2.float().cpu().numpy(), ref2.cpu().numpy()) <= TOL_F16


def test_mode_fp32_and_int_mm(dev):
    import torch
    from vkflame_amd import torch_mode as TM
    rng = np.random.default_rng(seed_for(6, 3))
    A = rng.integers(-127, 128, (64, 512)).astype(np.int8)
    B = rng.integers(-127, 128, (512, 96)).astype(np.int8)
    a32 = torch.randn(16, 32, device=dev)
    with TM.install() as mode:
        r32 = a32 @ a32.t()                 # fp32: PyTorch's own
        c = torch._int_mm(to_dev(A, dev), to_dev(B, dev))
    torch.cuda.synchronize()
    assert mode.calls == {"_int_mm": 1}
    assert c.dtype == torch.int32
    assert np.array_equal(c.cpu().numpy(), A.astype(np.int64) @ B.astype(np.int64))
    assert r32.shape == (16, 16)


def test_int8_linear_layer(dev):
    """Int8Linear: GPU weight quantisation equals the oracle's; the forward is
    the int8 linear's epilogue float(acc) * a_scale * w_scale + bias in fp32,
    rounded to fp16, bit for bit against a numpy restatement on the same
    quantised operands, and within int8 quantisation error of the fp32 layer."""
    import torch
    from vkflame_amd import torch_mode as TM
    g = torch.Generator().manual_seed(seed_for(6, 4))
    lin = torch.nn.Linear(1024, 768).half()
    with torch.no_grad():
        lin.weight.copy_((torch.randn(768, 1024, generator=g) * 0.03).half())
        lin.bias.copy_((torch.randn(768, generator=g) * 0.1).half())
    lin = lin.to(dev)
    ql = TM.Int8Linear.from_linear(lin)
    qo, so = O.np_quantize_rows_i8(lin.weight.detach().float().cpu().numpy())
    assert np.array_equal(ql.weight_int8.cpu().numpy(), qo)
    assert np.array_equal(ql.weight_scale.cpu().numpy(), so.astype(np.float16))
    x = torch.randn(3, 41, 1024, generator=g).half().to(dev)
    with torch.no_grad():
        y = ql(x)
    torch.cuda.synchronize()
    assert y.shape == (3, 41, 768) and y.dtype == torch.float16
    aq, as_ = O.np_quantize_rows_i8(x.reshape(-1, 1024).float().cpu().numpy())
    acc = aq.astype(np.int64) @ qo.astype(np.int64).T
    ws = so.astype(np.float16).astype(np.float32)
    v = (acc.astype(np.float32) * as_[:, None]).astype(np.float32)
    v = (v * ws[None, :]).astype(np.float32)
    v = (v + lin.bias.detach().float().cpu().numpy()[None, :]).astype(np.float32)
    ref = v.astype(np.float16)
    got = y.reshape(-1, 768).cpu().numpy()
    assert bits_equal(got, ref), first_mismatch(got, ref)
    full = (x.float() @ lin.weight.detach().float().t() + lin.bias.detach().float()).reshape(-1, 768).cpu().numpy()
    assert rel_err(got.astype(np.float32), full) <= 2e-2
