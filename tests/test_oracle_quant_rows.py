"""CPU: the per-row symmetric int8 quantiser of the oracle (the rule of the
reference's weight quantiser, tools/quantise.py:35-41), pinned by hand-worked
rows, by the reference's own expression evaluated in torch on the CPU, and by
the C restatement against its numpy twin."""
import numpy as np
import pytest
import torch

import oracle as O


def test_kat_rows():
    x = np.array([[127.0, -127.0, 0.5, 1.5, 2.5, -0.5, 126.4, -3.5],
                  [0.0] * 8,
                  [2.0, -1.0, 0.5, 0.0, 1.0, -2.0, 0.25, 1.5]], dtype=np.float32)
    q, s = O.np_quantize_rows_i8(x)
    # row 0: scale exactly 1, ties to even (0.5 -> 0, 1.5 -> 2, 2.5 -> 2, -3.5 -> -4)
    assert s[0] == np.float32(1.0)
    assert q[0].tolist() == [127, -127, 0, 2, 2, 0, 126, -4]
    # zero row: the scale clamps to 1e-8 and every code is 0
    assert s[1] == np.float32(1e-8) and not q[1].any()
    # row 2: scale 2/127; the extremes map to +-127
    assert s[2] == np.float32(2.0) / np.float32(127.0)
    assert q[2, 0] == 127 and q[2, 5] == -127
    for fn in (O.np_quantize_rows_i8, O.c_quantize_rows_i8):
        qq, ss = fn(x)
        assert np.array_equal(qq, q) and np.array_equal(ss.view(np.uint32), s.view(np.uint32))


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_matches_reference_expression_in_torch(seed):
    """tools/quantise.py:35-41 evaluated by torch (fp32, CPU) on the same rows."""
    rng = np.random.default_rng(seed)
    x = (rng.normal(0, 1, (37, 301)) * rng.uniform(1e-3, 10, (37, 1))).astype(np.float32)
    x[5] = 0.0
    w = torch.from_numpy(x)
    scale = (w.abs().max(dim=1).values / 127.0).clamp(min=1e-8)
    qt = (w / scale.unsqueeze(1)).round().clamp(-127, 127).to(torch.int8)
    q, s = O.np_quantize_rows_i8(x)
    assert np.array_equal(s.view(np.uint32), scale.numpy().view(np.uint32))
    assert np.array_equal(q, qt.numpy())
    qc, sc = O.c_quantize_rows_i8(x)
    assert np.array_equal(qc, q) and np.array_equal(sc.view(np.uint32), s.view(np.uint32))


def test_invariants():
    rng = np.random.default_rng(7)
    x = rng.normal(0, 3, (64, 512)).astype(np.float32)
    q, s = O.np_quantize_rows_i8(x)
    assert np.abs(q.astype(np.int32)).max() <= 127
    assert (np.abs(q).max(axis=1) == 127).all()                   # each row's extreme hits +-127
    err = np.abs(q.astype(np.float64) * s[:, None] - x)
    assert (err <= 0.5 * s[:, None] * (1 + 1e-6)).all()           # round-to-nearest bound
