"""GPU: weights read from a GGUF file feed the GEMV / GEMM directly (no
repacking), matching the oracle on the same blocks."""
import numpy as np
import pytest

import oracle as O
from _util import TOL_F32, rel_err, seed_for, to_dev

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("qt,M", [(O.Q4_K, 1), (O.Q4_K, 64), (O.Q6_K, 1), (O.Q4_0, 4), (O.Q8_0, 1)])
def test_gguf_weight_to_gemm(dev, tmp_path, qt, M):
    import torch
    from vkflame_amd import gguf as G
    from vkflame_amd import ops
    N, K = 1000, 2048
    b = O.gen_weight(qt, N, K, seed_for(7, qt))
    p = str(tmp_path / "w.gguf")
    G.write_gguf(p, {"blk.0.ffn_up.weight": (G.GGML_OF_LIBRARY[qt], (K, N), b)}, {"general.architecture": "test"})
    w, q, NN, KK = G.GGUFFile(p).weight_to_device("blk.0.ffn_up.weight", dev)
    assert (q, NN, KK) == (qt, N, K)
    x = np.random.default_rng(seed_for(7, 10 + qt)).normal(0, 1, (M, K)).astype(np.float32)
    if qt == O.Q6_K:
        xq = ops.quantize_q8_1(to_dev(x, dev))
        y = ops.gemm_q(w, q, xq, N, K)
        xr = O.np_dequant(O.Q8_1, O.np_quantize_q8_1(x)).reshape(M, K)
    else:
        y = ops.gemm_q(w, q, to_dev(x.astype(np.float16), dev), N, K)
        xr = x.astype(np.float16)
    torch.cuda.synchronize()
    ref = O.ref_gemv(xr.astype(np.float64), O.np_dequant(qt, b.reshape(-1)).reshape(N, K))
    assert rel_err(y.cpu().numpy(), ref) <= TOL_F32
