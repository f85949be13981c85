"""Writes tests/golden/fixtures.npz: small frozen input/output vectors.

The reference ships no golden vectors for this path (SURVEY: its tests cover
fp16 GEMM only), so these fixtures freeze the oracle's outputs on seeded and
hand-built inputs after the oracle itself has been pinned by
tests/test_oracle_*.py.  They anchor later rounds (a change to the oracle or
the kernels that moves a bit fails tests/test_golden.py and
tests/test_gpu_golden.py).  Data only: numpy arrays, no pickles.

Run: python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "..", "..", "oracle"))
import oracle as O  # noqa: E402


def main():
    out = {}
    for qt in range(8):
        name = O.QNAMES[qt]
        rng = np.random.default_rng(9000 + qt)
        b = np.concatenate([O.gen_blocks(qt, 6, rng), O.special_blocks(qt)[::4]])
        out[f"{name}_blocks"] = b
        out[f"{name}_f32"] = O.c_dequant(qt, b)
        out[f"{name}_f16"] = O.c_dequant(qt, b, out_f16=True)
    rng = np.random.default_rng(9100)
    x = np.concatenate([rng.normal(0, 1, 32 * 13), np.zeros(32), np.arange(32) - 15.5,
                        rng.normal(0, 1e-6, 32)]).astype(np.float32).reshape(-1, 64)
    out["quant_x"] = x
    out["quant_blocks"] = O.c_quantize_q8_1(x).reshape(x.shape[0], -1)
    A = rng.integers(-127, 128, (20, 96), dtype=np.int8)
    B = rng.integers(-127, 128, (12, 96), dtype=np.int8)
    out["i8_A"], out["i8_B"], out["i8_C"] = A, B, O.c_gemm_i8_nt(A, B)
    w = O.gen_weight(O.Q6_K, 6, 512, 9200)
    xq = O.c_quantize_q8_1(rng.normal(0, 1, (3, 512)).astype(np.float32)).reshape(3, -1)
    out["q6k_w"], out["q6k_xq"], out["q6k_P"] = w, xq, O.c_q6k_q8_1_partials(w, xq, 3, 6, 512)
    np.savez_compressed(os.path.join(HERE, "fixtures.npz"), **out)
    print("wrote", os.path.join(HERE, "fixtures.npz"), sum(v.nbytes for v in out.values()), "bytes")


if __name__ == "__main__":
    main()
