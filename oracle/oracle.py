"""CPU oracle for vkflame's quantized-linear path — TEST INFRASTRUCTURE ONLY.

Only tests/, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline leg
may import this module, and only as the checker.  The shipped library never
imports, links or calls it.

Two restatements of the same arithmetic live here:

* ``C`` — ctypes binding of ``oracle/libvkf_oracle.so`` (vkf_oracle.c), a
  scalar restatement of the reference's GLSL formulas, built with
  ``-ffp-contract=off``;
* the numpy twin (``np_dequant``, ``np_quantize_q8_1``, ...), vectorised for
  the timed CPU baseline.  tests/test_oracle_*.py check the two bit-for-bit.

Block formats and element order follow the reference shaders
(kernels/dequant_*.glsl, cited per function); generators follow the seeded
input recipes of the benchmark configurations.
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))

# Quant type codes: the reference's VKF_DEQUANT_* (runtime/dispatch.h:14-21).
Q4_0, Q4_1, Q8_0, Q5_0, Q4_K, Q5_K, Q6_K, Q8_1 = range(8)
QNAMES = {Q4_0: "q4_0", Q4_1: "q4_1", Q8_0: "q8_0", Q5_0: "q5_0",
          Q4_K: "q4_k", Q5_K: "q5_k", Q6_K: "q6_k", Q8_1: "q8_1"}
BLOCK_BYTES = {Q4_0: 18, Q4_1: 20, Q8_0: 34, Q5_0: 22, Q4_K: 144, Q5_K: 176,
               Q6_K: 210, Q8_1: 36}
BLOCK_ELEMS = {Q4_0: 32, Q4_1: 32, Q8_0: 32, Q5_0: 32, Q4_K: 256, Q5_K: 256,
               Q6_K: 256, Q8_1: 32}


# --------------------------------------------------------------------------
# C restatement (ctypes)
# --------------------------------------------------------------------------

class _C:
    _lib = None

    @classmethod
    def lib(cls):
        if cls._lib is None:
            path = os.path.join(HERE, "libvkf_oracle.so")
            if not os.path.exists(path):
                raise RuntimeError(f"oracle not built: {path} (run make -C oracle)")
            lib = ctypes.CDLL(path)
            P = ctypes.c_void_p
            lib.vkfo_h2f.argtypes = [ctypes.c_uint16]
            lib.vkfo_h2f.restype = ctypes.c_float
            lib.vkfo_f2h.argtypes = [ctypes.c_float]
            lib.vkfo_f2h.restype = ctypes.c_uint16
            lib.vkfo_dequant_f32.argtypes = [ctypes.c_int, P, ctypes.c_size_t, P]
            lib.vkfo_dequant_f16.argtypes = [ctypes.c_int, P, ctypes.c_size_t, P]
            lib.vkfo_quantize_q8_1.argtypes = [P, ctypes.c_size_t, P]
            lib.vkfo_quantize_q8_1.restype = None
            lib.vkfo_quantize_rows_i8.argtypes = [P, ctypes.c_int, ctypes.c_int, P, P]
            lib.vkfo_quantize_rows_i8.restype = None
            lib.vkfo_gemm_i8_nt.argtypes = [P, P, P, ctypes.c_int, ctypes.c_int, ctypes.c_int]
            lib.vkfo_q6k_q8_1_partials.argtypes = [P, P, P, ctypes.c_int, ctypes.c_int, ctypes.c_int]
            lib.vkfo_q6k_q8_1_partials.restype = None
            lib.vkfo_act.argtypes = [ctypes.c_int, ctypes.c_float]
            lib.vkfo_act.restype = ctypes.c_float
            cls._lib = lib
        return cls._lib


def _ptr(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.c_void_p)


def c_h2f(h: int) -> float:
    return _C.lib().vkfo_h2f(h)


def c_f2h(f: float) -> int:
    return _C.lib().vkfo_f2h(f)


def c_dequant(qtype: int, blocks: np.ndarray, out_f16: bool = False) -> np.ndarray:
    """Dequantise a uint8 array of whole blocks; returns flat fp32 (or fp16)."""
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    nb = blocks.size // BLOCK_BYTES[qtype]
    assert nb * BLOCK_BYTES[qtype] == blocks.size
    n = nb * BLOCK_ELEMS[qtype]
    if out_f16:
        out = np.empty(n, dtype=np.float16)
        rc = _C.lib().vkfo_dequant_f16(qtype, _ptr(blocks), nb, _ptr(out))
    else:
        out = np.empty(n, dtype=np.float32)
        rc = _C.lib().vkfo_dequant_f32(qtype, _ptr(blocks), nb, _ptr(out))
    assert rc == 0
    return out


def c_quantize_q8_1(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    assert x.size % 32 == 0
    out = np.empty(x.size // 32 * 36, dtype=np.uint8)
    _C.lib().vkfo_quantize_q8_1(_ptr(x), x.size, _ptr(out))
    return out


def c_quantize_rows_i8(x: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Per-row symmetric int8 quantiser (tools/quantise.py:35-41 rule)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    M, K = x.shape
    q = np.empty((M, K), dtype=np.int8)
    scale = np.empty(M, dtype=np.float32)
    _C.lib().vkfo_quantize_rows_i8(_ptr(x), M, K, _ptr(q), _ptr(scale))
    return q, scale


def c_gemm_i8_nt(A: np.ndarray, B: np.ndarray) -> np.ndarray:
    A = np.ascontiguousarray(A, dtype=np.int8)
    B = np.ascontiguousarray(B, dtype=np.int8)
    M, K = A.shape
    N = B.shape[0]
    C = np.empty((M, N), dtype=np.int32)
    rc = _C.lib().vkfo_gemm_i8_nt(_ptr(A), _ptr(B), _ptr(C), M, N, K)
    assert rc == 0, "int32 overflow"
    return C


def c_q6k_q8_1_partials(w: np.ndarray, xq: np.ndarray, M: int, N: int, K: int) -> np.ndarray:
    w = np.ascontiguousarray(w, dtype=np.uint8)
    xq = np.ascontiguousarray(xq, dtype=np.uint8)
    P = np.empty((M, N, K // 32), dtype=np.int32)
    _C.lib().vkfo_q6k_q8_1_partials(_ptr(w), _ptr(xq), _ptr(P), M, N, K)
    return P


def np_q8_0_q8_1_partials(w: np.ndarray, xq: np.ndarray, M: int, N: int, K: int) -> np.ndarray:
    """Exact integer block dots of Q8_0 weights [N, K] x Q8_1 activations
    [M, K]: P[m, n, kb] = sum over block kb of q8x * q8w (the integer core of
    ggml's vec_dot_q8_0_q8_1; codes at byte 2 of a Q8_0 block,
    kernels/dequant_q8_0.glsl:23-27, and byte 4 of a Q8_1 block,
    kernels/dequant_q8_1.glsl:26-31)."""
    nb = K // 32
    qw = np.ascontiguousarray(w, np.uint8).reshape(N, nb, 34)[:, :, 2:34].view(np.int8).astype(np.int64)
    qx = np.ascontiguousarray(xq, np.uint8).reshape(M, nb, 36)[:, :, 4:36].view(np.int8).astype(np.int64)
    return np.einsum("mbk,nbk->mnb", qx, qw).astype(np.int32)


def c_act(act: int, x: float) -> float:
    return _C.lib().vkfo_act(act, x)


# --------------------------------------------------------------------------
# numpy twin (vectorised; same arithmetic in float32)
# --------------------------------------------------------------------------

F32 = np.float32


def _h(b: np.ndarray, off: int) -> np.ndarray:
    """fp16 field at byte offset ``off`` of every block row -> float32."""
    return b[:, off:off + 2].copy().view(np.float16).reshape(-1).astype(F32)


def scale_min_k4(s: np.ndarray):
    """get_scale_min_k4 for all 8 sub-blocks (kernels/dequant_q4_k.glsl:16-24).
    s: (nb, 12) uint8 -> sc, m: (nb, 8) uint32."""
    s = s.astype(np.uint32)
    sc = np.empty((s.shape[0], 8), np.uint32)
    mn = np.empty((s.shape[0], 8), np.uint32)
    sc[:, :4] = s[:, 0:4] & 63
    mn[:, :4] = s[:, 4:8] & 63
    sc[:, 4:] = (s[:, 8:12] & 0xF) | ((s[:, 0:4] >> 6) << 4)
    mn[:, 4:] = (s[:, 8:12] >> 4) | ((s[:, 4:8] >> 6) << 4)
    return sc, mn


def q6k_fields(b: np.ndarray):
    """(v - 32, scale index) for all 256 elements of every Q6_K block
    (kernels/dequant_q6_k.glsl:19-58); returns v (nb,256) int32, sc (nb,256)."""
    nb = b.shape[0]
    ql = b[:, 0:128].astype(np.int32)
    qh = b[:, 128:192].astype(np.int32)
    scales = b[:, 192:208].view(np.int8).astype(np.int32)
    v = np.empty((nb, 256), np.int32)
    sci = np.empty(256, np.int64)
    for ip in range(2):
        q0 = ql[:, 64 * ip:64 * ip + 32]
        q32 = ql[:, 64 * ip + 32:64 * ip + 64]
        h = qh[:, 32 * ip:32 * ip + 32]
        base = 128 * ip
        v[:, base + 0:base + 32] = ((q0 & 15) | (((h >> 0) & 3) << 4)) - 32
        v[:, base + 32:base + 64] = ((q32 & 15) | (((h >> 2) & 3) << 4)) - 32
        v[:, base + 64:base + 96] = ((q0 >> 4) | (((h >> 4) & 3) << 4)) - 32
        v[:, base + 96:base + 128] = ((q32 >> 4) | (((h >> 6) & 3) << 4)) - 32
        l = np.arange(32)
        for t in range(4):
            sci[base + 32 * t + l] = 8 * ip + l // 16 + 2 * t
    return v, scales[:, sci]


def np_dequant(qtype: int, blocks: np.ndarray) -> np.ndarray:
    """Vectorised twin of c_dequant (fp32)."""
    bb = BLOCK_BYTES[qtype]
    b = np.ascontiguousarray(blocks, dtype=np.uint8).reshape(-1, bb)
    nb = b.shape[0]
    if qtype in (Q4_0, Q4_1, Q5_0):
        off = {Q4_0: 2, Q4_1: 4, Q5_0: 6}[qtype]
        qs = b[:, off:off + 16]
        q = np.concatenate([qs & 15, qs >> 4], axis=1).astype(np.uint32)
        d = _h(b, 0)[:, None]
        if qtype == Q4_0:
            return (d * q.astype(F32) + (F32(-8.0) * d)).reshape(-1)
        if qtype == Q4_1:
            return (d * q.astype(F32) + _h(b, 2)[:, None]).reshape(-1)
        qh = b[:, 2:6].copy().view(np.uint32).astype(np.uint32)  # (nb,1)
        bits = (qh >> np.arange(32, dtype=np.uint32)[None, :]) & 1
        x = (q | (bits << 4)).astype(F32)
        return (x * d + (F32(-16.0) * d)).reshape(-1)
    if qtype in (Q8_0, Q8_1):
        off = 2 if qtype == Q8_0 else 4
        q = b[:, off:off + 32].view(np.int8).astype(F32)
        return (_h(b, 0)[:, None] * q).reshape(-1)
    if qtype in (Q4_K, Q5_K):
        dall = _h(b, 0)[:, None]
        dmin = _h(b, 2)[:, None]
        sc, mn = scale_min_k4(b[:, 4:16])
        dj = dall * sc.astype(F32)          # (nb, 8), exact
        mj = dmin * mn.astype(F32)
        qoff = 16 if qtype == Q4_K else 48
        qs = b[:, qoff:qoff + 128].reshape(nb, 4, 32).astype(np.uint32)
        lo = qs & 15
        hi = qs >> 4
        if qtype == Q5_K:
            qh = b[:, 16:48].astype(np.uint32)[:, None, :]   # (nb,1,32)
            il = np.arange(4, dtype=np.uint32)[None, :, None]
            lo = lo + ((qh >> (2 * il)) & 1) * 16
            hi = hi + ((qh >> (2 * il + 1)) & 1) * 16
        q = np.stack([lo, hi], axis=2).reshape(nb, 8, 32).astype(F32)  # sub-block j
        y = dj[:, :, None] * q - mj[:, :, None]
        return y.reshape(-1)
    if qtype == Q6_K:
        v, sc = q6k_fields(b)
        d = _h(b, 208)[:, None]
        return (d * (sc * v).astype(F32)).reshape(-1)
    raise ValueError(qtype)


def np_quantize_q8_1(x: np.ndarray) -> np.ndarray:
    """Vectorised twin of c_quantize_q8_1 (ggml quantize_row_q8_1_ref)."""
    xb = np.ascontiguousarray(x, dtype=F32).reshape(-1, 32)
    amax = np.abs(xb).max(axis=1)
    d = (amax / F32(127.0)).astype(F32)
    with np.errstate(divide="ignore"):
        inv = np.where(d != 0, F32(1.0) / np.where(d != 0, d, F32(1.0)), F32(0.0)).astype(F32)
    v = (xb * inv[:, None]).astype(F32).astype(np.float64)
    q = np.trunc(v + np.copysign(0.5, v)).astype(np.int32)     # roundf
    s = (q.sum(axis=1).astype(F32) * d).astype(F32)
    out = np.empty((xb.shape[0], 36), np.uint8)
    out[:, 0:2] = d.astype(np.float16).view(np.uint8).reshape(-1, 2)
    with np.errstate(over="ignore"):
        out[:, 2:4] = s.astype(np.float16).view(np.uint8).reshape(-1, 2)
    out[:, 4:36] = q.astype(np.int8).view(np.uint8)
    return out.reshape(-1)


def np_quantize_rows_i8(x: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Vectorised twin of c_quantize_rows_i8: the reference's per-output-channel
    weight quantiser (tools/quantise.py:35-41) -- scale = max|row|/127 clamped
    to >= 1e-8, q = round(x/scale) (half to even, as torch.round) clamped to
    +-127 -- applied to each row (weights per channel, activations per token)."""
    x = np.ascontiguousarray(x, dtype=F32)
    scale = np.maximum((np.abs(x).max(axis=1) / F32(127.0)).astype(F32), F32(1e-8))
    q = np.clip(np.rint((x / scale[:, None]).astype(F32)), -127, 127).astype(np.int8)
    return q, scale


def np_quantize_act_i8(x: np.ndarray, act_scale: float) -> np.ndarray:
    """Activation quantisation of the reference's int8 linear
    (kernels/linear_int8.glsl:63-70): q = clamp(round(x / act_scale), -127,
    127) on fp16 activations, in float32 with an IEEE division.  GLSL's
    round() leaves halves to the implementation; this build rounds them to
    even (the GPU's v_rndne_f32)."""
    x = np.asarray(x, dtype=np.float16).astype(F32)
    return np.clip(np.rint((x / F32(act_scale)).astype(F32)), -127, 127).astype(np.int8)


def ref_linear_int8_fp16a(A16: np.ndarray, W: np.ndarray, act_scale: float, w_scale, act: int = 0):
    """The reference's int8 linear contract (kernels/linear_int8.glsl:48-101):
    fp16 A quantised by act_scale, int8 W [N, K], exact int32 acc, then
    act(f32(acc) * w_scale[n] * act_scale) (the reference omits act_scale
    from the product and only ever passes 1).  Returns (acc int32, D float32
    before the fp16 rounding)."""
    q = np_quantize_act_i8(A16, act_scale)
    acc = q.astype(np.int64) @ np.asarray(W, np.int64).T
    assert np.abs(acc).max() < 2 ** 31
    ws = np.ones(W.shape[0], F32) if w_scale is None else np.asarray(w_scale, F32)
    y = (acc.astype(np.float64) * ws.astype(np.float64)[None, :] * float(act_scale)).astype(F32)
    return acc.astype(np.int32), np_act(act, y)


def np_act(act: int, x: np.ndarray) -> np.ndarray:
    """Activation epilogue in float32 (kernels/linear_fp16.glsl:22-36)."""
    x = x.astype(F32)
    if act == 1:
        return (x * (F32(1.0) / (F32(1.0) + np.exp(-x)))).astype(F32)
    if act == 2:
        return np.maximum(x, F32(0.0))
    if act == 3:
        t = F32(1.0) / (F32(1.0) + F32(0.3275911) * np.abs(x * F32(0.70710678118654)))
        z = x * F32(0.70710678118654)
        y = F32(1.0) - ((((F32(1.061405429) * t - F32(1.453152027)) * t + F32(1.421413741)) * t
                          - F32(0.284496736)) * t + F32(0.254829592)) * t * np.exp(-z * z)
        erf = np.where(z >= 0, y, -y)
        return (F32(0.5) * x * (F32(1.0) + erf)).astype(F32)
    return x


def ref_gemv(x: np.ndarray, w_deq: np.ndarray) -> np.ndarray:
    """y = x @ W^T in float64 from the exact dequantised operands (the
    reference's intended dequant -> GEMM, shim/hip_runtime_shim.cpp:1127-1166)."""
    return np.asarray(x, np.float64) @ np.asarray(w_deq, np.float64).T


def max_rel_err(y, r) -> float:
    """max|y - r| / max|r|: the tolerance metric for float outputs."""
    y = np.asarray(y, np.float64)
    r = np.asarray(r, np.float64)
    den = np.abs(r).max()
    return float(np.abs(y - r).max() / (den if den > 0 else 1.0))


# --------------------------------------------------------------------------
# seeded generators (benchmark configuration recipes)
# --------------------------------------------------------------------------

def _f16_bytes(v: np.ndarray) -> np.ndarray:
    return np.asarray(v, np.float64).astype(np.float16).view(np.uint8).reshape(-1, 2)


def pack_scale_min_k4(sc: np.ndarray, mn: np.ndarray) -> np.ndarray:
    """Inverse of get_scale_min_k4: 8 six-bit scales and mins -> 12 bytes."""
    sc = sc.astype(np.uint32)
    mn = mn.astype(np.uint32)
    s = np.empty((sc.shape[0], 12), np.uint32)
    s[:, 0:4] = sc[:, 0:4] | ((sc[:, 4:8] >> 4) << 6)
    s[:, 4:8] = mn[:, 0:4] | ((mn[:, 4:8] >> 4) << 6)
    s[:, 8:12] = (sc[:, 4:8] & 15) | ((mn[:, 4:8] & 15) << 4)
    return s.astype(np.uint8)


def gen_blocks(qtype: int, nb: int, rng: np.random.Generator, sigma: float | None = None) -> np.ndarray:
    """nb random blocks of qtype -> uint8 array (nb, block_bytes)."""
    b = np.empty((nb, BLOCK_BYTES[qtype]), np.uint8)
    if qtype == Q8_0:
        s = 0.02 if sigma is None else sigma
        b[:, 0:2] = _f16_bytes(np.abs(rng.normal(0, s, nb)) / 127.0)
        b[:, 2:34] = rng.integers(-127, 128, (nb, 32), dtype=np.int8).view(np.uint8)
    elif qtype in (Q4_0, Q4_1, Q5_0):
        s = 0.01 if sigma is None else sigma
        b[:, 0:2] = _f16_bytes(np.abs(rng.normal(0, s, nb)))
        if qtype == Q4_0:
            b[:, 2:18] = rng.integers(0, 256, (nb, 16), dtype=np.uint8)
        elif qtype == Q4_1:
            b[:, 2:4] = _f16_bytes(rng.normal(0, s, nb))
            b[:, 4:20] = rng.integers(0, 256, (nb, 16), dtype=np.uint8)
        else:
            b[:, 2:22] = rng.integers(0, 256, (nb, 20), dtype=np.uint8)
    elif qtype in (Q4_K, Q5_K):
        s = 1e-3 if sigma is None else sigma
        b[:, 0:2] = _f16_bytes(np.abs(rng.normal(0, s, nb)))
        b[:, 2:4] = _f16_bytes(np.abs(rng.normal(0, s, nb)))
        b[:, 4:16] = pack_scale_min_k4(rng.integers(0, 64, (nb, 8), dtype=np.uint8),
                                        rng.integers(0, 64, (nb, 8), dtype=np.uint8))
        b[:, 16:] = rng.integers(0, 256, (nb, BLOCK_BYTES[qtype] - 16), dtype=np.uint8)
    elif qtype == Q6_K:
        s = 1e-3 if sigma is None else sigma
        b[:, 0:192] = rng.integers(0, 256, (nb, 192), dtype=np.uint8)
        b[:, 192:208] = rng.integers(-32, 32, (nb, 16), dtype=np.int8).view(np.uint8)
        b[:, 208:210] = _f16_bytes(np.abs(rng.normal(0, s, nb)))
    elif qtype == Q8_1:
        x = rng.normal(0, 1, nb * 32).astype(np.float32)
        b[:] = np_quantize_q8_1(x).reshape(nb, 36)
    else:
        raise ValueError(qtype)
    return b


def gen_weight(qtype: int, N: int, K: int, seed: int, sigma: float | None = None) -> np.ndarray:
    """Row-major quantised weight [N, K/block] -> uint8 (N, row_bytes)."""
    be = BLOCK_ELEMS[qtype]
    assert K % be == 0
    rng = np.random.default_rng(seed)
    nb = N * (K // be)
    return gen_blocks(qtype, nb, rng, sigma).reshape(N, (K // be) * BLOCK_BYTES[qtype])


@dataclass
class Int8LinearInputs:
    A: np.ndarray        # int8 [M, K]
    a_scale: np.ndarray  # fp32 [M]
    W: np.ndarray        # int8 [N, K]
    w_scale: np.ndarray  # fp32 [N]
    bias: np.ndarray     # fp16 [N]


def gen_int8_linear(M: int, N: int, K: int, seed: int) -> Int8LinearInputs:
    rng = np.random.default_rng(seed)
    return Int8LinearInputs(
        A=rng.integers(-127, 128, (M, K), dtype=np.int8),
        a_scale=np.abs(rng.normal(0, 0.02, M)).astype(np.float32),
        W=rng.integers(-127, 128, (N, K), dtype=np.int8),
        w_scale=np.abs(rng.normal(0, 0.01, N)).astype(np.float32),
        bias=rng.normal(0, 0.1, N).astype(np.float16),
    )


def ref_linear_int8(inp: Int8LinearInputs, act: int = 0, with_bias: bool = True):
    """D = f16(act(f32(acc) * a_scale[m] * w_scale[n] + bias[n])).
    acc is the exact int32 product (kernels/linear_int8.glsl:54-100 with the
    per-token scale and bias the reference binds but drops,
    shim/hipblaslt_shim.cpp:254-262).  Returns (acc int32, D float32 before
    the fp16 rounding, D fp16)."""
    acc = inp.A.astype(np.int64) @ inp.W.astype(np.int64).T
    assert np.abs(acc).max() < 2 ** 31
    acc = acc.astype(np.int32)
    y = acc.astype(F32) * inp.a_scale[:, None] * inp.w_scale[None, :]
    if with_bias:
        y = y + inp.bias.astype(F32)[None, :]
    y = np_act(act, y.astype(F32))
    return acc, y, y.astype(np.float16)


def special_blocks(qtype: int) -> np.ndarray:
    """Hand-built edge-case blocks: zero block, smallest fp16 subnormal and
    largest normal scales, negative scales, all-min and all-max codes, and
    (K-quants) all-0 / all-63 six-bit scale bytes covering both branches of
    get_scale_min_k4."""
    bb = BLOCK_BYTES[qtype]
    out = []
    scales = [0x0000, 0x0001, 0x03FF, 0x0400, 0x3C00, 0x7BFF, 0x8001, 0xBC00]
    fills = [0x00, 0xFF, 0x0F, 0xF0, 0x80, 0x7F, 0x55, 0xAA]
    for sc in scales:
        for fill in fills:
            b = np.full(bb, fill, np.uint8)
            if qtype in (Q4_0, Q8_0, Q5_0, Q8_1):
                b[0:2] = np.array([sc], np.uint16).view(np.uint8)
                if qtype == Q8_1:
                    b[2:4] = np.array([0x3C00], np.uint16).view(np.uint8)
            elif qtype == Q4_1:
                b[0:2] = np.array([sc], np.uint16).view(np.uint8)
                b[2:4] = np.array([scales[(scales.index(sc) + 3) % len(scales)]], np.uint16).view(np.uint8)
            elif qtype in (Q4_K, Q5_K):
                b[0:2] = np.array([sc], np.uint16).view(np.uint8)
                b[2:4] = np.array([scales[(scales.index(sc) + 5) % len(scales)]], np.uint16).view(np.uint8)
            elif qtype == Q6_K:
                b[208:210] = np.array([sc], np.uint16).view(np.uint8)
            out.append(b)
    return np.stack(out)
