"""CPU: pins the oracle's dequantisers (oracle/vkf_oracle.c and its numpy twin).

The reference ships no test, fixture or golden vector for any quant format
(its tests cover fp16 GEMM only), so the restatement of
kernels/dequant_*.glsl is pinned by checks that do not retype its formulas:

* known-answer blocks whose expected values were worked out by hand;
* round trips through ENCODERS written from the writer's side of each format
  (ggml's quantize_row_* byte layouts: where each code goes), so a wrong
  index, nibble half or bit position in the decoder fails;
* closed forms: products of an fp16 scale and small integers are exact in
  fp32, so Q8_0/Q8_1/Q4_0/Q5_0/Q6_K values equal their float64 values, and
  Q4_1/Q4_K/Q5_K values equal the float64 value rounded once to fp32;
* fp16 outputs are the fp32 values rounded to nearest even (numpy's
  conversion), and the C oracle equals the numpy twin bit for bit.
"""
import numpy as np
import pytest

import oracle as O

F16 = lambda v: np.array([v], np.float16).view(np.uint8)  # noqa: E731


# ---------------------------------------------------------------------------
# encoders (writer's side of each layout)
# ---------------------------------------------------------------------------

def enc_nibble32(L):
    """32 four-bit codes -> 16 bytes: qs[j] = L[j] | L[j+16] << 4."""
    L = np.asarray(L, np.uint8)
    return (L[:16] | (L[16:] << 4)).astype(np.uint8)


def enc_q5_0(L):
    """32 five-bit codes -> (qh u32, qs[16]): bit j of qh = bit 4 of L[j]."""
    L = np.asarray(L, np.uint32)
    qh = 0
    for j in range(32):
        qh |= int((L[j] >> 4) & 1) << j
    return np.array([qh], np.uint32).view(np.uint8), enc_nibble32(L & 15)


def enc_k_nibbles(L):
    """256 four-bit codes -> 128 bytes: chunk il, l<32:
    qs[32il + l] = L[64il + l] | L[64il + 32 + l] << 4."""
    L = np.asarray(L, np.uint8).reshape(4, 2, 32)
    return (L[:, 0, :] | (L[:, 1, :] << 4)).reshape(-1).astype(np.uint8)


def enc_q5_k_high(L):
    """256 five-bit codes -> qh[32]: bit 2il of qh[l] = bit 4 of L[64il+l],
    bit 2il+1 = bit 4 of L[64il+32+l]."""
    L = np.asarray(L, np.uint32).reshape(4, 2, 32)
    qh = np.zeros(32, np.uint32)
    for il in range(4):
        qh |= ((L[il, 0] >> 4) & 1) << (2 * il)
        qh |= ((L[il, 1] >> 4) & 1) << (2 * il + 1)
    return qh.astype(np.uint8)


def enc_q6_k(L):
    """256 six-bit codes -> (ql[128], qh[64]) as ggml's quantize_row_q6_K
    writes them: for half ip and l < 32, codes a,b,c,d at 128ip + l + {0,32,64,96}:
    ql[64ip+l] = a&15 | (c&15)<<4, ql[64ip+l+32] = b&15 | (d&15)<<4,
    qh[32ip+l] = a>>4 | (b>>4)<<2 | (c>>4)<<4 | (d>>4)<<6."""
    L = np.asarray(L, np.uint32)
    ql = np.zeros(128, np.uint32)
    qh = np.zeros(64, np.uint32)
    for ip in range(2):
        for l in range(32):
            a, b, c, d = (L[128 * ip + l + 32 * t] for t in range(4))
            ql[64 * ip + l] = (a & 15) | ((c & 15) << 4)
            ql[64 * ip + l + 32] = (b & 15) | ((d & 15) << 4)
            qh[32 * ip + l] = (a >> 4) | ((b >> 4) << 2) | ((c >> 4) << 4) | ((d >> 4) << 6)
    return ql.astype(np.uint8), qh.astype(np.uint8)


def both(qt, blocks):
    """C oracle output, after asserting the numpy twin agrees bit for bit."""
    c = O.c_dequant(qt, blocks)
    n = O.np_dequant(qt, blocks)
    assert np.array_equal(c.view(np.uint32), n.view(np.uint32))
    return c


# ---------------------------------------------------------------------------
# known answers (worked by hand)
# ---------------------------------------------------------------------------

def test_kat_q4_0():
    # d = 1, qs[i] = i | (15 - i) << 4: elements 0..15 are i - 8, 16..31 are 7 - i
    b = np.concatenate([F16(1.0), np.array([i | ((15 - i) << 4) for i in range(16)], np.uint8)])
    expect = list(range(-8, 8)) + list(range(7, -9, -1))
    assert both(O.Q4_0, b).tolist() == expect


def test_kat_q4_1():
    # d = 0.5, m = -1: y = 0.5*q - 1 with q as in test_kat_q4_0
    b = np.concatenate([F16(0.5), F16(-1.0), np.array([i | ((15 - i) << 4) for i in range(16)], np.uint8)])
    expect = [0.5 * i - 1 for i in range(16)] + [0.5 * (15 - i) - 1 for i in range(16)]
    assert both(O.Q4_1, b).tolist() == expect


def test_kat_q8_0_and_q8_1():
    q = np.array([-127, -64, -1, 0, 1, 2, 63, 127] * 4, np.int8)
    b = np.concatenate([F16(2.0), q.view(np.uint8)])
    assert both(O.Q8_0, b).tolist() == [2.0 * v for v in q.tolist()]
    b1 = np.concatenate([F16(-0.25), F16(99.0), q.view(np.uint8)])      # s must be ignored
    assert both(O.Q8_1, b1).tolist() == [-0.25 * v for v in q.tolist()]


def test_kat_q5_0():
    # d = 1, qh = 0xAAAAAAAA (odd bits set), nibble of element e is e % 16
    qh = np.array([0xAAAAAAAA], np.uint32).view(np.uint8)
    qs = np.array([i | (i << 4) for i in range(16)], np.uint8)
    b = np.concatenate([F16(1.0), qh, qs])
    expect = [(e % 16) + (16 if e % 2 else 0) - 16 for e in range(32)]
    assert both(O.Q5_0, b).tolist() == expect


# Hand-decoded scale bytes covering both branches of get_scale_min_k4:
#   j < 4 : sc = s[j] & 63 = 1,2,3,4          m = s[j+4] & 63 = 5,6,7,8
#   j >= 4: sc = s[j+4]&15 | (s[j-4]>>6)<<4 = 17,35,53,7
#           m  = s[j+4]>>4 | (s[j]>>6)<<4   = 18,36,54,8
K_SCALES = np.array([0x41, 0x82, 0xC3, 0x04, 0x45, 0x86, 0xC7, 0x08, 0x21, 0x43, 0x65, 0x87], np.uint8)
K_SC = [1, 2, 3, 4, 17, 35, 53, 7]
K_M = [5, 6, 7, 8, 18, 36, 54, 8]


def test_kat_q4_k():
    # dall = dmin = 1, every qs byte 0x21: low nibble 1 (even sub-blocks), high 2 (odd)
    b = np.concatenate([F16(1.0), F16(1.0), K_SCALES, np.full(128, 0x21, np.uint8)])
    per_sub = [-4, -2, -4, 0, -1, 34, -1, 6]            # sc*q - m worked by hand
    assert both(O.Q4_K, b).tolist() == [v for v in per_sub for _ in range(32)]


def test_kat_q5_k():
    # as Q4_K plus qh[l] = 0x55: bit 2il set (+16 on every even sub-block)
    b = np.concatenate([F16(1.0), F16(1.0), K_SCALES, np.full(32, 0x55, np.uint8), np.full(128, 0x21, np.uint8)])
    per_sub = [12, -2, 44, 0, 271, 34, 847, 6]
    assert both(O.Q5_K, b).tolist() == [v for v in per_sub for _ in range(32)]


def test_kat_q6_k_scale_index():
    # d = 1, codes all 0 (v = -32), scale i = i - 8: element e uses scale e // 16,
    # so y = -32 * (e//16 - 8) = 32 * (8 - e//16)
    sc = np.arange(16, dtype=np.int8) - 8
    b = np.concatenate([np.zeros(192, np.uint8), sc.view(np.uint8), F16(1.0)])
    assert both(O.Q6_K, b).tolist() == [32.0 * (8 - e // 16) for e in range(256)]


# ---------------------------------------------------------------------------
# encoder round trips
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("seed", range(5))
def test_roundtrip_q4_0_q4_1_q5_0(seed):
    rng = np.random.default_rng(seed)
    L = rng.integers(0, 16, 32)
    y = both(O.Q4_0, np.concatenate([F16(1.0), enc_nibble32(L)]))
    assert y.tolist() == (L - 8).tolist()
    y = both(O.Q4_1, np.concatenate([F16(1.0), F16(0.0), enc_nibble32(L)]))
    assert y.tolist() == L.tolist()
    L5 = rng.integers(0, 32, 32)
    qh, qs = enc_q5_0(L5)
    y = both(O.Q5_0, np.concatenate([F16(1.0), qh, qs]))
    assert y.tolist() == (L5 - 16).tolist()


@pytest.mark.parametrize("seed", range(5))
def test_roundtrip_q4_k_q5_k(seed):
    rng = np.random.default_rng(100 + seed)
    sc = rng.integers(0, 64, 8)
    mn = rng.integers(0, 64, 8)
    s = O.pack_scale_min_k4(sc[None], mn[None])[0]
    # decoded (sc, m) must be the packed ones
    dsc, dm = O.scale_min_k4(s[None])
    assert dsc[0].tolist() == sc.tolist() and dm[0].tolist() == mn.tolist()
    L = rng.integers(0, 16, 256)
    y = both(O.Q4_K, np.concatenate([F16(1.0), F16(1.0), s, enc_k_nibbles(L)]))
    j = np.arange(256) // 32
    assert y.tolist() == (sc[j] * L - mn[j]).tolist()
    L5 = rng.integers(0, 32, 256)
    y = both(O.Q5_K, np.concatenate([F16(1.0), F16(1.0), s, enc_q5_k_high(L5), enc_k_nibbles(L5 & 15)]))
    assert y.tolist() == (sc[j] * L5 - mn[j]).tolist()


@pytest.mark.parametrize("seed", range(5))
def test_roundtrip_q6_k(seed):
    rng = np.random.default_rng(200 + seed)
    L = rng.integers(0, 64, 256)
    sc = rng.integers(-128, 128, 16).astype(np.int8)
    ql, qh = enc_q6_k(L)
    y = both(O.Q6_K, np.concatenate([ql, qh, sc.view(np.uint8), F16(1.0)]))
    assert y.tolist() == (sc[np.arange(256) // 16].astype(np.int64) * (L - 32)).tolist()


# ---------------------------------------------------------------------------
# closed forms on random blocks
# ---------------------------------------------------------------------------

def _f64_values(qt, b):
    """The exact real value of every element, from independently decoded
    integer fields (encoders' inverse via the round-trip-pinned helpers)."""
    h = lambda off: b[:, off:off + 2].copy().view(np.float16).astype(np.float64)  # noqa: E731
    if qt in (O.Q8_0, O.Q8_1):
        off = 2 if qt == O.Q8_0 else 4
        return h(0) * b[:, off:off + 32].view(np.int8).astype(np.float64)
    if qt in (O.Q4_0, O.Q4_1):
        off = 2 if qt == O.Q4_0 else 4
        q = np.concatenate([b[:, off:off + 16] & 15, b[:, off:off + 16] >> 4], 1).astype(np.float64)
        return h(0) * (q - 8) if qt == O.Q4_0 else h(0) * q + h(2)
    if qt == O.Q5_0:
        qh = b[:, 2:6].copy().view(np.uint32).astype(np.int64)
        q = np.concatenate([b[:, 6:22] & 15, b[:, 6:22] >> 4], 1).astype(np.int64)
        q |= ((qh >> np.arange(32)) & 1) << 4
        return h(0) * (q - 16)
    if qt in (O.Q4_K, O.Q5_K):
        sc, mn = O.scale_min_k4(b[:, 4:16])
        qoff = 16 if qt == O.Q4_K else 48
        qs = b[:, qoff:qoff + 128].reshape(-1, 4, 32).astype(np.int64)
        q = np.stack([qs & 15, qs >> 4], 2).reshape(-1, 8, 32)
        if qt == O.Q5_K:  # sub-block j = 2il + half takes bit j of qh[l]
            qh = b[:, 16:48].astype(np.int64)
            q = q + 16 * np.stack([(qh >> j) & 1 for j in range(8)], 1)
        y = h(0)[:, :, None] * sc[:, :, None] * q - h(2)[:, :, None] * mn[:, :, None]
        return y.reshape(-1, 256)
    if qt == O.Q6_K:
        v, sc = O.q6k_fields(b)
        return h(208) * (sc * v)
    raise ValueError(qt)


EXACT = [O.Q8_0, O.Q8_1, O.Q4_0, O.Q5_0, O.Q6_K]
ONE_ROUNDING = [O.Q4_1, O.Q4_K, O.Q5_K]


@pytest.mark.parametrize("qt", EXACT + ONE_ROUNDING, ids=[O.QNAMES[q] for q in EXACT + ONE_ROUNDING])
def test_closed_form(qt):
    rng = np.random.default_rng(300 + qt)
    b = np.concatenate([O.gen_blocks(qt, 400, rng), O.special_blocks(qt)])
    y = both(qt, b).reshape(b.shape[0], -1)
    exact = _f64_values(qt, b)
    fin = np.isfinite(exact)
    if qt in EXACT:
        assert np.array_equal(y[fin].astype(np.float64), exact[fin])
    else:  # one rounding of the exact value to fp32
        assert np.array_equal(y[fin], exact[fin].astype(np.float32))


@pytest.mark.parametrize("qt", list(range(8)), ids=[O.QNAMES[q] for q in range(8)])
def test_f16_output_is_rne_of_f32(qt):
    rng = np.random.default_rng(400 + qt)
    b = np.concatenate([O.gen_blocks(qt, 300, rng), O.special_blocks(qt)])
    y32 = O.c_dequant(qt, b)
    y16 = O.c_dequant(qt, b, out_f16=True)
    with np.errstate(over="ignore"):
        assert np.array_equal(y16.view(np.uint16), y32.astype(np.float16).view(np.uint16))
