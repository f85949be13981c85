"""CPU: GGUF files (vkflame_amd.gguf) -- a hand-assembled file parsed against
the format's byte layout, writer/reader round trips of quantised tensors and
typed metadata, and the error checks."""
import struct

import numpy as np
import pytest

import oracle as O
from vkflame_amd import gguf as G


def _s(x: str) -> bytes:
    b = x.encode()
    return struct.pack("<Q", len(b)) + b


def test_hand_assembled_file(tmp_path):
    """Bytes laid out field by field: magic, version 3, counts, one string
    key/value, one u32 array, one Q8_0 tensor info (ne = 32 x 2), padding to
    32, data."""
    blocks = O.gen_weight(O.Q8_0, 2, 32, 5).reshape(-1)        # 2 rows x 1 block x 34 B
    head = struct.pack("<IIQQ", 0x46554747, 3, 1, 2)
    head += _s("general.architecture") + struct.pack("<I", 8) + _s("llama")
    head += _s("x.ids") + struct.pack("<I", 9) + struct.pack("<IQ", 4, 3) + struct.pack("<3I", 7, 8, 9)
    head += _s("blk.0.w") + struct.pack("<I", 2) + struct.pack("<QQ", 32, 2) + struct.pack("<IQ", 8, 0)
    pad = (-len(head)) % 32
    p = tmp_path / "hand.gguf"
    p.write_bytes(head + b"\0" * pad + blocks.tobytes())
    f = G.GGUFFile(str(p))
    assert f.version == 3 and f.alignment == 32 and f.data_offset == len(head) + pad
    assert f.metadata["general.architecture"] == "llama"
    assert f.metadata["x.ids"].tolist() == [7, 8, 9] and f.metadata["x.ids"].dtype == np.uint32
    ti = f.tensors["blk.0.w"]
    assert ti.shape == (32, 2) and ti.ggml_type == 8 and ti.nbytes == 68
    w, qt, N, K = f.weight("blk.0.w")
    assert (qt, N, K) == (O.Q8_0, 2, 32) and w.shape == (2, 34)
    assert np.array_equal(np.asarray(w).reshape(-1), blocks)


@pytest.mark.parametrize("alignment", [32, 64])
def test_round_trip(tmp_path, alignment):
    tensors, want = {}, {}
    for i, (qt, N, K) in enumerate([(O.Q4_K, 7, 512), (O.Q6_K, 3, 256), (O.Q4_0, 5, 96), (O.Q8_0, 2, 64),
                                    (O.Q5_K, 2, 256), (O.Q4_1, 4, 32), (O.Q5_0, 3, 64)]):
        b = O.gen_weight(qt, N, K, 100 + i)
        tensors[f"w{i}"] = (G.GGML_OF_LIBRARY[qt], (K, N), b)
        want[f"w{i}"] = (qt, N, K, b)
    f32 = np.arange(10, dtype=np.float32)
    f16 = np.linspace(-1, 1, 6, dtype=np.float16).reshape(2, 3)
    tensors["norm"] = (G.GGML_F32, (10,), f32)
    tensors["emb"] = (G.GGML_F16, (3, 2), f16)
    meta = {"general.name": "t", "n": 5, "neg": -3, "eps": 1e-5, "flag": True,
            "u32": np.uint32(7), "f32s": np.array([1.5, 2.5], dtype=np.float32),
            "toks": ["a", "bc", ""], "ints": [1, 2, 3]}
    p = str(tmp_path / "rt.gguf")
    G.write_gguf(p, tensors, meta, alignment=alignment)
    f = G.GGUFFile(p)
    assert f.alignment == alignment and f.data_offset % alignment == 0
    for k in ("general.name", "n", "neg", "eps", "flag", "u32", "toks"):
        assert f.metadata[k] == meta[k]
    assert np.array_equal(f.metadata["f32s"], meta["f32s"]) and list(f.metadata["ints"]) == [1, 2, 3]
    for name, (qt, N, K, b) in want.items():
        assert f.tensors[name].offset % alignment == 0
        w, qq, NN, KK = f.weight(name)
        assert (qq, NN, KK) == (qt, N, K)
        assert np.array_equal(np.asarray(w).reshape(-1), b.reshape(-1))
        assert np.array_equal(O.np_dequant(qt, np.asarray(w).reshape(-1)), O.np_dequant(qt, b.reshape(-1)))
    assert np.array_equal(f.raw("norm").view(np.float32), f32)
    assert np.array_equal(f.raw("emb").view(np.float16).reshape(2, 3), f16)


def test_errors(tmp_path):
    b = O.gen_weight(O.Q4_K, 2, 256, 1)
    p = str(tmp_path / "e.gguf")
    G.write_gguf(p, {"w": (12, (256, 2), b)})
    raw = open(p, "rb").read()
    bad = tmp_path / "bad.gguf"
    bad.write_bytes(b"GGUX" + raw[4:])
    with pytest.raises(G.GGUFError, match="not a GGUF"):
        G.GGUFFile(str(bad))
    bad.write_bytes(raw[:4] + struct.pack("<I", 1) + raw[8:])
    with pytest.raises(G.GGUFError, match="version"):
        G.GGUFFile(str(bad))
    bad.write_bytes(raw[:-10])
    with pytest.raises(G.GGUFError, match="past the end"):
        G.GGUFFile(str(bad))
    bad.write_bytes(raw[:30])
    with pytest.raises(G.GGUFError, match="truncated"):
        G.GGUFFile(str(bad))
    with pytest.raises(G.GGUFError, match="bytes given"):
        G.write_gguf(p, {"w": (12, (256, 3), b)})
    with pytest.raises(G.GGUFError, match="not one this library runs"):
        G.write_gguf(p, {"w": (17, (256, 1), np.zeros(10, np.uint8))})
