"""GGUF tensor files: the on-disk source of the ggml blocks this library runs.

A GGUF file (version 2 or 3, little-endian) is a header, typed metadata
key/values, one info record per tensor (name, dimensions ne[0..n) with ne[0]
the contiguous row length, ggml type, offset) and the tensor data, each
tensor at an offset aligned to ``general.alignment`` (default 32) from the
start of the data section.  Quantised tensors are stored exactly as the
kernels read them (rows of whole ggml blocks along ne[0]), so a weight goes
from the file to the GPU as one memory-mapped byte range and one copy, with
no repacking:

    f = GGUFFile("model.gguf")
    w, qt, N, K = f.weight_to_device("blk.0.ffn_up.weight", "cuda")
    y = ops.gemm_q(w, qt, x, N, K)

``write_gguf`` writes the same format (tests, tools).  The reference has no
loader (it receives ggml's buffers through its hipLaunchKernel shim); this
module is the "on-disk format" step next to the path.
"""
from __future__ import annotations

import os
import struct
from dataclasses import dataclass

import numpy as np

from . import _lib as L

GGUF_MAGIC = 0x46554747  # "GGUF"
DEFAULT_ALIGNMENT = 32

# ggml_type ids of the formats this library runs -> (library code, elements per
# block, bytes per block); F32 / F16 are plain arrays.
GGML_F32, GGML_F16 = 0, 1
GGML_TYPES = {
    2: (L.Q4_0, 32, 18), 3: (L.Q4_1, 32, 20), 6: (L.Q5_0, 32, 22), 8: (L.Q8_0, 32, 34), 9: (L.Q8_1, 32, 36),
    12: (L.Q4_K, 256, 144), 13: (L.Q5_K, 256, 176), 14: (L.Q6_K, 256, 210),
}
GGML_OF_LIBRARY = {v[0]: k for k, v in GGML_TYPES.items()}

# metadata value types
(T_U8, T_I8, T_U16, T_I16, T_U32, T_I32, T_F32, T_BOOL, T_STR, T_ARR, T_U64, T_I64, T_F64) = range(13)
_SCALAR = {T_U8: "<B", T_I8: "<b", T_U16: "<H", T_I16: "<h", T_U32: "<I", T_I32: "<i", T_F32: "<f",
           T_BOOL: "<?", T_U64: "<Q", T_I64: "<q", T_F64: "<d"}


class GGUFError(ValueError):
    pass


@dataclass
class TensorInfo:
    name: str
    shape: tuple  # ggml order: shape[0] = ne0, the contiguous row length
    ggml_type: int
    offset: int   # from the start of the data section

    @property
    def nbytes(self) -> int:
        n = int(np.prod(self.shape, dtype=np.int64))
        if self.ggml_type == GGML_F32:
            return 4 * n
        if self.ggml_type == GGML_F16:
            return 2 * n
        if self.ggml_type not in GGML_TYPES:
            raise GGUFError(f"{self.name}: ggml type {self.ggml_type} is not one this library runs")
        _, be, bb = GGML_TYPES[self.ggml_type]
        if self.shape[0] % be:
            raise GGUFError(f"{self.name}: row length {self.shape[0]} is not a multiple of {be}")
        return n // be * bb


class _Reader:
    def __init__(self, buf: memoryview):
        self.b = buf
        self.p = 0

    def take(self, n: int) -> memoryview:
        if self.p + n > len(self.b):
            raise GGUFError("truncated GGUF file")
        v = self.b[self.p:self.p + n]
        self.p += n
        return v

    def scalar(self, t: int):
        fmt = _SCALAR[t]
        return struct.unpack(fmt, self.take(struct.calcsize(fmt)))[0]

    def string(self) -> str:
        n = self.scalar(T_U64)
        return bytes(self.take(n)).decode("utf-8")

    def value(self, t: int):
        if t == T_STR:
            return self.string()
        if t == T_ARR:
            et = self.scalar(T_U32)
            n = self.scalar(T_U64)
            if et in _SCALAR and et != T_BOOL:
                dt = np.dtype(_SCALAR[et])
                return np.frombuffer(self.take(n * dt.itemsize), dtype=dt).copy()
            return [self.value(et) for _ in range(n)]
        if t in _SCALAR:
            return self.scalar(t)
        raise GGUFError(f"unknown metadata value type {t}")


class GGUFFile:
    """Parses a GGUF file and memory-maps its tensor data (private mapping:
    the file is never written)."""

    def __init__(self, path: str):
        self.path = path
        # copy-on-write private mapping: writable views (torch.from_numpy
        # takes them without a copy), the file itself is never modified
        self._mm = np.memmap(path, dtype=np.uint8, mode="c")
        r = _Reader(memoryview(self._mm))
        if r.scalar(T_U32) != GGUF_MAGIC:
            raise GGUFError(f"{path}: not a GGUF file")
        self.version = r.scalar(T_U32)
        if self.version not in (2, 3):
            raise GGUFError(f"{path}: GGUF version {self.version} is not supported (2 or 3)")
        n_tensors = r.scalar(T_U64)
        n_kv = r.scalar(T_U64)
        self.metadata: dict = {}
        for _ in range(n_kv):
            key = r.string()
            self.metadata[key] = r.value(r.scalar(T_U32))
        self.tensors: dict[str, TensorInfo] = {}
        for _ in range(n_tensors):
            name = r.string()
            nd = r.scalar(T_U32)
            shape = tuple(r.scalar(T_U64) for _ in range(nd))
            ti = TensorInfo(name, shape, r.scalar(T_U32), r.scalar(T_U64))
            self.tensors[name] = ti
        self.alignment = int(self.metadata.get("general.alignment", DEFAULT_ALIGNMENT))
        if self.alignment <= 0 or self.alignment & (self.alignment - 1):
            raise GGUFError(f"{path}: alignment {self.alignment} is not a power of two")
        self.data_offset = (r.p + self.alignment - 1) // self.alignment * self.alignment
        for ti in self.tensors.values():
            if ti.offset % self.alignment:
                raise GGUFError(f"{ti.name}: offset {ti.offset} not aligned to {self.alignment}")
            if self.data_offset + ti.offset + ti.nbytes > len(self._mm):
                raise GGUFError(f"{ti.name}: data runs past the end of the file")

    def raw(self, name: str) -> np.ndarray:
        """The tensor's bytes (a view into the mapped file)."""
        ti = self.tensors[name]
        o = self.data_offset + ti.offset
        return self._mm[o:o + ti.nbytes]

    def weight(self, name: str):
        """(blocks uint8 [N, row_bytes] view, library quant code, N, K) of a
        quantised matrix stored as ne = (K, N): N rows of K elements."""
        ti = self.tensors[name]
        if ti.ggml_type not in GGML_TYPES or len(ti.shape) != 2:
            raise GGUFError(f"{name}: not a quantised matrix (type {ti.ggml_type}, shape {ti.shape})")
        qt, be, bb = GGML_TYPES[ti.ggml_type]
        K, N = ti.shape
        return self.raw(name).reshape(N, K // be * bb), qt, N, K

    def weight_to_device(self, name: str, device="cuda"):
        """weight() copied to a device tensor: (uint8 [N, row_bytes], quant code, N, K)."""
        import torch
        blocks, qt, N, K = self.weight(name)
        t = torch.from_numpy(np.ascontiguousarray(blocks)).to(device)
        return t, qt, N, K


def write_gguf(path: str, tensors: dict, metadata: dict | None = None, alignment: int = DEFAULT_ALIGNMENT,
               version: int = 3) -> None:
    """Write a GGUF file.  tensors: name -> (ggml_type, shape in ggml order
    (ne0 first), uint8/float bytes of the whole tensor).  metadata values: str,
    bool, int (written as int64 / uint64), float (float64), numpy scalars
    (their own type), lists / 1-D numpy arrays (arrays)."""
    metadata = dict(metadata or {})
    if alignment != DEFAULT_ALIGNMENT:
        metadata["general.alignment"] = np.uint32(alignment)

    def s(x: str) -> bytes:
        b = x.encode("utf-8")
        return struct.pack("<Q", len(b)) + b

    np_types = {np.uint8: T_U8, np.int8: T_I8, np.uint16: T_U16, np.int16: T_I16, np.uint32: T_U32,
                np.int32: T_I32, np.float32: T_F32, np.uint64: T_U64, np.int64: T_I64, np.float64: T_F64,
                np.bool_: T_BOOL}

    def typed(v):
        if isinstance(v, bool):
            return T_BOOL, struct.pack("<?", v)
        if isinstance(v, str):
            return T_STR, s(v)
        if isinstance(v, np.generic) and type(v) in np_types:
            t = np_types[type(v)]
            return t, struct.pack(_SCALAR[t], v.item())
        if isinstance(v, int):
            return (T_I64, struct.pack("<q", v)) if v < 0 else (T_U64, struct.pack("<Q", v))
        if isinstance(v, float):
            return T_F64, struct.pack("<d", v)
        if isinstance(v, np.ndarray) and v.dtype.type in np_types and v.ndim == 1:
            et = np_types[v.dtype.type]
            return T_ARR, struct.pack("<IQ", et, v.size) + v.astype(v.dtype.newbyteorder("<")).tobytes()
        if isinstance(v, (list, tuple)):
            items = [typed(x) for x in v]
            et = items[0][0] if items else T_U8
            if any(t != et for t, _ in items):
                raise GGUFError("array items must share one type")
            return T_ARR, struct.pack("<IQ", et, len(items)) + b"".join(b for _, b in items)
        raise GGUFError(f"unsupported metadata value {v!r}")

    head = struct.pack("<IIQQ", GGUF_MAGIC, version, len(tensors), len(metadata))
    for k, v in metadata.items():
        t, b = typed(v)
        head += s(k) + struct.pack("<I", t) + b
    infos, blobs, off = b"", [], 0
    for name, (gt, shape, data) in tensors.items():
        data = np.ascontiguousarray(data).view(np.uint8).reshape(-1)
        ti = TensorInfo(name, tuple(int(d) for d in shape), int(gt), off)
        if ti.nbytes != data.size:
            raise GGUFError(f"{name}: {data.size} bytes given, {ti.nbytes} expected for type {gt} shape {shape}")
        infos += s(name) + struct.pack("<I", len(shape)) + b"".join(struct.pack("<Q", int(d)) for d in shape)
        infos += struct.pack("<IQ", int(gt), off)
        blobs.append((off, data))
        off = (off + data.size + alignment - 1) // alignment * alignment
    head += infos
    data_start = (len(head) + alignment - 1) // alignment * alignment
    with open(path, "wb") as f:
        f.write(head)
        f.write(b"\0" * (data_start - len(head)))
        pos = 0
        for o, data in blobs:
            f.write(b"\0" * (o - pos))
            f.write(data.tobytes())
            pos = o + data.size
        f.flush()
        os.fsync(f.fileno())
