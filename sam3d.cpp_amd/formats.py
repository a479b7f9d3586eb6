"""On-disk tensor formats for replaying the path on captured data.

SAMT (the reference's raw tensor file, src/objects_runtime/common.cpp:59-116,
written by scripts/objects/capture_mesh_reference.py:41-59):

    u32 magic 0x544D4153 ("SAMT") | i32 ndims (1..8) | i64 ne[ndims] | i32 ggml type | data

`ne` is in ggml order (ne[0] varies fastest), so the row-major numpy shape is
reversed(ne).  Types: 0 F32, 1 F16, 26 I32 (writers have also used 30 for
int32, which the reference's loader maps to I32, common.cpp:97-100).

GGUF (v2/v3, the weight container of the reference's converters): a header,
key/value metadata, tensor infos (name, ne, type, offset) and the tensor data
at general.alignment (default 32).  `GgufFile` memory-maps it and returns F32,
F16, BF16 and I32 tensors as numpy arrays.  `conv_weight` turns the
converters' sparse-conv tensors into the layouts `SparseConv.set_weights`
takes:

    SLat SubMConv3d  (Cout, 27*Cin)    gguf_schema.py:326-334  -> WEIGHT_SLAT [Cout][27][Cin]
    mesh conv k=3    (27, Cout*Cin)    convert_sam3d_to_gguf.py:486-492 -> WEIGHT_MESH [27][Cout][Cin]
    mesh conv k=1    (1, Cout*Cin)     same lines; the converter already applied
                                       spconv's (IC, OC) 1x1 reading -> WEIGHT_MESH [1][Cout][Cin]
"""
from __future__ import annotations

import struct
from pathlib import Path

import numpy as np

SAMT_MAGIC = 0x544D4153
GGML_F32, GGML_F16, GGML_I32, GGML_BF16 = 0, 1, 26, 30
_SAMT_DTYPES = {GGML_F32: np.float32, GGML_F16: np.float16, GGML_I32: np.int32}


def read_samt(path) -> np.ndarray:
    """A SAMT file as a numpy array of shape reversed(ne).  Raises ValueError on
    a malformed file (the reference's loader returns false)."""
    raw = Path(path).read_bytes()
    if len(raw) < 8:
        raise ValueError("SAMT: truncated header")
    magic, nd = struct.unpack_from("<Ii", raw, 0)
    if magic != SAMT_MAGIC or not 0 < nd <= 8:
        raise ValueError("SAMT: bad magic or ndims")
    off = 8
    if len(raw) < off + 8 * nd + 4:
        raise ValueError("SAMT: truncated header")
    ne = struct.unpack_from(f"<{nd}q", raw, off)
    off += 8 * nd
    (gtype,) = struct.unpack_from("<i", raw, off)
    off += 4
    if gtype == 30:  # int32 as some writers store it (common.cpp:97-100)
        gtype = GGML_I32
    if gtype not in _SAMT_DTYPES:
        raise ValueError(f"SAMT: unsupported ggml type {gtype}")
    dt = np.dtype(_SAMT_DTYPES[gtype])
    count = int(np.prod(ne))
    if len(raw) < off + count * dt.itemsize:
        raise ValueError("SAMT: truncated data")
    return np.frombuffer(raw, dt, count, off).reshape(tuple(reversed(ne))).copy()


def write_samt(path, array: np.ndarray) -> None:
    """save_raw_tensor (common.cpp:61-74) for float32 / float16 / int32 arrays."""
    a = np.ascontiguousarray(array)
    types = {np.dtype(np.float32): GGML_F32, np.dtype(np.float16): GGML_F16, np.dtype(np.int32): GGML_I32}
    if a.dtype not in types or not 0 < a.ndim <= 8:
        raise ValueError("SAMT: float32, float16 or int32 arrays of 1..8 dims")
    ne = tuple(reversed(a.shape))
    head = struct.pack("<Ii", SAMT_MAGIC, a.ndim) + struct.pack(f"<{a.ndim}q", *ne) + struct.pack("<i", types[a.dtype])
    Path(path).write_bytes(head + a.tobytes())


# ---- GGUF ---------------------------------------------------------------------
_GGUF_SCALAR = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<?", 10: "<Q",
                11: "<q", 12: "<d"}
_GGUF_TENSOR = {GGML_F32: np.float32, GGML_F16: np.float16, GGML_I32: np.int32, GGML_BF16: np.uint16}


class GgufFile:
    """Memory-mapped GGUF: `kv` (metadata) and `tensor(name)` (numpy, shape
    reversed(ne); BF16 comes back as float32)."""

    def __init__(self, path):
        self.path = Path(path)
        self._mm = np.memmap(self.path, np.uint8, "r")
        buf = self._mm
        if bytes(buf[:4]) != b"GGUF":
            raise ValueError("GGUF: bad magic")
        self._off = 4
        self.version = self._u("<I")
        if self.version not in (2, 3):
            raise ValueError(f"GGUF: unsupported version {self.version}")
        n_tensors, n_kv = self._u("<Q"), self._u("<Q")
        self.kv = {}
        for _ in range(n_kv):
            key = self._str()
            self.kv[key] = self._value(self._u("<I"))
        self.infos = {}
        for _ in range(n_tensors):
            name = self._str()
            nd = self._u("<I")
            ne = tuple(self._u("<Q") for _ in range(nd))
            gtype = self._u("<I")
            self.infos[name] = (ne, gtype, self._u("<Q"))
        align = int(self.kv.get("general.alignment", 32))
        self._data = (self._off + align - 1) // align * align

    def _u(self, fmt):
        v = struct.unpack_from(fmt, self._mm, self._off)[0]
        self._off += struct.calcsize(fmt)
        return v

    def _str(self):
        n = self._u("<Q")
        s = bytes(self._mm[self._off:self._off + n]).decode("utf-8")
        self._off += n
        return s

    def _value(self, vtype):
        if vtype in _GGUF_SCALAR:
            return self._u(_GGUF_SCALAR[vtype])
        if vtype == 8:
            return self._str()
        if vtype == 9:
            etype, n = self._u("<I"), self._u("<Q")
            return [self._value(etype) for _ in range(n)]
        raise ValueError(f"GGUF: unknown value type {vtype}")

    def tensor(self, name) -> np.ndarray:
        ne, gtype, off = self.infos[name]
        if gtype not in _GGUF_TENSOR:
            raise ValueError(f"GGUF: tensor {name} has unsupported type {gtype}")
        dt = np.dtype(_GGUF_TENSOR[gtype])
        count = int(np.prod(ne))
        a = np.frombuffer(self._mm, dt, count, self._data + off).reshape(tuple(reversed(ne)))
        if gtype == GGML_BF16:
            return (a.astype(np.uint32) << 16).view(np.float32)
        return np.array(a)


def conv_weight(t: np.ndarray, kind: str, cin: int, cout: int) -> np.ndarray:
    """A converter's sparse-conv tensor as float32 in the set_weights layout:
    kind "slat" -> [Cout][27][Cin], "mesh" -> [27][Cout][Cin], "mesh_1x1" ->
    [1][Cout][Cin]."""
    a = np.asarray(t, np.float32)
    if kind == "slat":
        if a.shape != (cout, 27 * cin):
            raise ValueError(f"SLat conv weight: expected {(cout, 27 * cin)}, got {a.shape}")
        return a.reshape(cout, 27, cin)
    if kind in ("mesh", "mesh_1x1"):
        k = 27 if kind == "mesh" else 1
        if a.shape != (k, cout * cin):
            raise ValueError(f"mesh conv weight: expected {(k, cout * cin)}, got {a.shape}")
        return a.reshape(k, cout, cin)
    raise ValueError(f"unknown conv weight kind {kind}")
