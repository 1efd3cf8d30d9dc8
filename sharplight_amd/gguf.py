"""GGUF files: the reader and the weight upload of libsharplight_hip, with the reference's object model.

``GgufFile`` mirrors ``Sharplight.Import.Gguf.GgufFile`` (src/Sharplight.Import.Gguf/GgufFile.cs:16-294):
``open`` maps the file and parses it natively (``slhip_gguf_open``); ``version``, ``alignment``,
``data_offset``, ``metadata``, ``tensors``, ``architecture``, ``find_tensor`` / ``get_tensor`` and
``close`` (``Dispose``) behave as there. A ``GgufTensorInfo`` (GgufTensorInfo.cs:7-79) reads its bytes
on the host (``IWeightSource.Read``) and uploads them to device memory (``WeightUploader.Upload``,
src/Sharplight.Vulkan/WeightUploader.cs:48-74) through the library's staged uploader.

``GgufModelFiles`` opens a model split over shards (GgufModelFiles.cs:9-110).
``read_metadata`` / ``read_tensor_table`` are ``GgufHeaderProbe.ReadMetadata`` / ``ReadTensorTable``
(GgufHeaderProbe.cs:17-135) over the first bytes of a file. ``GgufWriter`` is the reference's fixture
writer (GgufWriter.cs:7-191).

Metadata values come back typed as the reference's CLR values: numpy scalars of the stored width for
numbers, ``bool``, ``str``; numpy arrays for numeric and bool arrays, lists of ``str`` for string arrays,
lists for arrays of arrays. Errors: ``SlhipFormatError`` (InvalidDataException) for a malformed file,
``SlhipNotSupported`` for an unsupported version or type id, ``ValueError`` after ``close``.
"""
from __future__ import annotations

import ctypes
import os
import re
import struct

import numpy as np

from . import native

# slhip_gguf_vtype
UINT8, INT8, UINT16, INT16, UINT32, INT32, FLOAT32, BOOL, STRING, ARRAY, UINT64, INT64, FLOAT64 = range(13)
_NP = {UINT8: np.uint8, INT8: np.int8, UINT16: np.uint16, INT16: np.int16, UINT32: np.uint32, INT32: np.int32,
       FLOAT32: np.float32, UINT64: np.uint64, INT64: np.int64, FLOAT64: np.float64}
_FORMAT_NAMES = {v: k for k, v in native.FORMATS.items()}


def _decode(h, node: int):
    v = native.GgufValue()
    native.call("slhip_gguf_get_value", h, node, ctypes.byref(v))
    t = v.type
    if t in (UINT8, UINT16, UINT32, UINT64):
        return _NP[t](v.u)
    if t in (INT8, INT16, INT32, INT64):
        return _NP[t](v.i)
    if t in (FLOAT32, FLOAT64):
        return _NP[t](v.f)
    if t == BOOL:
        return bool(v.u)
    if t == STRING:
        return ctypes.string_at(v.data, v.count).decode("utf-8", errors="replace") if v.count else ""
    # ARRAY
    e, n = v.elem_type, v.count
    if e in _NP:
        dt = np.dtype(_NP[e]).newbyteorder("<")
        return np.frombuffer(ctypes.string_at(v.data, n * dt.itemsize), dt).astype(dt.newbyteorder("="))
    if e == BOOL:
        return np.frombuffer(ctypes.string_at(v.data, n), np.uint8) != 0
    return [_decode(h, v.first_child + k) for k in range(n)]


class GgufTensorInfo:
    """One tensor of the table (GgufTensorInfo.cs:7-79); valid while its file is open."""

    def __init__(self, file: "GgufFile", index: int, t: native.GgufTensor):
        self._file = file
        self.index = index
        self.name = t.name.decode("utf-8", errors="replace")
        self.ggml_type = t.ggml_type
        self.data_type = t.type_name.decode()         # the reference's DataType name
        self.format = _FORMAT_NAMES.get(t.format)     # the slhip format the kernels read it as, or None
        self.block_size, self.block_bytes = t.block_size, t.block_bytes
        self.ne = [t.ne[d] for d in range(t.n_dims)]  # ggml order, innermost first
        self.shape = tuple(reversed(self.ne))         # outermost first
        self.relative_offset, self.offset = t.relative_offset, t.offset
        self.byte_size, self.stored_bytes = t.byte_size, t.stored_bytes

    def read(self, offset: int = 0, size: int | None = None) -> bytes:
        """Bytes [offset, offset + size) as the element type (IWeightSource.Read)."""
        n = self.byte_size - offset if size is None else size
        buf = ctypes.create_string_buffer(max(n, 1))
        native.call("slhip_gguf_read", self._file._handle(), self.index, offset, buf, n)
        return buf.raw[:n]

    def pointer(self) -> int:
        """The bytes in the file mapping, 0 when they are read in another layout (TryGetPointer)."""
        p = ctypes.c_void_p(0)
        native.call("slhip_gguf_tensor_pointer", self._file._handle(), self.index, ctypes.byref(p))
        return p.value or 0

    def upload(self, dst: int, dst_bytes: int | None = None, stream=None) -> None:
        """Copies the whole tensor (as ``read`` returns it) to device memory ``dst``; ordered on ``stream``."""
        native.call("slhip_gguf_upload", self._file._handle(), self.index, dst,
                    self.byte_size if dst_bytes is None else dst_bytes, stream)

    def __repr__(self):
        return f"{self.name} {self.data_type}{list(self.shape)} @{self.offset} ({self.byte_size} B)"


class GgufFile:
    """A memory-mapped, read-only GGUF file (versions 2 and 3)."""

    def __init__(self, handle, path):
        self._h = handle
        self.path = path
        info = native.GgufInfo()
        native.call("slhip_gguf_get_info", handle, ctypes.byref(info))
        self.version, self.alignment = info.version, info.alignment
        self.data_offset, self.file_length = info.data_offset, info.file_length
        self.tensor_table_complete = bool(info.table_complete)
        self._n_kv, self._n_tensors = info.n_kv, info.n_tensors
        self._metadata = None
        self._tensors = None

    @classmethod
    def open(cls, path) -> "GgufFile":
        h = ctypes.c_void_p(0)
        native.call("slhip_gguf_open", str(path).encode(), ctypes.byref(h))
        return cls(h.value, str(path))

    @classmethod
    def from_prefix(cls, prefix: bytes) -> "GgufFile":
        """The first bytes of a file: the metadata pairs it holds whole, the tensor table when complete."""
        h = ctypes.c_void_p(0)
        buf = ctypes.create_string_buffer(bytes(prefix), len(prefix))
        native.call("slhip_gguf_open_prefix", buf, len(prefix), ctypes.byref(h))
        return cls(h.value, None)

    def _handle(self):
        if self._h is None:
            raise ValueError("the GGUF file is closed")  # ObjectDisposedException
        return self._h

    @property
    def metadata(self) -> dict:
        if self._metadata is None:
            h, md = self._handle(), {}
            key, node = ctypes.c_char_p(), ctypes.c_int64()
            for k in range(self._n_kv):
                native.call("slhip_gguf_kv", h, k, ctypes.byref(key), ctypes.byref(node))
                md[key.value.decode("utf-8", errors="replace")] = _decode(h, node.value)
            self._metadata = md
        return self._metadata

    @property
    def tensors(self) -> list:
        if self._tensors is None:
            h, out = self._handle(), []
            for k in range(self._n_tensors):
                t = native.GgufTensor()
                native.call("slhip_gguf_tensor_info", h, k, ctypes.byref(t))
                out.append(GgufTensorInfo(self, k, t))
            self._tensors = out
        return self._tensors

    @property
    def architecture(self):
        a = self.metadata.get("general.architecture")
        return a if isinstance(a, str) else None

    def find_tensor(self, name: str):
        i = ctypes.c_int64(-1)
        native.call("slhip_gguf_find_tensor", self._handle(), name.encode(), ctypes.byref(i))
        return None if i.value < 0 else self.tensors[i.value]

    def get_tensor(self, name: str) -> GgufTensorInfo:
        t = self.find_tensor(name)
        if t is None:
            raise KeyError(f"Tensor '{name}' not found.")
        return t

    def close(self) -> None:
        if self._h is not None:
            native.call("slhip_gguf_close", self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class GgufModelFiles:
    """One model that may be split over several shards (``name-00001-of-00003.gguf``): metadata of the
    first shard, tensors of all shards in order (GgufModelFiles.cs:9-110)."""

    _SHARD = re.compile(r"^(?P<prefix>.*)-(?P<idx>\d{5})-of-(?P<n>\d{5})\.gguf$", re.IGNORECASE)

    def __init__(self, files):
        self.files = files
        self.tensors = [t for f in files for t in f.tensors]
        self._by_name = {t.name: t for t in self.tensors}

    @classmethod
    def open(cls, path) -> "GgufModelFiles":
        """A single file, or every shard when `path` names the first shard of a split model; ValueError for
        another shard (ArgumentException)."""
        path = str(path)
        m = cls._SHARD.match(os.path.basename(path))
        files = []
        try:
            first = GgufFile.open(path)
            files.append(first)
            if m:
                index, count = int(m["idx"]), int(m["n"])
                declared = first.metadata.get("split.count")
                if isinstance(declared, np.integer) and 0 < int(declared) <= 2**31 - 1:
                    count = int(declared)
                if index != 1:
                    raise ValueError("Pass the first shard (-00001-of-N) of a split model.")
                width = len(m["idx"])
                for i in range(2, count + 1):
                    name = f"{m['prefix']}-{i:0{width}d}-of-{count:0{width}d}.gguf"
                    files.append(GgufFile.open(os.path.join(os.path.dirname(path) or ".", name)))
            return cls(files)
        except BaseException:
            for f in files:
                f.close()
            raise

    @property
    def first(self) -> GgufFile:
        return self.files[0]

    @property
    def metadata(self) -> dict:
        return self.first.metadata

    @property
    def architecture(self):
        return self.first.architecture

    def find_tensor(self, name: str):
        return self._by_name.get(name)

    def close(self) -> None:
        for f in self.files:
            f.close()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


def read_metadata(prefix: bytes) -> dict:
    """GgufHeaderProbe.ReadMetadata: the pairs the prefix holds whole ({} when it is not GGUF)."""
    with GgufFile.from_prefix(prefix) as f:
        return dict(f.metadata)


def read_tensor_table(prefix: bytes):
    """GgufHeaderProbe.ReadTensorTable: [(name, ggml type id, ne)] when the prefix holds the whole table,
    else None."""
    with GgufFile.from_prefix(prefix) as f:
        if not f.tensor_table_complete:
            return None
        return [(t.name, t.ggml_type, list(t.ne)) for t in f.tensors]


def ggml_type(type_id: int) -> dict:
    """GgmlTypes.GetDataType with the type's block geometry; SlhipNotSupported for an unknown id."""
    t = native.GgufTensor()
    native.call("slhip_gguf_type", type_id, ctypes.byref(t))
    return dict(name=t.type_name.decode(), block_size=t.block_size, block_bytes=t.block_bytes,
                format=_FORMAT_NAMES.get(t.format))


def upload(dst: int, src, nbytes: int | None = None, stream=None) -> None:
    """Staged copy of pageable host memory (an address, or a buffer-protocol object) to device memory."""
    if isinstance(src, int):
        if nbytes is None:
            raise ValueError("nbytes is required with an address")
        native.call("slhip_upload", dst, src, nbytes, stream)
        return
    a = np.frombuffer(src, np.uint8) if not isinstance(src, np.ndarray) else src.reshape(-1).view(np.uint8)
    native.call("slhip_upload", dst, a.ctypes.data, a.nbytes if nbytes is None else nbytes, stream)


# ---- writer ---------------------------------------------------------------------------------------

_SCALAR_FMT = {UINT8: "<B", INT8: "<b", UINT16: "<H", INT16: "<h", UINT32: "<I", INT32: "<i", FLOAT32: "<f",
               UINT64: "<Q", INT64: "<q", FLOAT64: "<d"}
_NP_TO_VT = {np.dtype(v): k for k, v in _NP.items()}


def _vtype(v):
    if isinstance(v, (bool, np.bool_)):
        return BOOL
    if isinstance(v, str):
        return STRING
    if isinstance(v, np.generic):
        return _NP_TO_VT[v.dtype]
    if isinstance(v, int):
        return INT32 if -2**31 <= v < 2**31 else INT64
    if isinstance(v, float):
        return FLOAT64
    if isinstance(v, (list, tuple, np.ndarray)):
        return ARRAY
    raise TypeError(f"cannot write metadata of type {type(v)}")


def _elem_type(a):
    if isinstance(a, np.ndarray):
        return BOOL if a.dtype == np.bool_ else _NP_TO_VT[a.dtype]
    if all(isinstance(e, str) for e in a) and len(a):
        return STRING
    if all(isinstance(e, (list, tuple, np.ndarray)) for e in a) and len(a):
        return ARRAY
    if len(a) == 0:
        return INT32
    return _vtype(a[0])


def _string(s: str) -> bytes:
    b = s.encode("utf-8")
    return struct.pack("<Q", len(b)) + b


def _value(v, t) -> bytes:
    if t in _SCALAR_FMT:
        return struct.pack(_SCALAR_FMT[t], v.item() if isinstance(v, np.generic) else v)
    if t == BOOL:
        return bytes([1 if v else 0])
    if t == STRING:
        return _string(v)
    e = _elem_type(v)
    out = struct.pack("<IQ", e, len(v))
    if isinstance(v, np.ndarray) and e != BOOL:
        return out + np.ascontiguousarray(v, v.dtype.newbyteorder("<")).tobytes()
    return out + b"".join(_value(x, e) for x in v)


class GgufWriter:
    """Minimal GGUF v3 writer (GgufWriter.cs:7-191): metadata in the order added, then the tensor table,
    then each tensor's bytes padded to the alignment."""

    def __init__(self, alignment: int = 32):
        self.alignment = alignment
        self._kv = []
        self._tensors = []

    def add_metadata(self, key: str, value, vtype: int | None = None) -> "GgufWriter":
        """Python int -> int32 (int64 beyond), float -> float64, numpy scalars and arrays keep their width;
        `vtype` forces a scalar's type."""
        self._kv.append((key, value, vtype))
        return self

    def add_tensor_ne(self, name: str, type_id: int, data, ne, layout_type: int | None = None) -> "GgufWriter":
        """A tensor with ggml-order dimensions; `layout_type` sizes ids stored in another type's layout."""
        data = bytes(data)
        t = ggml_type(type_id if layout_type is None else layout_type)
        n = int(np.prod(ne, dtype=np.int64)) if len(ne) else 1
        expected = n // t["block_size"] * t["block_bytes"]
        if len(data) != expected:
            raise ValueError(f"Tensor '{name}': expected {expected} bytes, got {len(data)}.")
        self._tensors.append((name, type_id, list(ne), data))
        return self

    def add_tensor(self, name: str, type_id: int, data, dims) -> "GgufWriter":
        """A tensor with row-major (outermost-first) dimensions."""
        return self.add_tensor_ne(name, type_id, data, list(reversed(list(dims))))

    def _align(self, n):
        return (n + self.alignment - 1) // self.alignment * self.alignment

    def to_bytes(self) -> bytes:
        kv = list(self._kv)
        if self.alignment != 32 and not any(k == "general.alignment" for k, _, _ in kv):
            kv.append(("general.alignment", np.uint32(self.alignment), None))
        out = bytearray(struct.pack("<IIQQ", 0x46554747, 3, len(self._tensors), len(kv)))
        for key, value, vtype in kv:
            t = _vtype(value) if vtype is None else vtype
            out += _string(key) + struct.pack("<I", t) + _value(value, t)
        off = 0
        for name, type_id, ne, data in self._tensors:
            out += _string(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", n) for n in ne)
            out += struct.pack("<IQ", type_id, off)
            off += self._align(len(data))
        out += bytes(self._align(len(out)) - len(out))
        for _, _, _, data in self._tensors:
            out += data
            out += bytes(self._align(len(out)) - len(out))
        return bytes(out)

    def write(self, path) -> None:
        with open(path, "wb") as f:
            f.write(self.to_bytes())
