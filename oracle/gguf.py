"""CPU oracle of GGUF reading -- TEST INFRASTRUCTURE ONLY.

A pure-Python restatement of the reference's GGUF reader, the checker of the native reader and uploader
(``slhip_gguf_*``, ``slhip_upload``). Only ``tests/`` and ``bench.py``'s ``cpu_baseline`` leg use it.

Follows:
- ``src/Sharplight.Import.Gguf/GgufFile.cs:72-245``: header, metadata, alignment, tensor table, data
  offset, byte sizes and the bounds of every tensor.
- ``GgufReader.cs:34-175``: the bounds-checked cursor, the value types, the guards on array counts.
- ``GgmlTypes.cs:52-119``: ggml type ids and what each is read as, with the block geometry of
  ``src/Sharplight.Core/Tensors/DataType.cs:76-244``.
- ``GgufHeaderProbe.cs:17-135``: metadata and tensor table from a prefix of a file.
- ``GgufInterleavedQ4_0Source.cs:43-79``, ``GgufI2sSource.cs:11-64`` and ``GgmlNarrowIq1.cs:55-86``: the
  types read in another layout than they are stored in.

Metadata values come back typed as the reference's CLR values are: numpy scalars of the exact width
for numbers, ``bool``, ``str``; numpy arrays for numeric and bool arrays, ``list`` of ``str`` for string
arrays, ``list`` for arrays of arrays.
"""
from __future__ import annotations

import struct

import numpy as np

MAGIC = 0x46554747
DEFAULT_ALIGNMENT = 32
HEADER_BYTES = 24
MAX_DIMS = 8
INT_MAX = 2**31 - 1


class GgufFormatError(ValueError):
    """InvalidDataException (and the OverflowException of a checked conversion)."""


class GgufUnsupported(ValueError):
    """NotSupportedException / UnsupportedWeightFormatException."""


# id -> (DataType name, block size, block bytes); GgmlTypes.Build and the DataType registrations
_PLAIN = {
    0: ("f32", 1, 4), 1: ("f16", 1, 2), 2: ("q4_0", 32, 18), 3: ("q4_1", 32, 20), 6: ("q5_0", 32, 22),
    7: ("q5_1", 32, 24), 8: ("q8_0", 32, 34), 9: ("q8_1", 32, 36), 10: ("q2_k", 256, 84), 11: ("q3_k", 256, 110),
    12: ("q4_k", 256, 144), 13: ("q5_k", 256, 176), 14: ("q6_k", 256, 210), 15: ("q8_k", 256, 292),
    16: ("iq2_xxs", 256, 66), 17: ("iq2_xs", 256, 74), 18: ("iq3_xxs", 256, 98), 19: ("iq1_s", 256, 50),
    20: ("iq4_nl", 32, 18), 21: ("iq3_s", 256, 110), 22: ("iq2_s", 256, 82), 23: ("iq4_xs", 256, 136),
    24: ("i8", 1, 1), 25: ("i16", 1, 2), 26: ("i32", 1, 4), 27: ("i64", 1, 8), 28: ("f64", 1, 8),
    29: ("iq1_m", 256, 56), 30: ("bf16", 1, 2), 34: ("tq1_0", 256, 54), 35: ("tq2_0", 256, 66),
    36: ("q2s_g128", 128, 36), 39: ("mxfp4", 32, 17), 40: ("nvfp4", 64, 36), 41: ("q1_0", 128, 18),
    42: ("q2_0", 64, 18), 43: ("f8_e4m3", 1, 1),
    142: ("q2_0_g128", 128, 34), 143: ("tern1_g128", 128, 28),
    144: ("trellis_v4k8_g128", 128, 34), 145: ("trellis_v4k6_g128", 128, 26), 146: ("trellis_v4k7_g128", 128, 30),
    147: ("trellis_v2k5_g128", 128, 42), 148: ("trellis_v2k6_g128", 128, 50), 149: ("trellis_v2k7_g128", 128, 58),
}
INTERLEAVED_Q4_0 = {31: (4, 4), 32: (4, 8), 33: (8, 8)}  # id -> (rows per group, nibble bytes kept together)
NARROW_IQ1 = {64: 46, 65: 42, 66: 38}                    # id -> stored bytes per 256-value block
I2S = 36


def type_of(ggml_type: int):
    """GgmlTypes.TryGetDataType: (name, block size, block bytes) of what the id is read as, or None."""
    if ggml_type in INTERLEAVED_Q4_0:
        return _PLAIN[2]
    if ggml_type in NARROW_IQ1:
        return _PLAIN[19]
    return _PLAIN.get(ggml_type)


def compute_byte_size(t, ne, name):
    """GgufFile.ComputeByteSize (GgufFile.cs:215-230)."""
    elements = 1
    for n in ne:
        elements *= n
    if elements > 2**63 - 1:
        raise GgufFormatError("Arithmetic operation resulted in an overflow.")
    row = ne[0] if ne else 1
    if row % t[1] != 0:
        raise GgufFormatError(f"Tensor '{name}': row length {row} is not a multiple of {t[0]} block size {t[1]}.")
    return elements // t[1] * t[2]


def stored_byte_size(ggml_type, size):
    """GgufFile.StoredByteSize (GgufFile.cs:207-213)."""
    if ggml_type in NARROW_IQ1:
        return size // 50 * NARROW_IQ1[ggml_type]
    if ggml_type == I2S:
        return size // 36 * 32 + 32
    return size


class _Cursor:
    """GgufReader: every read checks the remaining length."""

    def __init__(self, data, length=None):
        self.data = data
        self.length = len(data) if length is None else length
        self.pos = 0

    def take(self, n):
        if n < 0 or self.pos + n > self.length:
            raise GgufFormatError("Unexpected end of GGUF file.")
        b = self.data[self.pos:self.pos + n]
        self.pos += n
        return b

    def u32(self):
        return struct.unpack("<I", self.take(4))[0]

    def u64(self):
        return struct.unpack("<Q", self.take(8))[0]

    def len64(self):  # checked((long)ReadU64())
        v = self.u64()
        if v > 2**63 - 1:
            raise GgufFormatError("Arithmetic operation resulted in an overflow.")
        return v

    def string(self):
        n = self.len64()
        if n > INT_MAX:
            raise GgufFormatError("String too long.")
        return bytes(self.take(n)).decode("utf-8", errors="replace") if n else ""

    _SCALAR = {0: "<u1", 1: "<i1", 2: "<u2", 3: "<i2", 4: "<u4", 5: "<i4", 6: "<f4", 10: "<u8", 11: "<i8", 12: "<f8"}

    def value(self, vtype):
        """GgufReader.ReadValue."""
        if vtype in self._SCALAR:
            dt = np.dtype(self._SCALAR[vtype])
            return np.frombuffer(bytes(self.take(dt.itemsize)), dt)[0].astype(dt.newbyteorder("="))
        if vtype == 7:
            return self.take(1)[0] != 0
        if vtype == 8:
            return self.string()
        if vtype == 9:
            return self.array()
        raise GgufFormatError(f"Unknown GGUF value type {vtype}.")

    def array(self):
        """GgufReader.ReadArray (GgufReader.cs:99-127)."""
        elem = self.u32()
        count = self.len64()
        if count > INT_MAX:
            raise GgufFormatError("Array too large.")
        if elem in self._SCALAR:
            dt = np.dtype(self._SCALAR[elem])
            return np.frombuffer(bytes(self.take(count * dt.itemsize)), dt).astype(dt.newbyteorder("="))
        if elem == 7:
            return np.frombuffer(bytes(self.take(count)), np.uint8) != 0
        if elem == 8:
            if count * 8 > self.length - self.pos:
                raise GgufFormatError("String array larger than file.")
            return [self.string() for _ in range(count)]
        if elem == 9:
            if count * 12 > self.length - self.pos:
                raise GgufFormatError("Array larger than file.")
            return [self.array() for _ in range(count)]
        raise GgufFormatError(f"Unknown GGUF array element type {elem}.")

    def pair(self):
        key = self.string()
        return key, self.value(self.u32())

    def tensor_entry(self):
        """One entry of GgufFile.ReadTensorHeaders (GgufFile.cs:150-177)."""
        name = self.string()
        dims = self.u32()
        if dims > MAX_DIMS:
            raise GgufFormatError(f"Tensor '{name}' has {dims} dimensions.")
        ne = [self.len64() for _ in range(dims)]
        return name, self.u32(), ne, self.len64()


def _alignment(metadata):
    """GgufFile.ReadAlignment: general.alignment when numeric and positive (Convert.ToInt32)."""
    v = metadata.get("general.alignment")
    if v is None or isinstance(v, (str, list, np.ndarray)):
        return DEFAULT_ALIGNMENT
    if isinstance(v, (np.floating, float)):
        f = float(v)
        if not (-2147483648.5 <= f < 2147483647.5):
            raise GgufFormatError("Value was either too large or too small for an Int32.")
        v = round(f)  # half to even, as Convert.ToInt32
    v = int(v)
    if not (-2**31 <= v <= INT_MAX):
        raise GgufFormatError("Value was either too large or too small for an Int32.")
    return v if v > 0 else DEFAULT_ALIGNMENT


def parse_file(data, file_length=None):
    """GgufFile.Open on the file bytes `data`: dict(version, alignment, data_offset, metadata, keys,
    tensors), tensors as dicts in file order. `file_length` (default len(data)) is the size of the whole
    file when `data` holds only its first bytes: the header is read from `data`, the tensors' bounds are
    checked against the file."""
    length = len(data) if file_length is None else file_length
    if length < HEADER_BYTES:
        raise GgufFormatError("File too small to be GGUF.")
    c = _Cursor(data, min(len(data), length))
    if c.u32() != MAGIC:
        raise GgufFormatError("Not a GGUF file (bad magic).")
    version = c.u32()
    if version not in (2, 3):
        raise GgufUnsupported(f"Unsupported GGUF version {version}.")
    n_tensors, n_kv = c.len64(), c.len64()
    if n_tensors > length or n_kv > length:
        raise GgufFormatError("Implausible tensor/KV count.")
    metadata, keys = {}, []
    for _ in range(n_kv):
        k, v = c.pair()
        metadata[k] = v
        keys.append(k)
    alignment = _alignment(metadata)
    entries = [c.tensor_entry() for _ in range(n_tensors)]
    data_offset = (c.pos + alignment - 1) // alignment * alignment
    tensors = []
    for name, ggml, ne, rel in entries:
        t = type_of(ggml)
        if t is None:
            raise GgufUnsupported(f"Unsupported ggml tensor type id {ggml}.")
        size = compute_byte_size(t, ne, name)
        if ggml in INTERLEAVED_Q4_0:
            rows = size // t[2] * t[1] // max(1, ne[0] if ne else 1)
            if rows % INTERLEAVED_Q4_0[ggml][0]:
                raise GgufFormatError(f"Tensor '{name}': {rows} rows are not a multiple of the "
                                      f"{INTERLEAVED_Q4_0[ggml][0]} rows its type interleaves.")
        stored = stored_byte_size(ggml, size)
        off = data_offset + rel
        if off < 0 or off + stored > length:
            raise GgufFormatError(f"Tensor '{name}' extends beyond the end of the file (offset {off}, size {stored}, "
                                  f"file {length}).")
        tensors.append(dict(name=name, ggml_type=ggml, type_name=t[0], block_size=t[1], block_bytes=t[2], ne=list(ne),
                            shape=tuple(reversed(ne)), relative_offset=rel, offset=off, byte_size=size,
                            stored_bytes=stored))
    return dict(version=version, alignment=alignment, data_offset=data_offset, metadata=metadata, keys=keys,
                tensors=tensors)


def probe_metadata(prefix):
    """GgufHeaderProbe.ReadMetadata: the pairs the prefix holds whole (empty when it is not GGUF)."""
    out = {}
    if len(prefix) < HEADER_BYTES:
        return out
    c = _Cursor(prefix)
    if c.u32() != MAGIC or c.u32() not in (2, 3):
        return out
    c.u64()
    n_kv = min(c.u64(), INT_MAX)
    for _ in range(n_kv):
        try:
            k, v = c.pair()
        except GgufFormatError:
            break
        out[k] = v
    return out


def probe_tensor_table(prefix):
    """GgufHeaderProbe.ReadTensorTable: [(name, ggml type, ne)] when the prefix holds the whole table,
    else None."""
    if len(prefix) < HEADER_BYTES:
        return None
    c = _Cursor(prefix)
    try:
        if c.u32() != MAGIC or c.u32() not in (2, 3):
            return None
        n_tensors, n_kv = c.u64(), c.u64()
        if n_tensors > len(prefix) or n_kv > len(prefix):
            return None
        for _ in range(n_kv):
            c.pair()
        table = []
        for _ in range(n_tensors):
            name, ggml, ne, _ = c.tensor_entry()
            table.append((name, ggml, ne))
        return table
    except GgufFormatError:
        return None


def read_tensor(data, t):
    """IWeightSource.Read of the whole tensor: its bytes as the type it is read as."""
    raw = bytes(data[t["offset"]:t["offset"] + t["stored_bytes"]])
    g = t["ggml_type"]
    if g in INTERLEAVED_Q4_0:
        return deinterleave_q4_0(raw, t["ne"][0] // 32, *INTERLEAVED_Q4_0[g])
    if g == I2S:
        blocks = t["byte_size"] // 36
        out = np.empty((blocks, 36), np.uint8)
        out[:, :4] = np.frombuffer(raw[blocks * 32:blocks * 32 + 4], np.uint8)
        out[:, 4:] = np.frombuffer(raw[:blocks * 32], np.uint8).reshape(blocks, 32)
        return out.tobytes()
    if g in NARROW_IQ1:
        sb = NARROW_IQ1[g]
        return b"".join(widen_narrow_iq1(g, raw[b * sb:(b + 1) * sb]) for b in range(t["byte_size"] // 50))
    return raw


_NARROW_GRIDS = {}


def _narrow_grid(g):
    """The narrow type's codebook as IQ1_S grid positions, from the library's generated table header
    (sharplight_amd/csrc/narrow_iq1_grids.h: data of the format, pinned by the fork's decoded fixture)."""
    if not _NARROW_GRIDS:
        import os
        import re
        text = open(os.path.join(os.path.dirname(os.path.abspath(__file__)), "..", "sharplight_amd", "csrc",
                                 "narrow_iq1_grids.h")).read()
        for gid, name in ((64, "kNarrowIq1Xs"), (65, "kNarrowIq1Xxs"), (66, "kNarrowIq1Xxxs")):
            body = text[text.index(name + "["):]
            body = body[body.index("{") + 1:body.index("}")]
            _NARROW_GRIDS[gid] = [int(v) for v in re.findall(r"\d+", body)]
    return _NARROW_GRIDS[g]


def widen_narrow_iq1(g, narrow: bytes) -> bytes:
    """GgmlNarrowIq1.Widen (src/Sharplight.Import.Gguf/GgmlNarrowIq1.cs:55-86): one narrow block (46, 42 or 38
    bytes) as the 50-byte IQ1_S block with the same values."""
    grid = _narrow_grid(g)
    wide = bytearray(50)
    wide[0:2] = narrow[0:2]
    qs, tail = narrow[2:34], narrow[34:]
    for ib in range(8):
        if g == 65:
            ss = tail[ib] >> 4
        else:
            ss = (tail[8 + ib // 2 if g == 64 else ib // 2] >> (4 * (ib & 1))) & 0xF
        qh = (ss & 7) << 12 | (ss >> 3) << 15
        for l in range(4):
            high = (tail[ib] >> (2 * l)) & 3 if g == 64 else ((tail[ib] >> l) & 1 if g == 65 else 0)
            index = grid[qs[4 * ib + l] | high << 8]
            wide[2 + 4 * ib + l] = index & 0xFF
            qh |= (index >> 8) << (3 * l)
        wide[34 + 2 * ib:36 + 2 * ib] = struct.pack("<H", qh)
    return bytes(wide)


def deinterleave_q4_0(raw, blocks_per_row, rows, chunk):
    """GgufInterleavedQ4_0Source.Read (GgufInterleavedQ4_0Source.cs:43-79) over the whole tensor: for each
    group of `rows` rows and block column, the rows' f16 scales, then their nibble arrays in `chunk`-byte
    pieces interleaved row by row, XOR 0x88. Returns the plain Q4_0 rows."""
    a = np.frombuffer(raw, np.uint8)
    groups = len(a) // (18 * rows * blocks_per_row)
    g = a.reshape(groups, blocks_per_row, rows * 18)
    scales = g[:, :, :2 * rows].reshape(groups, blocks_per_row, rows, 2)
    nib = g[:, :, 2 * rows:].reshape(groups, blocks_per_row, 16 // chunk, rows, chunk) ^ 0x88
    out = np.empty((groups, rows, blocks_per_row, 18), np.uint8)
    out[..., :2] = scales.transpose(0, 2, 1, 3)
    out[..., 2:] = nib.transpose(0, 3, 1, 2, 4).reshape(groups, rows, blocks_per_row, 16)
    return out.tobytes()
