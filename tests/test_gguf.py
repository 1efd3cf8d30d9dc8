"""GGUF reading: the native reader (slhip_gguf_*) against the oracle restatement, and both against the
reference's fixtures and known answers.

Fixtures: ``tests/golden/gguf/*.header.gguf`` are data files of the reference's tests
(tests/Sharplight.Import.Gguf.Tests/Fixtures: headers of released checkpoints written by llama.cpp and
its forks, tokenizer arrays emptied), copied unchanged. Known answers follow the reference's tests:
GgufRoundTripTests.cs, GgufValidationTests.cs:16-27, InterleavedQ4_0Tests.cs, I2sTests.cs:17-53.

What pins the oracle (and through it the native reader):
- llama.cpp writes tensor data back to back: in file order, each tensor's relative offset is the previous
  one's plus its stored bytes rounded up to the alignment (restarting at 0 for the next shard of a split
  model, whose fixtures list every shard's table). Over the fixtures that fixes the block geometry of
  every ggml type they hold (30 ids, the interleaved, narrow IQ1 and trellis ids among them).
- A file assembled byte by byte in the test (not by the writer) reads back with the offsets and values
  the GGUF layout gives.
- The reference's facts about its fixtures (tensor count and a tensor's dimensions of the gemma-4 header).
- The interleaved Q4_0 layout: llama.cpp's repack (restated from InterleavedQ4_0Tests.Interleave) undone.
- I2_S: blocks decode to (code - 1) * scale with the reference test's code order.
"""
import glob
import math
import os
import struct

import numpy as np
import pytest

from oracle import gguf as og
from sharplight_amd import gguf, native

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "gguf")
FIXTURES = sorted(glob.glob(os.path.join(GOLDEN, "*.header.gguf")))


def _fx(name):
    return open(os.path.join(GOLDEN, name + ".header.gguf"), "rb").read()


def _same(a, b, path="value"):
    """Equal values of the same CLR-like type (numpy dtype / bool / str / list), floats bit for bit."""
    if isinstance(a, list):
        assert isinstance(b, list) and len(a) == len(b), path
        for k, (x, y) in enumerate(zip(a, b)):
            _same(x, y, f"{path}[{k}]")
    elif isinstance(a, np.ndarray):
        assert isinstance(b, np.ndarray) and a.dtype == b.dtype and a.shape == b.shape, path
        assert a.tobytes() == b.tobytes(), path
    elif isinstance(a, np.generic):
        assert type(a) is type(b) and a.tobytes() == b.tobytes(), f"{path}: {a!r} vs {b!r}"
    else:
        assert type(a) is type(b) and a == b, f"{path}: {a!r} vs {b!r}"


def _same_md(a: dict, b: dict):
    assert list(a) == list(b)
    for k in a:
        _same(a[k], b[k], k)


def _entries(data):
    c = og._Cursor(data)
    c.u32(), c.u32()
    nt, nk = c.u64(), c.u64()
    md = {}
    for _ in range(nk):
        k, v = c.pair()
        md[k] = v
    return md, [c.tensor_entry() for _ in range(nt)]


# ---- the oracle against the fixtures ------------------------------------------------------------

@pytest.mark.parametrize("path", FIXTURES, ids=lambda p: os.path.basename(p)[:40])
def test_fixture_tensors_are_back_to_back(path):
    data = open(path, "rb").read()
    md, ents = _entries(data)
    al = og._alignment(md)
    assert ents[0][3] == 0
    for (name, ggml, ne, rel), (_, _, _, nxt) in zip(ents, ents[1:]):
        t = og.type_of(ggml)
        assert t is not None, f"{name}: ggml type {ggml}"
        if nxt == 0:  # the next shard
            continue
        stored = og.stored_byte_size(ggml, og.compute_byte_size(t, ne, name))
        assert (rel + stored + al - 1) // al * al == nxt, f"{name} (type {ggml})"


def test_fixtures_cover_the_type_ids():
    ids = set()
    for p in FIXTURES:
        ids |= {e[1] for e in _entries(open(p, "rb").read())[1]}
    assert {0, 1, 2, 3, 6, 7, 8, 11, 12, 13, 14, 16, 17, 18, 19, 20, 22, 23, 26, 30, 31, 39, 40, 42, 65,
            144, 145, 146, 147, 148, 149} <= ids


def test_gemma4_header_facts():
    """GgufValidationTests.Gemma4Moe_HeaderTensorTable_IsReadCompletely (GgufValidationTests.cs:16-27)."""
    data = _fx("gemma-4-26B-A4B-it-UD-Q4_K_XL")
    for table in (og.probe_tensor_table(data), gguf.read_tensor_table(data)):
        assert len(table) == 658
        assert any(t[0] == "blk.29.ffn_gate_up_exps.weight" for t in table)
        assert [t[2] for t in table if t[0] == "blk.0.ffn_gate_up_exps.weight"] == [[2816, 1408, 128]]
    assert og.probe_tensor_table(data[:-1]) is None
    assert gguf.read_tensor_table(data[:-1]) is None


def test_hand_assembled_file():
    """A v2 file built byte by byte: alignment 64 from metadata, two tensors, data offset rounded up."""
    def s(x):
        b = x.encode()
        return struct.pack("<Q", len(b)) + b
    hdr = struct.pack("<IIQQ", 0x46554747, 2, 2, 3)
    hdr += s("general.alignment") + struct.pack("<II", 4, 64)
    hdr += s("general.architecture") + struct.pack("<I", 8) + s("toy")
    hdr += s("v") + struct.pack("<IIQ", 9, 6, 2) + struct.pack("<ff", 0.25, -3.0)
    hdr += s("a") + struct.pack("<IQQIQ", 2, 4, 2, 0, 0)          # f32 [2, 4]: 32 bytes at 0
    hdr += s("b") + struct.pack("<IQIQ", 1, 32, 8, 64)            # q8_0 [32]: 34 bytes at 64
    data_offset = (len(hdr) + 63) // 64 * 64
    a = np.arange(8, dtype=np.float32).tobytes()
    b = bytes(range(34))
    blob = hdr + bytes(data_offset - len(hdr)) + a + bytes(32) + b
    o = og.parse_file(blob)
    assert (o["version"], o["alignment"], o["data_offset"]) == (2, 64, data_offset)
    assert [(t["name"], t["offset"], t["byte_size"], t["shape"]) for t in o["tensors"]] == [
        ("a", data_offset, 32, (2, 4)), ("b", data_offset + 64, 34, (32,))]
    assert o["metadata"]["v"].tolist() == [0.25, -3.0]
    assert og.read_tensor(blob, o["tensors"][1]) == b
    n = _native_from_bytes(blob)
    assert (n.version, n.alignment, n.data_offset) == (2, 64, data_offset)
    assert n.get_tensor("a").read() == a and n.get_tensor("b").read() == b
    _same_md(n.metadata, o["metadata"])
    n.close()


# ---- native against oracle ----------------------------------------------------------------------

def _native_from_bytes(blob):
    import tempfile
    d = tempfile.mkdtemp(prefix="slgguf-")
    p = os.path.join(d, "f.gguf")
    with open(p, "wb") as f:
        f.write(blob)
    g = gguf.GgufFile.open(p)
    os.unlink(p)  # the mapping keeps the data
    os.rmdir(d)
    return g


@pytest.mark.parametrize("path", FIXTURES, ids=lambda p: os.path.basename(p)[:40])
def test_prefix_probe_matches_oracle(path):
    data = open(path, "rb").read()
    _same_md(gguf.read_metadata(data), og.probe_metadata(data))
    assert gguf.read_tensor_table(data) == og.probe_tensor_table(data)
    # cut inside the metadata, inside the table, and one byte short of its end
    for cut in (24, 100, len(data) // 3, len(data) // 2, len(data) - 40, len(data) - 1):
        _same_md(gguf.read_metadata(data[:cut]), og.probe_metadata(data[:cut]))
        assert gguf.read_tensor_table(data[:cut]) == og.probe_tensor_table(data[:cut])


@pytest.mark.parametrize("name", ["gemma-4-26B-A4B-it-UD-Q4_K_XL", "Llama-3.2-1B-Instruct-Q4_0_4_4",
                                  "NVIDIA-Nemotron-3.5-Lightning-30B-A3B-Q4_0",
                                  "dflash-NVIDIA-Nemotron-3.5-Bolt-74B-A9B-NVFP4",
                                  "Qwen3.8-Flash-Next-Gyro-S-TQ1_0"])
def test_sparse_padded_header_opens_like_oracle(tmp_path, name):
    """The header padded (sparsely) to the size its table needs opens as a whole file
    (GgufValidationTests.Gemma4Moe_Header_MapsLikeTheImporter); one byte less and the last tensor is
    past the end."""
    data = _fx(name)
    need = og.parse_file(data, file_length=1 << 50)
    length = max(t["offset"] + t["stored_bytes"] for t in need["tensors"])
    o = og.parse_file(data, file_length=length)
    p = tmp_path / "h.gguf"
    with open(p, "wb") as f:
        f.write(data)
        f.truncate(length)
    with gguf.GgufFile.open(p) as g:
        assert (g.version, g.alignment, g.data_offset) == (o["version"], o["alignment"], o["data_offset"])
        assert len(g.tensors) == len(o["tensors"])
        for a, b in zip(g.tensors, o["tensors"]):
            assert (a.name, a.ggml_type, a.data_type, a.block_size, a.block_bytes, a.ne, a.shape,
                    a.relative_offset, a.offset, a.byte_size, a.stored_bytes) == (
                b["name"], b["ggml_type"], b["type_name"], b["block_size"], b["block_bytes"], b["ne"], b["shape"],
                b["relative_offset"], b["offset"], b["byte_size"], b["stored_bytes"])
        _same_md(g.metadata, o["metadata"])
    with open(p, "r+b") as f:
        f.truncate(length - 1)
    with pytest.raises(native.SlhipFormatError, match="extends beyond the end of the file"):
        gguf.GgufFile.open(p)
    with pytest.raises(og.GgufFormatError, match="extends beyond the end of the file"):
        og.parse_file(data, file_length=length - 1)


def _roundtrip_writer():
    return (gguf.GgufWriter()
            .add_metadata("general.architecture", "toy")
            .add_metadata("u8", np.uint8(200)).add_metadata("i8", np.int8(-5))
            .add_metadata("u16", np.uint16(65000)).add_metadata("i16", np.int16(-30000))
            .add_metadata("u32", np.uint32(4000000000)).add_metadata("i32", np.int32(-2000000000))
            .add_metadata("f32", np.float32(1.5)).add_metadata("bool", True)
            .add_metadata("u64", np.uint64(2**64 - 1)).add_metadata("i64", np.int64(-2**63))
            .add_metadata("f64", math.pi).add_metadata("str", "héllo wörld")
            .add_metadata("toy.block_count", np.uint32(12))
            .add_metadata("strs", ["a", "", "ünï"])
            .add_metadata("ints", np.array([1, -2, 3], np.int32))
            .add_metadata("uints", np.array([1, 2], np.uint32))
            .add_metadata("floats", np.array([0.5, 1.5], np.float32))
            .add_metadata("bools", np.array([True, False, True]))
            .add_metadata("bytes", np.array([1, 2, 3], np.uint8))
            .add_metadata("nested", [np.array([1, 2], np.int32), ["x"], [np.array([1.0], np.float32)]]))


def test_scalars_arrays_nested_round_trip(tmp_path):
    """GgufRoundTripTests.Scalars_Arrays_Nested_RoundTrip."""
    p = tmp_path / "a.gguf"
    _roundtrip_writer().write(p)
    with gguf.GgufFile.open(p) as f:
        md = f.metadata
        assert f.version == 3 and f.architecture == "toy"
        expect = {"u8": np.uint8(200), "i8": np.int8(-5), "u16": np.uint16(65000), "i16": np.int16(-30000),
                  "u32": np.uint32(4000000000), "i32": np.int32(-2000000000), "f32": np.float32(1.5),
                  "bool": True, "u64": np.uint64(2**64 - 1), "i64": np.int64(-2**63), "f64": np.float64(math.pi),
                  "str": "héllo wörld", "strs": ["a", "", "ünï"], "ints": np.array([1, -2, 3], np.int32),
                  "uints": np.array([1, 2], np.uint32), "floats": np.array([0.5, 1.5], np.float32),
                  "bools": np.array([True, False, True]), "bytes": np.array([1, 2, 3], np.uint8),
                  "nested": [np.array([1, 2], np.int32), ["x"], [np.array([1.0], np.float32)]]}
        for k, v in expect.items():
            _same(md[k], v, k)
        _same_md(md, og.parse_file(open(p, "rb").read())["metadata"])


def _pattern(n, seed=1):
    return bytes((i * 7 + seed) & 255 for i in range(n))


def test_tensors_shapes_sizes_and_sources(tmp_path):
    """GgufRoundTripTests.Tensors_ShapesSizesAndSources."""
    f32, q8, q4k, f16 = _pattern(48), _pattern(2 * 3 * 34, 3), _pattern(144 * 5, 9), _pattern(14, 11)
    p = tmp_path / "t.gguf"
    (gguf.GgufWriter().add_metadata("general.architecture", "toy")
     .add_tensor("w.f32", 0, f32, [3, 4]).add_tensor("w.q8", 8, q8, [2, 96])
     .add_tensor("w.q4k", 12, q4k, [5, 256]).add_tensor("v.f16", 1, f16, [7]).write(p))
    with gguf.GgufFile.open(p) as f:
        assert len(f.tensors) == 4 and f.data_offset % 32 == 0
        assert all(t.offset % 32 == 0 for t in f.tensors)
        t0 = f.get_tensor("w.f32")
        assert (t0.ne, t0.shape, t0.data_type, t0.ggml_type, t0.byte_size) == ([4, 3], (3, 4), "f32", 0, 48)
        tq = f.get_tensor("w.q8")
        assert (tq.shape, tq.byte_size, tq.ggml_type, tq.format) == ((2, 96), 6 * 34, 8, "q8_0")
        assert f.get_tensor("w.q4k").byte_size == 720 and f.get_tensor("v.f16").shape == (7,)
        assert f.find_tensor("nope") is None
        with pytest.raises(KeyError):
            f.get_tensor("nope")
        for name, data in (("w.f32", f32), ("w.q8", q8), ("w.q4k", q4k), ("v.f16", f16)):
            t = f.get_tensor(name)
            assert t.read() == data and t.read(3, 5) == data[3:8]
            assert t.pointer() != 0
            with pytest.raises(native.SlhipIndexError):
                t.read(len(data) - 1, 2)


def test_custom_alignment(tmp_path):
    p = tmp_path / "al.gguf"
    d1, d2 = _pattern(16), _pattern(16, 5)
    w = gguf.GgufWriter(alignment=128).add_metadata("general.architecture", "toy")
    w.add_tensor("a", 0, d1, [4]).add_tensor("b", 0, d2, [4]).write(p)
    with gguf.GgufFile.open(p) as f:
        assert f.alignment == 128 and f.data_offset % 128 == 0
        assert f.get_tensor("b").relative_offset == 128 and f.get_tensor("b").read() == d2


def test_type_table_matches_oracle_and_reference_facts():
    """GgufRoundTripTests.AllGgmlTypes_HaveConsistentLayout / GroupBitFormats_HaveGgmlIds."""
    known = 0
    for i in list(range(44)) + [64, 65, 66] + list(range(142, 150)):
        o = og.type_of(i)
        if o is None:
            with pytest.raises(native.SlhipNotSupported, match=f"Unsupported ggml tensor type id {i}"):
                gguf.ggml_type(i)
            continue
        n = gguf.ggml_type(i)
        assert (n["name"], n["block_size"], n["block_bytes"]) == o
        known += i < 44
    assert known == 44 - 4  # 4, 5, 37 and 38 removed
    assert gguf.ggml_type(16)["block_size"] == 256 and gguf.ggml_type(16)["block_bytes"] == 66
    assert (gguf.ggml_type(40)["block_size"], gguf.ggml_type(40)["block_bytes"]) == (64, 36)
    assert gguf.ggml_type(14)["name"] == "q6_k" and gguf.ggml_type(30)["name"] == "bf16"
    assert gguf.ggml_type(39)["name"] == "mxfp4" and gguf.ggml_type(31)["name"] == "q4_0"
    for i, geo in ((41, (128, 18)), (42, (64, 18)), (142, (128, 34)), (143, (128, 28))):
        assert (gguf.ggml_type(i)["block_size"], gguf.ggml_type(i)["block_bytes"]) == geo
    # the formats this library's kernels read
    assert [gguf.ggml_type(i)["format"] for i in (0, 1, 30, 8, 2, 3, 6, 7, 10, 11, 12, 13, 14, 20, 23, 31)] == [
        "f32", "f16", "bf16", "q8_0", "q4_0", "q4_1", "q5_0", "q5_1", "q2_k", "q3_k", "q4_k", "q5_k", "q6_k",
        "iq4_nl", "iq4_xs", "q4_0"]


def test_many_tensor_types_round_trip(tmp_path):
    p = tmp_path / "many.gguf"
    ids = [2, 7, 10, 14, 23, 21, 34, 40, 39, 30, 26, 41, 42, 142, 143]
    w = gguf.GgufWriter().add_metadata("general.architecture", "toy")
    for i in ids:
        t = og.type_of(i)
        w.add_tensor(f"t.{t[0]}", i, _pattern(2 * t[2]), [2, t[1]])
    w.write(p)
    with gguf.GgufFile.open(p) as f:
        for i in ids:
            t = og.type_of(i)
            info = f.get_tensor(f"t.{t[0]}")
            assert (info.data_type, info.shape, info.byte_size) == (t[0], (2, t[1]), 2 * t[2])


# ---- errors -------------------------------------------------------------------------------------

def _both_raise(blob, exc_native, exc_oracle, match):
    with pytest.raises(exc_oracle, match=match):
        og.parse_file(blob)
    with pytest.raises(exc_native, match=match):
        _native_from_bytes(blob)


def test_bad_magic_small_file_and_versions():
    _both_raise(bytes(64), native.SlhipFormatError, og.GgufFormatError, r"bad magic")
    _both_raise(bytes(10), native.SlhipFormatError, og.GgufFormatError, "too small")
    good = gguf.GgufWriter().add_metadata("general.architecture", "toy").to_bytes()
    _both_raise(good[:4] + struct.pack("<I", 4) + good[8:], native.SlhipNotSupported, og.GgufUnsupported,
                "Unsupported GGUF version 4")


def test_every_truncation_fails_like_the_oracle():
    """GgufRoundTripTests.BadMagic_And_Truncation_Throw, at every length."""
    blob = (_roundtrip_writer().add_tensor("a", 0, _pattern(64), [16]).to_bytes())
    for cut in range(24, len(blob)):
        with pytest.raises(og.GgufFormatError) as eo:
            og.parse_file(blob[:cut])
        with pytest.raises(native.SlhipFormatError) as en:
            _native_from_bytes(blob[:cut])
        assert str(en.value) == str(eo.value), cut


def test_malformed_tables_and_values():
    def file_with(kv_bytes=b"", n_kv=0, tensors=b"", n_t=0):
        return struct.pack("<IIQQ", 0x46554747, 3, n_t, n_kv) + kv_bytes + tensors + bytes(64)
    key = struct.pack("<Q", 1) + b"k"
    cases = [
        (file_with(key + struct.pack("<I", 13), 1), native.SlhipFormatError, "Unknown GGUF value type 13"),
        (file_with(key + struct.pack("<IIQ", 9, 8, 10**6), 1), native.SlhipFormatError, "String array larger than file"),
        (file_with(key + struct.pack("<IIQ", 9, 9, 10**6), 1), native.SlhipFormatError, "Array larger than file"),
        (file_with(key + struct.pack("<IIQ", 9, 0, 2**31), 1), native.SlhipFormatError, "Array too large"),
        (file_with(key + struct.pack("<IIQ", 9, 14, 1), 1), native.SlhipFormatError, "Unknown GGUF array element type 14"),
        (file_with(key + struct.pack("<IQ", 8, 2**31), 1), native.SlhipFormatError, "String too long"),
        (file_with(n_kv=10**6), native.SlhipFormatError, "Implausible tensor/KV count"),
        (file_with(tensors=key + struct.pack("<I", 9), n_t=1), native.SlhipFormatError, "has 9 dimensions"),
        (file_with(tensors=key + struct.pack("<IQIQ", 1, 32, 37, 0), n_t=1), native.SlhipNotSupported,
         "Unsupported ggml tensor type id 37"),
        (file_with(tensors=key + struct.pack("<IQIQ", 1, 48, 8, 0), n_t=1), native.SlhipFormatError,
         "row length 48 is not a multiple of q8_0 block size 32"),
        (file_with(tensors=key + struct.pack("<IQQIQ", 2, 32, 3, 31, 0), n_t=1), native.SlhipFormatError,
         "3 rows are not a multiple of the 4 rows its type interleaves"),
    ]
    for blob, exc, match in cases:
        oexc = og.GgufUnsupported if exc is native.SlhipNotSupported else og.GgufFormatError
        _both_raise(blob, exc, oexc, match)


def test_deeply_nested_arrays_fail_without_recursing_away():
    """Arrays of arrays nest at most 64 deep; deeper nesting is a format error, not a stack overflow.

    The reference recurses without a limit in managed code; a native reader must not, since a file of
    a few MB could nest 10^5 deep. 64 levels still open."""
    def nested(depth):
        key = struct.pack("<Q", 1) + b"k"
        body = struct.pack("<I", 9) + struct.pack("<IQ", 9, 1) * (depth - 1) + struct.pack("<IQ", 4, 1) + \
            struct.pack("<I", 7)
        return struct.pack("<IIQQ", 0x46554747, 3, 0, 1) + key + body + bytes(64)
    f = _native_from_bytes(nested(64))
    assert f is not None
    with pytest.raises(native.SlhipFormatError, match="nested deeper than 64"):
        _native_from_bytes(nested(65))
    with pytest.raises(native.SlhipFormatError, match="nested deeper than 64"):
        _native_from_bytes(nested(200000))


def test_closed_file_refuses_reads(tmp_path):
    """GgufRoundTripTests.Dispose_InvalidatesSources."""
    p = tmp_path / "d.gguf"
    gguf.GgufWriter().add_tensor("a", 0, _pattern(16), [4]).write(p)
    f = gguf.GgufFile.open(p)
    t = f.get_tensor("a")
    f.close()
    with pytest.raises(ValueError, match="closed"):
        t.read()


# ---- types read in another layout -----------------------------------------------------------------

def interleave_q4_0(plain: bytes, row_count: int, blocks: int, rows: int, chunk: int) -> bytes:
    """llama.cpp's repack into the interleaved Q4_0 types, as InterleavedQ4_0Tests.Interleave states it."""
    out = bytearray()
    for group in range(row_count // rows):
        for column in range(blocks):
            for r in range(rows):
                src = ((group * rows + r) * blocks + column) * 18
                out += plain[src:src + 2]
            for i in range(rows * 16 // chunk):
                src = ((group * rows + i % rows) * blocks + column) * 18 + 2 + i // rows * chunk
                out += bytes(b ^ 0x88 for b in plain[src:src + chunk])
    return bytes(out)


@pytest.mark.parametrize("type_id,rows,chunk", [(31, 4, 4), (32, 4, 8), (33, 8, 8)])
def test_interleaved_q4_0_reads_as_plain(tmp_path, type_id, rows, chunk):
    columns, row_count = 96, 2 * rows
    plain = np.random.default_rng(type_id).integers(0, 256, row_count * columns // 32 * 18, dtype=np.uint8).tobytes()
    inter = interleave_q4_0(plain, row_count, columns // 32, rows, chunk)
    p = tmp_path / "q40x.gguf"
    gguf.GgufWriter().add_metadata("general.architecture", "toy").add_tensor_ne(
        "w", type_id, inter, [columns, row_count], layout_type=2).write(p)
    blob = open(p, "rb").read()
    o = og.parse_file(blob)
    assert og.read_tensor(blob, o["tensors"][0]) == plain
    with gguf.GgufFile.open(p) as f:
        t = f.get_tensor("w")
        assert (t.data_type, t.format, t.ggml_type) == ("q4_0", "q4_0", type_id)
        assert t.read() == plain and t.read(25, 50) == plain[25:75]
        assert t.pointer() == 0


def test_i2s_reads_as_scaled_blocks(tmp_path):
    """I2sTests.Source_SpreadsTheTensorScaleOverTheBlocks: 3 x 256 ternary values, scale 1.7."""
    rows, columns = 3, 256
    rng = np.random.default_rng(5)
    c = rng.integers(0, 3, (rows * columns // 4, 4))
    codes = (c[:, 0] << 6 | c[:, 1] << 4 | c[:, 2] << 2 | c[:, 3]).astype(np.uint8).tobytes()
    stored = codes + struct.pack("<f", 1.7) + bytes(28)
    hdr = struct.pack("<IIQQ", 0x46554747, 3, 1, 0) + struct.pack("<Q", 1) + b"w"
    hdr += struct.pack("<IQQIQ", 2, columns, rows, 36, 0)
    blob = hdr + bytes((len(hdr) + 31) // 32 * 32 - len(hdr)) + stored
    p = tmp_path / "i2s.gguf"
    p.write_bytes(blob)
    with gguf.GgufFile.open(p) as f:
        t = f.tensors[0]
        assert (t.data_type, t.byte_size, t.stored_bytes) == ("q2s_g128", rows * columns // 128 * 36, len(stored))
        blocks = t.read()
        assert t.read(41, 50) == blocks[41:91]
        assert blocks == og.read_tensor(blob, og.parse_file(blob)["tensors"][0])
    # decode the q2s_g128 blocks: (code - 1) * scale, byte j of a group holding values j, 32+j, 64+j, 96+j
    b = np.frombuffer(blocks, np.uint8).reshape(-1, 36)
    scale = b[:, :4].copy().view(np.float32)[:, 0]
    assert np.all(scale == np.float32(1.7))
    within = np.arange(128)
    got = ((b[:, 4:][:, within % 32] >> (6 - 2 * (within // 32))) & 3).astype(np.float32) - 1
    cb = np.frombuffer(codes, np.uint8).reshape(-1, 32)
    want = ((cb[:, within % 32] >> (6 - 2 * (within // 32))) & 3).astype(np.float32) - 1
    assert np.array_equal(got * scale[:, None], want * np.float32(1.7))


def _narrow_records():
    import oracle  # noqa: F401  (the C oracle decodes the widened IQ1_S blocks)
    fx = np.load(os.path.join(os.path.dirname(__file__), "golden", "ggml_narrow_iq1.npz"))
    n = len([k for k in fx.files if k.endswith("_type")])
    return [(int(fx[f"r{i}_type"][0]), int(fx[f"r{i}_type"][1]), int(fx[f"r{i}_type"][2]), fx[f"r{i}_blocks"].tobytes(),
             fx[f"r{i}_deq"]) for i in range(n)]


def test_narrow_iq1_widening_decodes_like_the_fork():
    """NarrowIq1Tests.WidenedBlocks_DecodeLikeTheFork: blocks of the three narrow types (gaussian data and random
    bytes), widened to IQ1_S, decode to the fork's own floats -- here bit for bit (the reference allows 1e-6)."""
    import oracle
    recs = _narrow_records()
    assert sorted({r[0] for r in recs}) == [64, 65, 66]
    for g, rows, cols, blocks, want in recs:
        sb = og.NARROW_IQ1[g]
        wide = b"".join(og.widen_narrow_iq1(g, blocks[k * sb:(k + 1) * sb]) for k in range(rows * cols // 256))
        got = oracle.dequant("iq1_s", np.frombuffer(wide, np.uint8), rows * cols).reshape(rows, cols)
        nan = np.isnan(want)
        assert np.array_equal(np.isnan(got), nan)
        assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32)), g


def test_narrow_iq1_reads_widened_at_any_offset(tmp_path):
    """NarrowIq1Tests.Source_ReadsWidenedBlocksAtAnyOffset, for every narrow type and fixture record: the
    native reader returns the oracle's widened blocks, whole and from a range inside blocks."""
    for i, (g, rows, cols, blocks, _) in enumerate(_narrow_records()):
        hdr = struct.pack("<IIQQ", 0x46554747, 3, 1, 0) + struct.pack("<Q", 1) + b"w"
        hdr += struct.pack("<IQQIQ", 2, cols, rows, g, 0)
        blob = hdr + bytes((len(hdr) + 31) // 32 * 32 - len(hdr)) + blocks
        p = tmp_path / f"n{i}.gguf"
        p.write_bytes(blob)
        want = og.read_tensor(blob, og.parse_file(blob)["tensors"][0])
        with gguf.GgufFile.open(p) as f:
            t = f.tensors[0]
            assert (t.data_type, t.format, t.byte_size, t.stored_bytes) == ("iq1_s", "iq1_s", len(want), len(blocks))
            assert t.read() == want and t.read(37, 61) == want[37:98]
            assert t.pointer() == 0


def test_narrow_iq1_header_prefix_has_no_data():
    data = _fx("Kimi-K3-UD-TQ1_0")
    with gguf.GgufFile.from_prefix(data) as f:
        t = next(t for t in f.tensors if t.ggml_type == 65)
        assert (t.data_type, t.block_bytes, t.format) == ("iq1_s", 50, "iq1_s")
        assert t.stored_bytes == t.byte_size // 50 * 42
        with pytest.raises(native.SlhipArgumentError, match="header prefix"):
            t.read(0, 1)


def test_split_files_are_merged(tmp_path):
    """GgufRoundTripTests.Split_Files_AreMerged; a later shard refuses to open the model."""
    p1, p2 = tmp_path / "m-00001-of-00002.gguf", tmp_path / "m-00002-of-00002.gguf"
    (gguf.GgufWriter().add_metadata("general.architecture", "toy").add_metadata("split.count", np.uint16(2))
     .add_tensor("a", 0, _pattern(8), [2]).write(p1))
    gguf.GgufWriter().add_metadata("split.no", np.uint16(1)).add_tensor("b", 0, _pattern(8, 2), [2]).write(p2)
    with gguf.GgufModelFiles.open(p1) as m:
        assert len(m.files) == 2 and len(m.tensors) == 2 and m.architecture == "toy"
        assert m.find_tensor("b").read() == _pattern(8, 2)
    with pytest.raises(ValueError, match="first shard"):
        gguf.GgufModelFiles.open(p2)
    single = tmp_path / "one.gguf"
    gguf.GgufWriter().add_tensor("c", 0, _pattern(4), [1]).write(single)
    with gguf.GgufModelFiles.open(single) as m:
        assert [t.name for t in m.tensors] == ["c"]
