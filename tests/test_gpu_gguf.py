"""The on-disk -> device path on the GPU: tensors of GGUF files uploaded by the staged uploader
(slhip_gguf_upload, slhip_upload) hold exactly the bytes the oracle reads from the file, and a table
uploaded that way gathers as the oracle dequantizes it.

Small staging buffers (SLHIP_UPLOAD_STAGING_MB, read on every call) put chunk boundaries inside blocks of
the types read in another layout than stored; back-to-back uploads reuse a staging buffer while the copy
out of the other one may still be running.
"""
import struct

import numpy as np
import pytest

import oracle
from oracle import gguf as og
from sharplight_amd import gguf, native, synth
from tests.devutil import Dev, log
from tests.test_gguf import interleave_q4_0

pytestmark = pytest.mark.gpu


def _rand(n, seed):
    return np.random.default_rng(seed).integers(0, 256, n, dtype=np.uint8).tobytes()


def _download(addr, n):
    return Dev.get(addr, (n,), np.uint8).tobytes()


@pytest.fixture()
def staging(monkeypatch):
    def set_(mb, threads=None):
        monkeypatch.setenv("SLHIP_UPLOAD_STAGING_MB", str(mb))
        if threads is not None:
            monkeypatch.setenv("SLHIP_UPLOAD_THREADS", str(threads))
    return set_


@pytest.mark.parametrize("mb,threads", [(64, 8), (1, 3), (2, 1)])
def test_upload_tensors_of_a_file(device, tmp_path, staging, mb, threads):
    staging(mb, threads)
    rows = 8
    q40 = _rand(rows * 4096 // 32 * 18, 2)
    w = gguf.GgufWriter().add_metadata("general.architecture", "toy")
    w.add_tensor("big.bf16", 30, _rand(5 * 1024 * 1024 + 6, 1), [1, (5 * 1024 * 1024 + 6) // 2])
    w.add_tensor_ne("inter.q4_0", 33, interleave_q4_0(q40, rows, 4096 // 32, 8, 8), [4096, rows], layout_type=2)
    w.add_tensor("q6k", 14, _rand(210 * 3 * 7, 3), [3, 7 * 256])
    w.add_tensor("tiny", 0, _rand(4, 4), [1])
    p = tmp_path / "up.gguf"
    w.write(p)
    blob = p.read_bytes()
    o = {t["name"]: t for t in og.parse_file(blob)["tensors"]}
    with gguf.GgufFile.open(p) as f, Dev() as d:
        for t in f.tensors:
            log(f"gguf upload {t.name} {t.data_type} {t.byte_size} B staging={mb} MiB threads={threads}")
            dst = d.empty(t.byte_size)
            t.upload(dst)
            native.synchronize()
            assert _download(dst, t.byte_size) == og.read_tensor(blob, o[t.name]), t.name
        assert f.get_tensor("inter.q4_0").read() == q40


def test_i2s_upload(device, tmp_path, staging):
    staging(1, 2)
    rows, columns = 64, 4096  # 2 MiB of blocks as read: chunk boundaries fall inside 36-byte blocks
    codes = _rand(rows * columns // 4, 7)
    hdr = struct.pack("<IIQQ", 0x46554747, 3, 1, 0) + struct.pack("<Q", 1) + b"w"
    hdr += struct.pack("<IQQIQ", 2, columns, rows, 36, 0)
    blob = hdr + bytes((len(hdr) + 31) // 32 * 32 - len(hdr)) + codes + struct.pack("<f", -0.5) + bytes(28)
    p = tmp_path / "i2s.gguf"
    p.write_bytes(blob)
    want = og.read_tensor(blob, og.parse_file(blob)["tensors"][0])
    with gguf.GgufFile.open(p) as f, Dev() as d:
        t = f.tensors[0]
        log(f"gguf upload i2s {t.byte_size} B")
        dst = d.empty(t.byte_size)
        t.upload(dst)
        native.synchronize()
        assert _download(dst, t.byte_size) == want


@pytest.mark.parametrize("n", [1, 7, 4096, 4097, 3 * 1024 * 1024 + 5, 9 * 1024 * 1024 + 3])
def test_upload_host_buffers(device, staging, n):
    staging(2, 4)
    src = _rand(n, n)
    with Dev() as d:
        log(f"slhip_upload {n} B")
        dst = d.empty(n)
        gguf.upload(dst, src)
        native.synchronize()
        assert _download(dst, n) == src


def test_back_to_back_uploads_reuse_staging(device, staging):
    """Four uploads in a row without waiting: each must see its own bytes although the staging buffers are
    refilled while earlier copies may still run."""
    staging(1, 2)
    srcs = [_rand(3 * 1024 * 1024 + k, 100 + k) for k in range(4)]
    with Dev() as d:
        dsts = [d.empty(len(s)) for s in srcs]
        log("slhip_upload x4 back to back")
        for dst, s in zip(dsts, srcs):
            gguf.upload(dst, s)
        native.synchronize()
        for dst, s in zip(dsts, srcs):
            assert _download(dst, len(s)) == s


def test_upload_rejects_short_destination(device, tmp_path):
    p = tmp_path / "s.gguf"
    gguf.GgufWriter().add_tensor("a", 0, _rand(64, 1), [16]).write(p)
    with gguf.GgufFile.open(p) as f, Dev() as d:
        dst = d.empty(64)
        with pytest.raises(native.SlhipArgumentError, match="needs 64 bytes"):
            f.get_tensor("a").upload(dst, 63)


@pytest.mark.parametrize("fmt,type_id", [("q4_k", 12), ("q8_0", 8), ("iq4_xs", 23)])
def test_embedding_table_from_file_gathers_like_oracle(device, tmp_path, staging, fmt, type_id):
    """token_embd.weight written to a GGUF file, uploaded, gathered: bit-exact against the oracle's gather
    of the same bytes."""
    staging(1, 4)
    V, D = 640, 2048
    table = synth.quant_table(fmt, V, D, seed=3, tid=9)
    p = tmp_path / "emb.gguf"
    gguf.GgufWriter().add_metadata("general.architecture", "toy").add_tensor(
        "token_embd.weight", type_id, table.tobytes(), [V, D]).write(p)
    ids = np.random.default_rng(4).integers(0, V, 300).astype(np.int32)
    with gguf.GgufFile.open(p) as f, Dev() as d:
        t = f.get_tensor("token_embd.weight")
        assert t.format == fmt
        log(f"gguf upload + gather {fmt} V={V} D={D}")
        tab = d.empty(t.byte_size)
        t.upload(tab)
        pid = d.put(ids)
        y = d.empty(ids.size * D * 4)
        native.gather(fmt, tab, V, D, pid, ids.size, "f32", y)
        native.synchronize()
        got = Dev.get(y, (ids.size, D), np.float32)
    want = oracle.gather(fmt, table, V, D, ids)
    assert got.tobytes() == want.tobytes()


def test_narrow_iq1_upload_gathers_like_the_fork(device, tmp_path, staging):
    """Narrow IQ1 tensors (GGUF ids 64-66) uploaded -- widened to IQ1_S on the way -- and gathered: the fork's
    own decoded floats (ggml_narrow_iq1.bin), bit for bit."""
    import os
    staging(1, 3)
    fx = np.load(os.path.join(os.path.dirname(__file__), "golden", "ggml_narrow_iq1.npz"))
    for i in range(len([k for k in fx.files if k.endswith("_type")])):
        g, rows, cols = (int(v) for v in fx[f"r{i}_type"])
        blocks, want = fx[f"r{i}_blocks"].tobytes(), fx[f"r{i}_deq"]
        hdr = struct.pack("<IIQQ", 0x46554747, 3, 1, 0) + struct.pack("<Q", 1) + b"w"
        hdr += struct.pack("<IQQIQ", 2, cols, rows, g, 0)
        p = tmp_path / f"n{i}.gguf"
        p.write_bytes(hdr + bytes((len(hdr) + 31) // 32 * 32 - len(hdr)) + blocks)
        with gguf.GgufFile.open(p) as f, Dev() as d:
            t = f.tensors[0]
            log(f"narrow IQ1 upload + gather type {g} [{rows}, {cols}]")
            tab = d.empty(t.byte_size)
            t.upload(tab)
            ids = np.arange(rows, dtype=np.int32)
            pid = d.put(ids)
            y = d.empty(rows * cols * 4)
            native.gather("iq1_s", tab, rows, cols, pid, rows, "f32", y)
            native.synchronize()
            got = Dev.get(y, (rows, cols), np.float32)
        nan = np.isnan(want)
        assert np.array_equal(np.isnan(got), nan)
        assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32)), (i, g)
