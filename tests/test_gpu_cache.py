"""GPU parity of the KV-cache writes: rope (with the fused q/k norm) written straight into a cache, and the
standalone cache write, against the oracle's CacheWriteOp (src/Sharplight.Cpu/CacheWriteOp.cs) applied to
its RmsNorm-then-Rope result -- the reference's FusionTests.NormRopeIntoCache pattern
(tests/Sharplight.Vulkan.Tests/FusionTests.cs:138-175: GPU cache contents vs the CPU provider's) for the
contiguous (n_past), multi-sequence and paged row maps, and the reference's overflow errors."""
import zlib

import numpy as np
import pytest

import oracle
from sharplight_amd import native, synth
from tests.devutil import Dev, log
from tests.parity import assert_bf16_close, assert_bits_equal, assert_f16_close, assert_f32_close

pytestmark = pytest.mark.gpu

NP = {"f32": np.float32, "f16": np.uint16, "bf16": np.uint16}
SENTINEL = {"f32": np.float32(-7.5), "f16": np.uint16(0x7BFF), "bf16": np.uint16(0x4242)}


def _seed(*parts) -> int:
    return zlib.crc32(repr(parts).encode())


def _to(ct, y32):
    return {"f32": lambda a: a, "f16": oracle.to_f16, "bf16": oracle.to_bf16}[ct](y32)


def _close(ct, got, ref, what):
    if ct == "f32":
        assert_f32_close(got, ref, what=what)
    elif ct == "f16":
        assert_f16_close(got, ref, what=what)
    else:
        assert_bf16_close(got, ref, what=what)


def _rows_case(mode, T, ctx, rng, slots=2, bs=4):
    """(device CacheRows kwargs builder, oracle kwargs): a row map of T tokens into a ctx-row cache."""
    if mode == "past":
        n_past = int(rng.integers(0, ctx - T + 1))
        return dict(n_past=n_past), dict(n_past=n_past), None, None
    if mode == "seq":
        seq = np.zeros((T, 4), np.int32)
        seq[:, 0] = rng.integers(0, slots, T)
        seq[:, 1] = rng.integers(0, ctx // slots, T)
        # distinct (slot, position) pairs: a cache row written twice would depend on write order
        _, keep = np.unique(seq[:, 0] * ctx + seq[:, 1], return_index=True)
        seq = seq[np.sort(keep)]
        return dict(slots=slots), dict(slots=slots), seq, None
    blocks = ctx // bs
    bps = blocks // slots
    table = rng.permutation(blocks)[: slots * bps].reshape(slots, bps).astype(np.int32)
    seq = np.zeros((T, 4), np.int32)
    seq[:, 0] = rng.integers(0, slots, T)
    seq[:, 1] = rng.integers(0, bps * bs, T)
    _, keep = np.unique(seq[:, 0] * ctx + seq[:, 1], return_index=True)
    seq = seq[np.sort(keep)]
    return (dict(page_slots=slots, blocks_per_slot=bps, block_size=bs), dict(block_size=bs), seq, table)


@pytest.mark.parametrize("mode", ["past", "seq", "paged"])
@pytest.mark.parametrize("din,ct", [("bf16", "bf16"), ("bf16", "f16"), ("f32", "f32"), ("f32", "f16")])
def test_norm_rope_into_cache(device, mode, din, ct):
    """k of a Qwen3-style layer: per-head RmsNorm then neox rope, stored into the K cache rows; q in the
    same launch to a plain output (FusionTests.cs:142-157 with a single-axis rope)."""
    rng = np.random.default_rng(_seed(mode, din, ct))
    T, Hq, Hk, D, ctx = 37, 4, 2, 128, 96
    q = synth.normal(1, 0, (T, Hq, D), dtype=din)
    k = synth.normal(1, 1, (T, Hk, D), dtype=din)
    wq, wk = synth.normal(1, 2, (D,), 1.0, 0.1), synth.normal(1, 3, (D,), 1.0, 0.1)
    dev_kw, orc_kw, seq, table = _rows_case(mode, T, ctx, rng)
    T = len(seq) if seq is not None else T
    q, k = q[:T], k[:T]
    pos = (seq[:, 1] if seq is not None else orc_kw["n_past"] + np.arange(T)).astype(np.int32)
    with Dev() as d:
        pseq = d.put(seq) if seq is not None else None
        ppages = d.put(table) if table is not None else None
        rows = native.cache_rows(mode, ctx, seq=pseq, pages=ppages, **dev_kw)
        cache0 = np.full((ctx, Hk, D), SENTINEL[ct], NP[ct])
        pc = d.put(cache0)
        py = d.empty(T * Hq * D * np.dtype(NP[ct]).itemsize)
        pp = d.put(pos)
        log(f"rope into {ct} cache, {mode} rows, {din} in, T={T}")
        native.rope(din, ct, [dict(x=d.put(q), y=py, heads=Hq, norm_w=d.put(wq)),
                              dict(x=d.put(k), y=pc, heads=Hk, norm_w=d.put(wk), rows=rows)],
                    pp, T, D, neox=True, base=1e6, norm=True, eps=1e-6)
        native.synchronize()
        got_c = d.get(pc, cache0.shape, NP[ct])
        got_q = d.get(py, (T, Hq, D), NP[ct])
    # the oracle's f32 rope result (before any output rounding), written through CacheWriteOp
    k32 = oracle.rope(oracle.rmsnorm(oracle.from_bf16(k) if din == "bf16" else k, wk, 1e-6), pos, base=1e6)
    q32 = oracle.rope(oracle.rmsnorm(oracle.from_bf16(q) if din == "bf16" else q, wq, 1e-6), pos, base=1e6)
    r = oracle.cache_rows(mode, T, ctx, seq=seq, pages=table, **orc_kw)
    want = cache0.copy()
    oracle.cache_write(want.reshape(ctx, -1), k32.reshape(T, -1), r, ct)
    untouched = np.setdiff1d(np.arange(ctx), r)
    assert_bits_equal(got_c[untouched], want[untouched], what="rows not written")
    _close(ct, got_c[r], want[r], f"k cache {mode}")
    _close(ct, got_q, _to(ct, q32), "q output")


@pytest.mark.parametrize("mode", ["past", "seq", "paged"])
@pytest.mark.parametrize("din,ct", [("f32", "f32"), ("f32", "f16"), ("f32", "bf16"), ("bf16", "f16"), ("bf16", "bf16")])
@pytest.mark.parametrize("inner", [1024, 96, 37])
def test_cache_write_bits(device, mode, din, ct, inner):
    """CacheWrite of V (no producer absorbed): a conversion, so bit-exact; inner 37 takes the general path."""
    rng = np.random.default_rng(_seed(mode, din, ct, inner))
    T, ctx = 29, 80
    x = synth.normal(2, 0, (T, inner), dtype=din)
    dev_kw, orc_kw, seq, table = _rows_case(mode, T, ctx, rng)
    T = len(seq) if seq is not None else T
    x = x[:T]
    with Dev() as d:
        rows = native.cache_rows(mode, ctx, seq=d.put(seq) if seq is not None else None,
                                 pages=d.put(table) if table is not None else None, **dev_kw)
        cache0 = np.full((ctx, inner), SENTINEL[ct], NP[ct])
        pc = d.put(cache0)
        log(f"cache_write {din}->{ct} {mode} inner={inner} T={T}")
        native.cache_write(din, ct, d.put(x), T, inner, pc, rows)
        native.synchronize()
        got = d.get(pc, cache0.shape, NP[ct])
    x32 = oracle.from_bf16(x) if din == "bf16" else x
    want = cache0.copy()
    oracle.cache_write(want, x32, oracle.cache_rows(mode, T, ctx, seq=seq, pages=table, **orc_kw), ct)
    assert_bits_equal(got, want, what=f"cache {mode} {din}->{ct}")


def test_past_overflow_is_refused_at_the_call(device):
    with Dev() as d:
        rows = native.cache_rows("past", 16, n_past=10)
        x, c = d.put(np.zeros((7, 64), np.float32)), d.empty(16 * 64 * 4)
        with pytest.raises(native.SlhipCacheError, match=r"n_past 10 \+ T 7 > context 16"):
            native.cache_write("f32", "f32", x, 7, 64, c, rows)


@pytest.mark.parametrize("case", ["seq", "page_table", "block"])
def test_bad_rows_are_skipped_and_reported(device, case):
    """A row outside the cache is not written; the others are, and the next sync reports the reference's
    message (CacheWriteOp.cs:103-117, KvPages.cs:38-49)."""
    T, ctx, inner = 4, 32, 64
    x = np.arange(T * inner, dtype=np.float32).reshape(T, inner)
    seq = np.int32([[0, 1, 0, 0], [1, 2, 0, 0], [0, 3, 0, 0], [1, 4, 0, 0]])
    table = np.int32([[0, 1], [2, 3]])  # 2 slots x 2 blocks of 8 rows
    if case == "seq":
        seq[2] = (0, 16, 0, 0)  # slot context is 32 / 2 = 16
        msg = "KV cache overflow: sequence row 2 slot 0 position 16"
    elif case == "page_table":
        seq[2] = (2, 0, 0, 0)  # only 2 slots in the table
        msg = r"Sequence slot 2 / position 0 outside the block table \[2, 2\]"
    else:
        table[1, 0] = 4  # block 4 ends at row 40 > 32: token 1 (slot 1, position 2) maps there
        seq[3] = (1, 9, 0, 0)  # slot 1's second block, still inside
        msg = r"Block 4 of slot 1 \(position 2\) is outside the KV cache of 32 rows"
    with Dev() as d:
        kw = (dict(slots=2) if case == "seq" else dict(page_slots=2, blocks_per_slot=2, block_size=8))
        rows = native.cache_rows("seq" if case == "seq" else "paged", ctx, seq=d.put(seq), pages=d.put(table), **kw)
        pc = d.put(np.full((ctx, inner), -1.0, np.float32))
        log(f"cache_write bad rows: {case}")
        native.cache_write("f32", "f32", d.put(x), T, inner, pc, rows)
        with pytest.raises(native.SlhipCacheError, match=msg):
            native.synchronize()
        got = d.get(pc, (ctx, inner), np.float32)
        native.synchronize()  # reported once: the record is clear again
    bad = 1 if case == "block" else 2
    for t in range(T):
        if t == bad:
            continue
        s, p = seq[t, :2]
        row = s * 16 + p if case == "seq" else table[s, p // 8] * 8 + p % 8
        assert np.array_equal(got[row], x[t]), (case, t)
    assert (got == -1.0).all(axis=1).sum() == ctx - (T - 1)  # nothing else written
