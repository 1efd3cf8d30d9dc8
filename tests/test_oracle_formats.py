"""Pins of the oracle's decoders for the reference's own table formats (Q1_0 .. F8E4M3_B128,
src/Sharplight.Cpu/Quant.cs:287-362 and Quant.Grouped/Absmax/Fp4/Fp8/Ternary.cs), which no ggml fixture covers:
brute force over every code byte and a spread of scales against closed forms computed here with numpy's own
IEEE f32 arithmetic, the code books against their published construction, and invariants tying a format to
one the fixtures do pin (NVFP4_GS with g = 2^k is NVFP4 times 2^k; Tern1's digits invert ggml's base-3 packing)."""
import numpy as np
import pytest

import oracle

F32 = np.float32
SCALES = np.array([1.0, 0.013, -0.75, 6.1e-5, 3.0e-8, 65504.0, 2.0 ** -24], np.float16)  # incl. f16 subnormals


def _h(v):
    return np.frombuffer(np.float16(v).tobytes(), np.uint8)


def _deq(fmt, blocks, values):
    return oracle.dequant(fmt, np.ascontiguousarray(blocks, np.uint8).reshape(-1), values)


def test_q1_0_every_byte_every_scale():
    """Bit i of byte j is value 8j + i: +d if set, -d if clear (Quant.Q1_0)."""
    for d in SCALES:
        blocks = np.zeros((16, 18), np.uint8)
        blocks[:, 0:2] = _h(d)
        blocks[:, 2:] = np.arange(256, dtype=np.uint8).reshape(16, 16)
        got = _deq("q1_0", blocks, 16 * 128).reshape(16, 16, 8)
        bits = (np.arange(256).reshape(16, 16, 1) >> np.arange(8)) & 1
        want = np.where(bits == 1, F32(d), -F32(d)).astype(F32)
        assert np.array_equal(got, want)


@pytest.mark.parametrize("fmt,qb", [("q2_0", 16), ("q2_0_g128", 32)])
def test_q2_0_every_byte(fmt, qb):
    """Byte j holds values 4j..4j+3, value 4j+i in bits 2i, 2i+1: (code - 1) * d."""
    codes = np.arange(256, dtype=np.uint8)
    n = 256 // qb
    for d in SCALES:
        blocks = np.zeros((n, 2 + qb), np.uint8)
        blocks[:, 0:2] = _h(d)
        blocks[:, 2:] = codes.reshape(n, qb)
        got = _deq(fmt, blocks, n * 4 * qb).reshape(256, 4)
        c = (codes[:, None] >> (2 * np.arange(4))) & 3
        want = ((c.astype(F32) - F32(1)) * F32(d)).astype(F32)
        assert np.array_equal(got, want)


def test_tern1_digits_invert_the_base3_packing():
    """Five digits t0..t4 (t0 most significant) pack as q = ceil(v 256 / 243), v = sum t_n 3^(4-n), the packing
    of ggml's TQ1_0 that Tern1_G128 shares; every byte of each region decodes back to t_n - 1: digit n of byte m
    at value n*16 + m (bytes 0..15), 80 + n*8 + m (16..23), 120 + 2n + h (24, 25, four digits)."""
    v = np.arange(243)
    q = ((v * 256 + 242) // 243).astype(np.uint8)
    digits = np.stack([(v // 3 ** (4 - n)) % 3 for n in range(5)], 1) - 1
    for d in (1.0, -0.02):
        blocks = np.zeros((243, 28), np.uint8)
        blocks[:, :26] = q[:, None]
        blocks[:, 26:28] = _h(d)
        got = _deq("tern1_g128", blocks, 243 * 128).reshape(243, 128)
        want = np.empty((243, 128), F32)
        for n in range(5):
            want[:, n * 16:(n + 1) * 16] = digits[:, n:n + 1]
            want[:, 80 + n * 8:80 + (n + 1) * 8] = digits[:, n:n + 1]
        for n in range(4):
            want[:, 120 + 2 * n:122 + 2 * n] = digits[:, n:n + 1]
        assert np.array_equal(got, (want * F32(np.float16(d))).astype(F32))


def test_nvfp4_gs_with_power_of_two_g_is_scaled_nvfp4():
    """g = 2^k scales exactly: NVFP4_GS(g, block) == 2^k * NVFP4(block) (NVFP4 is pinned by ggml's fixture)."""
    rng = np.random.default_rng(3)
    body = rng.integers(0, 256, (50, 36), dtype=np.uint8)
    body[:, :4] = rng.integers(0x08, 0x70, (50, 4), dtype=np.uint8)
    base = _deq("nvfp4", body, 50 * 64)
    for k in (0, 3, -5):
        blocks = np.zeros((50, 40), np.uint8)
        blocks[:, :4] = np.frombuffer(F32(2.0 ** k).tobytes(), np.uint8)
        blocks[:, 4:] = body
        assert np.array_equal(_deq("nvfp4_gs", blocks, 50 * 64), (base * F32(2.0 ** k)).astype(F32))
    # a g that is not a power of two rounds the sub-block multiplier once: ue4m3 * g, then * code
    g = F32(0.3)
    blocks[:, :4] = np.frombuffer(g.tobytes(), np.uint8)
    got = _deq("nvfp4_gs", blocks, 50 * 64).reshape(50, 4, 16)
    x = body[:, :4].astype(np.int64)
    e, m = (x >> 3) & 15, x & 7
    ue = np.where(e == 0, m * 2.0 ** -9, (1 + m / 8) * np.ldexp(1.0, e - 7)) / 2
    ue[(x == 0) | (x == 0x7F)] = 0
    mult = (ue.astype(F32) * g).astype(F32)
    codes = np.concatenate([body[:, 4:].reshape(50, 4, 8) & 15, body[:, 4:].reshape(50, 4, 8) >> 4], axis=2)
    e2m1 = np.array([0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12], F32)
    assert np.array_equal(got, (e2m1[codes] * mult[..., None]).astype(F32))


@pytest.mark.parametrize("fmt,group", [("q4z_g32", 32), ("q4z_g128", 128)])
def test_q4z_closed_form(fmt, group):
    """{f16 d; f16 z; nibbles}: value j of a 32-value run the low nibble of byte j, j + 16 the high nibble;
    (q - z) * d, the subtraction rounded before the product."""
    rng = np.random.default_rng(4)
    n = 64
    blocks = rng.integers(0, 256, (n, 4 + group // 2), dtype=np.uint8)
    d = rng.uniform(-0.05, 0.05, n).astype(np.float16)
    z = np.concatenate([rng.uniform(0, 16, n - 2), [2.0 ** -24, 7.5]]).astype(np.float16)  # a tiny z rounds q - z
    blocks[:, 0:2] = d.view(np.uint8).reshape(n, 2)
    blocks[:, 2:4] = z.view(np.uint8).reshape(n, 2)
    got = _deq(fmt, blocks, n * group).reshape(n, group // 32, 32)
    qs = blocks[:, 4:].reshape(n, group // 32, 16)
    q = np.concatenate([qs & 15, qs >> 4], axis=2).astype(F32)
    want = ((q - z.astype(F32)[:, None, None]).astype(F32) * d.astype(F32)[:, None, None]).astype(F32)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("fmt,group", [("q8z_g32", 32), ("q8z_g128", 128)])
def test_q8z_every_code(fmt, group):
    rng = np.random.default_rng(5)
    n = 256 // group + 8
    blocks = np.zeros((n, 4 + group), np.uint8)
    blocks[:, 4:] = np.resize(np.arange(256, dtype=np.uint8), (n, group))
    d = rng.uniform(-0.05, 0.05, n).astype(np.float16)
    z = rng.uniform(0, 255, n).astype(np.float16)
    blocks[:, 0:2] = d.view(np.uint8).reshape(n, 2)
    blocks[:, 2:4] = z.view(np.uint8).reshape(n, 2)
    got = _deq(fmt, blocks, n * group).reshape(n, group)
    want = ((blocks[:, 4:].astype(F32) - z.astype(F32)[:, None]).astype(F32) * d.astype(F32)[:, None]).astype(F32)
    assert np.array_equal(got, want)


def test_nf4_fp4_code_books():
    """FP4_B64's book: the magnitudes 0, 0.0625, 8, 12, 4, 6, 2, 3 over 12, then negated (code 8 is +0); NF4_B64's:
    bitsandbytes' normal map -- standard-normal quantiles at 8 points from 0.9677083 to 0.5 (positive side) and
    7 points (negative side), each normalized by its largest -- ascending from -1 to 1 with 0 at code 7."""
    from scipy.stats import norm
    fp4 = np.array([0, 0.0625, 8, 12, 4, 6, 2, 3], np.float64) / 12
    want_fp4 = np.concatenate([fp4, -fp4]).astype(F32)
    want_fp4[8] = 0.0
    d = F32(1.0)
    blocks = np.zeros((1, 36), np.uint8)
    blocks[0, :4] = np.frombuffer(d.tobytes(), np.uint8)
    blocks[0, 4:20] = (np.arange(16) | (np.arange(16) << 4)).astype(np.uint8)
    got = _deq("fp4_b64", blocks, 64)[:16]
    assert np.array_equal(got, want_fp4)
    offset = 0.9677083
    pos = norm.ppf(np.linspace(offset, 0.5, 9)[:-1])
    neg = -norm.ppf(np.linspace(offset, 0.5, 8)[:-1])
    v = np.sort(np.concatenate([pos, [0.0], neg]))
    v /= np.abs(v).max()
    got = _deq("nf4_b64", blocks, 64)[:16]
    assert np.allclose(got, v, rtol=0, atol=2e-7) and got[7] == 0 and got[0] == -1 and got[15] == 1
    assert (np.diff(got) > 0).all()


@pytest.mark.parametrize("fmt", ["nf4_b64", "fp4_b64"])
def test_lookup_b64_layout_and_scale(fmt):
    """Two 32-value runs of 16 bytes, value j the low nibble of byte j, j + 16 the high one; book[q] * d."""
    rng = np.random.default_rng(6)
    n = 40
    blocks = rng.integers(0, 256, (n, 36), dtype=np.uint8)
    d = rng.uniform(-3, 3, n).astype(F32)
    blocks[:, :4] = d.view(np.uint8).reshape(n, 4)
    book = _deq(fmt, np.concatenate([np.frombuffer(F32(1).tobytes(), np.uint8), (np.arange(16) * 17).astype(np.uint8),
                                     np.zeros(16, np.uint8)]).reshape(1, 36), 64)[:16]
    got = _deq(fmt, blocks, n * 64).reshape(n, 2, 32)
    qs = blocks[:, 4:].reshape(n, 2, 16)
    q = np.concatenate([qs & 15, qs >> 4], axis=2)
    assert np.array_equal(got, (book[q] * d[:, None, None]).astype(F32))


def test_q8a_g32_every_code():
    """{f32 d; i8 q[32]}: (q * d) * f32(1/127), rounded after each product."""
    rng = np.random.default_rng(7)
    n = 24
    blocks = np.zeros((n, 36), np.uint8)
    blocks[:, 4:] = np.resize(np.arange(256, dtype=np.uint8), (n, 32))
    d = rng.uniform(-2, 2, n).astype(F32)
    blocks[:, :4] = d.view(np.uint8).reshape(n, 4)
    got = _deq("q8a_g32", blocks, n * 32).reshape(n, 32)
    q = blocks[:, 4:].view(np.int8).astype(F32)
    want = ((q * d[:, None]).astype(F32) * F32(7.874015718698502e-3)).astype(F32)
    assert np.array_equal(got, want)
    assert F32(7.874015718698502e-3) == F32(1 / 127)


def test_q2s_g128_every_byte():
    """{f32 d; u8 qs[32]}: byte j holds values j, 32 + j, 64 + j, 96 + j in bits 6, 4, 2, 0; (code - 1) * d."""
    blocks = np.zeros((8, 36), np.uint8)
    blocks[:, 4:] = np.arange(256, dtype=np.uint8).reshape(8, 32)
    d = np.array([1, -0.5, 3e-39, 7.25, 1e30, -2, 0.1, 4], F32)
    blocks[:, :4] = d.view(np.uint8).reshape(8, 4)
    got = _deq("q2s_g128", blocks, 8 * 128).reshape(8, 4, 32)
    b = blocks[:, 4:]
    for grp, sh in enumerate((6, 4, 2, 0)):
        want = ((((b >> sh) & 3).astype(F32) - F32(1)) * d[:, None]).astype(F32)
        assert np.array_equal(got[:, grp], want)


def test_fp8_every_code():
    """E4M3FN: sign, 4 exponent bits (bias 7), 3 mantissa bits, exponent 0 subnormal, 0x7F/0xFF NaN, no infinity
    -- checked against the formula in f64 and against the oracle's nearest-even E4M3 encoder (a round trip on
    every finite code); E5M2 is the top byte of an IEEE half (numpy's float16)."""
    codes = np.arange(256, dtype=np.uint8)
    e4 = np.array([oracle.lib().orc_e4m3_value(int(c)) for c in codes], F32)
    e, m, s = (codes >> 3) & 15, codes & 7, np.where(codes & 0x80, -1.0, 1.0)
    want = s * np.where(e == 0, m * 2.0 ** -9, (1 + m / 8) * np.ldexp(1.0, e.astype(int) - 7))
    nan = (codes & 0x7F) == 0x7F
    assert np.isnan(e4[nan]).all() and np.array_equal(e4[~nan], want[~nan].astype(F32))
    finite = np.nonzero(~nan & ((codes & 0x7F) != 0))[0]  # the encoder maps -0 to +0
    assert all(oracle.lib().orc_e4m3_code(float(e4[c])) == c for c in finite)
    e5 = np.array([oracle.lib().orc_e5m2_value(int(c)) for c in codes], F32)
    ref5 = (codes.astype(np.uint16) << 8).view(np.float16).astype(F32)
    assert np.array_equal(e5, ref5, equal_nan=True)
    got = _deq("f8e4m3", codes, 256)
    assert np.array_equal(got, e4, equal_nan=True)
    assert np.array_equal(_deq("f8e5m2", codes, 256), ref5, equal_nan=True)


@pytest.mark.parametrize("fmt,block", [("f8e4m3_b32", 32), ("f8e4m3_b128", 128)])
def test_scaled_e4m3_blocks(fmt, block):
    rng = np.random.default_rng(8)
    n = 12
    blocks = np.zeros((n, 4 + block), np.uint8)
    blocks[:, 4:] = np.resize(np.arange(256, dtype=np.uint8), (n, block))
    d = rng.uniform(-4, 4, n).astype(F32)
    blocks[:, :4] = d.view(np.uint8).reshape(n, 4)
    got = _deq(fmt, blocks, n * block).reshape(n, block)
    e4 = np.array([oracle.lib().orc_e4m3_value(int(c)) for c in range(256)], F32)
    want = (e4[blocks[:, 4:]] * d[:, None]).astype(F32)
    assert np.array_equal(got, want, equal_nan=True)


TRELLIS_IDS = {144: "trellis_v4k8_g128", 145: "trellis_v4k6_g128", 146: "trellis_v4k7_g128",
               147: "trellis_v2k5_g128", 148: "trellis_v2k6_g128", 149: "trellis_v2k7_g128"}


def trellis_fixture():
    """tests/golden/trellis_ref.bin, a data file of the reference's tests (tests/Sharplight.Cpu.Tests/Fixtures,
    read by TrellisDequantTests.cs:49-69): random blocks of each trellis format (ggml ids 144-149 of the
    fork that introduced them) with the values the fork's decoders give, as (format, rows, cols, block bytes,
    expected f32 values)."""
    import os
    import struct
    from sharplight_amd import synth
    b = open(os.path.join(os.path.dirname(__file__), "golden", "trellis_ref.bin"), "rb").read()
    n, o = struct.unpack_from("<i", b, 0)[0], 4
    out = []
    for _ in range(n):
        t, rows, cols = struct.unpack_from("<iii", b, o)
        o += 12
        fmt = TRELLIS_IDS[t]
        nb = rows * synth.row_bytes(fmt, cols)
        blocks = np.frombuffer(b, np.uint8, nb, o).reshape(rows, -1)
        o += nb
        expected = np.frombuffer(b, np.float32, rows * cols, o).reshape(rows, cols)
        o += 4 * rows * cols
        out.append((fmt, rows, cols, blocks, expected))
    assert o == len(b)
    return out


def test_trellis_matches_the_reference_fixture_bit_for_bit():
    """TrellisDequantTests.EveryFormat_DequantizesLikeTheReference: every format, every value, same bits."""
    seen = set()
    for fmt, rows, cols, blocks, expected in trellis_fixture():
        got = _deq(fmt, blocks, rows * cols).reshape(rows, cols)
        assert np.array_equal(got.view(np.uint32), expected.view(np.uint32)), fmt
        seen.add(fmt)
    assert seen == set(TRELLIS_IDS.values())


@pytest.mark.parametrize("fmt", list(TRELLIS_IDS.values()))
def test_trellis_scale_is_a_plain_factor(fmt):
    """value = d * point: with d a power of two every value scales exactly, and d = 0 gives zeros (+-0);
    the path bytes alone select the points (a block's values with d = 1 are codebook entries)."""
    from sharplight_amd import synth
    t = synth.quant_table(fmt, 4, 512, seed=5, tid=9)
    bb = synth.row_bytes(fmt, 128)
    blocks = t.reshape(-1, bb).copy()
    blocks[:, 0:2] = _h(1.0)
    one = _deq(fmt, blocks, blocks.shape[0] * 128)
    import os
    import re
    text = open(os.path.join(os.path.dirname(__file__), "..", "sharplight_amd", "csrc", "trellis_codebook.h")).read()
    book = np.array([int(v, 16) for v in re.findall(r"0x[0-9a-f]+", text.split("{", 1)[1])], np.uint16)
    assert book.size == 4096
    assert np.isin(one, book.view(np.float16).astype(F32)).all()
    for k in (-3, 0, 5):
        blocks[:, 0:2] = _h(2.0 ** k)
        assert np.array_equal(_deq(fmt, blocks, blocks.shape[0] * 128), one * F32(2.0 ** k))
    blocks[:, 0:2] = _h(0.0)
    assert not np.any(_deq(fmt, blocks, blocks.shape[0] * 128))
