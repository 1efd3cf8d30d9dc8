"""Seeded synthetic inputs of the benchmark configurations (C1..C5) and of the parity tests.

Every tensor comes from its own numpy PCG64 stream keyed by (seed, tensor id), so a tensor's bits do not
depend on which other tensors were generated. N(0,1) values are drawn in f32 and stored to bf16 by
round-to-nearest-even; quantized tables are built block by block in ggml's layout (f16 scale first).
bf16 arrays are carried as raw uint16 bits.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np


def rng(seed: int, tensor_id: int) -> np.random.Generator:
    return np.random.default_rng([seed, tensor_id])


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """f32 -> bf16 bits, round to nearest even, NaN quieted."""
    b = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    r = ((b + np.uint32(0x7FFF) + ((b >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)).astype(np.uint16)
    nan = (b & np.uint32(0x7FFFFFFF)) > np.uint32(0x7F800000)
    if nan.any():
        r[nan] = ((b[nan] >> np.uint32(16)) | np.uint32(0x40)).astype(np.uint16)
    return r


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(bits, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def normal(seed, tid, shape, mean=0.0, std=1.0, dtype="f32"):
    x = rng(seed, tid).standard_normal(size=shape, dtype=np.float32)
    if std != 1.0 or mean != 0.0:
        x = (x * np.float32(std) + np.float32(mean)).astype(np.float32)
    return bf16_bits(x) if dtype == "bf16" else x


BLOCK = {"q8_0": 34, "q4_0": 18, "q4_1": 20, "q5_0": 22, "q5_1": 24, "iq4_nl": 18}
# 256-value super-blocks: bytes per block, and the byte offsets of their f16 fields (d, dmin)
KBLOCK = {"q2_k": (84, (80, 82)), "q3_k": (110, (108,)), "q4_k": (144, (0, 2)), "q5_k": (176, (0, 2)),
          "q6_k": (210, (208,)), "iq4_xs": (136, (0,)), "tq1_0": (54, (52,)), "tq2_0": (66, (64,)),
          "iq2_xxs": (66, (0,)), "iq2_xs": (74, (0,)), "iq2_s": (82, (0,)), "iq3_xxs": (98, (0,)), "iq3_s": (110, (0,)),
          "iq1_s": (50, (0,)), "iq1_m": (56, ())}
# 4-bit float blocks: bytes, values, and the scale bytes at the block start (E8M0 exponent / UE4M3 scales)
FP4BLOCK = {"mxfp4": (17, 32, 1), "nvfp4": (36, 64, 4)}
# The reference's own formats: bytes, values, and the scale fields ("h" f16 at an offset, "f" f32 at an offset,
# "ue" UE4M3 bytes at 4..7) -- every other byte random.
REFBLOCK = {"q1_0": (18, 128, (("h", 0),)), "q2_0": (18, 64, (("h", 0),)), "q2_0_g128": (34, 128, (("h", 0),)),
            "tern1_g128": (28, 128, (("h", 26),)), "nvfp4_gs": (40, 64, (("f", 0), ("ue", 4))),
            "q4z_g32": (20, 32, (("h", 0), ("z", 2))), "q4z_g128": (68, 128, (("h", 0), ("z", 2))),
            "q8z_g32": (36, 32, (("h", 0), ("z8", 2))), "q8z_g128": (132, 128, (("h", 0), ("z8", 2))),
            "nf4_b64": (36, 64, (("f", 0),)), "fp4_b64": (36, 64, (("f", 0),)), "q8a_g32": (36, 32, (("f", 0),)),
            "q2s_g128": (36, 128, (("f", 0),)), "f8e4m3": (1, 1, ()), "f8e5m2": (1, 1, ()),
            "f8e4m3_b32": (36, 32, (("f", 0),)), "f8e4m3_b128": (132, 128, (("f", 0),)),
            "trellis_v4k8_g128": (34, 128, (("h", 0),)), "trellis_v4k6_g128": (26, 128, (("h", 0),)),
            "trellis_v4k7_g128": (30, 128, (("h", 0),)), "trellis_v2k5_g128": (42, 128, (("h", 0),)),
            "trellis_v2k6_g128": (50, 128, (("h", 0),)), "trellis_v2k7_g128": (58, 128, (("h", 0),))}


def block_values(fmt: str) -> int:
    if fmt in REFBLOCK:
        return REFBLOCK[fmt][1]
    if fmt in FP4BLOCK:
        return FP4BLOCK[fmt][1]
    return 256 if fmt in KBLOCK else 32


def row_bytes(fmt: str, D: int) -> int:
    if fmt in REFBLOCK:
        bb, bs, _ = REFBLOCK[fmt]
        assert D % bs == 0
        return D // bs * bb
    if fmt == "f32":
        return 4 * D
    if fmt in ("f16", "bf16"):
        return 2 * D
    if fmt in KBLOCK:
        assert D % 256 == 0
        return D // 256 * KBLOCK[fmt][0]
    if fmt in FP4BLOCK:
        bb, bs, _ = FP4BLOCK[fmt]
        assert D % bs == 0
        return D // bs * bb
    assert D % 32 == 0
    return D // 32 * BLOCK[fmt]


def quant_table(fmt: str, V: int, D: int, seed: int = 0, tid: int = 0, scale_lo=0.001, scale_hi=0.02):
    """Raw [V, row_bytes] uint8 image of a table in ``fmt``.

    q8_0: int8 codes ~ U{-127..127}; q4_*/q5_*/iq4_nl: bytes ~ U{0..255} (so nibbles ~ U{0..15}); scales and
    mins f16 ~ U[scale_lo, scale_hi]; K-quants / iq4_xs: random bytes with their f16 fields ~ U[scale_lo,
    scale_hi] (the packed sub-block scales are any bytes); tq1_0 / tq2_0 likewise; mxfp4: codes any bytes,
    E8M0 exponents ~ U{118..126} (scales 2^-10..2^-2); nvfp4: codes any bytes, UE4M3 scales ~ U{0x20..0x3F}
    (2^-4 .. 1.9); f16: values N(0,1)*0.02; bf16 / f32: N(0,1)*0.02."""
    g = rng(seed, tid)
    if fmt in REFBLOCK:  # random code bytes; scales ~ U[scale_lo, scale_hi] (f32 ones x 64: their codes are small)
        bb, bs, fields = REFBLOCK[fmt]
        nb = D // bs
        t = g.integers(0, 256, size=(V, nb, bb), dtype=np.uint8)
        if fmt == "f8e4m3":  # no NaN codes (0x7F, 0xFF) in the synthetic table
            t[t & 0x7F == 0x7F] = 0x7E
        for kind, off in fields:
            if kind == "h":
                t[:, :, off:off + 2] = g.uniform(scale_lo, scale_hi, size=(V, nb)).astype(np.float16).view(np.uint8).reshape(V, nb, 2)
            elif kind in ("z", "z8"):  # a zero point near the code range's middle
                mid = 8.0 if kind == "z" else 128.0
                t[:, :, off:off + 2] = g.uniform(mid - 2, mid + 2, size=(V, nb)).astype(np.float16).view(np.uint8).reshape(V, nb, 2)
            elif kind == "f":
                t[:, :, off:off + 4] = (g.uniform(scale_lo, scale_hi, size=(V, nb)) * 64).astype(np.float32).view(np.uint8).reshape(V, nb, 4)
            elif kind == "ue":
                t[:, :, off:off + 4] = g.integers(0x20, 0x40, size=(V, nb, 4), dtype=np.uint8)
        if fmt == "f8e4m3_b32" or fmt == "f8e4m3_b128":
            c = t[:, :, 4:]
            c[c & 0x7F == 0x7F] = 0x7E
        return t.reshape(V, nb * bb)
    if fmt in FP4BLOCK:
        bb, bs, ns = FP4BLOCK[fmt]
        nb = D // bs
        t = g.integers(0, 256, size=(V, nb, bb), dtype=np.uint8)
        lo, hi = (118, 127) if fmt == "mxfp4" else (0x20, 0x40)
        t[:, :, :ns] = g.integers(lo, hi, size=(V, nb, ns), dtype=np.uint8)
        return t.reshape(V, nb * bb)
    if fmt in KBLOCK:
        bb, fields = KBLOCK[fmt]
        nb = D // 256
        t = g.integers(0, 256, size=(V, nb, bb), dtype=np.uint8)
        for f in fields:
            v = g.uniform(scale_lo, scale_hi, size=(V, nb)).astype(np.float16)
            t[:, :, f:f + 2] = v.view(np.uint8).reshape(V, nb, 2)
        if fmt == "iq1_m":  # the f16 scale lives in the top nibbles of the four u16 scale words
            bits = g.uniform(scale_lo, scale_hi, size=(V, nb)).astype(np.float16).view(np.uint16).astype(np.uint32)
            w = t[:, :, 48:56].copy().view(np.uint16).astype(np.uint32)
            for i in range(4):
                w[..., i] = (w[..., i] & 0x0FFF) | (((bits >> (4 * i)) & 0xF) << 12)
            t[:, :, 48:56] = w.astype(np.uint16).view(np.uint8).reshape(V, nb, 8)
        return t.reshape(V, nb * bb)
    if fmt in ("f16", "bf16", "f32"):
        x = (g.standard_normal(size=(V, D), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
        if fmt == "f16":
            return x.astype(np.float16).view(np.uint8).reshape(V, -1)
        if fmt == "bf16":
            return bf16_bits(x).view(np.uint8).reshape(V, -1)
        return x.view(np.uint8).reshape(V, -1)
    nb = D // 32
    bb = BLOCK[fmt]
    t = np.empty((V, nb, bb), np.uint8)
    d = g.uniform(scale_lo, scale_hi, size=(V, nb)).astype(np.float16)
    t[:, :, 0:2] = d.view(np.uint8).reshape(V, nb, 2)
    if fmt == "q8_0":
        t[:, :, 2:34] = g.integers(-127, 128, size=(V, nb, 32), dtype=np.int8).view(np.uint8)
    else:
        off = 2
        if fmt in ("q4_1", "q5_1"):
            m = g.uniform(-scale_hi, scale_hi, size=(V, nb)).astype(np.float16)
            t[:, :, 2:4] = m.view(np.uint8).reshape(V, nb, 2)
            off = 4
        t[:, :, off:] = g.integers(0, 256, size=(V, nb, bb - off), dtype=np.uint8)
    return t.reshape(V, nb * bb)


@dataclass(frozen=True)
class Config:
    name: str
    description: str


CONFIGS = {
    "c1_rmsnorm_f32": Config("c1_rmsnorm_f32", "RMSNorm f32 x[512,1024], gamma ~ N(1,0.1), eps 1e-6 (Qwen3-0.6B)"),
    "c2_add_rmsnorm_bf16": Config("c2_add_rmsnorm_bf16",
                                  "residual add + RMSNorm bf16 x,res[8192,4096], gamma f32, eps 1e-5 (Llama-3-8B)"),
    "c3_swiglu_bf16": Config("c3_swiglu_bf16", "SwiGLU bf16 gate,up[8192,14336] (Llama-3-8B FFN)"),
    "c3_geglu_bf16": Config("c3_geglu_bf16", "GeGLU (tanh GELU) bf16 gate,up[8192,14336]"),
    "c3_geglu_erf_bf16": Config("c3_geglu_erf_bf16", "GeGLU (erf GELU) bf16 gate,up[8192,14336]"),
    "layernorm_vit_f32": Config("layernorm_vit_f32", "LayerNorm f32 x[197,768], gamma/beta, eps 1e-6 (ViT-B/16)"),
    "layernorm_bf16": Config("layernorm_bf16", "LayerNorm bf16 x[8192,4096], f32 gamma/beta, eps 1e-5 (C2 shape)"),
    "bias_add_bf16": Config("bias_add_bf16", "Add bf16 x[8192,4096] + bias[4096] (broadcast) -> bf16"),
    "c4_qknorm_rope_bf16": Config("c4_qknorm_rope_bf16",
                                  "q[4096,32,128], k[4096,8,128] bf16: per-head RMSNorm + neox RoPE theta 1e6 (Qwen3-8B)"),
    "c5_gather_q8_0": Config("c5_gather_q8_0", "gather 16384 ids from Q8_0 [151936,4096] -> bf16"),
    "c5_gather_q4_0": Config("c5_gather_q4_0", "gather 16384 ids from Q4_0 [151936,4096] -> bf16"),
    "c5_gather_f16": Config("c5_gather_f16", "gather 16384 ids from F16 [151936,4096] -> bf16"),
    "c5_gather_q4_k": Config("c5_gather_q4_k", "gather 16384 ids from Q4_K [151936,4096] -> bf16 (C5 shape, K-quant)"),
    "c5_gather_q6_k": Config("c5_gather_q6_k", "gather 16384 ids from Q6_K [151936,4096] -> bf16 (C5 shape, K-quant)"),
    "c5_gather_mxfp4": Config("c5_gather_mxfp4", "gather 16384 ids from MXFP4 [151936,4096] -> bf16 (C5 shape, 4-bit float)"),
    "c5_gather_nvfp4": Config("c5_gather_nvfp4", "gather 16384 ids from NVFP4 [151936,4096] -> bf16 (C5 shape, 4-bit float)"),
    "c5_gather_iq2_xxs": Config("c5_gather_iq2_xxs", "gather 16384 ids from IQ2_XXS [151936,4096] -> bf16 (C5 shape, grid IQ)"),
    "c5_gather_iq3_s": Config("c5_gather_iq3_s", "gather 16384 ids from IQ3_S [151936,4096] -> bf16 (C5 shape, grid IQ)"),
}


def c1(seed=0, rows=512, D=1024):
    return dict(x=normal(seed, 0, (rows, D)), w=normal(seed, 1, (D,), 1.0, 0.1), eps=1e-6)


def c2(seed=0, rows=8192, D=4096):
    return dict(x=normal(seed, 0, (rows, D), dtype="bf16"), res=normal(seed, 1, (rows, D), dtype="bf16"),
                w=normal(seed, 2, (D,), 1.0, 0.1), eps=1e-5)


def layernorm(seed=0, rows=197, D=768, dtype="f32"):
    return dict(x=normal(seed, 0, (rows, D), dtype=dtype), w=normal(seed, 1, (D,), 1.0, 0.1),
                b=normal(seed, 2, (D,), 0.0, 0.1), eps=1e-6 if dtype == "f32" else 1e-5)


def c3(seed=0, rows=8192, cols=14336):
    return dict(gate=normal(seed, 0, (rows, cols), dtype="bf16"), up=normal(seed, 1, (rows, cols), dtype="bf16"))


def c4(seed=0, T=4096, Hq=32, Hk=8, D=128, max_pos=32768):
    return dict(q=normal(seed, 0, (T, Hq, D), dtype="bf16"), k=normal(seed, 1, (T, Hk, D), dtype="bf16"),
                wq=normal(seed, 2, (D,), 1.0, 0.1), wk=normal(seed, 3, (D,), 1.0, 0.1),
                pos=rng(seed, 4).integers(0, max_pos, size=T, dtype=np.int32), eps=1e-6, base=1e6)


def c5(fmt="q8_0", seed=0, V=151936, D=4096, N=16384):
    return dict(table=quant_table(fmt, V, D, seed, 0), ids=rng(seed, 1).integers(0, V, size=N, dtype=np.int32),
                V=V, D=D, fmt=fmt)
