"""CPU oracle for the fused layer ops -- TEST INFRASTRUCTURE ONLY.

A numpy/ctypes face over ``liboracle.so`` (``sl_oracle.c``), the C restatement of the reference CPU
provider's arithmetic (``src/Sharplight.Cpu``). Only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s ``cpu_baseline`` leg import this package; it is the checker, never the thing measured
or shipped.

The composite functions (``add_rmsnorm``, ``gated``, ``qk_norm_rope``, ``gather``) run the
reference's *unfused* f32 decomposition -- the CPU provider executes ``Add`` then ``RmsNorm``,
``Silu`` then ``Mul``, ``RmsNorm`` then ``Rope`` as separate ops -- and, for bf16 tensors, convert
with the provider's own casts (``Simd.BFloatToFloat`` on the way in, ``Simd.FloatToBFloat`` on the
way out, ``src/Sharplight.Cpu/Simd.cs:527-540``). bf16 arrays are carried as ``uint16``.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")

(F32, F16, BF16, Q8_0, Q4_0, Q4_1, Q5_0, Q5_1, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, IQ4_NL, IQ4_XS, TQ1_0, TQ2_0, MXFP4,
 NVFP4, IQ2_XXS, IQ2_XS, IQ2_S, IQ3_XXS, IQ3_S, IQ1_S, IQ1_M) = range(26)
# the reference's own formats, numbered like the C ABI
REF_FORMATS = ["q1_0", "q2_0", "q2_0_g128", "tern1_g128", "nvfp4_gs", "q4z_g32", "q4z_g128", "q8z_g32", "q8z_g128",
               "nf4_b64", "fp4_b64", "q8a_g32", "q2s_g128", "f8e4m3", "f8e5m2", "f8e4m3_b32", "f8e4m3_b128",
               "trellis_v4k8_g128", "trellis_v4k6_g128", "trellis_v4k7_g128", "trellis_v2k5_g128", "trellis_v2k6_g128", "trellis_v2k7_g128"]
FORMATS = {"f32": F32, "f16": F16, "bf16": BF16, "q8_0": Q8_0, "q4_0": Q4_0, "q4_1": Q4_1, "q5_0": Q5_0,
           "q5_1": Q5_1, "q2_k": Q2_K, "q3_k": Q3_K, "q4_k": Q4_K, "q5_k": Q5_K, "q6_k": Q6_K, "iq4_nl": IQ4_NL,
           "iq4_xs": IQ4_XS, "tq1_0": TQ1_0, "tq2_0": TQ2_0, "mxfp4": MXFP4, "nvfp4": NVFP4,
           "iq2_xxs": IQ2_XXS, "iq2_xs": IQ2_XS, "iq2_s": IQ2_S, "iq3_xxs": IQ3_XXS, "iq3_s": IQ3_S, "iq1_s": IQ1_S,
           "iq1_m": IQ1_M, **{n: 26 + i for i, n in enumerate(REF_FORMATS)}}
ACTS = {"silu": 0, "gelu_tanh": 1, "gelu_erf": 2}

_lib = None


def build() -> str:
    """Compile liboracle.so with the committed Makefile (gcc)."""
    import subprocess
    subprocess.run(["make", "-s", "-C", _HERE, "liboracle.so"], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        _declare(_lib)
    return _lib


_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_F = ctypes.c_float
_I = ctypes.c_int


def _declare(L):
    sig = {
        "orc_f32_to_bf16_n": (None, [_P, _P, _I64]),
        "orc_bf16_to_f32_n": (None, [_P, _P, _I64]),
        "orc_f16_to_f32_n": (None, [_P, _P, _I64]),
        "orc_sumsq": (_F, [_P, _I64]),
        "orc_sum": (_F, [_P, _I64]),
        "orc_rmsnorm": (None, [_P, _P, _P, _I64, _I64, _F, _I]),
        "orc_layernorm": (None, [_P, _P, _P, _P, _I64, _I64, _F]),
        "orc_add": (None, [_P, _P, _P, _I64]),
        "orc_mul": (None, [_P, _P, _P, _I64]),
        "orc_unary": (None, [_I, _P, _P, _I64]),
        "orc_erf": (ctypes.c_double, [ctypes.c_double]),
        "orc_e4m3_value": (_F, [ctypes.c_uint8]),
        "orc_e5m2_value": (_F, [ctypes.c_uint8]),
        "orc_unary_kind": (None, [_I, _P, _P, _I64, _F, _F]),
        "orc_binary": (None, [_I, _P, _P, _P, _P, _P, _P, _I]),
        "orc_align": (None, [_P, _I, _I, _P]),
        "orc_erf_rational": (_F, [_F]),
        "orc_rope": (None, [_P, _P, _P, _P, _I64, _I64, _I64, _I, _I, _F, _F, _F]),
        "orc_rope_multi": (None, [_P, _P, _I, _P, _I, _I, _P, _P, _I64, _I64, _I64, _I, _I, _F, _F, _F]),
        "orc_rope_axis_of": (_I, [_I, _P, _I]),
        "orc_row_bytes": (_I64, [_I, _I64]),
        "orc_dequant": (_I, [_I, _P, _I64, _P]),
        "orc_gather": (_I, [_I, _P, _I64, _I64, _P, _I64, _P, ctypes.POINTER(_I64)]),
        "orc_set_threads": (None, [_I]),
        "orc_get_threads": (_I, []),
        "orc_rmsnorm_mt": (None, [_P, _P, _P, _I64, _I64, _F, _I]),
        "orc_layernorm_mt": (None, [_P, _P, _P, _P, _I64, _I64, _F]),
        "orc_add_mt": (None, [_P, _P, _P, _I64]),
        "orc_mul_mt": (None, [_P, _P, _P, _I64]),
        "orc_unary_mt": (None, [_I, _P, _P, _I64]),
        "orc_rope_mt": (None, [_P, _P, _P, _P, _I64, _I64, _I64, _I, _I, _F, _F, _F]),
        "orc_gather_mt": (_I, [_I, _P, _I64, _I64, _P, _I64, _P, ctypes.POINTER(_I64)]),
        "orc_f32_to_f16_n": (None, [_P, _P, _I64]),
        "orc_cache_rows": (_I, [_I, _I64, _I64, _I64, _P, _I64, _P, _I64, _I64, _I64, _P, ctypes.c_char_p, _I64]),
        "orc_cache_write": (None, [_I, _P, _I64, _P, _I64, _P]),
        "orc_cache_write_mt": (None, [_I, _P, _I64, _P, _I64, _P]),
        "orc_e4m3_code": (ctypes.c_uint8, [_F]),
        "orc_quantize_fp8_rows": (None, [_P, _I64, _I64, _P]),
        "orc_quantize_fp8_rows_mt": (None, [_P, _I64, _I64, _P]),
        "orc_f32_to_f16_mt": (None, [_P, _P, _I64]),
        "orc_matvec": (ctypes.c_int, [ctypes.c_int, _P, _I64, _I64, _P, _I64, _P]),
        "orc_matvec_mt": (ctypes.c_int, [ctypes.c_int, _P, _I64, _I64, _P, _I64, _P]),
        "orc_q8_quantize": (_I, [_P, _I64, _I64, _P, _P, _P]),
        "orc_intdot_decode": (_I, [_I, _P, _I64, _P, _P, _P]),
        "orc_intdot_dot": (_F, [_P, _P, _P, _P, _P, _P, _I64]),
        "orc_intdot_supported": (_I, [_I]),
        "orc_matvec_q8": (_I, [_I, _P, _I64, _I64, _P, _I64, _P, _P]),
        "orc_matvec_q8_mt": (_I, [_I, _P, _I64, _I64, _P, _I64, _P]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args


def _p(a):
    return None if a is None else a.ctypes.data


def _c(a, dtype):
    return None if a is None else np.ascontiguousarray(a, dtype=dtype)


class OutOfRange(IndexError):
    """The reference's GatherOp throws ArgumentOutOfRangeException (GatherOp.cs:60-63)."""


# ---- casts ---------------------------------------------------------------------------------------

def to_bf16(x):
    x = _c(x, np.float32)
    y = np.empty(x.shape, np.uint16)
    lib().orc_f32_to_bf16_n(_p(x), _p(y), x.size)
    return y


def from_bf16(x):
    x = _c(x, np.uint16)
    y = np.empty(x.shape, np.float32)
    lib().orc_bf16_to_f32_n(_p(x), _p(y), x.size)
    return y


def f16_bits_to_f32(x):
    x = _c(x, np.uint16)
    y = np.empty(x.shape, np.float32)
    lib().orc_f16_to_f32_n(_p(x), _p(y), x.size)
    return y


def _as_f32(x, dtype):
    return from_bf16(x) if dtype == "bf16" else _c(x, np.float32)


def _out(y, dtype):
    return to_bf16(y) if dtype == "bf16" else y


# ---- primitives ----------------------------------------------------------------------------------

def sumsq(x):
    x = _c(x, np.float32)
    return float(lib().orc_sumsq(_p(x), x.size))


def rmsnorm(x, w=None, eps=1e-6, mode=0, threads=None):
    """RowOp RmsNorm (mode 0) / L2Norm (mode 1) over the last axis, f32."""
    x = _c(x, np.float32)
    w = _c(w, np.float32)
    n = x.shape[-1]
    rows = x.size // n if n else 0
    y = np.empty_like(x)
    fn = lib().orc_rmsnorm_mt if threads else lib().orc_rmsnorm
    fn(_p(x), _p(w), _p(y), rows, n, eps, mode)
    return y


def layernorm(x, w=None, b=None, eps=1e-5, threads=None):
    x = _c(x, np.float32)
    w = _c(w, np.float32)
    b = _c(b, np.float32)
    n = x.shape[-1]
    rows = x.size // n if n else 0
    y = np.empty_like(x)
    fn = lib().orc_layernorm_mt if threads else lib().orc_layernorm
    fn(_p(x), _p(w), _p(b), _p(y), rows, n, eps)
    return y


def add(a, b, threads=None):
    a = _c(a, np.float32)
    b = _c(b, np.float32)
    y = np.empty_like(a)
    (lib().orc_add_mt if threads else lib().orc_add)(_p(a), _p(b), _p(y), a.size)
    return y


def mul(a, b, threads=None):
    a = _c(a, np.float32)
    b = _c(b, np.float32)
    y = np.empty_like(a)
    (lib().orc_mul_mt if threads else lib().orc_mul)(_p(a), _p(b), _p(y), a.size)
    return y


def unary(act, x, threads=None):
    x = _c(x, np.float32)
    y = np.empty_like(x)
    (lib().orc_unary_mt if threads else lib().orc_unary)(ACTS[act], _p(x), _p(y), x.size)
    return y


# The reference's UnaryKind and BinaryKind, by name (src/Sharplight.Cpu/UnaryKind.cs:4-6, BinaryKind.cs:4).
UNARY_KINDS = ["Neg", "Exp", "Log", "Sqrt", "Rsqrt", "Sigmoid", "Silu", "Gelu", "GeluTanh", "Tanh", "Softplus", "Relu",
               "Abs", "Square", "Recip", "Scale", "Erf", "HardSwish", "HardSigmoid", "Clip", "Sin", "Cos", "Tan",
               "Asin", "Acos", "Atan", "Sinh", "Cosh", "Asinh", "Acosh", "Atanh", "Floor", "Ceil", "Round", "Sign",
               "Softsign", "Mish", "Elu", "Celu", "Selu", "LeakyRelu", "ThresholdedRelu", "Not", "IsNaN", "IsInf"]
BINARY_KINDS = ["Add", "Sub", "Mul", "Div", "Max", "Min", "Pow", "Mod", "PRelu", "Equal", "NotEqual", "Less",
                "LessEqual", "Greater", "GreaterEqual", "And", "Or", "Xor", "Atan2", "FMod"]


def unary_kind(kind, x, p0=1.0, p1=0.0):
    """ScalarMath.Unary of one contiguous range (vector forms on whole groups of 8, then the tail form)."""
    x = _c(x, np.float32)
    y = np.empty(x.shape, np.float32)
    lib().orc_unary_kind(UNARY_KINDS.index(kind), _p(x), _p(y), x.size, p0, p1)
    return y


def align(a_shape, y_rank):
    """BinaryOp.Align: element strides of a dense operand of a_shape against an output of rank y_rank."""
    d = np.asarray(a_shape, np.int64)
    s = np.empty(max(y_rank, 1), np.int64)
    lib().orc_align(_p(d), len(a_shape), y_rank, _p(s))
    return s[:y_rank]


def binary(kind, a, b):
    """BinaryOp on dense f32 operands with numpy broadcasting; returns y of the broadcast shape."""
    sha, shb = np.shape(a), np.shape(b)
    a = _c(a, np.float32)  # (a 0-d operand becomes 1-d here; its shape is kept above)
    b = _c(b, np.float32)
    shape = np.broadcast_shapes(sha, shb)
    r = len(shape)
    y = np.empty(shape, np.float32)
    dims = np.asarray(shape if r else [1], np.int64)
    sa, sb = align(sha, r), align(shb, r)
    if r == 0:
        sa = sb = np.zeros(1, np.int64)
    lib().orc_binary(BINARY_KINDS.index(kind), _p(a), _p(sa), _p(b), _p(sb), _p(y), _p(dims), r)
    return y


def rope(x, pos, dims=None, neox=True, base=10000.0, freq_scale=1.0, attn_factor=1.0, ff=None, threads=None):
    """RopeOp over x [T, H, D] (f32) with int32 positions [T]."""
    x = _c(x, np.float32)
    T, H, D = x.shape
    pos = _c(pos, np.int32).reshape(-1)
    assert pos.size == T
    ff = _c(ff, np.float32)
    dims = D if not dims else dims
    y = np.empty_like(x)
    fn = lib().orc_rope_mt if threads else lib().orc_rope
    fn(_p(x), _p(pos), _p(ff), _p(y), T, H, D, dims, int(bool(neox)), base, freq_scale, attn_factor)
    return y


def rope_multi(x, pos, sections=None, interleaved=False, per_element=False, dims=None, neox=True, base=10000.0,
               freq_scale=1.0, attn_factor=1.0, ff=None):
    """Multi-axis RopeOp: x [T, H, D] f32, positions int32 [T, A] (A <= 4), sections of 4 entries or None."""
    x = _c(x, np.float32)
    T, H, D = x.shape
    pos = _c(pos, np.int32).reshape(T, -1)
    sec = None if sections is None else _c(sections, np.int32)
    ff = _c(ff, np.float32)
    dims = D if not dims else dims
    y = np.empty_like(x)
    lib().orc_rope_multi(_p(x), _p(pos), pos.shape[1], _p(sec), int(bool(interleaved)), int(bool(per_element)),
                         _p(ff), _p(y), T, H, D, dims, int(bool(neox)), base, freq_scale, attn_factor)
    return y


def rope_axis_of(i, sections, interleaved=False):
    sec = _c(sections, np.int32)
    return int(lib().orc_rope_axis_of(i, _p(sec), int(bool(interleaved))))


def row_bytes(fmt, d):
    return int(lib().orc_row_bytes(FORMATS[fmt], d))


def dequant(fmt, raw, count):
    raw = _c(raw, np.uint8)
    y = np.empty(count, np.float32)
    if lib().orc_dequant(FORMATS[fmt], _p(raw), count, _p(y)):
        raise ValueError(f"cannot dequantize {count} values of {fmt}")
    return y


def gather(fmt, table, V, D, ids, threads=None):
    """GatherOp with f32 output: table is the raw [V, row_bytes] byte image."""
    table = _c(table, np.uint8)
    ids = _c(ids, np.int32).reshape(-1)
    y = np.empty((ids.size, D), np.float32)
    bad = _I64(0)
    fn = lib().orc_gather_mt if threads else lib().orc_gather
    st = fn(FORMATS[fmt], _p(table), V, D, _p(ids), ids.size, _p(y), ctypes.byref(bad))
    if st == -1:
        raise OutOfRange(f"Gather index {bad.value} out of range [0,{V}).")
    if st:
        raise ValueError(f"gather: unsupported format/shape {fmt} D={D}")
    return y


def set_threads(n):
    lib().orc_set_threads(int(n))


# ---- composites: the reference's unfused decomposition ------------------------------------------

def add_rmsnorm(x, res, w, eps, dtype="f32", mode=0):
    """Add then RmsNorm (CPU provider order); returns (y, h) in ``dtype``. The norm reads the f32 sum."""
    h = add(_as_f32(x, dtype), _as_f32(res, dtype))
    y = rmsnorm(h, w, eps, mode)
    return _out(y, dtype), _out(h, dtype)


def norm(x, w, eps, dtype="f32", mode=0):
    return _out(rmsnorm(_as_f32(x, dtype), w, eps, mode), dtype)


def add_layernorm(x, res, w, b, eps, dtype="f32"):
    h = add(_as_f32(x, dtype), _as_f32(res, dtype)) if res is not None else _as_f32(x, dtype)
    y = layernorm(h, w, b, eps)
    return _out(y, dtype), (_out(h, dtype) if res is not None else None)


def gated(act, gate, up, dtype="f32", threads=None):
    """Mul(act(gate), up) as two ops (IMlpActivation.cs:12)."""
    return _out(mul(unary(act, _as_f32(gate, dtype), threads=threads), _as_f32(up, dtype), threads=threads), dtype)


def qk_norm_rope(x, pos, w=None, eps=1e-6, dtype="f32", **rope_kw):
    """RmsNorm over each head row (if w is given or norm requested) then Rope, x [T, H, D]."""
    xf = _as_f32(x, dtype)
    if w is not None:
        xf = rmsnorm(xf, w, eps)
    return _out(rope(xf, pos, **rope_kw), dtype)


def gather_as(fmt, table, V, D, ids, dtype="f32"):
    return _out(gather(fmt, table, V, D, ids), dtype)


# ---- KV cache writes -------------------------------------------------------------------------------

ROWS = {"past": 0, "seq": 1, "paged": 2}


class CacheOverflow(RuntimeError):
    """The reference's CacheWriteOp / KvPages throw InvalidOperationException (CacheWriteOp.cs:103-127,
    KvPages.cs:38-49)."""


def to_f16(x):
    x = _c(x, np.float32)
    y = np.empty(x.shape, np.uint16)
    lib().orc_f32_to_f16_n(_p(x), _p(y), x.size)
    return y


def cache_rows(mode, T, ctx, n_past=0, seq=None, slots=1, pages=None, block_size=16):
    """Cache row of each token (CacheWriteOp's mapping); raises CacheOverflow like the reference."""
    seq = _c(seq, np.int32)
    pages = _c(pages, np.int32)
    page_slots, bps = (pages.shape if pages is not None else (0, 0))
    rows = np.empty(max(T, 1), np.int64)
    err = ctypes.create_string_buffer(256)
    st = lib().orc_cache_rows(ROWS[mode], T, ctx, n_past, _p(seq), slots, _p(pages), page_slots, bps, block_size,
                              _p(rows), err, len(err))
    if st:
        raise CacheOverflow(err.value.decode())
    return rows[:T]


def cache_write(cache, x, rows, cache_type):
    """CacheWriteOp.Body: x [T, inner] f32 into ``cache`` (numpy array: f32, or uint16 bits of f16/bf16)
    at rows[t]; in place."""
    x = _c(x, np.float32)
    T = x.shape[0]
    inner = x.size // max(T, 1)
    rows = _c(rows, np.int64)
    lib().orc_cache_write(FORMATS[cache_type], _p(cache), inner, _p(x), T, _p(rows))
    return cache


# ---- E4M3 activation rows ---------------------------------------------------------------------------

def e4m3_code(v: float) -> int:
    return int(lib().orc_e4m3_code(float(v)))


def quantize_fp8(x):
    """quantize_fp8 (Kernels/gemm_fp8.slang:36-55): rows [R, K] f32 (K % 128 == 0) -> [R, K + K/32] bytes,
    K E4M3 codes then K/128 f32 scales (amax / 448) per row."""
    x = _c(x, np.float32)
    K = x.shape[-1]
    rows = x.size // K
    out = np.empty((rows, K + K // 32), np.uint8)
    lib().orc_quantize_fp8_rows(_p(x), rows, K, _p(out))
    return out.reshape(x.shape[:-1] + (K + K // 32,))


def matvec(fmt, w_raw, N, K, x, threads=None):
    """MatMulOp's float-row path: y [T, N] f32 = x [T, K] f32 . W^T, W = N rows of the raw ``fmt`` bytes."""
    x = _c(np.atleast_2d(x), np.float32)
    w_raw = np.ascontiguousarray(w_raw).view(np.uint8)
    T = x.shape[0]
    y = np.empty((T, N), np.float32)
    fn = lib().orc_matvec_mt if threads else lib().orc_matvec
    if fn(FORMATS[fmt], _p(w_raw), N, K, _p(x), T, _p(y)):
        raise ValueError(f"matvec: bad format/size {fmt} K={K}")
    return y


def dual_matvec(act, fmt, wg_raw, wu_raw, N, K, x, dtype="f32"):
    """The unfused decode FFN the dual matvec replaces: act(x . Wg^T) * (x . Wu^T) as MatMul, MatMul, the
    activation (UnaryOp) and Mul (BinaryOp), all f32; ``dtype`` "bf16" rounds the result."""
    g = matvec(fmt, wg_raw, N, K, x)
    u = matvec(fmt, wu_raw, N, K, x)
    y = mul(unary(act, g), u)
    return to_bf16(y) if dtype == "bf16" else y


# ---- integer-dot matvec (q8 activations) ---------------------------------------------------------------

INTDOT_FORMATS = ("q8_0", "q4_0", "q4_1", "q5_0", "q5_1", "q4_k", "q5_k", "q6_k", "iq4_nl", "iq4_xs", "mxfp4")


def q8_quantize(x):
    """IntDot.Quantize per row: x [rows, K] f32 -> (q int8 [rows, K], d f32 [rows, K/32], gs f32 [rows, K/16])."""
    x = _c(np.atleast_2d(x), np.float32)
    rows, K = x.shape
    q = np.empty((rows, K), np.int8)
    d = np.empty((rows, K // 32), np.float32)
    gs = np.empty((rows, K // 16), np.float32)
    if lib().orc_q8_quantize(_p(x), rows, K, _p(q), _p(d), _p(gs)):
        raise ValueError(f"q8_quantize: K={K} is not a multiple of 32")
    return q, d, gs


def intdot_decode(fmt, row_raw, K):
    """IntDot.Decode of one weight row: (u uint8 [K], a f32 [K/16], b f32 [K/16]), value = a u + b."""
    row_raw = np.ascontiguousarray(row_raw).view(np.uint8)
    u = np.empty(K, np.uint8)
    a = np.empty(K // 16, np.float32)
    b = np.empty(K // 16, np.float32)
    if lib().orc_intdot_decode(FORMATS[fmt], _p(row_raw), K, _p(u), _p(a), _p(b)):
        raise ValueError(f"intdot_decode: {fmt} has no integer-dot decoder")
    return u, a, b


def intdot_dot(u, a, b, q, d, gs):
    """IntDot.DotScalar: one decoded weight row with one quantized activation row."""
    u, a, b = _c(u, np.uint8), _c(a, np.float32), _c(b, np.float32)
    q, d, gs = _c(q, np.int8), _c(d, np.float32), _c(gs, np.float32)
    return float(lib().orc_intdot_dot(_p(u), _p(a), _p(b), _p(q), _p(d), _p(gs), u.size))


def matvec_q8(fmt, w_raw, N, K, x, threads=None, with_abs=False):
    """MatMulOp's integer-dot path: x [T, K] quantized per 32 values, y [T, N] f32. with_abs: also the
    per-output sum of |a d s| + |b gs| (f64), the magnitude bound of the f32 accumulation."""
    x = _c(np.atleast_2d(x), np.float32)
    w_raw = np.ascontiguousarray(w_raw).view(np.uint8)
    T = x.shape[0]
    y = np.empty((T, N), np.float32)
    if threads:
        r = lib().orc_matvec_q8_mt(FORMATS[fmt], _p(w_raw), N, K, _p(x), T, _p(y))
        yabs = None
    else:
        yabs = np.empty((T, N), np.float64) if with_abs else None
        r = lib().orc_matvec_q8(FORMATS[fmt], _p(w_raw), N, K, _p(x), T, _p(y), _p(yabs))
    if r:
        raise ValueError(f"matvec_q8: {fmt} K={K} not supported")
    return (y, yabs) if with_abs else y
