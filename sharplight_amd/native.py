"""ctypes binding of libsharplight_hip (include/sharplight_hip.h).

This is the Python twin of the managed provider's ``[LibraryImport]`` declarations: one typed foreign
function per C entry point, statuses turned into the exceptions the reference's providers throw
(``ArgumentException`` -> ``ValueError``, ``NotSupportedException`` -> ``NotImplementedError``,
``ArgumentOutOfRangeException`` -> ``IndexError``, ``InvalidDataException`` -> ``SlhipFormatError``, a
``ValueError``). There is no fallback: if the library is not built
or cannot load, every call raises.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libsharplight_hip.so")

OK, ERR_INVALID, ERR_UNSUPPORTED, ERR_HIP, ERR_INDEX, ERR_NO_DEVICE, ERR_CACHE, ERR_FORMAT = 0, -1, -2, -3, -4, -5, -6, -7
F32, F16, BF16 = 0, 1, 2
DTYPES = {"f32": F32, "f16": F16, "bf16": BF16}
NP_DTYPES = {F32: np.float32, F16: np.float16, BF16: np.uint16}  # bf16 travels as raw uint16 bits
(FMT_F32, FMT_F16, FMT_BF16, FMT_Q8_0, FMT_Q4_0, FMT_Q4_1, FMT_Q5_0, FMT_Q5_1, FMT_Q2_K, FMT_Q3_K, FMT_Q4_K,
 FMT_Q5_K, FMT_Q6_K, FMT_IQ4_NL, FMT_IQ4_XS, FMT_TQ1_0, FMT_TQ2_0, FMT_MXFP4, FMT_NVFP4, FMT_IQ2_XXS, FMT_IQ2_XS,
 FMT_IQ2_S, FMT_IQ3_XXS, FMT_IQ3_S, FMT_IQ1_S, FMT_IQ1_M) = range(26)
# the reference's own formats (slhip_format 26..48, the trellis formats last)
REF_FORMATS = ["q1_0", "q2_0", "q2_0_g128", "tern1_g128", "nvfp4_gs", "q4z_g32", "q4z_g128", "q8z_g32", "q8z_g128",
               "nf4_b64", "fp4_b64", "q8a_g32", "q2s_g128", "f8e4m3", "f8e5m2", "f8e4m3_b32", "f8e4m3_b128",
               "trellis_v4k8_g128", "trellis_v4k6_g128", "trellis_v4k7_g128", "trellis_v2k5_g128", "trellis_v2k6_g128", "trellis_v2k7_g128"]
FORMATS = {"f32": FMT_F32, "f16": FMT_F16, "bf16": FMT_BF16, "q8_0": FMT_Q8_0, "q4_0": FMT_Q4_0,
           "q4_1": FMT_Q4_1, "q5_0": FMT_Q5_0, "q5_1": FMT_Q5_1, "q2_k": FMT_Q2_K, "q3_k": FMT_Q3_K,
           "q4_k": FMT_Q4_K, "q5_k": FMT_Q5_K, "q6_k": FMT_Q6_K, "iq4_nl": FMT_IQ4_NL, "iq4_xs": FMT_IQ4_XS,
           "tq1_0": FMT_TQ1_0, "tq2_0": FMT_TQ2_0, "mxfp4": FMT_MXFP4, "nvfp4": FMT_NVFP4, "iq2_xxs": FMT_IQ2_XXS,
           "iq2_xs": FMT_IQ2_XS, "iq2_s": FMT_IQ2_S, "iq3_xxs": FMT_IQ3_XXS, "iq3_s": FMT_IQ3_S, "iq1_s": FMT_IQ1_S,
           "iq1_m": FMT_IQ1_M, **{n: 26 + i for i, n in enumerate(REF_FORMATS)}}
NORM_RMS, NORM_L2, NORM_LAYER = 0, 1, 2
NORMS = {"rms": NORM_RMS, "l2": NORM_L2, "layer": NORM_LAYER}
ACT_SILU, ACT_GELU_TANH, ACT_GELU_ERF = 0, 1, 2
ACTS = {"silu": ACT_SILU, "gelu_tanh": ACT_GELU_TANH, "gelu_erf": ACT_GELU_ERF}
# slhip_unary_op / slhip_binary_op: the reference's UnaryKind and BinaryKind order, by StandardOps name
UNARY_OPS = {n: i for i, n in enumerate(
    ["Neg", "Exp", "Log", "Sqrt", "Rsqrt", "Sigmoid", "Silu", "Gelu", "GeluTanh", "Tanh", "Softplus", "Relu", "Abs",
     "Square", "Recip", "Scale", "Erf", "HardSwish", "HardSigmoid", "Clip", "Sin", "Cos", "Tan", "Asin", "Acos",
     "Atan", "Sinh", "Cosh", "Asinh", "Acosh", "Atanh", "Floor", "Ceil", "Round", "Sign", "Softsign", "Mish", "Elu",
     "Celu", "Selu", "LeakyRelu", "ThresholdedRelu", "Not", "IsNaN", "IsInf"])}
BINARY_OPS = {n: i for i, n in enumerate(
    ["Add", "Sub", "Mul", "Div", "Max", "Min", "Pow", "Mod", "PRelu", "Equal", "NotEqual", "Less", "LessEqual",
     "Greater", "GreaterEqual", "And", "Or", "Xor", "Atan2", "FMod"])}


class SlhipError(RuntimeError):
    """A HIP runtime failure (SLHIP_ERR_HIP) or a missing device (SLHIP_ERR_NO_DEVICE)."""


class SlhipArgumentError(ValueError):
    pass


class SlhipNotSupported(NotImplementedError):
    pass


class SlhipIndexError(IndexError):
    pass


class SlhipFormatError(ValueError):
    """Malformed file data (the reference throws InvalidDataException)."""


class SlhipCacheError(SlhipError):
    """A KV-cache row outside the cache or block table (the reference throws InvalidOperationException)."""


class DeviceProps(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char * 256), ("arch", ctypes.c_char * 64), ("total_memory", ctypes.c_int64),
                ("compute_units", ctypes.c_int32), ("wavefront_size", ctypes.c_int32),
                ("pci_domain", ctypes.c_int32), ("pci_bus", ctypes.c_int32), ("pci_device", ctypes.c_int32),
                ("clock_khz", ctypes.c_int32), ("l2_bytes", ctypes.c_int64),
                ("max_threads_per_block", ctypes.c_int32), ("lds_bytes_per_block", ctypes.c_int32)]


class CacheRows(ctypes.Structure):
    """slhip_cache_rows: where token t of a cache write goes (ROWS_PAST / ROWS_SEQ / ROWS_PAGED)."""
    _fields_ = [("mode", ctypes.c_int32), ("reserved", ctypes.c_int32), ("ctx", ctypes.c_int64),
                ("n_past", ctypes.c_int64), ("seq", ctypes.c_void_p), ("slots", ctypes.c_int64),
                ("pages", ctypes.c_void_p), ("page_slots", ctypes.c_int64), ("blocks_per_slot", ctypes.c_int64),
                ("block_size", ctypes.c_int64)]


class NormCopies(ctypes.Structure):
    """slhip_norm_copies: the f16 and E4M3 GEMM activation copies a row norm writes (either may be NULL)."""
    _fields_ = [("y16", ctypes.c_void_p), ("y16_stride", ctypes.c_int64), ("yq", ctypes.c_void_p),
                ("yq_stride", ctypes.c_int64)]


EW_MAX_INPUTS, EW_MAX_OPS, EW_MAX_OUTPUTS, EW_MAX_REGS = 8, 16, 4, 16
EWI_FULL, EWI_ROW, EWI_COL, EWI_SCALAR = 0, 1, 2, 3
EWK_BINARY, EWK_UNARY = 0, 1
EW_NORMS = {"rms": 1, "l2": 2}


class EwInput(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("dtype", ctypes.c_int), ("mode", ctypes.c_int)]


class EwOp(ctypes.Structure):
    _fields_ = [("kind", ctypes.c_int), ("op", ctypes.c_int), ("a", ctypes.c_int), ("b", ctypes.c_int),
                ("dst", ctypes.c_int), ("round", ctypes.c_int), ("p0", ctypes.c_float), ("p1", ctypes.c_float)]


class EwOutput(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("dtype", ctypes.c_int), ("reg", ctypes.c_int)]


class EwNorm(ctypes.Structure):
    _fields_ = [("kind", ctypes.c_int), ("reg", ctypes.c_int), ("w", ctypes.c_void_p), ("eps", ctypes.c_float),
                ("y", ctypes.c_void_p), ("dtype_y", ctypes.c_int)]


class EwProgram(ctypes.Structure):
    """slhip_ew_program: a fused elementwise group with an optional norm head or tail."""
    _fields_ = [("n_inputs", ctypes.c_int), ("n_ops", ctypes.c_int), ("n_outputs", ctypes.c_int),
                ("inputs", EwInput * EW_MAX_INPUTS), ("ops", EwOp * EW_MAX_OPS),
                ("outputs", EwOutput * EW_MAX_OUTPUTS), ("head", EwNorm), ("tail", EwNorm)]


class GgufInfo(ctypes.Structure):
    """slhip_gguf_info."""
    _fields_ = [("version", ctypes.c_uint32), ("alignment", ctypes.c_uint32), ("n_tensors", ctypes.c_int64),
                ("n_kv", ctypes.c_int64), ("data_offset", ctypes.c_int64), ("file_length", ctypes.c_int64),
                ("has_data", ctypes.c_int32), ("table_complete", ctypes.c_int32)]


class GgufValue(ctypes.Structure):
    """slhip_gguf_value: one node of a metadata value tree."""
    _fields_ = [("type", ctypes.c_uint32), ("elem_type", ctypes.c_uint32), ("count", ctypes.c_int64),
                ("u", ctypes.c_uint64), ("i", ctypes.c_int64), ("f", ctypes.c_double), ("data", ctypes.c_void_p),
                ("first_child", ctypes.c_int64)]


class GgufTensor(ctypes.Structure):
    """slhip_gguf_tensor."""
    _fields_ = [("name", ctypes.c_char_p), ("type_name", ctypes.c_char_p), ("ggml_type", ctypes.c_int32),
                ("format", ctypes.c_int32), ("block_size", ctypes.c_int32), ("block_bytes", ctypes.c_int32),
                ("n_dims", ctypes.c_int32), ("reserved", ctypes.c_int32), ("ne", ctypes.c_int64 * 8),
                ("relative_offset", ctypes.c_int64), ("offset", ctypes.c_int64), ("byte_size", ctypes.c_int64),
                ("stored_bytes", ctypes.c_int64)]


ROWS = {"past": 0, "seq": 1, "paged": 2}


def cache_rows(mode, ctx, *, n_past=0, seq=None, slots=1, pages=None, page_slots=0, blocks_per_slot=0,
               block_size=16) -> CacheRows:
    return CacheRows(ROWS.get(mode, mode), 0, ctx, n_past, ptr(seq), slots, ptr(pages), page_slots, blocks_per_slot,
                     block_size)


class RopeTensor(ctypes.Structure):
    _fields_ = [("x", ctypes.c_void_p), ("y", ctypes.c_void_p), ("norm_w", ctypes.c_void_p),
                ("heads", ctypes.c_int64), ("x_stride_t", ctypes.c_int64), ("x_stride_h", ctypes.c_int64),
                ("y_stride_t", ctypes.c_int64), ("y_stride_h", ctypes.c_int64),
                ("rows", ctypes.POINTER(CacheRows))]


class RopeCfg(ctypes.Structure):
    _fields_ = [("dims", ctypes.c_int32), ("neox", ctypes.c_int32), ("base", ctypes.c_float),
                ("freq_scale", ctypes.c_float), ("attn_factor", ctypes.c_float), ("norm", ctypes.c_int32),
                ("eps", ctypes.c_float), ("pos_axes", ctypes.c_int32), ("sections", ctypes.c_int32 * 4),
                ("interleaved", ctypes.c_int32), ("per_element", ctypes.c_int32)]


_P = ctypes.c_void_p
_I = ctypes.c_int
_I64 = ctypes.c_int64
_F = ctypes.c_float
_SZ = ctypes.c_size_t

SIGNATURES = {
    "slhip_last_error": (ctypes.c_char_p, []),
    "slhip_abi_version": (_I, []),
    "slhip_device_count": (_I, [ctypes.POINTER(_I)]),
    "slhip_device_props_get": (_I, [_I, ctypes.POINTER(DeviceProps)]),
    "slhip_set_device": (_I, [_I]),
    "slhip_get_device": (_I, [ctypes.POINTER(_I)]),
    "slhip_mem_info": (_I, [ctypes.POINTER(_SZ), ctypes.POINTER(_SZ)]),
    "slhip_malloc": (_I, [ctypes.POINTER(_P), _SZ]),
    "slhip_free": (_I, [_P]),
    "slhip_host_malloc": (_I, [ctypes.POINTER(_P), _SZ]),
    "slhip_host_free": (_I, [_P]),
    "slhip_memcpy_h2d": (_I, [_P, _P, _SZ, _P]),
    "slhip_memcpy_d2h": (_I, [_P, _P, _SZ, _P]),
    "slhip_memcpy_d2d": (_I, [_P, _P, _SZ, _P]),
    "slhip_memset": (_I, [_P, _I, _SZ, _P]),
    "slhip_stream_create": (_I, [ctypes.POINTER(_P)]),
    "slhip_stream_destroy": (_I, [_P]),
    "slhip_stream_sync": (_I, [_P]),
    "slhip_event_create": (_I, [ctypes.POINTER(_P)]),
    "slhip_event_destroy": (_I, [_P]),
    "slhip_event_record": (_I, [_P, _P]),
    "slhip_event_synchronize": (_I, [_P]),
    "slhip_event_elapsed_ms": (_I, [ctypes.POINTER(_F), _P, _P]),
    "slhip_graph_begin": (_I, [_P]),
    "slhip_graph_end": (_I, [_P, ctypes.POINTER(_P)]),
    "slhip_graph_launch": (_I, [_P, _P]),
    "slhip_graph_destroy": (_I, [_P]),
    "slhip_rownorm": (_I, [_I, _I, _I, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _F, _P]),
    "slhip_rownorm_copies": (_I, [_I, _I, _I, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _F,
                                  ctypes.POINTER(NormCopies), _P]),
    "slhip_matvec": (_I, [_I, _I, _I, _P, _I64, _I64, _I64, _P, _I64, _P, _I64, _P]),
    "slhip_dual_matvec": (_I, [_I, _I, _I, _I, _P, _I64, _I64, _I64, _P, _P, _I64, _P, _I64, _P]),
    "slhip_matvec_bias": (_I, [_I, _I, _I, _P, _I64, _I64, _I64, _P, _I64, _P, _P, _I64, _P]),
    "slhip_q8_row_bytes": (_I64, [_I64]),
    "slhip_ew_program_run": (_I, [ctypes.POINTER(EwProgram), _I64, _I64, _P]),
    "slhip_dual_matvec_int8": (_I, [_I, _I, _I, _I, _P, _I64, _I64, _I64, _P, _P, _I64, _P, _I64, _P, _I64, _P]),
    "slhip_dual_matvec_int8_noalloc": (_I, [_I, _I, _I, _I, _P, _I64, _I64, _I64, _P, _P, _I64, _P, _I64, _P]),
    "slhip_quantize_q8": (_I, [_I, _P, _I64, _I64, _I64, _P, _P]),
    "slhip_matvec_q8": (_I, [_I, _I, _P, _I64, _I64, _P, _I64, _P, _I64, _P, _P]),
    "slhip_dual_matvec_q8": (_I, [_I, _I, _I, _P, _I64, _I64, _P, _P, _I64, _P, _I64, _P]),
    "slhip_gated_act": (_I, [_I, _I, _I, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _P]),
    "slhip_rope": (_I, [_I, _I, ctypes.POINTER(RopeTensor), _I, _P, _P, _I64, _I64, ctypes.POINTER(RopeCfg), _P]),
    "slhip_gather": (_I, [_I, _P, _I64, _I64, _P, _I64, _I, _P, _I64, _P]),
    "slhip_convert": (_I, [_I, _I, _P, _P, _I64, _P]),
    "slhip_binary": (_I, [_I, _I, _I, _I, _P, _P, _P, _P, _P, _P, _I, _P]),
    "slhip_unary": (_I, [_I, _I, _I, _P, _P, _I64, _I64, _I64, _I64, _F, _F, _P]),
    "slhip_cache_write": (_I, [_I, _I, _P, _I64, _I64, _I64, _P, ctypes.POINTER(CacheRows), _P]),
    "slhip_provider_check": (_I, [ctypes.c_char_p, _SZ]),
    "slhip_node_supports": (_I, [ctypes.c_char_p, _I, ctypes.POINTER(_I), ctypes.c_char_p, _SZ]),
    "slhip_segment_compile": (_I, [ctypes.c_char_p, _I64, ctypes.POINTER(_P)]),
    "slhip_segment_set_input": (_I, [_P, _I, _P, _SZ]),
    "slhip_segment_execute": (_I, [_P, _I64]),
    "slhip_segment_get_output": (_I, [_P, _I, _P, _SZ]),
    "slhip_segment_reset_state": (_I, [_P]),
    "slhip_segment_set_scalar": (_I, [_P, ctypes.c_char_p, _I64]),
    "slhip_segment_device_bytes": (_I, [_P, ctypes.POINTER(_I64)]),
    "slhip_segment_launches": (_I, [_P, ctypes.c_char_p, _SZ]),
    "slhip_segment_launches_at": (_I, [_P, _I64, ctypes.c_char_p, _SZ]),
    "slhip_segment_plan": (_I, [ctypes.c_char_p, ctypes.c_char_p, _SZ]),
    "slhip_segment_describe": (_I, [ctypes.c_char_p, ctypes.c_char_p, _SZ]),
    "slhip_segment_destroy": (_I, [_P]),
    "slhip_gguf_open": (_I, [ctypes.c_char_p, ctypes.POINTER(_P)]),
    "slhip_gguf_open_prefix": (_I, [_P, _SZ, ctypes.POINTER(_P)]),
    "slhip_gguf_close": (_I, [_P]),
    "slhip_gguf_get_info": (_I, [_P, ctypes.POINTER(GgufInfo)]),
    "slhip_gguf_kv": (_I, [_P, _I64, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(_I64)]),
    "slhip_gguf_find_kv": (_I, [_P, ctypes.c_char_p, ctypes.POINTER(_I64)]),
    "slhip_gguf_get_value": (_I, [_P, _I64, ctypes.POINTER(GgufValue)]),
    "slhip_gguf_tensor_info": (_I, [_P, _I64, ctypes.POINTER(GgufTensor)]),
    "slhip_gguf_find_tensor": (_I, [_P, ctypes.c_char_p, ctypes.POINTER(_I64)]),
    "slhip_gguf_type": (_I, [_I, ctypes.POINTER(GgufTensor)]),
    "slhip_gguf_read": (_I, [_P, _I64, _I64, _P, _SZ]),
    "slhip_gguf_tensor_pointer": (_I, [_P, _I64, ctypes.POINTER(_P)]),
    "slhip_gguf_upload": (_I, [_P, _I64, _P, _SZ, _P]),
    "slhip_upload": (_I, [_P, _P, _SZ, _P]),
}

_lib = None


def lib():
    """The loaded library; raises if it is not built (no fallback path exists)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise SlhipError(f"{LIB_PATH} is not built: run `python -m sharplight_amd.build`")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def last_error() -> str:
    return lib().slhip_last_error().decode(errors="replace")


def check(status: int) -> None:
    if status == OK:
        return
    msg = last_error()
    if status == ERR_INVALID:
        raise SlhipArgumentError(msg)
    if status == ERR_UNSUPPORTED:
        raise SlhipNotSupported(msg)
    if status == ERR_INDEX:
        raise SlhipIndexError(msg)
    if status == ERR_CACHE:
        raise SlhipCacheError(msg)
    if status == ERR_FORMAT:
        raise SlhipFormatError(msg)
    raise SlhipError(f"status {status}: {msg}")


def call(name: str, *args) -> None:
    check(getattr(lib(), name)(*args))


# ---- devices ----------------------------------------------------------------------------------------

def device_count() -> int:
    n = _I(0)
    call("slhip_device_count", ctypes.byref(n))
    return n.value


def device_props(index: int = 0) -> DeviceProps:
    p = DeviceProps()
    call("slhip_device_props_get", index, ctypes.byref(p))
    return p


def set_device(index: int) -> None:
    call("slhip_set_device", index)


def synchronize(stream=None) -> None:
    call("slhip_stream_sync", stream)


# ---- memory -----------------------------------------------------------------------------------------

class DeviceBuffer:
    """Owning device allocation (slhip_malloc / slhip_free)."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = _P(0)
        call("slhip_malloc", ctypes.byref(p), self.nbytes)
        self.ptr = p.value or 0

    @classmethod
    def from_numpy(cls, arr: np.ndarray, stream=None) -> "DeviceBuffer":
        arr = np.ascontiguousarray(arr)
        buf = cls(arr.nbytes)
        buf.upload(arr, stream)
        return buf

    def upload(self, arr: np.ndarray, stream=None, offset: int = 0) -> None:
        arr = np.ascontiguousarray(arr)
        if offset + arr.nbytes > self.nbytes:
            raise ValueError("upload past the end of the buffer")
        call("slhip_memcpy_h2d", self.ptr + offset, arr.ctypes.data, arr.nbytes, stream)
        call("slhip_stream_sync", stream)

    def download(self, shape, dtype, stream=None, offset: int = 0) -> np.ndarray:
        out = np.empty(shape, dtype)
        if offset + out.nbytes > self.nbytes:
            raise ValueError("download past the end of the buffer")
        call("slhip_memcpy_d2h", out.ctypes.data, self.ptr + offset, out.nbytes, stream)
        call("slhip_stream_sync", stream)
        return out

    def zero(self, stream=None) -> None:
        call("slhip_memset", self.ptr, 0, self.nbytes, stream)

    def free(self) -> None:
        if self.ptr:
            call("slhip_free", self.ptr)
            self.ptr = 0

    def __del__(self):
        try:
            if self.ptr and _lib is not None:
                _lib.slhip_free(self.ptr)
                self.ptr = 0
        except Exception:
            pass

    def __int__(self):
        return self.ptr


def ptr(x) -> int | None:
    """Device address of a DeviceBuffer / int / None."""
    if x is None:
        return None
    if isinstance(x, DeviceBuffer):
        return x.ptr
    return int(x)


class Event:
    def __init__(self):
        e = _P(0)
        call("slhip_event_create", ctypes.byref(e))
        self.handle = e.value

    def record(self, stream=None):
        call("slhip_event_record", self.handle, stream)

    def synchronize(self):
        call("slhip_event_synchronize", self.handle)

    def elapsed_ms(self, end: "Event") -> float:
        ms = _F(0)
        call("slhip_event_elapsed_ms", ctypes.byref(ms), self.handle, end.handle)
        return ms.value

    def __del__(self):
        try:
            if self.handle and _lib is not None:
                _lib.slhip_event_destroy(self.handle)
        except Exception:
            pass


class Stream:
    def __init__(self):
        s = _P(0)
        call("slhip_stream_create", ctypes.byref(s))
        self.handle = s.value

    def sync(self):
        call("slhip_stream_sync", self.handle)

    def __del__(self):
        try:
            if self.handle and _lib is not None:
                _lib.slhip_stream_destroy(self.handle)
        except Exception:
            pass


class Graph:
    """Launches recorded once on a stream (slhip_graph_begin/end), replayed with launch()."""

    def __init__(self, stream: "Stream", record):
        call("slhip_graph_begin", stream.handle)
        try:
            record()
        finally:
            g = _P(0)
            st = lib().slhip_graph_end(stream.handle, ctypes.byref(g))
        check(st)
        self.handle = g.value

    def launch(self, stream: "Stream"):
        call("slhip_graph_launch", self.handle, stream.handle)

    def __del__(self):
        try:
            if self.handle and _lib is not None:
                _lib.slhip_graph_destroy(self.handle)
        except Exception:
            pass


# ---- ops (device pointers in, nothing synchronous) -------------------------------------------------

def rownorm(kind, dtype_in, dtype_out, x, y, rows, D, *, res=None, w=None, b=None, h_out=None, eps=1e-6,
            x_stride=None, res_stride=None, y_stride=None, h_stride=None, y16=None, y16_stride=None, yq=None,
            yq_stride=None, stream=None):
    """slhip_rownorm; with y16 (f16 rows) or yq (E4M3 rows: D codes then D/128 f32 scales) it calls
    slhip_rownorm_copies, and y may then be None."""
    args = (NORMS.get(kind, kind), DTYPES.get(dtype_in, dtype_in), DTYPES.get(dtype_out, dtype_out),
            ptr(x), ptr(res), ptr(w), ptr(b), ptr(y), ptr(h_out), rows, D,
            D if x_stride is None else x_stride, D if res_stride is None else res_stride,
            D if y_stride is None else y_stride, D if h_stride is None else h_stride, eps)
    if y16 is None and yq is None:
        call("slhip_rownorm", *args, stream)
        return
    copies = NormCopies(ptr(y16), D if y16_stride is None else y16_stride, ptr(yq),
                        D + D // 32 if yq_stride is None else yq_stride)
    call("slhip_rownorm_copies", *args, ctypes.byref(copies), stream)


def matvec(fmt, dtype_x, dtype_y, x, T, K, w, N, y, *, x_stride=None, y_stride=None, stream=None):
    """y [T, N] = x [T, K] . W^T, W = N rows of K weights in ``fmt``."""
    call("slhip_matvec", FORMATS.get(fmt, fmt), DTYPES.get(dtype_x, dtype_x), DTYPES.get(dtype_y, dtype_y), ptr(x),
         K if x_stride is None else x_stride, T, K, ptr(w), N, ptr(y), N if y_stride is None else y_stride, stream)


def matvec_bias(fmt, dtype_x, dtype_y, x, T, K, w, N, bias, y, *, x_stride=None, y_stride=None, stream=None):
    """y [T, N] = x [T, K] . W^T + bias[N] (one launch)."""
    call("slhip_matvec_bias", FORMATS.get(fmt, fmt), DTYPES.get(dtype_x, dtype_x), DTYPES.get(dtype_y, dtype_y),
         ptr(x), K if x_stride is None else x_stride, T, K, ptr(w), N, ptr(bias), ptr(y),
         N if y_stride is None else y_stride, stream)


def dual_matvec(act, fmt, dtype_x, dtype_y, x, T, K, w_gate, w_up, N, y, *, x_stride=None, y_stride=None,
                stream=None):
    """y [T, N] = act(x . Wg^T) * (x . Wu^T)."""
    call("slhip_dual_matvec", ACTS.get(act, act), FORMATS.get(fmt, fmt), DTYPES.get(dtype_x, dtype_x),
         DTYPES.get(dtype_y, dtype_y), ptr(x), K if x_stride is None else x_stride, T, K, ptr(w_gate), ptr(w_up), N,
         ptr(y), N if y_stride is None else y_stride, stream)


def ew_program(inputs, ops, outputs, rows, cols, *, head=None, tail=None, stream=None):
    """A fused elementwise group (slhip_ew_program_run). inputs: [(ptr, dtype, mode)]; ops: [(kind, op, a, b,
    round dtype, p0, p1)] with kind "binary"/"unary" and op a BINARY_OPS / UNARY_OPS name; outputs:
    [(ptr, dtype, reg)]; head / tail: dict(kind="rms"|"l2", reg, w, eps, y, dtype_y)."""
    p = EwProgram()
    p.n_inputs, p.n_ops, p.n_outputs = len(inputs), len(ops), len(outputs)
    for i, (d, dt, mode) in enumerate(inputs):
        p.inputs[i] = EwInput(ptr(d), DTYPES.get(dt, dt), mode)
    for k, (kind, op, a, b, dst, rnd, p0, p1) in enumerate(ops):
        code = BINARY_OPS[op] if kind == "binary" else UNARY_OPS[op]
        p.ops[k] = EwOp(EWK_BINARY if kind == "binary" else EWK_UNARY, code, a, b, dst, DTYPES.get(rnd, rnd), p0, p1)
    for j, (d, dt, reg) in enumerate(outputs):
        p.outputs[j] = EwOutput(ptr(d), DTYPES.get(dt, dt), reg)
    for name, nm in (("head", head), ("tail", tail)):
        if nm:
            setattr(p, name, EwNorm(EW_NORMS[nm["kind"]], nm["reg"], ptr(nm.get("w")), nm.get("eps", 1e-6),
                                    ptr(nm.get("y")), DTYPES.get(nm.get("dtype_y", "f32"), nm.get("dtype_y", "f32"))))
    call("slhip_ew_program_run", ctypes.byref(p), rows, cols, stream)


def q8_row_bytes(K) -> int:
    """Bytes of one quantized activation row of K values (slhip_quantize_q8's layout)."""
    return int(lib().slhip_q8_row_bytes(K))


def quantize_q8(dtype_x, x, T, K, xq, *, x_stride=None, stream=None):
    """x [T, K] (f32 / bf16) -> the int-dot matvec's quantized rows at xq ([T, q8_row_bytes(K)] bytes)."""
    call("slhip_quantize_q8", DTYPES.get(dtype_x, dtype_x), ptr(x), K if x_stride is None else x_stride, T, K,
         ptr(xq), stream)


def matvec_q8(fmt, dtype_y, xq, T, K, w, N, y, *, y_stride=None, bias=None, stream=None):
    """y [T, N] = x . W^T + bias on the quantized rows xq (integer dots)."""
    call("slhip_matvec_q8", FORMATS.get(fmt, fmt), DTYPES.get(dtype_y, dtype_y), ptr(xq), T, K, ptr(w), N, ptr(y),
         N if y_stride is None else y_stride, ptr(bias), stream)


def dual_matvec_q8(act, fmt, dtype_y, xq, T, K, w_gate, w_up, N, y, *, y_stride=None, stream=None):
    """y [T, N] = act(x . Wg^T) * (x . Wu^T) on the quantized rows xq (integer dots)."""
    call("slhip_dual_matvec_q8", ACTS.get(act, act), FORMATS.get(fmt, fmt), DTYPES.get(dtype_y, dtype_y), ptr(xq), T,
         K, ptr(w_gate), ptr(w_up), N, ptr(y), N if y_stride is None else y_stride, stream)


def dual_matvec_int8(act, fmt, dtype_x, dtype_y, x, T, K, w_gate, w_up, N, y, work, work_bytes, *, x_stride=None,
                     y_stride=None, stream=None):
    """x -> q8 in `work`, then y = act(x . Wg^T) * (x . Wu^T) on integer dots (one call, two launches)."""
    call("slhip_dual_matvec_int8", ACTS.get(act, act), FORMATS.get(fmt, fmt), DTYPES.get(dtype_x, dtype_x),
         DTYPES.get(dtype_y, dtype_y), ptr(x), K if x_stride is None else x_stride, T, K, ptr(w_gate), ptr(w_up), N,
         ptr(y), N if y_stride is None else y_stride, ptr(work), work_bytes, stream)


def dual_matvec_int8_noalloc(act, fmt, dtype_x, dtype_y, x, T, K, w_gate, w_up, N, y, *, x_stride=None,
                             y_stride=None, stream=None):
    """dual_matvec_int8 on the library's static per-device workspace (allocates nothing)."""
    call("slhip_dual_matvec_int8_noalloc", ACTS.get(act, act), FORMATS.get(fmt, fmt), DTYPES.get(dtype_x, dtype_x),
         DTYPES.get(dtype_y, dtype_y), ptr(x), K if x_stride is None else x_stride, T, K, ptr(w_gate), ptr(w_up), N,
         ptr(y), N if y_stride is None else y_stride, stream)


def gated_act(act, dtype_in, dtype_out, gate, up, out, rows, cols, *, gate_stride=None, up_stride=None,
              out_stride=None, stream=None):
    call("slhip_gated_act", ACTS.get(act, act), DTYPES.get(dtype_in, dtype_in), DTYPES.get(dtype_out, dtype_out),
         ptr(gate), ptr(up), ptr(out), rows, cols, cols if gate_stride is None else gate_stride,
         cols if up_stride is None else up_stride, cols if out_stride is None else out_stride, stream)


def binary(op, dtype_a, dtype_b, dtype_out, a, b, y, dims, *, a_strides=None, b_strides=None, stream=None):
    """y [dims] = op(a, b); a_strides / b_strides: element strides aligned to y's rank (0 where broadcast),
    None for dense [dims]."""
    rank = len(dims)
    arr = lambda v: None if v is None else (_I64 * max(rank, 1))(*v) if rank else (_I64 * 1)(0)
    call("slhip_binary", BINARY_OPS.get(op, op), DTYPES.get(dtype_a, dtype_a), DTYPES.get(dtype_b, dtype_b),
         DTYPES.get(dtype_out, dtype_out), ptr(a), arr(a_strides), ptr(b), arr(b_strides), ptr(y),
         (_I64 * max(rank, 1))(*dims) if rank else None, rank, stream)


def unary(op, dtype_in, dtype_out, x, y, rows, cols, *, x_stride=None, y_stride=None, p0=1.0, p1=0.0, stream=None):
    """y [rows, cols] = op(x) with the reference's two unary parameters p0, p1."""
    call("slhip_unary", UNARY_OPS.get(op, op), DTYPES.get(dtype_in, dtype_in), DTYPES.get(dtype_out, dtype_out),
         ptr(x), ptr(y), rows, cols, cols if x_stride is None else x_stride, cols if y_stride is None else y_stride,
         p0, p1, stream)


def rope(dtype_in, dtype_out, tensors, pos, T, D, *, dims=0, neox=True, base=10000.0, freq_scale=1.0,
         attn_factor=1.0, norm=False, eps=1e-6, ff=None, pos_axes=1, sections=None, interleaved=False,
         per_element=False, stream=None):
    """tensors: list of dicts with x, y, heads and optional norm_w / strides (elements) / rows (a CacheRows:
    y is then a KV cache [ctx, heads, D] written at those rows)."""
    arr = (RopeTensor * len(tensors))()
    for i, t in enumerate(tensors):
        H = t["heads"]
        rows = t.get("rows")
        arr[i] = RopeTensor(ptr(t["x"]), ptr(t["y"]), ptr(t.get("norm_w")), H,
                            t.get("x_stride_t", H * D), t.get("x_stride_h", D),
                            t.get("y_stride_t", H * D), t.get("y_stride_h", D),
                            ctypes.pointer(rows) if rows is not None else None)
    cfg = RopeCfg(dims, 1 if neox else 0, base, freq_scale, attn_factor, 1 if norm else 0, eps, pos_axes,
                  (ctypes.c_int32 * 4)(*(sections or (0, 0, 0, 0))), 1 if interleaved else 0, 1 if per_element else 0)
    call("slhip_rope", DTYPES.get(dtype_in, dtype_in), DTYPES.get(dtype_out, dtype_out), arr, len(tensors),
         ptr(pos), ptr(ff), T, D, ctypes.byref(cfg), stream)


def cache_write(dtype_in, dtype_cache, x, T, inner, cache, rows: CacheRows, *, x_stride=None, stream=None):
    call("slhip_cache_write", DTYPES.get(dtype_in, dtype_in), DTYPES.get(dtype_cache, dtype_cache), ptr(x),
         inner if x_stride is None else x_stride, T, inner, ptr(cache), ctypes.byref(rows), stream)


def gather(fmt, table, V, D, ids, N, dtype_out, y, *, y_stride=None, stream=None):
    call("slhip_gather", FORMATS.get(fmt, fmt), ptr(table), V, D, ptr(ids), N, DTYPES.get(dtype_out, dtype_out),
         ptr(y), D if y_stride is None else y_stride, stream)


def convert(dtype_in, dtype_out, x, y, n, stream=None):
    call("slhip_convert", DTYPES.get(dtype_in, dtype_in), DTYPES.get(dtype_out, dtype_out), ptr(x), ptr(y), n,
         stream)
