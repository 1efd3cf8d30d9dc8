"""Host-side face of the Sharplight HIP execution provider, over libsharplight_hip's provider C ABI.

Mirrors the reference's provider contracts for this path -- ``IExecutionProvider``
(src/Sharplight.Core/Runtime/IExecutionProvider.cs:25-74), ``IComputeDevice`` (IComputeDevice.cs:6-67) and
``ICompiledSegment`` (ICompiledSegment.cs:6-25) -- with the same names, argument meaning and error behaviour:
``check_availability`` never raises, ``get_devices`` is empty when unavailable, ``open_device`` raises
``ValueError`` for another provider's device and ``NotImplementedError`` when unavailable, ``supports``
answers per node, ``compile`` raises ``NotImplementedError`` for what it cannot run, ``execute`` rejects a
token count beyond the compiled bound. The lowering and fusion live in C++ (csrc/provider.hip); this module
only builds the segment text and moves bytes.

``GraphBuilder`` plays the part of the reference's GraphBuilder (src/Sharplight.Core/Graph/GraphBuilder.cs)
for the ops on this path, so graph-level tests read like the reference's NormTests / FusionTests.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, field

import numpy as np

from . import native

NP = {"f32": np.float32, "f16": np.float16, "bf16": np.uint16, "i32": np.int32}
BLOCKS = {"q8_0": (32, 34), "q4_0": (32, 18), "q4_1": (32, 20), "q5_0": (32, 22), "q5_1": (32, 24),
          "q2_k": (256, 84), "q3_k": (256, 110), "q4_k": (256, 144), "q5_k": (256, 176), "q6_k": (256, 210),
          "iq4_nl": (32, 18), "iq4_xs": (256, 136), "tq1_0": (256, 54), "tq2_0": (256, 66), "mxfp4": (32, 17),
          "nvfp4": (64, 36), "iq2_xxs": (256, 66), "iq2_xs": (256, 74), "iq2_s": (256, 82), "iq3_xxs": (256, 98),
          "iq3_s": (256, 110), "iq1_s": (256, 50), "iq1_m": (256, 56),
          "q1_0": (128, 18), "q2_0": (64, 18), "q2_0_g128": (128, 34), "tern1_g128": (128, 28), "nvfp4_gs": (64, 40),
          "q4z_g32": (32, 20), "q4z_g128": (128, 68), "q8z_g32": (32, 36), "q8z_g128": (128, 132), "nf4_b64": (64, 36),
          "fp4_b64": (64, 36), "q8a_g32": (32, 36), "q2s_g128": (128, 36), "f8e4m3": (1, 1), "f8e5m2": (1, 1),
          "f8e4m3_b32": (32, 36), "f8e4m3_b128": (128, 132), "trellis_v4k8_g128": (128, 34),
          "trellis_v4k6_g128": (128, 26), "trellis_v4k7_g128": (128, 30), "trellis_v2k5_g128": (128, 42),
          "trellis_v2k6_g128": (128, 50), "trellis_v2k7_g128": (128, 58)}
ELEM_BYTES = {"f32": 4, "f16": 2, "bf16": 2, "i32": 4}


@dataclass(frozen=True)
class Value:
    id: int
    type: str
    dims: tuple  # ints, or "T" for the symbolic token count

    def shape(self, T: int) -> tuple:
        return tuple(T if d == "T" else d for d in self.dims)

    def nbytes(self, T: int) -> int:
        n = int(np.prod(self.shape(T), dtype=np.int64)) if self.dims else 1
        if self.type in BLOCKS:
            bs, bb = BLOCKS[self.type]
            return n // bs * bb
        return n * ELEM_BYTES[self.type]


@dataclass
class Node:
    op: str
    inputs: list
    outputs: list
    attrs: dict = field(default_factory=dict)


class GraphBuilder:
    """Builds a graph segment for the provider (values, nodes, inputs, weights, outputs)."""

    def __init__(self):
        self.values: list[Value] = []
        self.nodes: list[Node] = []
        self.inputs: list[Value] = []
        self.weights: list[Value] = []
        self.outputs: list[Value] = []
        self.states: list[Value] = []
        # compile options: reduced_precision (CompileOptions.AllowReducedPrecision) and int_dot
        # ("lowerer" | "cpu" | "off": which rule picks the integer-dot matvec)
        self.options: dict = {}

    def value(self, type: str, *dims) -> Value:
        v = Value(len(self.values), type, tuple(dims))
        self.values.append(v)
        return v

    def input(self, type: str, *dims) -> Value:
        v = self.value(type, *dims)
        self.inputs.append(v)
        return v

    def weight(self, type: str, *dims) -> Value:
        v = self.value(type, *dims)
        self.weights.append(v)
        return v

    def state(self, type: str, *dims) -> Value:
        """A state (KV cache): fixed dims, persistent across runs, zero until written."""
        v = self.value(type, *dims)
        self.states.append(v)
        return v

    def output(self, v: Value) -> Value:
        self.outputs.append(v)
        return v

    def emit(self, op: str, inputs, out_type: str, out_dims, **attrs) -> Value:
        y = self.value(out_type, *out_dims)
        self.nodes.append(Node(op, [v for v in inputs if v is not None], [y], attrs))
        return y

    # the ops on this path (StandardOps names)
    def binary(self, op, a, b, out_type=None, **attrs):
        """A StandardOps binary op with numpy broadcasting (the symbolic "T" broadcasts against T or 1)."""
        return self.emit(op, [a, b], out_type or a.type, broadcast(a.dims, b.dims), **attrs)

    def unary(self, op, x, out_type=None, **attrs):
        return self.emit(op, [x], out_type or x.type, x.dims, **attrs)

    def add(self, a, b):
        return self.binary("Add", a, b)

    def mul(self, a, b):
        return self.binary("Mul", a, b)

    def scale(self, x, scale=1.0, bias=0.0):
        return self.unary("Scale", x, scale=scale, bias=bias)

    def clip(self, x, min=float("-inf"), max=float("inf")):
        return self.unary("Clip", x, min=min, max=max)

    def silu(self, x):
        return self.emit("Silu", [x], x.type, x.dims)

    def gelu_tanh(self, x):
        return self.emit("GeluTanh", [x], x.type, x.dims)

    def gelu(self, x):
        return self.emit("Gelu", [x], x.type, x.dims)

    def rms_norm(self, x, w=None, eps=1e-6, out_type=None):
        return self.emit("RmsNorm", [x, w], out_type or x.type, x.dims, eps=eps)

    def l2_norm(self, x, eps=1e-6, out_type=None):
        return self.emit("L2Norm", [x], out_type or x.type, x.dims, eps=eps)

    def layer_norm(self, x, w=None, b=None, eps=1e-5, out_type=None):
        if b is not None and w is None:
            raise ValueError("LayerNorm bias without weight")
        return self.emit("LayerNorm", [x, w, b], out_type or x.type, x.dims, eps=eps)

    def rope(self, x, pos, ff=None, dims=0, base=10000.0, style="neox", freq_scale=1.0, attn_factor=1.0,
             out_type=None, sections=None, interleaved=False, sections_per_element=False):
        """StandardOps.Rope; pos i32 [T] or [T, A] (multi-axis, with `sections` of four entries)."""
        attrs = dict(dims=dims, base=base, style=style, freq_scale=freq_scale, attn_factor=attn_factor)
        if sections is not None:
            attrs["sections"] = ",".join(str(int(v)) for v in sections)
        if interleaved:
            attrs["interleaved"] = "true"
        if sections_per_element:
            attrs["sections_per_element"] = "true"
        return self.emit("Rope", [x, pos, ff], out_type or x.type, x.dims, **attrs)

    def gather(self, table, ids, out_type="f32"):
        d = table.dims[1:]
        return self.emit("Gather", [table, ids], out_type, (ids.dims[0],) + tuple(d))

    def matmul(self, x, w, out_type="f32", f32_activations=None):
        """StandardOps.MatMul: x [.., K] . W^T, W a weight [N, K] -> [.., N]; f32_activations=True keeps x
        unquantized (StandardOps.F32ActivationsAttribute, src/Sharplight.Core/Graph/StandardOps.cs:135)."""
        attrs = {} if f32_activations is None else {"f32_activations": f32_activations}
        return self.emit("MatMul", [x, w], out_type, tuple(x.dims[:-1]) + (w.dims[0],), **attrs)

    def cast(self, x, to: str):
        return self.emit("Cast", [x], to, x.dims)

    def cache_write(self, state, x, rows=None, pages=None, offset="n_past", slots=None, block_size=None):
        """GraphBuilder.CacheWrite (src/Sharplight.Core/Graph/GraphBuilder.cs:330-336), with the inputs and
        attributes the multi-sequence / paged rewrite adds (MultiSequence.cs:201-233)."""
        attrs = {"offset": offset}
        if slots is not None:
            attrs["slots"] = slots
        if block_size is not None:
            attrs["block_size"] = block_size
        self.nodes.append(Node("CacheWrite", [v for v in (state, x, rows, pages) if v is not None], [], attrs))

    def to_ir(self) -> str:
        lines = [f"option {k}={_fmt(v)}" for k, v in self.options.items()]
        for v in self.values:
            lines.append(f"value {v.id} {v.type} " + " ".join(str(d) for d in v.dims))
        for v in self.inputs:
            lines.append(f"input {v.id}")
        for v in self.weights:
            lines.append(f"weight {v.id}")
        for v in self.outputs:
            lines.append(f"output {v.id}")
        for v in self.states:
            lines.append(f"state {v.id}")
        for n in self.nodes:
            attrs = " ".join(f"{k}={_fmt(v)}" for k, v in n.attrs.items())
            lines.append(f"node {n.op} {','.join(str(v.id) for v in n.inputs) or '-'} -> "
                         f"{','.join(str(v.id) for v in n.outputs) or '-'} {attrs}".rstrip())
        return "\n".join(lines) + "\n"


def broadcast(a: tuple, b: tuple) -> tuple:
    """numpy broadcasting of two dim tuples whose entries are ints or "T"."""
    r = max(len(a), len(b))
    a = (1,) * (r - len(a)) + tuple(a)
    b = (1,) * (r - len(b)) + tuple(b)
    out = []
    for x, y in zip(a, b):
        if x == y or y == 1:
            out.append(x)
        elif x == 1:
            out.append(y)
        else:
            raise ValueError(f"shapes {a} and {b} do not broadcast")
    return tuple(out)


def plan(graph: "GraphBuilder") -> list[str]:
    """The launches compile() would create for ``graph``, decided without a device (slhip_segment_plan)."""
    buf = ctypes.create_string_buffer(8192)
    native.call("slhip_segment_plan", graph.to_ir().encode(), buf, len(buf))
    return [s for s in buf.value.decode().split("\n") if s]


def describe(text: str) -> str:
    """The segment text as the provider parsed it, in canonical form (slhip_segment_describe)."""
    buf = ctypes.create_string_buffer(1 << 16)
    native.call("slhip_segment_describe", text.encode(), buf, len(buf))
    return buf.value.decode()


def _fmt(v) -> str:
    """An attribute value as segment text: floats round-trip (repr), booleans true/false, lists comma-joined."""
    if isinstance(v, bool):
        return "true" if v else "false"
    if isinstance(v, float):
        return repr(float(v))
    if isinstance(v, (list, tuple)):
        return ",".join(_fmt(x) for x in v)
    s = str(v)
    if not s or any(c.isspace() for c in s):
        raise ValueError(f"attribute value {v!r} cannot be written as one token")
    return s


@dataclass(frozen=True)
class ProviderAvailability:
    """ProviderAvailability (src/Sharplight.Core/Runtime/ProviderAvailability.cs)."""
    is_available: bool
    reason: str = ""


@dataclass(frozen=True)
class DeviceInfo:
    """DeviceInfo (src/Sharplight.Core/Runtime/DeviceInfo.cs:4-50) for a HIP device."""
    provider: str
    index: int
    name: str
    kind: str
    total_memory: int
    vendor: str
    driver: str
    uuid: str
    features: tuple
    concurrent_workgroups: int


@dataclass(frozen=True)
class OpSupport:
    is_supported: bool
    reason: str = ""


class HipExecutionProvider:
    """IExecutionProvider for HIP devices. Cheap to construct; touches the runtime only in
    check_availability / get_devices (IExecutionProvider.cs:3-6)."""

    name = "hip"
    portable_code_format = None  # kernels are prebuilt code objects: no portable stage

    def check_availability(self) -> ProviderAvailability:
        try:
            buf = ctypes.create_string_buffer(512)
            st = native.lib().slhip_provider_check(buf, len(buf))
        except Exception as e:  # a missing or unloadable library means "unavailable", never an exception
            return ProviderAvailability(False, str(e))
        return ProviderAvailability(st == native.OK, "" if st == native.OK else buf.value.decode())

    def get_devices(self) -> list[DeviceInfo]:
        if not self.check_availability().is_available:
            return []
        out = []
        for i in range(native.device_count()):
            p = native.device_props(i)
            if not p.arch.decode().startswith("gfx950"):
                continue  # the library's code objects are gfx950 only
            out.append(DeviceInfo(self.name, i, p.name.decode() or p.arch.decode(), "DiscreteGpu", p.total_memory,
                                  "AMD", "HIP", f"{p.pci_domain:04x}:{p.pci_bus:02x}:{p.pci_device:02x}",
                                  ("bf16", "f16", "subgroup_ops"), p.compute_units))
        return out

    def open_device(self, device: DeviceInfo, options=None) -> "HipDevice":
        if device.provider != self.name:
            raise ValueError(f"Device of provider '{device.provider}' cannot be opened by '{self.name}'.")
        avail = self.check_availability()
        if not avail.is_available:
            raise NotImplementedError(f"The HIP provider is unavailable: {avail.reason}")
        return HipDevice(device)

    def can_compile_for(self, profile) -> bool:
        return False


class HipDevice:
    """IComputeDevice: supports() per node, compile() a segment; close() releases it."""

    def __init__(self, info: DeviceInfo):
        self.info = info
        native.set_device(info.index)

    @property
    def available_memory(self) -> int:
        free = ctypes.c_size_t(0)
        native.call("slhip_mem_info", ctypes.byref(free), None)
        return free.value

    def supports(self, graph: GraphBuilder, node_index: int) -> OpSupport:
        ok = ctypes.c_int(0)
        buf = ctypes.create_string_buffer(512)
        native.call("slhip_node_supports", graph.to_ir().encode(), node_index, ctypes.byref(ok), buf, len(buf))
        return OpSupport(bool(ok.value), buf.value.decode())

    def compile(self, graph: GraphBuilder, max_tokens: int = 512) -> "CompiledSegment":
        native.set_device(self.info.index)
        seg = ctypes.c_void_p(0)
        native.call("slhip_segment_compile", graph.to_ir().encode(), max_tokens, ctypes.byref(seg))
        return CompiledSegment(seg.value, graph)

    def close(self):
        pass


class CompiledSegment:
    """ICompiledSegment: set_input, execute (asynchronous until an output is read), get_output."""

    def __init__(self, handle: int, graph: GraphBuilder):
        self.handle = handle
        self.graph = graph
        self.tokens = 0

    def set_input(self, value: Value, data: np.ndarray) -> None:
        data = np.ascontiguousarray(data)
        native.call("slhip_segment_set_input", self.handle, value.id, data.ctypes.data, data.nbytes)

    def execute(self, T: int) -> None:
        native.call("slhip_segment_execute", self.handle, T)
        self.tokens = T

    def get_output(self, value: Value) -> np.ndarray:
        shape = value.shape(self.tokens)
        if value.type in NP:
            out = np.empty(shape, NP[value.type])
        else:
            out = np.empty(value.nbytes(self.tokens), np.uint8)
        native.call("slhip_segment_get_output", self.handle, value.id, out.ctypes.data, out.nbytes)
        return out

    def reset_state(self) -> None:
        native.call("slhip_segment_reset_state", self.handle)

    def set_scalar(self, name: str, value: int) -> None:
        """A runtime scalar of the next runs (RunParameters.Scalars), e.g. n_past."""
        native.call("slhip_segment_set_scalar", self.handle, name.encode(), int(value))

    @property
    def device_memory_bytes(self) -> int:
        n = ctypes.c_int64(0)
        native.call("slhip_segment_device_bytes", self.handle, ctypes.byref(n))
        return n.value

    @property
    def launches(self) -> list[str]:
        buf = ctypes.create_string_buffer(8192)
        native.call("slhip_segment_launches", self.handle, buf, len(buf))
        return [s for s in buf.value.decode().split("\n") if s]

    def launches_at(self, tokens: int) -> list[str]:
        """The launches a run of ``tokens`` tokens makes (each matvec with the path it takes)."""
        buf = ctypes.create_string_buffer(8192)
        native.call("slhip_segment_launches_at", self.handle, tokens, buf, len(buf))
        return [s for s in buf.value.decode().split("\n") if s]

    def close(self) -> None:
        if self.handle:
            native.call("slhip_segment_destroy", self.handle)
            self.handle = 0

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            if self.handle and native._lib is not None:
                native._lib.slhip_segment_destroy(self.handle)
        except Exception:
            pass
