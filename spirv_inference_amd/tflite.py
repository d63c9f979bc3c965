"""TFLite front end: load a `.tflite` FlatBuffer and run it on the device kernels.

Counterpart of the reference's tflite_loader crate (source/tflite_loader/src):
* `parse_model` / `load_model` read the fields model.rs:255-363 reads (version, description,
  operator codes, the first subgraph's tensors / inputs / outputs / operators, buffers) and
  flag unsupported operators and quantized tensors the same way (model.rs:152-206, 334-350);
* `decode_options` decodes the builtin options op_decoder.rs decodes, with its defaults;
* `topological_order` keeps the ready-order rule of scheduler.rs:1454-1500;
* `validate_supported_graph` is graph.rs:5-34;
* `TfliteExecutor` replaces scheduler.rs:run_graph (29-1082): instead of one host round trip
  per operator, every tensor stays resident on the device in the model's own NHWC layout,
  weights are packed and uploaded once, and each operator is one registry launch (the
  reference's kernel names and push vectors, NHWC-native variants for Conv2D / Depthwise).
  Fused activations go into the producing kernel's epilogue (scheduler.rs:1146-1197 runs
  them as separate dispatches).

`TfliteWriter` builds TFL3 FlatBuffers with the same fields (the reference's fixture
generators, fixtures/make_synthetic_logistic_tflite.py:20-83, need the `flatbuffers`
package, which is not installed here).

Deviations kept on purpose, each documented where it happens: ResizeBilinear options are read
at the schema's field ids 2 and 3 (op_decoder.rs reads ids 0 and 1, which the schema marks as
the deprecated new_height / new_width); Softmax ignores beta as the reference does
(scheduler.rs:277-320 dispatches softmax10 / softmax1000, which have no beta).
"""
from __future__ import annotations

import dataclasses
import hashlib
import struct
from collections import OrderedDict
from typing import Dict, List, Optional, Tuple

import numpy as np

# ---- schema constants (schema.fbs) -------------------------------------------------------
TENSOR_TYPES = {0: "Float32", 2: "Int32", 3: "UInt8", 4: "Int64", 5: "String", 6: "Bool",
                7: "Int16", 8: "Complex64", 9: "Int8", 10: "Float16", 11: "Float64"}

# BuiltinOperator codes the reference recognises (model.rs:81-149), by schema name.
BUILTIN_NAMES = {
    0: "ADD", 1: "AVERAGE_POOL_2D", 2: "CONCATENATION", 3: "CONV_2D", 4: "DEPTHWISE_CONV_2D",
    7: "EMBEDDING_LOOKUP", 9: "FULLY_CONNECTED", 11: "L2_NORMALIZATION", 14: "LOGISTIC",
    17: "MAX_POOL_2D", 18: "MUL", 21: "RELU6", 22: "RESHAPE", 23: "RESIZE_BILINEAR",
    25: "SOFTMAX", 28: "TANH", 34: "PAD", 36: "GATHER", 39: "TRANSPOSE", 40: "MEAN", 41: "SUB",
    42: "DIV", 43: "SQUEEZE", 47: "EXP", 48: "TOPK_V2", 49: "SPLIT", 53: "CAST", 55: "MAXIMUM",
    56: "ARG_MAX", 57: "MINIMUM", 59: "NEG", 65: "SLICE", 67: "TRANSPOSE_CONV", 69: "TILE",
    70: "EXPAND_DIMS", 73: "LOG", 74: "SUM", 75: "SQRT", 76: "RSQRT", 78: "POW",
    82: "REDUCE_MAX", 83: "PACK", 88: "UNPACK", 97: "RESIZE_NEAREST_NEIGHBOR",
    98: "LEAKY_RELU", 101: "ABS", 126: "BATCH_MATMUL", 150: "GELU"}
BUILTIN_CODES = {v: k for k, v in BUILTIN_NAMES.items()}
CUSTOM_CODES = (32, 32768)
# Every recognised builtin is "supported" by the parser (model.rs:152-206); the scheduler
# lowers a subset and rejects the rest at run time (scheduler.rs:1003-1007).
SUPPORTED = frozenset(BUILTIN_NAMES.values())

# BuiltinOptions union indices (schema.fbs `union BuiltinOptions`, NONE = 0).
OPTIONS_TYPE = {"Conv2DOptions": 1, "DepthwiseConv2DOptions": 2, "Pool2DOptions": 5,
                "FullyConnectedOptions": 8, "SoftmaxOptions": 9, "ConcatenationOptions": 10,
                "AddOptions": 11, "L2NormOptions": 12, "ResizeBilinearOptions": 15,
                "ReshapeOptions": 17, "MulOptions": 21, "PadOptions": 22,
                "ReducerOptions": 27, "SubOptions": 28, "DivOptions": 29,
                "SqueezeOptions": 30, "ResizeNearestNeighborOptions": 74,
                "LeakyReluOptions": 75}
PADDING = {0: "same", 1: "valid"}
ACTIVATION = {0: "none", 1: "relu", 2: "relu_n1_to_1", 3: "relu6", 4: "tanh", 5: "sign_bit"}


# ---- FlatBuffer reading --------------------------------------------------------------------
class _Table:
    """A FlatBuffer table at byte position `pos` of `buf` (model.rs:365-540)."""

    def __init__(self, buf: bytes, pos: int):
        self.buf, self.pos = buf, pos
        self._check(pos, 4)
        self.vt = pos - struct.unpack_from("<i", buf, pos)[0]
        self._check(self.vt, 4)
        self.vt_len = struct.unpack_from("<H", buf, self.vt)[0]

    def _check(self, at: int, n: int) -> None:
        if at < 0 or at + n > len(self.buf):
            raise ValueError(f"FlatBuffer access [{at}, {at + n}) outside {len(self.buf)} bytes")

    def field(self, fid: int) -> Optional[int]:
        slot = 4 + 2 * fid
        if slot + 2 > self.vt_len:
            return None
        off = struct.unpack_from("<H", self.buf, self.vt + slot)[0]
        return self.pos + off if off else None

    def _scalar(self, fid: int, fmt: str):
        at = self.field(fid)
        if at is None:
            return None
        self._check(at, struct.calcsize(fmt))
        return struct.unpack_from("<" + fmt, self.buf, at)[0]

    def i8(self, fid):
        return self._scalar(fid, "b")

    def u8(self, fid):
        return self._scalar(fid, "B")

    def i32(self, fid):
        return self._scalar(fid, "i")

    def u32(self, fid):
        return self._scalar(fid, "I")

    def f32(self, fid):
        return self._scalar(fid, "f")

    def bool(self, fid):
        v = self._scalar(fid, "B")
        return None if v is None else v != 0

    def _ref(self, fid: int) -> Optional[int]:
        at = self.field(fid)
        if at is None:
            return None
        self._check(at, 4)
        return at + struct.unpack_from("<I", self.buf, at)[0]

    def _vector(self, fid: int) -> Optional[Tuple[int, int]]:
        at = self._ref(fid)
        if at is None:
            return None
        self._check(at, 4)
        return at + 4, struct.unpack_from("<I", self.buf, at)[0]

    def string(self, fid) -> Optional[str]:
        v = self._vector(fid)
        if v is None:
            return None
        self._check(v[0], v[1])
        return self.buf[v[0]:v[0] + v[1]].decode("utf-8", "replace")

    def vector_i32(self, fid) -> Optional[List[int]]:
        v = self._vector(fid)
        if v is None:
            return None
        self._check(v[0], 4 * v[1])
        return list(struct.unpack_from(f"<{v[1]}i", self.buf, v[0]))

    def vector_u8(self, fid) -> Optional[Tuple[int, bytes]]:
        v = self._vector(fid)
        if v is None:
            return None
        self._check(v[0], v[1])
        return v[0], bytes(self.buf[v[0]:v[0] + v[1]])

    def table(self, fid) -> Optional["_Table"]:
        at = self._ref(fid)
        return None if at is None else _Table(self.buf, at)

    def vector_tables(self, fid) -> List["_Table"]:
        v = self._vector(fid)
        if v is None:
            return []
        self._check(v[0], 4 * v[1])
        out = []
        for i in range(v[1]):
            at = v[0] + 4 * i
            out.append(_Table(self.buf, at + struct.unpack_from("<I", self.buf, at)[0]))
        return out


@dataclasses.dataclass
class Tensor:
    index: int
    name: str
    shape: List[int]
    tensor_type: str
    buffer: int


@dataclasses.dataclass
class Operator:
    index: int
    opcode_index: int
    builtin: str            # schema name, "CUSTOM:<code>" or "UNKNOWN_<n>"
    code: int
    inputs: List[int]
    outputs: List[int]
    options_type: Optional[int]
    options: Optional[_Table] = dataclasses.field(repr=False, default=None)


@dataclasses.dataclass
class Buffer:
    index: int
    data_offset: Optional[int]
    data: bytes = dataclasses.field(repr=False)

    @property
    def sha256(self) -> str:
        return hashlib.sha256(self.data).hexdigest()


@dataclasses.dataclass
class TfliteModel:
    path: str
    nbytes: int
    version: int
    description: Optional[str]
    tensors: List[Tensor]
    inputs: List[int]
    outputs: List[int]
    operators: List[Operator]
    buffers: List[Buffer]
    op_histogram: Dict[str, int]
    unsupported_ops: List[str]
    quantized_tensors: List[str]

    def summary(self) -> dict:
        """The `model` section of the report (the serialised ModelInfo of model.rs:238-253)."""
        return {
            "path": self.path, "bytes": self.nbytes, "version": self.version,
            "description": self.description,
            "tensors": [dataclasses.asdict(t) for t in self.tensors],
            "inputs": self.inputs, "outputs": self.outputs,
            "operators": [{"index": o.index, "opcode_index": o.opcode_index,
                           "builtin": o.builtin, "inputs": o.inputs, "outputs": o.outputs,
                           "builtin_options_type": o.options_type,
                           "builtin_options_table_pos": o.options.pos if o.options else None}
                          for o in self.operators],
            "buffers": [{"index": b.index, "data_offset": b.data_offset,
                         "data_len": len(b.data), "data_sha256": b.sha256}
                        for b in self.buffers],
            "op_histogram": dict(sorted(self.op_histogram.items())),
            "unsupported_ops": self.unsupported_ops,
            "quantized_tensors": self.quantized_tensors,
        }


def _builtin_name(code: int, custom: Optional[str]) -> str:
    if code in CUSTOM_CODES:
        return "CUSTOM:" + (custom or "CUSTOM")
    return BUILTIN_NAMES.get(code, f"UNKNOWN_{code}")


def parse_model(data: bytes, path: str = "<memory>") -> TfliteModel:
    """model.rs:260-363."""
    if len(data) < 8:
        raise ValueError(f"{path} is too small to be a TFLite FlatBuffer")
    if data[4:8] != b"TFL3":
        raise ValueError(f"{path} missing TFL3 FlatBuffer identifier")
    model = _Table(data, struct.unpack_from("<I", data, 0)[0])
    opcodes = model.vector_tables(1)
    subgraphs = model.vector_tables(2)
    buffers = []
    for i, b in enumerate(model.vector_tables(4)):
        v = b.vector_u8(0)
        buffers.append(Buffer(i, v[0] if v else None, v[1] if v else b""))
    if not subgraphs:
        raise ValueError("model has no subgraphs")
    sg = subgraphs[0]
    tensors = []
    for i, t in enumerate(sg.vector_tables(0)):
        ttype = t.i8(1) or 0
        tensors.append(Tensor(i, t.string(3) or f"tensor_{i}", t.vector_i32(0) or [],
                              TENSOR_TYPES.get(ttype, f"Unknown({ttype})"), t.u32(2) or 0))
    operators = []
    for i, op in enumerate(sg.vector_tables(3)):
        oi = op.u32(0) or 0
        if oi >= len(opcodes):
            raise ValueError("opcode index out of range")
        oc = opcodes[oi]
        new_code, old_code = oc.i32(3), oc.i8(0)
        code = new_code if new_code is not None else (old_code if old_code is not None else 0)
        operators.append(Operator(i, oi, _builtin_name(code, oc.string(1)), code,
                                  op.vector_i32(1) or [], op.vector_i32(2) or [], op.u8(3),
                                  op.table(4)))
    hist: Dict[str, int] = {}
    unsupported = []
    for op in operators:
        hist[op.builtin] = hist.get(op.builtin, 0) + 1
        if op.builtin not in SUPPORTED:
            unsupported.append(f"operator {op.index}: {op.builtin}")
    quantized = [f"{t.name}:{t.tensor_type}" for t in tensors
                 if t.tensor_type not in ("Float32", "Int32")]
    return TfliteModel(path, len(data), model.i32(0) or 0, model.string(3), tensors,
                       sg.vector_i32(1) or [], sg.vector_i32(2) or [], operators, buffers, hist,
                       unsupported, quantized)


def load_model(path) -> TfliteModel:
    with open(path, "rb") as f:
        return parse_model(f.read(), str(path))


def decode_options(op: Operator) -> dict:
    """op_decoder.rs: the options of one operator, with the reference's defaults."""
    t = op.options
    if t is None:
        return {"kind": "empty"}
    act = lambda fid: ACTIVATION.get(t.i8(fid) or 0, f"unknown({t.i8(fid)})")
    pad = lambda fid: PADDING.get(t.i8(fid) or 0, f"unknown({t.i8(fid)})")
    b = op.builtin
    if b == "CONV_2D":
        return {"kind": "conv2d", "padding": pad(0), "stride_w": _d(t.i32(1), 1),
                "stride_h": _d(t.i32(2), 1), "fused_activation": act(3),
                "dilation_w_factor": _d(t.i32(4), 1), "dilation_h_factor": _d(t.i32(5), 1)}
    if b == "DEPTHWISE_CONV_2D":
        return {"kind": "depthwise_conv2d", "padding": pad(0), "stride_w": _d(t.i32(1), 1),
                "stride_h": _d(t.i32(2), 1), "depth_multiplier": _d(t.i32(3), 1),
                "fused_activation": act(4), "dilation_w_factor": _d(t.i32(5), 1),
                "dilation_h_factor": _d(t.i32(6), 1)}
    if b in ("AVERAGE_POOL_2D", "MAX_POOL_2D"):
        return {"kind": "pool2d", "padding": pad(0), "stride_w": _d(t.i32(1), 1),
                "stride_h": _d(t.i32(2), 1), "filter_w": _d(t.i32(3), 1),
                "filter_h": _d(t.i32(4), 1), "fused_activation": act(5)}
    if b in ("ADD", "MUL", "SUB", "DIV"):
        return {"kind": "elementwise", "fused_activation": act(0)}
    if b == "CONCATENATION":
        return {"kind": "concatenation", "axis": _d(t.i32(0), 0), "fused_activation": act(1)}
    if b == "FULLY_CONNECTED":
        return {"kind": "fully_connected", "fused_activation": act(0)}
    if b == "SOFTMAX":
        return {"kind": "softmax", "beta": _d(t.f32(0), 1.0)}
    if b == "RESHAPE":
        return {"kind": "reshape", "new_shape": t.vector_i32(0) or []}
    if b == "LEAKY_RELU":
        return {"kind": "leaky_relu", "alpha": _d(t.f32(0), 0.2)}
    if b == "SQUEEZE":
        return {"kind": "squeeze", "squeeze_dims": t.vector_i32(0) or []}
    if b == "RESIZE_BILINEAR":
        # schema ids 2 and 3 (ids 0 and 1 are the deprecated new_height / new_width)
        return {"kind": "resize", "align_corners": bool(t.bool(2)),
                "half_pixel_centers": bool(t.bool(3))}
    if b == "RESIZE_NEAREST_NEIGHBOR":
        return {"kind": "resize", "align_corners": bool(t.bool(0)),
                "half_pixel_centers": bool(t.bool(1))}
    if b in ("MEAN", "SUM", "REDUCE_MAX"):
        return {"kind": "reducer", "keep_dims": bool(t.bool(0))}
    return {"kind": "empty"}


def _d(v, default):
    return default if v is None else v


def topological_order(model: TfliteModel) -> List[int]:
    """scheduler.rs:1454-1500: repeatedly take, in model order, every operator whose inputs are
    graph inputs, constants or produced by operators already taken."""
    producer: Dict[int, int] = {}
    for op in model.operators:
        for out in op.outputs:
            if out >= 0:
                if out in producer:
                    raise ValueError(f"tensor {out} has multiple producers: {producer[out]} "
                                     f"and {op.index}")
                producer[out] = op.index
    done, order = set(), []
    while len(order) < len(model.operators):
        progressed = False
        for op in model.operators:
            if op.index in done:
                continue
            if all(i < 0 or i in model.inputs or i not in producer or producer[i] in done
                   for i in op.inputs):
                done.add(op.index)
                order.append(op.index)
                progressed = True
        if not progressed:
            raise ValueError("operator graph has a cycle or an unresolvable input")
    return order


def validate_supported_graph(model: TfliteModel) -> dict:
    """graph.rs:5-34: raises for unsupported operators or quantized tensors."""
    if model.unsupported_ops:
        raise ValueError("unsupported TFLite ops: " + ", ".join(model.unsupported_ops))
    if model.quantized_tensors:
        raise ValueError("quantized tensors require dequantization support: " +
                         ", ".join(model.quantized_tensors))
    producers = {o for op in model.operators for o in op.outputs if o >= 0}
    return {"status": "pass", "operator_count": len(model.operators),
            "tensor_count": len(model.tensors),
            "topological_validation": "operator_order_with_single_producer_map",
            "producer_count": len(producers),
            "supported_ops": sum(1 for o in model.operators
                                 if not o.builtin.startswith("UNKNOWN_"))}


def default_input(elements: int) -> np.ndarray:
    """The deterministic input scheduler.rs:load_input uses when no file is given
    (value i = (i - n/2) * 0.25)."""
    i = np.arange(elements, dtype=np.float32)
    return ((i - np.float32(elements / 2.0)) * np.float32(0.25)).astype(np.float32)


def top1(values: np.ndarray) -> dict:
    """scheduler.rs:1637-1652: the last maximum (Rust max_by), 1001-class heads offset by 1."""
    v = np.asarray(values, np.float32).reshape(-1)
    off = 1 if v.size == 1001 else 0
    body = v[off:]
    if body.size == 0:
        return {"class": 0, "model_class": 0, "confidence": 0.0}
    last = body.size - 1 - int(np.argmax(body[::-1]))
    mc = last + off
    return {"class": mc - off, "model_class": mc, "confidence": float(v[mc]),
            "class_index_basis": "imagenet_1000_without_tflite_background" if off
            else "model_output_index"}


# ---- FlatBuffer writing --------------------------------------------------------------------
class _Out:
    """Front-to-back FlatBuffer serialiser: children are appended after their parents, so
    every unsigned offset points forward, as the format requires."""

    def __init__(self):
        self.b = bytearray()

    def align(self, n: int) -> None:
        while len(self.b) % n:
            self.b.append(0)

    def patch_ref(self, at: int, target: int) -> None:
        struct.pack_into("<I", self.b, at, target - at)


def _emit(out: _Out, obj) -> int:
    """Serialise obj at the end of out; returns its position.  obj is a `_T` table, a `_V`
    vector, a str, or bytes (a ubyte vector)."""
    if isinstance(obj, _T):
        return obj.emit(out)
    if isinstance(obj, str):
        obj = _V("B", list(obj.encode("utf-8")), nul=True)
    if isinstance(obj, (bytes, bytearray)):
        obj = _V("B", bytes(obj), align=16)
    return obj.emit(out)


class _V:
    """A vector of scalars (fmt 'i', 'B', 'I') or of tables (fmt 'T')."""

    def __init__(self, fmt: str, items, nul: bool = False, align: int = 4):
        self.fmt, self.items, self.nul, self.alignment = fmt, items, nul, align

    def emit(self, out: _Out) -> int:
        esize = 4 if self.fmt in "iIT" else 1
        # the element data must be aligned; the length word sits right before it
        out.align(4)
        while (len(out.b) + 4) % max(self.alignment, esize):
            out.b.append(0)
        pos = len(out.b)
        out.b += struct.pack("<I", len(self.items))
        if self.fmt == "T":
            slots = len(out.b)
            out.b += bytes(4 * len(self.items))
            for i, t in enumerate(self.items):
                out.patch_ref(slots + 4 * i, _emit(out, t))
        elif self.fmt == "B":
            out.b += bytes(self.items)
            if self.nul:
                out.b.append(0)
        else:
            out.b += struct.pack(f"<{len(self.items)}{self.fmt}", *self.items)
        return pos


class _T:
    """A table: fields {id: (kind, value)} with kind one of 'b','B','i','I','f' (scalars) or
    'ref' (a child table / vector / string)."""

    def __init__(self, **fields):
        self.fields: Dict[int, Tuple[str, object]] = {}

    def set(self, fid: int, kind: str, value) -> "_T":
        if value is not None:
            self.fields[fid] = (kind, value)
        return self

    def emit(self, out: _Out) -> int:
        nf = (max(self.fields) + 1) if self.fields else 0
        # vtable first (table offset to it is signed, so either side works), then the table
        out.align(2)
        vt = len(out.b)
        out.b += bytes(4 + 2 * nf)
        out.align(4)
        tpos = len(out.b)
        out.b += bytes(4)
        layout = []
        for fid in sorted(self.fields):
            kind, value = self.fields[fid]
            size = 4 if kind in ("i", "I", "f", "ref") else 1
            while len(out.b) % size:
                out.b.append(0)
            layout.append((fid, len(out.b), kind, value))
            out.b += bytes(size)
        out.align(4)
        tsize = len(out.b) - tpos
        struct.pack_into("<HH", out.b, vt, 4 + 2 * nf, tsize)
        struct.pack_into("<i", out.b, tpos, tpos - vt)
        for fid, at, kind, value in layout:
            struct.pack_into("<H", out.b, vt + 4 + 2 * fid, at - tpos)
            if kind != "ref":
                struct.pack_into("<" + kind, out.b, at, value)
        for fid, at, kind, value in layout:
            if kind == "ref":
                out.patch_ref(at, _emit(out, value))
        return tpos


class TfliteWriter:
    """Builds a one-subgraph TFL3 model (the fields parse_model reads, schema field ids)."""

    def __init__(self, description: str = "", version: int = 3):
        self.description, self.version = description, version
        self.tensors: List[_T] = []
        self.shapes: List[List[int]] = []
        self.buffers: List[bytes] = [b""]  # buffer 0: the empty sentinel
        self.opcodes: List[int] = []
        self.ops: List[_T] = []
        self.inputs: List[int] = []
        self.outputs: List[int] = []

    def tensor(self, name: str, shape, data: Optional[np.ndarray] = None,
               ttype: int = 0) -> int:
        buf = 0
        if data is not None:
            self.buffers.append(np.ascontiguousarray(data, np.float32).tobytes())
            buf = len(self.buffers) - 1
        t = _T().set(0, "ref", _V("i", [int(s) for s in shape])).set(1, "b", ttype)
        t.set(2, "I", buf).set(3, "ref", name)
        self.tensors.append(t)
        self.shapes.append([int(s) for s in shape])
        return len(self.tensors) - 1

    def op(self, builtin: str, inputs, outputs, options_type: Optional[str] = None,
           options: Optional[Dict[int, Tuple[str, object]]] = None) -> int:
        code = BUILTIN_CODES[builtin]
        if code not in self.opcodes:
            self.opcodes.append(code)
        t = _T().set(0, "I", self.opcodes.index(code))
        t.set(1, "ref", _V("i", list(inputs))).set(2, "ref", _V("i", list(outputs)))
        if options_type is not None:
            o = _T()
            for fid, (kind, value) in (options or {}).items():
                o.set(fid, kind, value)
            t.set(3, "B", OPTIONS_TYPE[options_type]).set(4, "ref", o)
        self.ops.append(t)
        return len(self.ops) - 1

    def finish(self) -> bytes:
        sg = _T().set(0, "ref", _V("T", self.tensors)).set(1, "ref", _V("i", self.inputs))
        sg.set(2, "ref", _V("i", self.outputs)).set(3, "ref", _V("T", self.ops))
        sg.set(4, "ref", "main")
        # deprecated_builtin_code (a byte, codes < 127) and builtin_code, like the reference's
        # fixture generator writes both
        codes = [_T().set(0, "b", c if c < 127 else 127).set(2, "i", 1).set(3, "i", c)
                 for c in self.opcodes]
        bufs = [_T().set(0, "ref", b) if b else _T() for b in self.buffers]
        model = _T().set(0, "I", self.version).set(1, "ref", _V("T", codes))
        model.set(2, "ref", _V("T", [sg])).set(3, "ref", self.description)
        model.set(4, "ref", _V("T", bufs))
        out = _Out()
        out.b += bytes(8)
        out.b[4:8] = b"TFL3"
        root = model.emit(out)
        struct.pack_into("<I", out.b, 0, root)
        return bytes(out.b)


# ---- execution on the device ------------------------------------------------------------------
_UNARY = {"ABS": "abs", "EXP": "exp", "LOG": "log", "LOGISTIC": "sigmoid", "NEG": "neg",
          "RSQRT": "rsqrt", "SQRT": "sqrt", "TANH": "tanh", "RELU6": "relu6"}
_BINARY = {"ADD": "add", "SUB": "sub", "MUL": "mul", "DIV": "div", "POW": "pow",
           "MINIMUM": "min", "MAXIMUM": "max"}
_ALIASES = ("RESHAPE", "SQUEEZE", "EXPAND_DIMS", "CAST")


def _same_pads(ih, iw, oh, ow, kh, kw, sh, sw, dh=1, dw=1):
    """TF SAME offsets, scheduler.rs:1597-1614 (with the dilated kernel extent)."""
    eh, ew = (kh - 1) * dh + 1, (kw - 1) * dw + 1
    return max((oh - 1) * sh + eh - ih, 0) // 2, max((ow - 1) * sw + ew - iw, 0) // 2


class TfliteExecutor:
    """Runs a parsed TFLite model on one Context with every tensor resident on the device.

    Lowerings (reference kernel names, NHWC-native where the reference relabels NHWC data as
    NCHW, scheduler.rs:58-62):
      CONV_2D            -> conv2d_nhwc (OHWI weights + bias tail, packed once; scheduler.rs:321-427)
      DEPTHWISE_CONV_2D  -> depthwise_conv2d_nhwc ([KH,KW,C] + bias tail; :428-548)
      FULLY_CONNECTED    -> fully_connected ([out,in] + bias tail; :914-1002)
      AVERAGE_POOL_2D / MEAN over H,W (global only) -> global_avg_pool_nhwc (:549-613)
      MAX_POOL_2D        -> hlo_reduce_window_rank4, kind max, SAME / VALID offsets (:614-709)
      SOFTMAX            -> softmax10 / softmax1000 over the whole output (:277-320)
      ADD/SUB/MUL/DIV/POW/MINIMUM/MAXIMUM (equal shapes) -> add … max (:144-211)
      ABS/EXP/LOG/LOGISTIC/NEG/RSQRT/SQRT/TANH/RELU6/LEAKY_RELU -> unary kernels (:82-143)
      RESHAPE/SQUEEZE/EXPAND_DIMS/CAST (f32) -> a view of the input, no copy (:212-276)
      CONCATENATION      -> hlo_concatenate_into per input (:710-794)
      L2_NORMALIZATION   -> l2_normalization (on-device norm; :795-836 computes it on the CPU)
    A fused activation runs in the producing kernel's epilogue where it has one, else as a
    unary launch.  A CONV_2D without activation whose output is read only by an ADD of an
    equal-sized tensor computed earlier (a residual connection) runs as one conv2d_nhwc launch
    with that tensor as the epilogue's residual and the ADD's activation; the ADD then
    dispatches nothing.  An inverted-residual chain, [1x1 CONV_2D] -> DEPTHWISE_CONV_2D ->
    1x1 CONV_2D [-> residual ADD], whose intermediates nothing else reads, runs as one
    inverted_residual_nhwc launch at the projection where the library expects that to beat
    the three launches (shp_block_plan), else, where that pays, the expand as its own launch
    and the depthwise + projection as one; fuse_blocks=True fuses every chain the kernel takes,
    False none.  A 1x1 CONV_2D read only by a global pool (the classifier head) runs as one
    conv1x1_gap_nhwc launch unless fuse_blocks is False.  Anything else raises, like the
    reference's scheduler.

    run(graph=True) replays the launch sequence from one hipGraph: the first such call runs
    eagerly if nothing ran yet (so every buffer, packed weight and split-K workspace exists),
    then captures the sequence once; later calls replay it.  Tensors keep their device
    buffers across runs, so set_input() between replays feeds the graph.
    """

    def __init__(self, ctx, model: TfliteModel, fuse_blocks: Optional[bool] = None):
        self.ctx, self.model = ctx, model
        self.order = topological_order(model)
        self.dev: Dict[int, object] = {}
        self.owned: List[object] = []
        self.consts: Dict[int, np.ndarray] = {}
        for t in model.tensors:
            if t.index in model.inputs or t.buffer == 0 or t.buffer >= len(model.buffers):
                continue
            data = model.buffers[t.buffer].data
            if data and t.tensor_type == "Float32":
                self.consts[t.index] = np.frombuffer(data, dtype="<f4").copy()
            elif data and t.tensor_type == "Int32":
                self.consts[t.index] = np.frombuffer(data, dtype="<i4").copy()
        self.packed: Dict[Tuple[int, int], object] = {}
        self.op_log: List[dict] = []
        self._check_aliases()
        self.residual_adds = self._find_residual_adds()
        self.blocks = self._find_blocks(fuse_blocks is None) if fuse_blocks is not False else {}
        self.heads = self._find_heads() if fuse_blocks is not False else {}
        self._graph = None
        self._warm = False

    def _check_aliases(self) -> None:
        """The view ops' rules (scheduler.rs:230-249), checked before anything runs: Cast
        only Float32 -> Float32, and the element count must not change (a view larger than
        its source would read past that allocation)."""
        for op in self.model.operators:
            if op.builtin not in _ALIASES:
                continue
            if not op.inputs or op.inputs[0] < 0 or len(op.outputs) != 1:
                raise ValueError(f"operator {op.index} {op.builtin} needs one data input and "
                                 "one output")
            src, dst = op.inputs[0], op.outputs[0]
            if op.builtin == "CAST":
                tin = self.model.tensors[src].tensor_type
                tout = self.model.tensors[dst].tensor_type
                if tin != "Float32" or tout != "Float32":
                    raise ValueError(f"operator {op.index} Cast only supports Float32->Float32, "
                                     f"got {tin}->{tout}")
            if self._elems(src) != self._elems(dst):
                raise ValueError(f"operator {op.index} {op.builtin} element count changed from "
                                 f"{self._elems(src)} to {self._elems(dst)}")

    def _find_residual_adds(self) -> Dict[int, Tuple[int, int]]:
        """{conv operator index: (add operator index, residual tensor)} for every CONV_2D
        that can take the ADD after it as its epilogue (see the class docstring)."""
        pos = {oi: k for k, oi in enumerate(self.order)}
        producer, readers = {}, {}
        for op in self.model.operators:
            for t in op.outputs:
                producer[t] = op.index
            for t in op.inputs:
                readers.setdefault(t, []).append(op.index)
        out = {}
        for op in self.model.operators:
            if op.builtin != "CONV_2D" or decode_options(op)["fused_activation"] != "none":
                continue
            t = op.outputs[0]
            r = readers.get(t, [])
            if len(r) != 1 or t in self.model.outputs:
                continue
            add = self.model.operators[r[0]]
            if add.builtin != "ADD" or len(add.inputs) != 2 or add.inputs.count(t) != 1:
                continue
            other = add.inputs[1] if add.inputs[0] == t else add.inputs[0]
            if self._elems(other) != self._elems(t) or self._elems(add.outputs[0]) != self._elems(t):
                continue
            if decode_options(add).get("fused_activation", "none") not in ("none", "relu", "relu6", "tanh"):
                continue
            p = producer.get(other)
            if p is not None and pos.get(p, 1 << 30) > pos[op.index]:
                continue  # the residual must exist when the convolution runs
            out[op.index] = (add.index, other)
        return out

    def _find_blocks(self, only_if_faster: bool = True) -> Dict[int, dict]:
        """{projection operator index: block} for every inverted-residual chain the fused
        kernel takes (see the class docstring): 1x1 stride-1 convolutions with constant
        weights, a depthwise with a square 3x3 or 5x5 kernel, stride 1 or 2, multiplier 1 and
        no dilation, ReLU / ReLU6 / no activation before the projection, intermediates read
        by the next operator only and not model outputs; the kernel's own plan query decides
        the rest (channel multiples, and with only_if_faster whether one launch pays)."""
        producer, readers = {}, {}
        for op in self.model.operators:
            for t in op.outputs:
                producer[t] = op.index
            for t in op.inputs:
                readers.setdefault(t, []).append(op.index)
        acts = ("none", "relu", "relu6")
        ops = self.model.operators

        def sole_reader(t):
            r = readers.get(t, [])
            return r[0] if len(r) == 1 and t not in self.model.outputs else None

        def const_bias(op):
            return len(op.inputs) < 3 or op.inputs[2] < 0 or op.inputs[2] in self.consts

        def pointwise(op):
            if op.builtin != "CONV_2D" or op.inputs[1] not in self.consts or not const_bias(op):
                return False
            o = decode_options(op)
            _, kh, kw, _ = self._shape(op.inputs[1])
            return (kh, kw, o["stride_h"], o["stride_w"], o["dilation_h_factor"],
                    o["dilation_w_factor"]) == (1, 1, 1, 1, 1, 1) and o["fused_activation"] in acts

        out = {}
        for dw in ops:
            if dw.builtin != "DEPTHWISE_CONV_2D" or dw.inputs[1] not in self.consts:
                continue
            o = decode_options(dw)
            _, kh, kw, c = self._shape(dw.inputs[1])
            if (o["depth_multiplier"] != 1 or kh != kw or kh not in (3, 5) or o["stride_h"] != o["stride_w"]
                    or o["stride_h"] not in (1, 2) or not const_bias(dw)
                    or (o["dilation_h_factor"], o["dilation_w_factor"]) != (1, 1)
                    or o["fused_activation"] not in acts):
                continue
            pi = sole_reader(dw.outputs[0])
            if pi is None or not pointwise(ops[pi]) or ops[pi].inputs[0] != dw.outputs[0]:
                continue
            src, ei = dw.inputs[0], producer.get(dw.inputs[0])
            if ei is not None and pointwise(ops[ei]) and sole_reader(src) == dw.index:
                src = ops[ei].inputs[0]
            else:
                ei = None
            blk = {"expand": ei, "dw": dw.index, "src": src}
            plan = self._block_plan(ops[pi], blk)
            if plan is not None and plan[7]:
                out[pi] = blk
            elif ei is not None and only_if_faster:
                # the expand as its own launch, the depthwise and projection as one where
                # that pays (as the model graphs decide)
                sub = {"expand": None, "dw": dw.index, "src": dw.inputs[0]}
                plan = self._block_plan(ops[pi], sub)
                if plan is not None and plan[7]:
                    out[pi] = sub
            elif plan is not None and not only_if_faster:
                out[pi] = blk
        return out

    def _find_heads(self) -> Dict[int, int]:
        """{pool operator index: conv operator index} for every classifier head the fused
        conv1x1_gap_nhwc kernel takes: a 1x1 stride-1 CONV_2D with constant weights and bias,
        no dilation, ReLU / ReLU6 / no activation and a channel count that is a multiple of
        4, whose output only a global pool reads (MEAN over H and W, or an AVERAGE_POOL_2D
        over the whole map without an activation of its own) and is not a model output."""
        readers = {}
        for op in self.model.operators:
            for t in op.inputs:
                readers.setdefault(t, []).append(op.index)
        ops = self.model.operators
        out = {}
        for conv in ops:
            if conv.builtin != "CONV_2D" or conv.inputs[1] not in self.consts:
                continue
            if len(conv.inputs) > 2 and conv.inputs[2] >= 0 and conv.inputs[2] not in self.consts:
                continue
            o = decode_options(conv)
            _, kh, kw, cin = self._shape(conv.inputs[1])
            if ((kh, kw, o["stride_h"], o["stride_w"], o["dilation_h_factor"],
                 o["dilation_w_factor"]) != (1, 1, 1, 1, 1, 1)
                    or o["fused_activation"] not in ("none", "relu", "relu6") or cin % 4):
                continue
            t = conv.outputs[0]
            r = readers.get(t, [])
            if len(r) != 1 or t in self.model.outputs:
                continue
            pool = ops[r[0]]
            if pool.inputs[0] != t or len(self._shape(t)) != 4:
                continue
            n, h, w_, c = self._shape(t)
            if self._elems(pool.outputs[0]) != n * c:
                continue
            if pool.builtin == "MEAN":
                if sorted(int(a) % 4 for a in self.consts.get(pool.inputs[1], [])) != [1, 2]:
                    continue
            elif pool.builtin == "AVERAGE_POOL_2D":
                po = decode_options(pool)
                if (po["filter_h"], po["filter_w"], po["fused_activation"]) != (h, w_, "none"):
                    continue
            else:
                continue
            out[pool.index] = conv.index
        return out

    def _run_head(self, pool: Operator, ci: int) -> None:
        conv = self.model.operators[ci]
        n, h, w_, cin = self._shape(conv.inputs[0])
        cout = self._shape(conv.inputs[1])[0]
        w = self._pack(conv.inputs[1], conv.inputs[2] if len(conv.inputs) > 2 else -1, cout)
        y = self._alloc(pool.outputs[0])
        self._launch("conv1x1_gap_nhwc", self._get(conv.inputs[0]), w, y,
                     [n, cin, h, w_, cout, n * cout],
                     act=decode_options(conv)["fused_activation"])

    def _block_push(self, proj: Operator, blk: dict) -> List[int]:
        from ._lib import ACT
        ops = self.model.operators
        dw = ops[blk["dw"]]
        od = decode_options(dw)
        n, h, w_, cin = self._shape(blk["src"])
        _, oh, ow, ce = self._shape(dw.outputs[0])
        cout = self._shape(proj.outputs[0])[3]
        k, s = self._shape(dw.inputs[1])[1], od["stride_h"]
        pt, pl = _same_pads(h, w_, oh, ow, k, k, s, s) if od["padding"] == "same" else (0, 0)
        act_e = (ACT[decode_options(ops[blk["expand"]])["fused_activation"]]
                 if blk["expand"] is not None else 0)
        return [n, cin, h, w_, ce, cout, oh, ow, k, s, pt, pl,
                0 if blk["expand"] is None else 1, act_e, ACT[od["fused_activation"]],
                n * oh * ow * cout]

    def _block_plan(self, proj: Operator, blk: dict):
        """shp_block_plan of the chain, or None if the fused kernel does not take it."""
        import ctypes as C
        from ._lib import lib
        push = self._block_push(proj, blk)
        out = (C.c_int32 * 8)()
        if lib().shp_block_plan((C.c_int32 * 16)(*push), 16, out) != 0:
            return None
        return list(out)

    def _block_weights(self, proj: Operator, blk: dict):
        """The packed weights of a fused block (the operators' tensors back to back),
        uploaded once."""
        key = ("block", proj.index)
        if key not in self.packed:
            parts = []
            for oi in (blk["expand"], blk["dw"], proj.index):
                if oi is None:
                    continue
                op = self.model.operators[oi]
                w = self.consts[op.inputs[1]].astype(np.float32)
                n_out = self._shape(op.inputs[1])[0 if op.builtin == "CONV_2D" else 3]
                b = (self.consts[op.inputs[2]].astype(np.float32)
                     if len(op.inputs) > 2 and op.inputs[2] >= 0 else np.zeros(n_out, np.float32))
                parts += [w.reshape(-1), b.reshape(-1)]
            t = self.ctx.tensor(np.concatenate(parts))
            self.owned.append(t)
            self.packed[key] = t
        return self.packed[key]

    def _residual_epilogue(self, op: Operator, out_idx: int, act: str):
        """(output tensor, residual, activation) of a CONV_2D, with its residual ADD folded in."""
        if op.index not in self.residual_adds:
            return out_idx, None, act
        add_i, r_idx = self.residual_adds[op.index]
        add = self.model.operators[add_i]
        return add.outputs[0], self._get(r_idx), decode_options(add).get("fused_activation", "none")

    def _run_block(self, proj: Operator, blk: dict) -> None:
        out_idx, residual, act = self._residual_epilogue(
            proj, proj.outputs[0], decode_options(proj)["fused_activation"])
        y = self._alloc(out_idx)
        self._launch("inverted_residual_nhwc", self._get(blk["src"]),
                     self._block_weights(proj, blk), y, self._block_push(proj, blk), act=act,
                     residual=residual)

    # -- helpers
    def _shape(self, idx: int) -> List[int]:
        return self.model.tensors[idx].shape

    def _elems(self, idx: int) -> int:
        return int(np.prod(self._shape(idx))) if self._shape(idx) else 1

    def _alloc(self, idx: int):
        """The device buffer of tensor idx, allocated on first use and kept across runs."""
        n = max(1, self._elems(idx))
        t = self.dev.get(idx)
        if t is not None and t.n == n:
            return t
        t = self.ctx.empty(n)
        self.owned.append(t)
        self.dev[idx] = t
        return t

    def _get(self, idx: int):
        if idx in self.dev:
            return self.dev[idx]
        if idx in self.consts:
            t = self.ctx.tensor(self.consts[idx].astype(np.float32))
            self.owned.append(t)
            self.dev[idx] = t
            return t
        raise ValueError(f"tensor {idx} not materialized")

    def _pack(self, w_idx: int, b_idx: int, n_out: int):
        """Weights followed by the bias tail (scheduler.rs:1327-1436), uploaded once."""
        key = (w_idx, b_idx)
        if key not in self.packed:
            if w_idx not in self.consts:
                raise ValueError(f"weight tensor {w_idx} is not a constant")
            w = self.consts[w_idx].astype(np.float32)
            b = (self.consts[b_idx].astype(np.float32) if b_idx >= 0
                 else np.zeros(n_out, np.float32))
            t = self.ctx.tensor(np.concatenate([w, b]))
            self.owned.append(t)
            self.packed[key] = t
        return self.packed[key]

    def _launch(self, kernel, in0, in1, out, push, **kw):
        self.ctx.launch(kernel, in0, in1, out, push, **kw)
        self.op_log[-1]["dispatches"].append({"kernel": kernel, "push": list(push)})

    def _activation(self, act: str, out):
        if act in ("none",):
            return
        k = {"relu": "relu", "relu6": "relu6", "tanh": "tanh"}.get(act)
        if k is None:
            raise ValueError(f"fused activation {act} is not supported")
        self._launch(k, out, None, out, [out.n])

    # -- running
    def set_input(self, values: np.ndarray, index: int = 0) -> None:
        idx = self.model.inputs[index]
        v = np.ascontiguousarray(values, np.float32).reshape(-1)
        if v.size != self._elems(idx):
            raise ValueError(f"input has {v.size} values, tensor {idx} holds {self._elems(idx)}")
        t = self._alloc(idx)
        t.upload(v)

    def run(self, graph: bool = False) -> None:
        if graph and self._graph is not None:
            self._graph.launch()
            return
        if graph and self._warm:
            self.ctx.capture_begin()
            try:
                self._run_ops()
            finally:
                self._graph = self.ctx.capture_end()
            self._graph.launch()
            return
        self._run_ops()
        self._warm = True

    def _run_ops(self) -> None:
        self.op_log = []  # the dispatches of this run
        fused = {a: c for c, (a, _) in self.residual_adds.items()}
        for pi, blk in self.blocks.items():
            fused[blk["dw"]] = pi
            if blk["expand"] is not None:
                fused[blk["expand"]] = pi
        for pool, conv in self.heads.items():
            fused[conv] = pool
        for oi in self.order:
            op = self.model.operators[oi]
            self.op_log.append({"index": op.index, "op": op.builtin,
                                "options": decode_options(op), "inputs": op.inputs,
                                "outputs": op.outputs, "dispatches": []})
            if op.index in fused:
                self.op_log[-1]["fused_into"] = fused[op.index]
                continue
            if op.index in self.blocks:
                self._run_block(op, self.blocks[op.index])
                continue
            if op.index in self.heads:
                self._run_head(op, self.heads[op.index])
                continue
            self._run_op(op, self.op_log[-1]["options"])

    def output(self, index: int = 0) -> np.ndarray:
        return self._get(self.model.outputs[index]).download()

    def tensor(self, idx: int) -> np.ndarray:
        return self._get(idx).download()

    def close(self) -> None:
        if self._graph is not None:
            self._graph.destroy()
            self._graph = None
        for t in self.owned:
            t.free()
        self.owned, self.dev, self.packed = [], {}, {}
        self._warm = False

    def _run_op(self, op: Operator, o: dict) -> None:
        b = op.builtin
        ins = [i for i in op.inputs]
        out_idx = op.outputs[0] if op.outputs else -1
        if b in _ALIASES:
            src = self._get(ins[0])
            from .runtime import DeviceTensor
            self.dev[out_idx] = DeviceTensor(self.ctx, self._elems(out_idx), ptr=src.ptr,
                                             owned=False)
            return
        if b == "CONV_2D":
            n, ih, iw, ic = self._shape(ins[0])
            oc, kh, kw, wic = self._shape(ins[1])
            _, oh, ow, _ = self._shape(out_idx)
            if (o["dilation_w_factor"], o["dilation_h_factor"]) != (1, 1):
                raise ValueError(f"operator {op.index}: Conv2D dilation is not supported")
            if wic != ic:
                raise ValueError(f"operator {op.index}: Conv2D channel mismatch")
            sh, sw = o["stride_h"], o["stride_w"]
            pt, pl = (_same_pads(ih, iw, oh, ow, kh, kw, sh, sw) if o["padding"] == "same"
                      else (0, 0))
            w = self._pack(ins[1], ins[2] if len(ins) > 2 else -1, oc)
            act = o["fused_activation"]
            fused = act if act in ("none", "relu", "relu6", "tanh") else None
            if fused is None:
                raise ValueError(f"operator {op.index}: fused activation {act} not supported")
            # conv + bias + residual, then the ADD's act
            out_idx, residual, fused = self._residual_epilogue(op, out_idx, fused)
            y = self._alloc(out_idx)
            self._launch("conv2d_nhwc", self._get(ins[0]), w, y,
                         [n, ic, ih, iw, oc, oh, ow, kh, kw, sh, sw,
                          1 if o["padding"] == "same" else 0, pt, pl, n * oh * ow * oc],
                         act=fused, residual=residual)
            return
        if b == "DEPTHWISE_CONV_2D":
            n, ih, iw, c = self._shape(ins[0])
            _, kh, kw, wc = self._shape(ins[1])
            _, oh, ow, oc = self._shape(out_idx)
            if o["depth_multiplier"] != 1 or wc != c or oc != c:
                raise ValueError(f"operator {op.index}: depth_multiplier must be 1 "
                                 "(scheduler.rs:457-462)")
            sh, sw = o["stride_h"], o["stride_w"]
            dh, dw = o["dilation_h_factor"], o["dilation_w_factor"]
            pt, pl = (_same_pads(ih, iw, oh, ow, kh, kw, sh, sw, dh, dw)
                      if o["padding"] == "same" else (0, 0))
            w = self._pack(ins[1], ins[2] if len(ins) > 2 else -1, c)
            y = self._alloc(out_idx)
            act = o["fused_activation"]
            if act not in ("none", "relu", "relu6", "tanh"):
                raise ValueError(f"operator {op.index}: fused activation {act} not supported")
            self._launch("depthwise_conv2d_nhwc", self._get(ins[0]), w, y,
                         [n, c, ih, iw, oh, ow, kh, kw, sh, sw,
                          1 if o["padding"] == "same" else 0, pt, pl, dh, dw, n * oh * ow * c],
                         act=act)
            return
        if b == "FULLY_CONNECTED":
            n_out, n_in = self._shape(ins[1])
            batches = self._elems(ins[0]) // n_in
            act = o["fused_activation"]
            if act not in ("none", "relu", "relu6", "tanh"):
                raise ValueError(f"operator {op.index}: fused activation {act} not supported")
            w = self._pack(ins[1], ins[2] if len(ins) > 2 and ins[2] >= 0 else -1, n_out)
            y = self._alloc(out_idx)
            self._launch("fully_connected", self._get(ins[0]), w, y,
                         [batches, n_in, n_out, batches * n_out], act=act)
            return
        if b in ("AVERAGE_POOL_2D", "MEAN"):
            n, h, w_, c = self._shape(ins[0])
            if self._elems(out_idx) != n * c:
                raise ValueError(f"operator {op.index}: {b} only supports a global pool to "
                                 "N*C outputs")
            if b == "MEAN":
                axes = sorted(int(a) % 4 for a in self.consts.get(ins[1], []))
                if axes != [1, 2]:
                    raise ValueError(f"operator {op.index}: MEAN only over the H and W axes")
            y = self._alloc(out_idx)
            self._launch("global_avg_pool_nhwc", self._get(ins[0]), None, y, [n, h, w_, c])
            if b == "AVERAGE_POOL_2D":
                self._activation(o["fused_activation"], y)
            return
        if b == "MAX_POOL_2D":
            n, ih, iw, c = self._shape(ins[0])
            _, oh, ow, _ = self._shape(out_idx)
            kh, kw, sh, sw = o["filter_h"], o["filter_w"], o["stride_h"], o["stride_w"]
            pt, pl = (_same_pads(ih, iw, oh, ow, kh, kw, sh, sw) if o["padding"] == "same"
                      else (0, 0))
            y = self._alloc(out_idx)
            self._launch("hlo_reduce_window_rank4", self._get(ins[0]), None, y,
                         [n, ih, iw, c, oh, ow, kh, kw, sh, sw, pt, pl, 1, n * oh * ow * c])
            self._activation(o["fused_activation"], y)
            return
        if b == "SOFTMAX":
            classes = self._elems(out_idx)
            y = self._alloc(out_idx)
            if classes == 10:
                self._launch("softmax10", self._get(ins[0]), None, y, [])
            else:
                self._launch("softmax1000", self._get(ins[0]), None, y, [classes])
            return
        if b in _BINARY:
            if self._elems(ins[0]) != self._elems(ins[1]):
                raise ValueError(f"operator {op.index}: {b} needs equal input sizes "
                                 "(scheduler.rs:172-180)")
            y = self._alloc(out_idx)
            self._launch(_BINARY[b], self._get(ins[0]), self._get(ins[1]), y,
                         [self._elems(out_idx)])
            self._activation(o.get("fused_activation", "none"), y)
            return
        if b in _UNARY or b == "LEAKY_RELU":
            y = self._alloc(out_idx)
            if b == "LEAKY_RELU":
                bits = int(np.array([o["alpha"]], np.float32).view(np.int32)[0])
                self._launch("leaky_relu", self._get(ins[0]), None, y,
                             [self._elems(out_idx), bits])
            else:
                self._launch(_UNARY[b], self._get(ins[0]), None, y, [self._elems(out_idx)])
            return
        if b == "CONCATENATION":
            out_shape = self._shape(out_idx)
            r = len(out_shape)
            axis = o["axis"] % r
            y = self._alloc(out_idx)
            off = 0
            for i in ins:
                s = self._shape(i)
                self._launch("hlo_concatenate_into", self._get(i), None, y,
                             [r, axis, off, *out_shape, *s], out_elems=y.n)
                off += s[axis]
            self._activation(o["fused_activation"], y)
            return
        if b == "L2_NORMALIZATION":
            y = self._alloc(out_idx)
            self._launch("l2_normalization", self._get(ins[0]), None, y, [self._elems(out_idx)])
            return
        raise ValueError(f"operator {op.index} {b} is recognized by the parser but has no "
                         "scheduler lowering")


def run_model(ctx, model: TfliteModel, input_values: Optional[np.ndarray] = None,
              input_source: Optional[dict] = None) -> Tuple[dict, np.ndarray]:
    """scheduler.rs:run_graph's report for one model input (without per-op host dumps;
    the CLI writes those)."""
    if len(model.inputs) != 1:
        raise ValueError(f"exactly one model input is supported, got {len(model.inputs)}")
    ex = TfliteExecutor(ctx, model)
    try:
        n_in = ex._elems(model.inputs[0])
        if input_values is None:
            input_values = default_input(n_in)
            input_source = {"kind": "deterministic_ramp", "formula": "(i - n/2) * 0.25"}
        ex.set_input(input_values)
        ex.run()
        ctx.sync()
        outs = OrderedDict((i, ex._get(i).download()) for i in model.outputs)
        primary = next(iter(outs.values()))
        report = {
            "status": "pass",
            "execution_kind": "tflite_graph_resident_hip_gfx950",
            "operator_count": len(model.operators),
            "inputs": [{"tensor": model.inputs[0], "shape": ex._shape(model.inputs[0]),
                        "elements": n_in, "source": input_source}],
            "topological_order": ex.order,
            "ops": ex.op_log,
            "outputs": [{"tensor": i, "elements": int(v.size),
                         "sha256": hashlib.sha256(v.astype("<f4").tobytes()).hexdigest()}
                        for i, v in outs.items()],
            "top1": top1(primary),
        }
        return report, primary
    finally:
        ex.close()


# ---- export of a resident TFLite-path model graph -------------------------------------------
_ACT_TO_TFL = {0: 0, 1: 1, 2: 3, 5: 4}  # registry epilogue code -> ActivationFunctionType


def model_to_tflite(m, description: str = "") -> bytes:
    """A TFL3 file of a resident model graph built on the TFLite path (MobileNetV2,
    EfficientNet-Lite0: conv2d_nhwc, depthwise_conv2d_nhwc or the fused
    inverted_residual_nhwc, global_avg_pool_nhwc or the fused conv1x1_gap_nhwc head,
    fully_connected, softmax1000), with its weights: CONV_2D / DEPTHWISE_CONV_2D (OHWI and
    [1,KH,KW,C] weights with separate bias tensors; a fused block as its three operators, a
    fused head as CONV_2D + MEAN), ADD for a residual the graph fuses into a convolution, MEAN
    over H and W, FULLY_CONNECTED, SOFTMAX."""
    w = TfliteWriter(description or f"{m.arch} exported from the resident graph")
    tfl: Dict[int, int] = {}          # model tensor id -> tflite tensor index
    host = lambda tid: m.download(tid)

    def conv(label, x, n, ic, oh, ow, oc, k, s, same, wts, bias, act, residual=None):
        wt = w.tensor(f"{label}/weights", [oc, k, k, ic], wts)
        bt = w.tensor(f"{label}/bias", [oc], bias)
        y = w.tensor(label, [n, oh, ow, oc])
        opts = {0: ("b", 0 if same else 1), 1: ("i", s), 2: ("i", s),
                3: ("b", 0 if residual is not None else act)}
        w.op("CONV_2D", [x, wt, bt], [y], "Conv2DOptions", opts)
        if residual is not None:
            z = w.tensor(label + "/add", [n, oh, ow, oc])
            w.op("ADD", [y, residual], [z], "AddOptions", {0: ("b", act)})
            y = z
        return y

    def depthwise(label, x, n, c, oh, ow, k, s, same, wts, bias, act, dh=1, dw=1):
        wt = w.tensor(f"{label}/weights", [1, k, k, c], wts)
        bt = w.tensor(f"{label}/bias", [c], bias)
        y = w.tensor(label, [n, oh, ow, c])
        opts = {0: ("b", 0 if same else 1), 1: ("i", s), 2: ("i", s), 3: ("i", 1),
                4: ("b", act), 5: ("i", dw), 6: ("i", dh)}
        w.op("DEPTHWISE_CONV_2D", [x, wt, bt], [y], "DepthwiseConv2DOptions", opts)
        return y

    def model_input(tid, shape):
        if tid not in tfl:
            tfl[tid] = w.tensor("input", shape)
            w.inputs.append(tfl[tid])
        return tfl[tid]

    for k, op in enumerate(m.ops()):
        q = op.push
        if op.kernel == "conv2d_nhwc":
            n, ic, ih, iw, oc, oh, ow, kh, kw, sh, sw, same = q[:12]
            if kh != kw or sh != sw:
                raise ValueError(f"op {k} ({op.label}): only square kernels and strides export")
            x = model_input(op.in0, [n, ih, iw, ic])
            packed = host(op.in1)
            K = kh * kw * ic
            tfl[op.out] = conv(op.label, x, n, ic, oh, ow, oc, kh, sh, same, packed[:oc * K],
                               packed[oc * K:oc * K + oc], _ACT_TO_TFL[op.act],
                               tfl[op.residual] if op.residual >= 0 else None)
        elif op.kernel == "depthwise_conv2d_nhwc":
            n, c, ih, iw, oh, ow, kh, kw, sh, sw, same, pt, pl, dh, dw = q[:15]
            packed = host(op.in1)
            tfl[op.out] = depthwise(op.label, tfl[op.in0], n, c, oh, ow, kh, sh, same,
                                    packed[:kh * kw * c], packed[kh * kw * c:kh * kw * c + c],
                                    _ACT_TO_TFL[op.act], dh, dw)
        elif op.kernel == "inverted_residual_nhwc":
            n, cin, h, w_, ce, cout, oh, ow, kk, s, pt, pl, expand, act_e, act_d = q[:15]
            packed, o = host(op.in1), 0
            x = model_input(op.in0, [n, h, w_, cin])
            base = op.label
            for suffix in ("_mbconv", "_dwproj"):
                if base.endswith(suffix):
                    base = base[:-len(suffix)]
            if expand:
                x = conv(f"{base}_expand", x, n, cin, h, w_, ce, 1, 1, True,
                         packed[:ce * cin], packed[ce * cin:ce * cin + ce], _ACT_TO_TFL[act_e])
                o = ce * cin + ce
            x = depthwise(f"{base}_depthwise", x, n, ce, oh, ow, kk, s, True,
                          packed[o:o + kk * kk * ce], packed[o + kk * kk * ce:o + kk * kk * ce + ce],
                          _ACT_TO_TFL[act_d])
            o += kk * kk * ce + ce
            tfl[op.out] = conv(f"{base}_project", x, n, ce, oh, ow, cout, 1, 1, True,
                               packed[o:o + cout * ce], packed[o + cout * ce:o + cout * ce + cout],
                               _ACT_TO_TFL[op.act], tfl[op.residual] if op.residual >= 0 else None)
        elif op.kernel == "conv1x1_gap_nhwc":  # the fused head: CONV_2D 1x1, then MEAN
            n, cin, h, w_, cout = q[:5]
            packed = host(op.in1)
            x = model_input(op.in0, [n, h, w_, cin])
            base = op.label[:-len("_pool")] if op.label.endswith("_pool") else op.label
            y = conv(base, x, n, cin, h, w_, cout, 1, 1, True, packed[:cout * cin],
                     packed[cout * cin:cout * cin + cout], _ACT_TO_TFL[op.act])
            axes = w.tensor(f"{op.label}/axes", [2], np.array([1, 2], np.int32).view(np.float32),
                            ttype=2)
            tfl[op.out] = w.tensor(op.label, [n, cout])
            w.op("MEAN", [y, axes], [tfl[op.out]], "ReducerOptions", {0: ("B", 0)})
        elif op.kernel == "global_avg_pool_nhwc":
            n, h, w_, c = q[:4]
            axes = w.tensor(f"{op.label}/axes", [2], np.array([1, 2], np.int32).view(np.float32),
                            ttype=2)
            y = w.tensor(op.label, [n, c])
            w.op("MEAN", [tfl[op.in0], axes], [y], "ReducerOptions", {0: ("B", 0)})
            tfl[op.out] = y
        elif op.kernel == "fully_connected":
            b, n_in, n_out = q[:3]
            packed = host(op.in1)
            wt = w.tensor(f"{op.label}/weights", [n_out, n_in], packed[:n_out * n_in])
            bt = w.tensor(f"{op.label}/bias", [n_out], packed[n_out * n_in:n_out * n_in + n_out])
            y = w.tensor(op.label, [b, n_out])
            w.op("FULLY_CONNECTED", [tfl[op.in0], wt, bt], [y], "FullyConnectedOptions",
                 {0: ("b", _ACT_TO_TFL[op.act])})
            tfl[op.out] = y
        elif op.kernel == "softmax1000":
            y = w.tensor(op.label, [q[0] // 1000, 1000] if q[0] % 1000 == 0 else [q[0]])
            w.op("SOFTMAX", [tfl[op.in0]], [y], "SoftmaxOptions", {0: ("f", 1.0)})
            tfl[op.out] = y
            w.outputs = [y]
        else:
            raise ValueError(f"op {k} ({op.kernel}) is not a TFLite-path op")
    return w.finish()
