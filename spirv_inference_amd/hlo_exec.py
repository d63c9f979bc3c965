"""Executor for XLA HLO text modules on resident device tensors (the HLO path's caller).

The reference's HLO runner (source/xla_hlo/src/parser.rs:5-110 + compiler.rs:267-640,
`run_graph`) parses the ENTRY computation of an HLO text module and executes it op by op:
elementwise ops, convolution, dot, reduce, reduce-window and pad through Vulkan kernels,
and broadcast, transpose, slice, concatenate, compare, select and rank > 4 reduce on the
host CPU between dispatches, with every tensor copied to and from the device per op.  This
module executes the same module text with the same lowering decisions, but every op is a
registry kernel launched on tensors that stay in HBM (reshape/convert/tuple are aliases).

The lowering is written against a small backend interface (upload / empty / launch /
alias / free / read) so the same walk can drive the device (`DeviceBackend`, the product) or
any other implementation of the registry kernels with the same names and push vectors.

    ops = parse_hlo_text(open("resnet50.stablehlo.txt").read())
    ex = HloExecutor(DeviceBackend(ctx), ops)
    out = ex.run(params)          # params: numpy arrays in parameter order
"""
from __future__ import annotations

import dataclasses
import re
from typing import Any, Sequence

import numpy as np

from . import hlo_ops as H
from .runtime import Context, DeviceTensor

# parser.rs:113-160 checks these names in this order, so compound names win over prefixes
_OPCODES = ("get-tuple-element", "reduce-window", "dynamic-slice", "dynamic-update-slice",
            "broadcast_in_dim", "dot_general", "parameter", "constant", "broadcast",
            "convolution", "transpose", "subtract", "multiply", "maximum", "minimum",
            "exponential", "reshape", "convert", "divide", "negate", "rsqrt", "sqrt", "tanh",
            "logistic", "compare", "select", "slice", "reduce", "tuple", "add", "dot", "abs",
            "log", "pad", "floor", "ceil", "round-nearest-even", "sine", "cosine", "remainder",
            "power", "iota", "gather", "scatter")
_ATTRS = ("window", "dim_labels", "dimensions", "padding", "lhs_batch_dims", "rhs_batch_dims",
          "lhs_contracting_dims", "rhs_contracting_dims", "feature_group_count",
          "batch_group_count", "to_apply", "direction", "index")

# opcode -> registry kernel, arity (compiler.rs:1155-1228 kernel_mapping)
ELEMENTWISE = {"add": ("add", 2), "subtract": ("sub", 2), "multiply": ("mul", 2),
               "divide": ("div", 2), "maximum": ("max", 2), "minimum": ("min", 2),
               "power": ("pow", 2), "abs": ("abs", 1), "exponential": ("exp", 1),
               "log": ("log", 1), "sqrt": ("sqrt", 1), "rsqrt": ("rsqrt", 1),
               "negate": ("neg", 1), "tanh": ("tanh", 1), "logistic": ("sigmoid", 1),
               "sine": ("sine", 1)}
ALIASES = ("reshape", "convert", "tuple", "get-tuple-element")


@dataclasses.dataclass
class HloOp:
    result: str
    opcode: str
    operands: list[str]
    shape: list[int]
    attrs: dict[str, str]
    raw: str
    result_type: str | None = None  # the type text before the opcode, e.g. f32[1,64]{1,0}


def _attr(line: str, key: str) -> str | None:
    """parser.rs:230-251 parse_attr_value: `{...}`, `"..."` or up to ',' / ' '."""
    i = line.find(key + "=")
    if i < 0:
        return None
    rest = line[i + len(key) + 1:]
    if rest.startswith("{"):
        j = rest.find("}")
        return rest[1:j] if j >= 0 else None
    if rest.startswith('"'):
        j = rest.find('"', 1)
        return rest[1:j] if j >= 0 else None
    ends = [k for k in (rest.find(","), rest.find(" ")) if k >= 0]
    return rest[:min(ends)].strip() if ends else rest.strip()


def _parse_op(line: str) -> HloOp | None:
    """parser.rs:86-110 parse_xla_hlo_op."""
    if "=" not in line:
        return None
    lhs, rhs = line.split("=", 1)
    opcode, before = None, None
    for op in _OPCODES:
        k = rhs.find(op + "(")
        if k >= 0:
            opcode, before = op, rhs[:k].strip()
            break
    if opcode is None:
        k = rhs.find("(")
        if k < 0:
            return None
        before = rhs[:k].strip()
        opcode = before.split()[-1] if before.split() else ""
    if not opcode or "[" in opcode or "{" in opcode:
        return None
    res = [t for t in lhs.strip().removeprefix("ROOT ").split() if t.startswith("%")]
    if not res:
        return None
    rtype = before.split()[0] if before.split() else ""
    m = re.search(r"\[([^\]]*)\]", rtype)
    shape = [int(d) for d in m.group(1).split(",") if d.strip().isdigit()] if m else []
    operands = [t.strip(",()") for t in rhs.split() if t.startswith("%")]
    attrs = {k: v for k in _ATTRS if (v := _attr(line, k)) is not None}
    return HloOp(res[0], opcode, operands, shape, attrs, line, rtype or None)


def parse_hlo_text(text: str) -> list[HloOp]:
    """The ENTRY computation's instructions, in order (parser.rs:5-60)."""
    ops, in_entry = [], False
    for line in text.splitlines():
        t = line.strip()
        if t.startswith("ENTRY "):
            in_entry = True
            continue
        if in_entry and t == "}":
            in_entry = False
            continue
        if in_entry and (op := _parse_op(t)) is not None:
            ops.append(op)
    return ops


def module_name(text: str) -> str:
    """The module's name as parser.rs:14-31 takes it: the token after `HloModule` (its
    trailing comma dropped), or after `module @`; "module" when neither is present."""
    name = "module"
    for line in text.splitlines():
        t = line.strip()
        if t.startswith("HloModule "):
            parts = t.split()
            name = parts[1].rstrip(",") if len(parts) > 1 else "module"
        if t.startswith("module @"):
            parts = t.split()
            name = parts[1].lstrip("@") if len(parts) > 1 else "@module"
    return name


def _ints(v: str | None) -> list[int]:
    return [int(x) for x in re.findall(r"\d+", v)] if v else []


def _window(v: str | None, key: str) -> list[int]:
    """compiler.rs:1328-1342 parse_window: `key=AxBx...`."""
    if not v or key + "=" not in v:
        return []
    part = v.split(key + "=", 1)[1].split(" ", 1)[0]
    return [int(x) for x in part.split("x") if x.lstrip("-").isdigit()]


def _pairs(v: str | None) -> list[tuple[int, int]]:
    """`lo_hi` pairs separated by 'x' (compiler.rs:1344-1359, :1704-1720)."""
    out = []
    for part in v.split("x") if v else []:
        nums = [int(x) for x in part.split("_") if x.lstrip("-").isdigit()]
        out.append((nums[0] if nums else 0, nums[1] if len(nums) > 1 else 0))
    return out


def _constant(raw: str) -> float:
    """compiler.rs:1254-1263 constant_scalar."""
    s = raw.split("constant(", 1)[1].split(")", 1)[0].strip()
    return {"inf": np.inf, "+inf": np.inf, "-inf": -np.inf, "-0": -0.0}.get(s, None) \
        if s in ("inf", "+inf", "-inf", "-0") else float(s)


def _slice_spec(raw: str):
    """compiler.rs:1897-1929 parse_slice_spec: `slice={[a:b], [c:d:e], ...}`."""
    spec = raw.split("slice={", 1)[1].split("}", 1)[0]
    starts, limits, strides = [], [], []
    for m in re.finditer(r"\[([^\]]*)\]", spec):
        parts = m.group(1).split(":")
        starts.append(int(parts[0]))
        limits.append(int(parts[1]))
        strides.append(int(parts[2]) if len(parts) > 2 else 1)
    return starts, limits, strides


def _n(shape: Sequence[int]) -> int:
    return int(np.prod(shape, dtype=np.int64)) if len(shape) else 1


class DeviceBackend:
    """Registry kernels on `ctx`'s stream; values are DeviceTensors."""

    def __init__(self, ctx: Context):
        self.ctx = ctx

    def upload(self, arr: np.ndarray) -> DeviceTensor:
        return self.ctx.tensor(np.ascontiguousarray(arr, np.float32).reshape(-1))

    def empty(self, n: int) -> DeviceTensor:
        return self.ctx.empty(max(1, n))

    def launch(self, kernel: str, in0, in1, out, push: Sequence[int], bias=None, residual=None,
               act: int = 0, alpha: float = 0.0, out_elems: int | None = None) -> None:
        self.ctx.launch(kernel, in0, in1, out, list(push), out_elems=out_elems, bias=bias,
                        residual=residual, act=act, alpha=alpha)

    def sub(self, t: DeviceTensor, offset: int, n: int) -> DeviceTensor:
        """Elements [offset, offset + n) of `t` (no copy; `t` keeps the memory)."""
        if offset == 0 and n == t.n:
            return t
        return DeviceTensor(self.ctx, n, ptr=t.ptr + 4 * int(offset), owned=False)

    def write(self, t: DeviceTensor, offset: int, arr: np.ndarray) -> None:
        self.sub(t, offset, arr.size).upload(arr)

    def read(self, t: DeviceTensor) -> np.ndarray:
        return t.download()

    def free(self, t: DeviceTensor) -> None:
        t.free()

    # hipGraph capture of a launch sequence on the context stream
    def capture_begin(self) -> None:
        self.ctx.capture_begin()

    def capture_end(self):
        return self.ctx.capture_end()

    def graph_launch(self, g) -> None:
        g.launch()

    def graph_destroy(self, g) -> None:
        g.destroy()


class _Recorder:
    """The backend with its launches noted by kernel name and element count, so every
    launch can be attributed to the HLO op that issued it."""

    def __init__(self, backend: Any):
        self._b, self._log = backend, []

    def __getattr__(self, name):
        return getattr(self._b, name)

    def launch(self, kernel, in0, in1, out, push, **kw):
        n = kw.get("out_elems")
        if n is None:
            n = getattr(out, "n", None) or getattr(out, "size", None)
        self._log.append((kernel, int(n) if n is not None else None))
        return self._b.launch(kernel, in0, in1, out, push, **kw)

    def take(self) -> list:
        log, self._log = self._log, []
        return log


class HloExecutor:
    """Runs an ENTRY op list with compiler.rs's lowering on a backend."""

    def __init__(self, backend: Any, ops: Sequence[HloOp]):
        self.b, self.ops = backend, list(ops)
        self.last_use: dict[str, int] = {}
        for i, op in enumerate(self.ops):
            for name in op.operands:
                self.last_use[name] = i

    def run(self, params: Sequence[np.ndarray], keep: bool = False, on_value=None):
        """Execute with `params` in parameter order; returns the last op's value (a backend
        tensor) and its shape.  keep=True keeps every intermediate in self.values.

        After each op, self.record holds (result, opcode, kernels launched for it) and
        on_value(op, tensor, shape), when given, sees the op's value before any buffer is
        released (the NaN trace of compiler.rs:613-623 hooks in here)."""
        backend = self.b
        self.b = _Recorder(backend)  # every launch, _dot's included, goes through it
        try:
            return self._run(params, keep, on_value)
        finally:
            self.b = backend

    def _run(self, params, keep, on_value):
        b = self.b
        vals: dict[str, tuple[Any, list[int]]] = {}
        owner: dict[str, str] = {}   # value -> the name whose buffer it is (aliases share)
        end: dict[str, int] = {}     # buffer owner -> last op index reading it or an alias
        scalars: dict[str, float] = {}
        self.values = vals
        self._orphans: dict[str, Any] = {}  # owners dropped from vals while an alias lives
        self.record = []
        next_param, last = 0, None
        for i, op in enumerate(self.ops):
            shape = op.shape
            n = _n(shape)
            oc = op.opcode
            get = lambda k: vals[op.operands[k]]
            if oc == "parameter":
                m = re.search(r"parameter\((\d+)\)", op.raw)
                idx = int(m.group(1)) if m else next_param
                next_param = max(next_param, idx + 1)
                a = np.asarray(params[idx], np.float32)
                if a.size != n:
                    raise ValueError(f"parameter({idx}) has {a.size} values, {op.result} needs {n}")
                out = b.upload(a)
            elif oc == "constant":
                c = _constant(op.raw)
                scalars[op.result] = c
                one = b.upload(np.array([c], np.float32))
                if n == 1:
                    out = one
                else:  # materialised over the result shape (compiler.rs:298-300)
                    out = b.empty(n)
                    b.launch("hlo_broadcast", one, None, out, H.broadcast_push((1,), shape, (0,)))
                    b.free(one)
            elif oc in ALIASES:
                b.take()
                src, _ = get(0)
                vals[op.result] = (src, shape)
                own = owner[op.operands[0]]
                owner[op.result] = own
                end[own] = max(end[own], self.last_use.get(op.result, i))
                if op.operands[0] in scalars:
                    scalars[op.result] = scalars[op.operands[0]]
                last = op.result
                self._release(i, vals, owner, end, keep)
                continue
            elif oc in ("broadcast", "broadcast_in_dim"):
                src, ss = get(0)
                out = b.empty(n)
                dims = _ints(op.attrs.get("dimensions"))
                if len(dims) != len(ss):  # only the copy / splat cases need no `dimensions`
                    dims = list(range(len(shape) - len(ss), len(shape)))
                b.launch("hlo_broadcast", src, None, out, H.broadcast_push(ss, shape, dims))
            elif oc == "transpose":
                src, ss = get(0)
                out = b.empty(n)
                b.launch("hlo_transpose", src, None, out,
                         H.transpose_push(ss, _ints(op.attrs.get("dimensions"))))
            elif oc == "slice":
                src, ss = get(0)
                out = b.empty(n)
                st, lim, sp = _slice_spec(op.raw)
                b.launch("hlo_slice", src, None, out, H.slice_push(ss, st, lim, sp))
            elif oc == "concatenate":
                dim = (_ints(op.attrs.get("dimensions")) or [0])[0]
                out = b.empty(n)
                off = 0
                for k in range(len(op.operands)):
                    src, ss = get(k)
                    b.launch("hlo_concatenate_into", src, None, out,
                             H.concatenate_into_push(shape, ss, dim, off))
                    off += ss[dim]
            elif oc == "compare":
                (a, sa), (c, sc) = get(0), get(1)
                out = b.empty(n)
                b.launch("hlo_compare", a, c, out,
                         H.compare_push(op.attrs.get("direction", "GT"), shape, sa, sc))
            elif oc == "select":
                (p, sp_), (t, st_), (f, sf) = get(0), get(1), get(2)
                out = b.empty(n)
                if _n(sf) == n:
                    b.launch("reshape", f, None, out, [n])
                else:
                    b.launch("hlo_broadcast", f, None, out, H.broadcast_push(
                        sf, shape, list(range(len(shape) - len(sf), len(shape)))))
                b.launch("hlo_select", p, t, out, H.select_push(shape, sp_, st_))
            elif oc == "pad":
                src, ss = get(0)
                pv, _ = get(1)
                pads = _pairs(op.attrs.get("padding")) or [(0, 0)] * len(ss)
                if len(ss) > 4:
                    raise NotImplementedError("pad supports rank <= 4 (compiler.rs:1097-1099)")
                off = 4 - len(ss)
                od, idim, pl = [1] * 4, [1] * 4, [0] * 4
                for k in range(len(ss)):
                    od[off + k], idim[off + k], pl[off + k] = shape[k], ss[k], pads[k][0]
                out = b.empty(n)
                b.launch("pad", src, pv, out, [*od, *idim, *pl, n])
            elif oc == "convolution":
                (x, sx), (w, sw) = get(0), get(1)
                if op.attrs.get("dim_labels") != "b01f_01io->b01f" or len(sx) != 4:
                    raise NotImplementedError(f"convolution {op.attrs.get('dim_labels')} "
                                              "(compiler.rs:785-790 takes b01f_01io->b01f)")
                win = op.attrs.get("window")
                stride = _window(win, "stride") or [1, 1]
                pads = _pairs(win.split("pad=", 1)[1].split(" ")[0]) if win and "pad=" in win else [(0, 0), (0, 0)]
                out = b.empty(n)
                b.launch("hlo_conv_nhwc_hwio", x, w, out,
                         [*sx, sw[0], sw[1], sw[3], shape[1], shape[2], stride[0], stride[1],
                          pads[0][0], pads[1][0], n])
            elif oc in ("dot", "dot_general"):
                out = self._dot(op, get(0), get(1), n)
            elif oc == "reduce":
                src, ss = get(0)
                init = scalars.get(op.operands[1], 0.0)
                dims = _ints(op.attrs.get("dimensions"))
                kind = 1 if ("to_apply=%max" in op.raw or init == -np.inf) else 0
                out = b.empty(n)
                if len(ss) > 4:  # reduce_tensor (compiler.rs:1730-1759) on the device
                    b.launch("hlo_reduce", src, None, out,
                             H.reduce_push("max" if kind else "sum", ss, dims, init))
                else:
                    d4, flags, od = [1] * 4, [0] * 4, [1] * 4
                    for k, d in enumerate(ss):
                        d4[k] = d
                    for d in dims:
                        flags[d] = 1
                    cur = 0
                    for k in range(len(ss)):
                        if not flags[k]:
                            od[k] = shape[cur] if cur < len(shape) else 1
                            cur += 1
                    # as vulkan_reduce (compiler.rs:939-1007): the kernel folds from 0 or
                    # -inf by kind; the init operand only selects the kind
                    b.launch("hlo_reduce_rank4", src, None, out,
                             [len(ss), *d4, *od, *flags, kind, n])
            elif oc == "reduce-window":
                src, ss = get(0)
                init = scalars.get(op.operands[1], 0.0)
                win = op.attrs.get("window")
                size = _window(win, "size") or [1] * 4
                stride = _window(win, "stride") or [1] * 4
                pads = _pairs(win.split("pad=", 1)[1].split(" ")[0]) if win and "pad=" in win else []
                pt = pads[1][0] if len(pads) > 1 else 0
                pl = pads[2][0] if len(pads) > 2 else 0
                kind = 1 if ("to_apply=%max" in op.raw or init == -np.inf) else 0
                out = b.empty(n)
                b.launch("hlo_reduce_window_rank4", src, None, out,
                         [*ss, shape[1], shape[2], size[1], size[2], stride[1], stride[2],
                          pt, pl, kind, n])
            elif oc in ELEMENTWISE:
                kernel, arity = ELEMENTWISE[oc]
                ins, tmp = [], []
                for k in range(arity):
                    src, ss = get(k)
                    if _n(ss) != n:  # binary_tensor's operand broadcast (compiler.rs:705-729)
                        t = b.empty(n)
                        b.launch("hlo_broadcast", src, None, t, H.broadcast_push(
                            ss, shape, list(range(len(shape) - len(ss), len(shape)))))
                        tmp.append(t)
                        src = t
                    ins.append(src)
                out = b.empty(n)
                b.launch(kernel, ins[0], ins[1] if arity == 2 else None, out, [n])
                for t in tmp:
                    b.free(t)
            else:
                raise NotImplementedError(f"no device lowering for HLO op {oc} ({op.result})")
            vals[op.result] = (out, shape)
            owner[op.result] = op.result
            end[op.result] = self.last_use.get(op.result, i)
            self.record.append((op.result, oc, b.take()))
            if on_value is not None:
                on_value(op, out, shape)
            last = op.result
            self._release(i, vals, owner, end, keep)
        if last is None:
            raise ValueError("HLO module has no ENTRY instructions")
        return vals[last]

    def _dot(self, op: HloOp, lhs, rhs, n: int):
        """compiler.rs:1009-1084: one contracting dim per side; operands permuted to
        [B, M, K] / [B, K, N] (here on the device, skipped when already in that order),
        then hlo_dot_batched."""
        b = self.b
        (a, sa), (c, sc) = lhs, rhs
        lc, rc = _ints(op.attrs.get("lhs_contracting_dims")), _ints(op.attrs.get("rhs_contracting_dims"))
        lb, rb = _ints(op.attrs.get("lhs_batch_dims")), _ints(op.attrs.get("rhs_batch_dims"))
        if len(lc) != 1 or len(rc) != 1:
            raise NotImplementedError("dot_general requires exactly one contracting dim per side")
        K = sa[lc[0]]
        if K != sc[rc[0]]:
            raise ValueError(f"dot contracting dim mismatch {K} vs {sc[rc[0]]}")
        bsz = _n([sa[d] for d in lb])
        lf = [d for d in range(len(sa)) if d not in lb and d not in lc]
        rf = [d for d in range(len(sc)) if d not in rb and d not in rc]
        M, N = _n([sa[d] for d in lf]), _n([sc[d] for d in rf])
        tmp = []

        def permuted(t, shape, order):
            if list(order) == list(range(len(shape))):
                return t
            o = b.empty(_n(shape))
            b.launch("hlo_transpose", t, None, o, H.transpose_push(shape, order))
            tmp.append(o)
            return o

        a2 = permuted(a, sa, lb + lf + lc)
        c2 = permuted(c, sc, rb + rc + rf)
        out = b.empty(n)
        b.launch("hlo_dot_batched", a2, c2, out, [bsz, M, K, N, bsz * M * N])
        for t in tmp:
            b.free(t)
        return out

    def _release(self, i, vals, owner, end, keep):
        """After op i: free every buffer whose owner and aliases have all been read for the
        last time (never the buffer of op i's own result)."""
        cur = owner[self.ops[i].result]
        for own in [o for o, e in end.items() if e <= i and o != cur]:
            del end[own]
            if not keep:
                self.b.free(vals[own][0] if own in vals else self._orphans.pop(own))
        for k in [k for k in vals if self.last_use.get(k, -1) <= i and k != self.ops[i].result]:
            o = owner[k]
            if o == k and o in end:  # an alias still reads this buffer: keep it by owner
                self._orphans[o] = vals[k][0]
            del vals[k]
