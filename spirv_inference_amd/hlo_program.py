"""Compiled execution of an XLA HLO text module: strided views, fused epilogues, row-kernel
fusion, liveness-pooled buffers and a replayable launch list (hipGraph on the device).

The reference's HLO runner (source/xla_hlo/src/compiler.rs:267-640 `run_graph`) walks the ENTRY
computation once per run: every op is its own Vulkan dispatch with a host round trip, and the
shape ops (broadcast, transpose, slice, ...) copy on the CPU.  `hlo_exec.HloExecutor` keeps
that op-by-op lowering on resident tensors.  This module compiles the same op list once into a
short list of registry launches and replays it:

* Views.  reshape / convert / transpose / broadcast / slice / tuple / get-tuple-element make no
  copy: a value is (buffer, element offset, shape, element strides).  A kernel that needs a
  contiguous operand gets one from `hlo_strided_copy`; `dot` reads any operand layout in place
  through `dot_general_strided` (compiler.rs:1043-1058 permutes on the CPU instead) and can
  write its result directly in the layout of a following transpose.
* Fused epilogues.  convolution / dot followed by a bias add (a vector broadcast along the last
  axis), a residual add and a unary activation region become one `shp_launch_ex`.  The
  activation is recognised by evaluating the region (any chain of elementwise / compare /
  select ops of the value and constants, such as the erfc expansion of GELU in
  bert_base.stablehlo.txt:55-144) on probe values in float64 and comparing it with the
  epilogue activations (scheduler.rs:1146-1197's ReLU/ReLU6 and the GELU/SiLU/sigmoid/tanh
  forms).
* Row kernels.  reduce(max) -> subtract -> exponential -> reduce(sum) -> divide over the last
  axis (with an optional preceding scale multiply and mask add) is `softmax_rows` (and a
  scores dot -> softmax -> context dot over the column blocks of a fused QKV activation, at
  sequence 128 and head dim 64, is one `attention_fused`); the mean /
  variance / rsqrt chain of a LayerNorm is `layernorm_rows`; x * rsqrt(mean(x*x) + eps) * w is
  `rmsnorm_rows`; reduce(sum over H, W) / (H*W) of an NHWC tensor is `global_avg_pool_nhwc`;
  a zero pad in front of a convolution becomes the convolution's padding.
* Buffers are allocated while compiling and reused by liveness (same element count); the
  recorded launches are replayed eagerly or, on the device, from one hipGraph capture.

Everything else lowers as `HloExecutor` does (same kernels, same push vectors).
"""
from __future__ import annotations

import math
import re
from typing import Any, Sequence

import numpy as np

from . import hlo_ops as H
from .hlo_exec import ELEMENTWISE, HloOp, _constant, _ints, _n, _pairs, _slice_spec, _window

_UNARY_REGION_OPS = {"add", "subtract", "multiply", "divide", "maximum", "minimum", "abs",
                     "negate", "exponential", "log", "sqrt", "rsqrt", "tanh", "logistic",
                     "compare", "select", "power", "sine", "cosine"}
# epilogue activations (SHP_ACT_*) the unary-region matcher can recognise
_ACT_CANDIDATES = {
    1: lambda x: np.maximum(x, 0.0),
    2: lambda x: np.minimum(np.maximum(x, 0.0), 6.0),
    4: lambda x: 1.0 / (1.0 + np.exp(-x)),
    5: np.tanh,
    6: lambda x: x / (1.0 + np.exp(-x)),
    7: lambda x: 0.5 * x * np.array([math.erfc(-v / math.sqrt(2.0)) if not math.isnan(v)
                                      else math.nan for v in x]),
}
# Probe values on which a region must equal an activation before it is fused: a dense sweep
# of [-12, 12], then magnitudes out to the float32 limit (a clamp at 20 or 1e4 that equals
# ReLU on the sweep differs there), the tiny and non-finite values.
_WIDE = np.array([12.5, 15.0, 19.99, 20.0, 20.01, 25.0, 50.0, 88.0, 100.0, 1e3, 1e4, 1e5, 1e10,
                  1e20, 1e30, 3.4e38, 1e-30, 1e-38])
_PROBES = np.concatenate([np.linspace(-12.0, 12.0, 2401), [0.0, 1e-4, -1e-4, 0.5, -0.5],
                          _WIDE, -_WIDE, [np.inf, -np.inf, np.nan]])


def _same(y: np.ndarray, ref: np.ndarray) -> bool:
    """y equals ref on every probe: within 1e-5 * (1 + |ref|) where ref is finite, the same
    infinity where it is infinite, NaN where it is NaN."""
    fin = np.isfinite(ref)
    with np.errstate(invalid="ignore"):
        close = np.abs(y[fin] - ref[fin]) <= 1e-5 * (1.0 + np.abs(ref[fin]))
    inf = np.isinf(ref)
    nan = np.isnan(ref)
    return bool(np.all(close) and np.all(y[inf] == ref[inf]) and np.all(np.isnan(y[nan])))


def _rm_strides(shape: Sequence[int]) -> tuple:
    st, s = [], 1
    for d in reversed(shape):
        st.append(s)
        s *= d
    return tuple(reversed(st))


class Buf:
    """One backend allocation (or a caller's tensor) and how many live values view it."""

    def __init__(self, handle, n: int, pinned: bool):
        self.handle, self.n, self.pinned, self.refs = handle, n, pinned, 0


class View:
    __slots__ = ("buf", "off", "shape", "strides")

    def __init__(self, buf: Buf, off: int, shape: Sequence[int], strides: Sequence[int]):
        self.buf, self.off, self.shape, self.strides = buf, int(off), tuple(shape), tuple(strides)

    @property
    def n(self) -> int:
        return _n(self.shape)

    def contiguous(self) -> bool:
        return all(d == 1 or s == r for d, s, r in zip(self.shape, self.strides,
                                                        _rm_strides(self.shape)))

    def extent(self) -> int:
        """Elements from the first to one past the last element the view touches."""
        return 1 + sum((d - 1) * s for d, s in zip(self.shape, self.strides))


def _reshape_view(v: View, shape: Sequence[int]) -> View | None:
    """The view of `v`'s elements in row-major order under a new shape, without a copy, or
    None if the strides do not allow it (numpy's no-copy reshape rule)."""
    shape = tuple(shape)
    if v.contiguous():
        return View(v.buf, v.off, shape, _rm_strides(shape))
    old = [(d, s) for d, s in zip(v.shape, v.strides) if d != 1]
    new_nz = [d for d in shape if d != 1]
    out_strides: list[int] = []
    i = j = 0
    while i < len(old) and j < len(new_nz):
        # group old dims [i, i2) and new dims [j, j2) with equal products
        po, pn, i2, j2 = old[i][0], new_nz[j], i + 1, j + 1
        while po != pn:
            if po < pn:
                if i2 >= len(old):
                    return None
                po *= old[i2][0]
                i2 += 1
            else:
                if j2 >= len(new_nz):
                    return None
                pn *= new_nz[j2]
                j2 += 1
        for k in range(i, i2 - 1):  # the old group must be one strided run
            if old[k][1] != old[k + 1][1] * old[k + 1][0]:
                return None
        st = old[i2 - 1][1]
        grp = []
        for k in range(j2 - 1, j - 1, -1):
            grp.append(st)
            st *= new_nz[k]
        out_strides.extend(reversed(grp))
        i, j = i2, j2
    if i != len(old) or j != len(new_nz):
        return None
    it = iter(out_strides)
    return View(v.buf, v.off, shape, tuple(next(it) if d != 1 else 0 for d in shape))


class HloProgram:
    """An HLO ENTRY op list compiled for a backend.

    backend: DeviceBackend (product) or any object with the same interface
             (upload, empty, sub, write, launch, read, free).
    params:  one entry per parameter: a numpy array (uploaded into a buffer the program owns),
             a backend tensor (used in place), or (backend tensor, element offset).
    run() executes the recorded launches (eager, or one hipGraph replay when graph=True on a
    backend that can capture); outputs() gives the ROOT values (a tuple ROOT gives several).
    """

    def __init__(self, backend: Any, ops: Sequence[HloOp], params: Sequence[Any],
                 fuse: bool = True):
        self.b, self.ops, self.fuse = backend, list(ops), fuse
        self.idx = {op.result: i for i, op in enumerate(self.ops)}
        self.consumers: dict[str, list[int]] = {op.result: [] for op in self.ops}
        for i, op in enumerate(self.ops):
            for o in op.operands:
                if o in self.consumers and i not in self.consumers[o]:
                    self.consumers[o].append(i)
        self.launches: list[tuple] = []
        self.launch_src: list[str] = []  # the HLO result each launch is recorded for
        self._cur = None
        self.pool: dict[int, list[Buf]] = {}
        self.owned: list[Buf] = []
        self.fused_counts: dict[str, int] = {}
        self._graph = None
        self._warm = False
        self._roots = self._root_names()
        self.groups = self._analyse() if fuse else {}
        self.absorbed = {j for g in self.groups.values() for j in g["members"]}
        self._compile(params)

    # ------------------------------------------------------------------ analysis helpers
    def _op(self, name: str) -> HloOp | None:
        i = self.idx.get(name)
        return self.ops[i] if i is not None else None

    def _root_names(self) -> list[str]:
        root = self.ops[-1]
        if root.opcode == "tuple":
            return list(root.operands)
        return [root.result]

    def _sole(self, name: str) -> int | None:
        """Index of the one consumer of `name`, or None (several, none, or a program output)."""
        c = self.consumers.get(name, [])
        if len(c) != 1 or name in self._roots:
            return None
        return c[0]

    def const_value(self, name: str) -> float | None:
        """Value of a scalar-constant expression (constants through reshape / convert /
        broadcast and elementwise ops of constants), else None."""
        op = self._op(name)
        if op is None:
            return None
        if op.opcode == "constant":
            if "{" in op.raw.split("constant(", 1)[1].split(")", 1)[0]:
                return None
            try:
                return float(_constant(op.raw))
            except ValueError:
                return None
        if op.opcode in ("reshape", "convert", "broadcast", "broadcast_in_dim"):
            return self.const_value(op.operands[0])
        if op.opcode in ELEMENTWISE:
            vals = [self.const_value(o) for o in op.operands]
            if any(v is None for v in vals):
                return None
            with np.errstate(all="ignore"):
                return float(_eval_elementwise(op.opcode, [np.float64(v) for v in vals]))
        return None

    def _trace_vector(self, name: str, out_shape: Sequence[int]) -> str | None:
        """If `name` is a vector broadcast along the last axis of `out_shape` (through reshape
        / convert / broadcast ops), the name of the vector's source value, else None."""
        n_last = out_shape[-1] if out_shape else 1
        cur, seen_bcast = name, False
        while True:
            op = self._op(cur)
            if op is None:
                return None
            if op.opcode in ("reshape", "convert"):
                src = self._op(op.operands[0])
                if src is None or _n(src.shape) != _n(op.shape):
                    return None
                cur = op.operands[0]
                continue
            if op.opcode in ("broadcast", "broadcast_in_dim"):
                src = self._op(op.operands[0])
                if src is None:
                    return None
                dims = _ints(op.attrs.get("dimensions"))
                nz = [(a, d) for a, d in enumerate(src.shape) if d != 1]
                if len(dims) != len(src.shape) or len(nz) != 1:
                    return None
                a, d = nz[0]
                if seen_bcast or d != n_last or dims[a] != len(op.shape) - 1:
                    return None
                seen_bcast = True
                cur = op.operands[0]
                continue
            break
        op = self._op(cur)
        if not seen_bcast or op is None or _n(op.shape) != n_last:
            return None
        return cur

    def _row_bcast_source(self, name: str, x_shape: Sequence[int]) -> str | None:
        """If `name` broadcasts a per-row value (shape x_shape[:-1]) along the last axis of
        x_shape (through reshape / broadcast ops), that per-row value's name."""
        rows = _n(x_shape[:-1])
        cur, ok = name, False
        while True:
            op = self._op(cur)
            if op is None:
                return None
            if op.opcode in ("reshape", "convert"):
                cur = op.operands[0]
                continue
            if op.opcode in ("broadcast", "broadcast_in_dim"):
                src = self._op(op.operands[0])
                if src is None:
                    return None
                dims = _ints(op.attrs.get("dimensions"))
                if _n(src.shape) == _n(op.shape):
                    if dims != list(range(len(src.shape))):
                        return None
                elif list(op.shape) == list(x_shape) and _n(src.shape) == rows and \
                        dims == list(range(len(x_shape) - 1))[:len(src.shape)] and \
                        list(src.shape) == list(x_shape[:len(src.shape)]):
                    ok = True
                else:
                    return None
                cur = op.operands[0]
                continue
            break
        op = self._op(cur)
        if not ok or op is None or _n(op.shape) != rows:
            return None
        return cur

    def _is_reduce(self, op: HloOp, x: str, kind: str, dims: list[int]) -> bool:
        if op is None or op.opcode != "reduce" or op.operands[0] != x:
            return False
        init = self.const_value(op.operands[1]) if len(op.operands) > 1 else None
        is_max = "to_apply=%max" in op.raw or init == -np.inf
        if kind == "max" and not is_max:
            return False
        if kind == "sum" and (is_max or init not in (0.0, None)):
            return False
        return _ints(op.attrs.get("dimensions")) == dims

    def _binary_other(self, op: HloOp, name: str) -> str | None:
        if op is None or len(op.operands) != 2 or name not in op.operands:
            return None
        a, b = op.operands
        if a == name and b == name:
            return name
        return b if a == name else a

    def _unary_region(self, x: str, limit: int = 512):
        """(member indices, exit name, act code) of the elementwise region computing one
        epilogue activation of `x`, or None."""
        xi = self.idx[x]
        inset, members, pending = {x}, [], set(self.consumers.get(x, []))
        while pending:
            j = min(pending)
            pending.discard(j)
            if j - xi > limit:
                return None
            op = self.ops[j]
            if op.opcode not in _UNARY_REGION_OPS:
                return self._close_region(x, members, inset)
            if not all(o in inset or self.const_value(o) is not None for o in op.operands):
                # an outside consumer of a region value: allowed only for the exit, which is
                # decided below; stop growing here
                return self._close_region(x, members, inset)
            members.append(j)
            inset.add(op.result)
            pending.update(self.consumers.get(op.result, []))
        return self._close_region(x, members, inset)

    def _close_region(self, x: str, members: list[int], inset: set):
        if not members:
            return None
        mset = set(members)
        exits = [self.ops[j].result for j in members
                 if self.ops[j].result in self._roots or
                 any(c not in mset for c in self.consumers.get(self.ops[j].result, []))]
        if len(exits) != 1 or any(c not in mset for c in self.consumers.get(x, [])):
            return None
        exit_name = exits[0]
        # every member must feed the exit (no dead side branches)
        act = self._identify(x, sorted(members), exit_name)
        if act is None:
            return None
        return sorted(members), exit_name, act

    def _identify(self, x: str, members: list[int], exit_name: str) -> int | None:
        env = {x: _PROBES.astype(np.float64)}
        with np.errstate(all="ignore"):
            for j in members:
                op = self.ops[j]
                args = []
                for o in op.operands:
                    if o in env:
                        args.append(env[o])
                    else:
                        args.append(np.float64(self.const_value(o)))
                if op.opcode == "compare":
                    env[op.result] = _compare(op.attrs.get("direction", "GT"), *args)
                elif op.opcode == "select":
                    env[op.result] = np.where(np.asarray(args[0]) != 0, args[1], args[2])
                else:
                    env[op.result] = _eval_elementwise(op.opcode, args)
            y = np.broadcast_to(env[exit_name], _PROBES.shape)
            for code, f in _ACT_CANDIDATES.items():
                if _same(y, f(_PROBES)):
                    return code
        return None

    # ------------------------------------------------------------------ pattern analysis
    def _analyse(self) -> dict[int, dict]:
        """Fusion groups keyed by their anchor (the op index where the fused launch is
        recorded): {"kind", "members" (absorbed op indices), "inputs", ...}."""
        groups: dict[int, dict] = {}
        taken: set[int] = set()
        self._taken = taken

        def free(js):
            return not any(j in taken for j in js)

        for i, op in enumerate(self.ops):
            if i in taken:
                continue
            g = None
            if op.opcode in ("convolution", "dot"):
                g = self._match_epilogue(i)
            elif op.opcode == "reduce":
                g = self._match_softmax(i) or self._match_layernorm(i) or self._match_meanpool(i)
            elif op.opcode == "multiply":
                g = self._match_rmsnorm(i)
            elif op.opcode == "pad":
                g = None
            if g is None:
                continue
            js = set(g["members"]) | {g["anchor"]}
            if not free(js):
                continue
            taken |= js
            groups[g["anchor"]] = g
        return groups

    def _match_epilogue(self, i: int) -> dict | None:
        head = self.ops[i]
        cur, members = head.result, []
        bias = residual = None
        act = 0
        pad_src = None
        if head.opcode == "convolution":  # a zero pad in front folds into the conv padding
            pop = self._op(head.operands[0])
            if pop is not None and pop.opcode == "pad" and self._sole(pop.result) == i and \
                    self.const_value(pop.operands[1]) == 0.0 and len(pop.shape) == 4:
                pads = _pairs(pop.attrs.get("padding"))
                if len(pads) == 4 and pads[0] == (0, 0) and pads[3] == (0, 0) and \
                        all(lo >= 0 and hi >= 0 for lo, hi in pads):
                    pad_src = (pop.operands[0], pads[1][0], pads[2][0], self.idx[pop.result])
        while True:
            j = self._sole(cur)
            c = self.ops[j] if j is not None else None
            if c is not None and c.opcode in ("reshape", "convert") and \
                    list(c.shape) == list(self._op(cur).shape):
                members.append(j); cur = c.result; continue
            if c is not None and c.opcode == "transpose" and \
                    _ints(c.attrs.get("dimensions")) == list(range(len(c.shape))):
                members.append(j); cur = c.result; continue
            if c is not None and c.opcode == "add" and bias is None and residual is None and \
                    act == 0:
                other = self._binary_other(c, cur)
                vec = self._trace_vector(other, c.shape) if other else None
                if vec is not None and vec != cur and self.idx.get(vec, 1 << 30) < j:
                    bias = vec; members.append(j); cur = c.result; continue
            if c is not None and c.opcode == "add" and residual is None and act == 0:
                # the residual must exist before the head, so the fused launch can read it
                other = self._binary_other(c, cur)
                oo = self._op(other) if other else None
                if other and other != cur and oo is not None and \
                        list(oo.shape) == list(c.shape) and self.idx[other] < i:
                    residual = other; members.append(j); cur = c.result; continue
            if act == 0:
                reg = self._unary_region(cur)
                if reg is not None:
                    rmem, exit_name, code = reg
                    members += rmem
                    cur, act = exit_name, code
                    continue
            break
        if not members and pad_src is None:
            return None
        anchor = self.idx[cur]
        absorbed = [m for m in members if m != anchor]
        if members:
            absorbed.append(i)
        inputs = [o for o in head.operands] + [x for x in (bias, residual) if x]
        if pad_src is not None:
            absorbed.append(pad_src[3])
            inputs[0] = pad_src[0]
        if not members:  # only the pad: the conv itself is the anchor
            anchor, absorbed = i, [pad_src[3]]
        return {"kind": "epilogue", "anchor": anchor, "head": i, "members": absorbed,
                "inputs": inputs, "bias": bias, "residual": residual, "act": act,
                "pad": pad_src, "out": cur}

    def _match_softmax(self, i: int) -> dict | None:
        m = self.ops[i]
        x = m.operands[0]
        xo = self._op(x)
        if xo is None or not xo.shape:
            return None
        r = len(xo.shape)
        if not self._is_reduce(m, x, "max", [r - 1]):
            return None
        # subtract(x, rowbcast(m))
        members = [i]
        sub = None
        for c in self.consumers.get(x, []):
            co = self.ops[c]
            if co.opcode == "subtract" and co.operands[0] == x and \
                    self._row_bcast_source(co.operands[1], xo.shape) == m.result:
                sub = c
        if sub is None:
            return None
        if not self._chain_only(m.result, self.ops[sub].operands[1], sub, members):
            return None
        members.append(sub)
        e = self._sole(self.ops[sub].result)
        if e is None or self.ops[e].opcode != "exponential":
            return None
        members.append(e)
        en = self.ops[e].result
        ce = self.consumers.get(en, [])
        if len(ce) != 2 or en in self._roots:
            return None
        zi = next((c for c in ce if self._is_reduce(self.ops[c], en, "sum", [r - 1])), None)
        di = next((c for c in ce if self.ops[c].opcode == "divide" and
                   self.ops[c].operands[0] == en), None)
        if zi is None or di is None:
            return None
        if self._row_bcast_source(self.ops[di].operands[1], xo.shape) != self.ops[zi].result:
            return None
        members.append(zi)
        if not self._chain_only(self.ops[zi].result, self.ops[di].operands[1], di, members):
            return None
        # x's consumers must be the max reduce and the subtract
        if sorted(self.consumers.get(x, [])) != sorted([i, sub]):
            return None
        scale, mask, src = 1.0, None, x
        expect = sorted([i, sub])
        a = self._op(src)
        if a is not None and a.opcode == "add" and src not in self._roots and \
                self.idx[a.result] not in self._taken:
            for k in (0, 1):
                vec = self._trace_vector(a.operands[1 - k], a.shape)
                if vec is not None and self._op(a.operands[k]) is not None and \
                        list(self._op(a.operands[k]).shape) == list(a.shape):
                    mask, src = vec, a.operands[k]
                    members.append(self.idx[a.result])
                    expect = [self.idx[a.result]]
                    break
        a = self._op(src)
        if a is not None and a.opcode == "multiply" and src not in self._roots and \
                self.idx[a.result] not in self._taken and \
                sorted(self.consumers.get(a.result, [])) == expect:
            for k in (0, 1):
                cv = self.const_value(a.operands[1 - k])
                if cv is not None and self._op(a.operands[k]) is not None and \
                        list(self._op(a.operands[k]).shape) == list(a.shape):
                    scale, src = cv, a.operands[k]
                    members.append(self.idx[a.result])
                    break
        return {"kind": "softmax", "anchor": di, "members": members, "inputs":
                [src] + ([mask] if mask else []), "x": src, "mask": mask, "scale": scale,
                "rows": _n(xo.shape[:-1]), "cols": xo.shape[-1]}

    def _chain_only(self, src: str, dst: str, user: int, members: list[int]) -> bool:
        """The reshape/broadcast chain from `src` to `dst` is used only on that path (and
        `dst` only by `user`); its ops are added to members."""
        chain, cur = [], dst
        while cur != src:
            op = self._op(cur)
            if op is None or op.opcode not in ("reshape", "convert", "broadcast",
                                               "broadcast_in_dim"):
                return False
            chain.append(self.idx[cur])
            cur = op.operands[0]
        for j in chain:
            r = self.ops[j].result
            cons = self.consumers.get(r, [])
            if len(cons) != 1 or r in self._roots:
                return False
        if len(self.consumers.get(src, [])) != 1 or src in self._roots:
            return False
        members.extend(chain)
        return True

    def _match_layernorm(self, i: int) -> dict | None:
        s1 = self.ops[i]
        x = s1.operands[0]
        xo = self._op(x)
        if xo is None or not xo.shape:
            return None
        r, D = len(xo.shape), xo.shape[-1]
        if not self._is_reduce(s1, x, "sum", [r - 1]):
            return None
        members = [i]
        mj = self._sole(s1.result)
        if mj is None or self.ops[mj].opcode != "divide" or self.ops[mj].operands[0] != s1.result \
                or self.const_value(self.ops[mj].operands[1]) != float(D):
            return None
        members.append(mj)
        mean = self.ops[mj].result
        sub = None
        for c in self.consumers.get(x, []):
            co = self.ops[c]
            if co.opcode == "subtract" and co.operands[0] == x and \
                    self._row_bcast_source(co.operands[1], xo.shape) == mean:
                sub = c
        if sub is None or not self._chain_only(mean, self.ops[sub].operands[1], sub, members):
            return None
        members.append(sub)
        d = self.ops[sub].result
        dc = self.consumers.get(d, [])
        sq = next((c for c in dc if self.ops[c].opcode == "multiply" and
                   self.ops[c].operands == [d, d]), None)
        if sq is None or len(dc) != 2 or d in self._roots:
            return None
        nj = next(c for c in dc if c != sq)
        members.append(sq)
        s2 = self._sole(self.ops[sq].result)
        if s2 is None or not self._is_reduce(self.ops[s2], self.ops[sq].result, "sum", [r - 1]):
            return None
        members.append(s2)
        vj = self._sole(self.ops[s2].result)
        if vj is None or self.ops[vj].opcode != "divide" or \
                self.const_value(self.ops[vj].operands[1]) != float(D):
            return None
        members.append(vj)
        aj = self._sole(self.ops[vj].result)
        if aj is None or self.ops[aj].opcode != "add":
            return None
        eps = self.const_value(self._binary_other(self.ops[aj], self.ops[vj].result) or "")
        if eps is None:
            return None
        members.append(aj)
        rj = self._sole(self.ops[aj].result)
        if rj is None or self.ops[rj].opcode != "rsqrt":
            return None
        members.append(rj)
        no = self.ops[nj]
        if no.opcode != "multiply" or self._row_bcast_source(
                self._binary_other(no, d) or "", xo.shape) != self.ops[rj].result:
            return None
        if not self._chain_only(self.ops[rj].result, self._binary_other(no, d), nj, members):
            return None
        members.append(nj)
        gj = self._sole(no.result)
        if gj is None or self.ops[gj].opcode != "multiply":
            return None
        gamma = self._trace_vector(self._binary_other(self.ops[gj], no.result) or "", xo.shape)
        if gamma is None:
            return None
        members.append(gj)
        bj = self._sole(self.ops[gj].result)
        if bj is None or self.ops[bj].opcode != "add":
            return None
        beta = self._trace_vector(self._binary_other(self.ops[bj], self.ops[gj].result) or "",
                                  xo.shape)
        if beta is None:
            return None
        if sorted(self.consumers.get(x, [])) != sorted([i, sub]):
            return None
        return {"kind": "layernorm", "anchor": bj, "members": members,
                "inputs": [x, gamma, beta], "x": x, "gamma": gamma, "beta": beta,
                "eps": eps, "rows": _n(xo.shape[:-1]), "cols": D}

    def _match_rmsnorm(self, i: int) -> dict | None:
        sq = self.ops[i]
        if len(sq.operands) != 2 or sq.operands[0] != sq.operands[1]:
            return None
        x = sq.operands[0]
        xo = self._op(x)
        if xo is None or not xo.shape:
            return None
        r, D = len(xo.shape), xo.shape[-1]
        members = [i]
        sj = self._sole(sq.result)
        if sj is None or not self._is_reduce(self.ops[sj], sq.result, "sum", [r - 1]):
            return None
        members.append(sj)
        mj = self._sole(self.ops[sj].result)
        if mj is None or self.ops[mj].opcode != "divide" or \
                self.const_value(self.ops[mj].operands[1]) != float(D):
            return None
        members.append(mj)
        aj = self._sole(self.ops[mj].result)
        if aj is None or self.ops[aj].opcode != "add":
            return None
        eps = self.const_value(self._binary_other(self.ops[aj], self.ops[mj].result) or "")
        if eps is None:
            return None
        members.append(aj)
        rj = self._sole(self.ops[aj].result)
        if rj is None or self.ops[rj].opcode != "rsqrt":
            return None
        members.append(rj)
        nj = None
        for c in self.consumers.get(x, []):
            co = self.ops[c]
            if co.opcode == "multiply" and c != i and \
                    self._row_bcast_source(self._binary_other(co, x) or "", xo.shape) == \
                    self.ops[rj].result:
                nj = c
        if nj is None or not self._chain_only(self.ops[rj].result,
                                              self._binary_other(self.ops[nj], x), nj, members):
            return None
        members.append(nj)
        wj = self._sole(self.ops[nj].result)
        if wj is None or self.ops[wj].opcode != "multiply":
            return None
        w = self._trace_vector(self._binary_other(self.ops[wj], self.ops[nj].result) or "",
                               xo.shape)
        if w is None:
            return None
        if sorted(self.consumers.get(x, [])) != sorted([i, nj]) and x not in self._roots:
            # x has other readers: fine, the fused kernel only reads it
            pass
        return {"kind": "rmsnorm", "anchor": wj, "members": members, "inputs": [x, w],
                "x": x, "w": w, "eps": eps, "rows": _n(xo.shape[:-1]), "cols": D}

    def _match_meanpool(self, i: int) -> dict | None:
        s = self.ops[i]
        x = s.operands[0]
        xo = self._op(x)
        if xo is None or len(xo.shape) != 4 or not self._is_reduce(s, x, "sum", [1, 2]):
            return None
        dj = self._sole(s.result)
        n, h, w, c = xo.shape
        if dj is None or self.ops[dj].opcode != "divide" or self.ops[dj].operands[0] != s.result \
                or self.const_value(self.ops[dj].operands[1]) != float(h * w):
            return None
        return {"kind": "meanpool", "anchor": dj, "members": [i], "inputs": [x], "x": x,
                "dims": [n, h, w, c]}

    # ------------------------------------------------------------------ compilation
    def _alloc(self, n: int) -> Buf:
        lst = self.pool.get(n)
        if lst:
            return lst.pop()
        b = Buf(self.b.empty(n), n, pinned=False)
        self.owned.append(b)
        return b

    def _hold(self, v):
        if isinstance(v, list):
            for x in v:
                self._hold(x)
        elif v is not None:
            v.buf.refs += 1

    def _drop(self, v):
        if isinstance(v, list):
            for x in v:
                self._drop(x)
            return
        if v is None:
            return
        v.buf.refs -= 1
        if v.buf.refs == 0 and not v.buf.pinned:
            self.pool.setdefault(v.buf.n, []).append(v.buf)

    def _h(self, v: View, n: int | None = None):
        """Backend handle of the elements a view starts at."""
        return self.b.sub(v.buf.handle, v.off, v.extent() if n is None else n)

    def _launch(self, kernel, in0, in1, out, push, bias=None, residual=None, act=0,
                alpha=0.0, out_elems=None):
        self.launches.append((kernel, in0, in1, out, [int(p) for p in push], bias, residual,
                              int(act), float(alpha), out_elems))
        self.launch_src.append(self._cur)

    def _new(self, shape: Sequence[int]) -> View:
        n = max(1, _n(shape))
        return View(self._alloc(n), 0, shape, _rm_strides(shape))

    def _contig(self, v: View, temps: list) -> View:
        """`v` itself if it is contiguous, else a contiguous copy (hlo_strided_copy)."""
        if v.contiguous():
            return v
        out = self._new(v.shape)
        out.buf.refs += 1
        temps.append(out)
        shape = list(v.shape) or [1]
        strides = list(v.strides) or [0]
        self._launch("hlo_strided_copy", self._h(v), None, self._h(out),
                     [len(shape), _n(shape), *shape, *strides], out_elems=out.n)
        return out

    def _compile(self, params: Sequence[Any]) -> None:
        # effective last use: an op absorbed into a group is read at the group's anchor
        eff: dict[str, int] = {}
        anchor_of = {}
        for a, g in self.groups.items():
            for m in g["members"]:
                anchor_of[m] = a
        for i, op in enumerate(self.ops):
            at = anchor_of.get(i, i)
            srcs = self.groups[i]["inputs"] if i in self.groups else op.operands
            for o in srcs:
                eff[o] = max(eff.get(o, -1), at)
            if i not in self.groups:
                for o in op.operands:
                    eff[o] = max(eff.get(o, -1), at)
        self.vals: dict[str, Any] = {}
        self.param_views: dict[int, View] = {}
        self._param_bufs: dict[Any, Buf] = {}
        next_param = 0
        for i, op in enumerate(self.ops):
            if i in self.absorbed and i not in self.groups:
                self._release_after(i, eff)
                continue
            self._cur = op.result
            if i in self.groups:
                v = self._lower_group(self.groups[i])
            elif op.opcode == "parameter":
                m = re.search(r"parameter\((\d+)\)", op.raw)
                pidx = int(m.group(1)) if m else next_param
                next_param = max(next_param, pidx + 1)
                v = self._bind_param(pidx, params[pidx], op.shape)
            else:
                v = self._lower(op)
            self.vals[op.result] = v
            self._hold(v)
            self._release_after(i, eff)
        outs = []
        for name in self._roots:
            self._cur = name
            v = self.vals[name]
            temps: list = []
            c = self._contig(v, temps)
            c.buf.pinned = True
            outs.append(c)
        self._outputs = outs

    def _release_after(self, i: int, eff: dict[str, int]) -> None:
        for name in [k for k in list(self.vals) if eff.get(k, -1) <= i and k not in self._roots]:
            self._drop(self.vals.pop(name))

    def _bind_param(self, idx: int, p: Any, shape: Sequence[int]) -> View:
        n = _n(shape)
        if isinstance(p, np.ndarray):
            a = np.ascontiguousarray(p, np.float32).reshape(-1)
            if a.size != n:
                raise ValueError(f"parameter({idx}) has {a.size} values, needs {n}")
            buf = Buf(self.b.upload(a), n, pinned=True)
            self.owned.append(buf)
        else:
            handle, off = (p if isinstance(p, tuple) else (p, 0))
            # parameters bound to one tensor share one Buf (so adjacent views are seen as such)
            key = getattr(handle, "ptr", None) or id(handle)
            buf = self._param_bufs.get(key)
            if buf is None:
                buf = Buf(handle, getattr(handle, "n", n + off), pinned=True)
                self._param_bufs[key] = buf
            v = View(buf, off, shape, _rm_strides(shape))
            self.param_views[idx] = v
            return v
        v = View(buf, 0, shape, _rm_strides(shape))
        self.param_views[idx] = v
        return v

    def set_param(self, idx: int, arr: np.ndarray) -> None:
        """Write new values into parameter `idx`'s buffer (the recorded launches keep it)."""
        v = self.param_views[idx]
        a = np.ascontiguousarray(arr, np.float32).reshape(-1)
        if a.size != v.n:
            raise ValueError(f"parameter({idx}) needs {v.n} values, got {a.size}")
        self.b.write(v.buf.handle, v.off, a)

    # ---- lowering of single ops
    def _get(self, name: str):
        return self.vals[name]

    def _lower(self, op: HloOp):
        oc, shape = op.opcode, op.shape
        n = _n(shape)
        temps: list = []
        try:
            if oc == "constant":
                c = float(_constant(op.raw))
                buf = Buf(self.b.upload(np.array([c], np.float32)), 1, pinned=True)
                self.owned.append(buf)
                return View(buf, 0, shape, (0,) * len(shape))
            if oc in ("tuple",):
                return [self._get(o) for o in op.operands]
            if oc == "get-tuple-element":
                src = self._get(op.operands[0])
                k = int(op.attrs.get("index", 0))
                return src[k] if isinstance(src, list) else src
            if oc in ("reshape", "convert"):
                src = self._get(op.operands[0])
                if list(src.shape) == list(shape):
                    return src
                v = _reshape_view(src, shape)
                if v is None:
                    c = self._contig(src, temps)
                    v = View(c.buf, c.off, shape, _rm_strides(shape))
                    temps.remove(c)  # the copy becomes this value's buffer
                    c.buf.refs -= 1
                return v
            if oc == "transpose":
                src = self._get(op.operands[0])
                perm = _ints(op.attrs.get("dimensions"))
                return View(src.buf, src.off, shape, tuple(src.strides[p] for p in perm))
            if oc in ("broadcast", "broadcast_in_dim"):
                src = self._get(op.operands[0])
                dims = _ints(op.attrs.get("dimensions"))
                if len(dims) != len(src.shape):
                    dims = list(range(len(shape) - len(src.shape), len(shape)))
                st = [0] * len(shape)
                for a, d in enumerate(dims):
                    if src.shape[a] != 1:
                        if src.shape[a] != shape[d]:
                            raise ValueError(f"broadcast {op.result}: dim {a} does not match")
                        st[d] += src.strides[a]
                return View(src.buf, src.off, shape, tuple(st))
            if oc == "slice":
                src = self._get(op.operands[0])
                st, lim, sp = _slice_spec(op.raw)
                off = src.off + sum(s * t for s, t in zip(st, src.strides))
                return View(src.buf, off, shape, tuple(t * s for t, s in zip(src.strides, sp)))
            if oc in ("dot", "dot_general"):
                return self._dot(op, None, None, 0, temps, None)
            out = self._new(shape)
            if oc == "concatenate":
                dim = (_ints(op.attrs.get("dimensions")) or [0])[0]
                off = 0
                for k in range(len(op.operands)):
                    src = self._contig(self._get(op.operands[k]), temps)
                    self._launch("hlo_concatenate_into", self._h(src), None, self._h(out),
                                 H.concatenate_into_push(shape, src.shape, dim, off), out_elems=n)
                    off += src.shape[dim]
            elif oc == "compare":
                a = self._full(self._get(op.operands[0]), shape, temps)
                c = self._full(self._get(op.operands[1]), shape, temps)
                self._launch("hlo_compare", self._h(a), self._h(c), self._h(out),
                             H.compare_push(op.attrs.get("direction", "GT"), shape, shape, shape),
                             out_elems=n)
            elif oc == "select":
                p = self._full(self._get(op.operands[0]), shape, temps)
                t = self._full(self._get(op.operands[1]), shape, temps)
                f = self._full(self._get(op.operands[2]), shape, temps)
                self._launch("reshape", self._h(f), None, self._h(out), [n], out_elems=n)
                self._launch("hlo_select", self._h(p), self._h(t), self._h(out),
                             H.select_push(shape, shape, shape), out_elems=n)
            elif oc == "pad":
                src = self._contig(self._get(op.operands[0]), temps)
                pv = self._contig(self._get(op.operands[1]), temps)
                ss = src.shape
                pads = _pairs(op.attrs.get("padding")) or [(0, 0)] * len(ss)
                if len(ss) > 4:
                    raise NotImplementedError("pad supports rank <= 4 (compiler.rs:1097-1099)")
                off = 4 - len(ss)
                od, idim, pl = [1] * 4, [1] * 4, [0] * 4
                for k in range(len(ss)):
                    od[off + k], idim[off + k], pl[off + k] = shape[k], ss[k], pads[k][0]
                self._launch("pad", self._h(src), self._h(pv, 1), self._h(out),
                             [*od, *idim, *pl, n], out_elems=n)
            elif oc == "convolution":
                self._conv(op, self._get(op.operands[0]), 0, 0, None, None, 0, out, temps)
            elif oc == "reduce":
                src = self._contig(self._get(op.operands[0]), temps)
                init = self.const_value(op.operands[1]) if len(op.operands) > 1 else 0.0
                init = 0.0 if init is None else init
                dims = _ints(op.attrs.get("dimensions"))
                kind = 1 if ("to_apply=%max" in op.raw or init == -np.inf) else 0
                ss = src.shape
                if len(ss) > 4:
                    self._launch("hlo_reduce", self._h(src), None, self._h(out),
                                 H.reduce_push("max" if kind else "sum", ss, dims, init),
                                 out_elems=n)
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
                    self._launch("hlo_reduce_rank4", self._h(src), None, self._h(out),
                                 [len(ss), *d4, *od, *flags, kind, n], out_elems=n)
            elif oc == "reduce-window":
                src = self._contig(self._get(op.operands[0]), temps)
                init = self.const_value(op.operands[1]) if len(op.operands) > 1 else 0.0
                win = op.attrs.get("window")
                size = _window(win, "size") or [1] * 4
                stride = _window(win, "stride") or [1] * 4
                pads = _pairs(win.split("pad=", 1)[1].split(" ")[0]) if win and "pad=" in win else []
                pt = pads[1][0] if len(pads) > 1 else 0
                pl = pads[2][0] if len(pads) > 2 else 0
                kind = 1 if ("to_apply=%max" in op.raw or init == -np.inf) else 0
                self._launch("hlo_reduce_window_rank4", self._h(src), None, self._h(out),
                             [*src.shape, shape[1], shape[2], size[1], size[2], stride[1],
                              stride[2], pt, pl, kind, n], out_elems=n)
            elif oc in ELEMENTWISE:
                kernel, arity = ELEMENTWISE[oc]
                ins = [self._full(self._get(op.operands[k]), shape, temps) for k in range(arity)]
                self._launch(kernel, self._h(ins[0]), self._h(ins[1]) if arity == 2 else None,
                             self._h(out), [n], out_elems=n)
            else:
                raise NotImplementedError(f"no device lowering for HLO op {oc} ({op.result})")
            return out
        finally:
            for t in temps:
                self._drop(t)

    def _full(self, v: View, shape: Sequence[int], temps: list) -> View:
        """A contiguous tensor of `shape` holding `v` (binary_tensor's operand broadcast,
        compiler.rs:705-729: trailing-axis alignment; flat when the counts agree)."""
        if list(v.shape) != list(shape):
            if v.n == _n(shape):
                v = _reshape_view(v, shape) or View(self._contig(v, temps).buf, 0, shape,
                                                    _rm_strides(shape))
            else:
                r = len(shape) - len(v.shape)
                st = [0] * len(shape)
                for a, d in enumerate(v.shape):
                    if d != 1:
                        if d != shape[r + a]:
                            raise ValueError("operand does not broadcast")
                        st[r + a] = v.strides[a]
                v = View(v.buf, v.off, shape, tuple(st))
        return self._contig(v, temps)

    # ---- dense ops
    def _conv(self, op: HloOp, x: View, pt_extra: int, pl_extra: int, bias, residual, act,
              out: View, temps: list) -> None:
        w = self._contig(self._get(op.operands[1]), temps)
        x = self._contig(x, temps)
        if op.attrs.get("dim_labels") != "b01f_01io->b01f" or len(x.shape) != 4:
            raise NotImplementedError(f"convolution {op.attrs.get('dim_labels')} "
                                      "(compiler.rs:785-790 takes b01f_01io->b01f)")
        win = op.attrs.get("window")
        stride = _window(win, "stride") or [1, 1]
        pads = _pairs(win.split("pad=", 1)[1].split(" ")[0]) if win and "pad=" in win else [(0, 0), (0, 0)]
        shape = op.shape
        ws = w.shape
        push = [*x.shape, ws[0], ws[1], ws[3], shape[1], shape[2], stride[0], stride[1],
                pads[0][0] + pt_extra, pads[1][0] + pl_extra, _n(shape)]
        self._launch("hlo_conv_nhwc_hwio", self._h(x), self._h(w), self._h(out), push,
                     bias=self._h(bias) if bias is not None else None,
                     residual=self._h(residual) if residual is not None else None,
                     act=act, out_elems=_n(shape))

    def _dot(self, op: HloOp, bias, residual, act, temps: list, out: View | None) -> View:
        """dot / dot_general (compiler.rs:1009-1084) reading both operands in place."""
        A, B = self._get(op.operands[0]), self._get(op.operands[1])
        lc, rc = _ints(op.attrs.get("lhs_contracting_dims")), _ints(op.attrs.get("rhs_contracting_dims"))
        lb, rb = _ints(op.attrs.get("lhs_batch_dims")), _ints(op.attrs.get("rhs_batch_dims"))
        if len(lc) != 1 or len(rc) != 1:
            raise NotImplementedError("dot_general requires exactly one contracting dim per side")
        K = A.shape[lc[0]]
        if K != B.shape[rc[0]]:
            raise ValueError(f"dot contracting dim mismatch {K} vs {B.shape[rc[0]]}")
        if len(lb) != len(rb):
            raise ValueError("dot: lhs and rhs batch dims differ in number")
        lf = [d for d in range(len(A.shape)) if d not in lb and d not in lc]
        rf = [d for d in range(len(B.shape)) if d not in rb and d not in rc]
        nb = len(lb)
        shape = list(op.shape)
        M = _n([A.shape[d] for d in lf])
        N = _n([B.shape[d] for d in rf])
        bsz = _n([A.shape[d] for d in lb])
        if out is None:
            out = self._out_layout(op, shape) if not (bias or residual or act) else None
            if out is None:
                out = self._new(shape)

        def layout(v: View, bd, fd, cd):
            bs, fs = _batch2(v, bd), _run(v, fd)
            return None if bs is None or fs is None else (bs, fs, v.strides[cd])

        la = layout(A, lb, lf, lc[0])
        if la is None:  # materialise as [batch, free, contract]
            order = lb + lf + lc
            A = self._contig(View(A.buf, A.off, [A.shape[d] for d in order],
                                  [A.strides[d] for d in order]), temps)
            la = layout(A, list(range(nb)), list(range(nb, nb + len(lf))), len(order) - 1)
        lbv = layout(B, rb, rf, rc[0])
        if lbv is None:  # materialise as [batch, contract, free]
            order = rb + rc + rf
            B = self._contig(View(B.buf, B.off, [B.shape[d] for d in order],
                                  [B.strides[d] for d in order]), temps)
            lbv = layout(B, list(range(nb)), list(range(nb + 1, len(order))), nb)
        oc = _batch2(out, list(range(nb)))
        om = _run(out, list(range(nb, nb + len(lf))))
        on = _run(out, list(range(nb + len(lf), len(shape))))
        if oc is None or om is None or on is None:
            raise NotImplementedError(f"dot {op.result}: output layout")
        (sa, am, ak), (sb, bn, bk), (sc, cm, cn) = la, lbv, (oc, om, on)
        # a size-1 M or N dim has no stride of its own: use the row-major one
        am, cm = (K if am == 0 else am), (N if cm == 0 else cm)
        bn, cn = (1 if bn == 0 and N == 1 else bn), (1 if cn == 0 and N == 1 else cn)
        bo = _n([A.shape[d] for d in lb[:-1]]) if nb else 1
        bi = A.shape[lb[-1]] if nb else 1
        e = dict(bias=self._h(bias) if bias is not None else None,
                 residual=self._h(residual) if residual is not None else None, act=act)
        if bsz == 1 and ak == 1 and am == K and bn == 1 and bk == N and cn == 1 and cm == N:
            self._launch("hlo_dot_rank2", self._h(A), self._h(B), self._h(out),
                         [M, K, N, M * N], out_elems=M * N, **e)
        else:
            push = [bo, bi, M, N, K, sa[0], sa[1], am, ak, sb[0], sb[1], bk, bn,
                    sc[0], sc[1], cm, cn]
            if not (bias or residual or act) and self._fuse_attention(A, B, out, push, op):
                return out
            self._launch("dot_general_strided", self._h(A), self._h(B), self._h(out), push,
                         out_elems=bsz * M * N, **e)
            self._last_dot = (len(self.launches) - 1, A, B, out, push, op.result)
        return out

    def _readers(self, name: str) -> tuple[set, bool]:
        """The ops that read `name`'s elements, looking through the view ops that alias it
        (reshape / convert / transpose), and whether `name` or one of those views is a
        program output."""
        out, root, todo, seen = set(), False, [name], set()
        while todo:
            cur = todo.pop()
            if cur in seen:
                continue
            seen.add(cur)
            root = root or cur in self._roots
            for c in self.consumers.get(cur, []):
                if self.ops[c].opcode in ("reshape", "convert", "transpose"):
                    todo.append(self.ops[c].result)
                else:
                    out.add(c)
        return out, root

    def _fuse_attention(self, P: View, V: View, out: View, push: list, ctx_op: HloOp) -> bool:
        """The context dot of an attention block: when the two launches before it are the
        scores dot (Q . K^T) and the row softmax that reads it, and this dot reads the softmax's
        output, with Q, K and V column blocks of one row-major buffer (sequence 128, head dim
        64, heads side by side, the layout of a fused QKV activation), replace the three by
        one `attention_fused` launch (the C++ graph's op for the same block).  The fused
        launch writes neither the scores nor the probabilities, so it is taken only when
        nothing else reads them: the probabilities only by this dot, the scores only by the
        softmax, and neither is a program output."""
        sm, dt = getattr(self, "_last_softmax", None), getattr(self, "_last_dot", None)
        n = len(self.launches)
        if sm is None or dt is None or sm[0] != n - 1 or dt[0] != n - 2:
            return False
        _, x, y, mask, bits, g = sm
        _, Q, K, S_out, sp, scores_name = dt
        probs, root = self._readers(self.ops[g["anchor"]].result)
        if root or probs != {self.idx[ctx_op.result]}:
            return False
        scores, root = self._readers(scores_name)
        if root or not scores <= set(g["members"]) | {g["anchor"]}:
            return False
        B, H, S, _, HD = sp[:5]
        if S != 128 or HD != 64 or push[:5] != [B, H, S, HD, S]:
            return False
        if not (P.buf is y.buf and P.off == y.off and x.buf is S_out.buf and x.off == S_out.off):
            return False
        if not (Q.buf is K.buf is V.buf):
            return False
        ld = sp[7]  # Q row stride
        if B == 1:  # a size-1 batch dim has no stride of its own: use the row-major one
            sp, push = list(sp), list(push)
            sp[5] = sp[9] = S * ld
            sp[13], push[5], push[9] = H * S * S, H * S * S, S * ld
            push[13] = S * push[15]
        want_scores = [B, H, S, S, HD, S * ld, HD, ld, 1, S * ld, HD, 1, ld]
        if sp[:13] != want_scores or sp[13:] != [H * S * S, S * S, S, 1]:
            return False
        if push[5:13] != [H * S * S, S * S, S, 1, S * ld, HD, ld, 1]:
            return False
        ld_out = push[15]
        if push[13:] != [S * ld_out, HD, ld_out, 1] or ld_out < H * HD:
            return False
        base = min(Q.off, K.off, V.off)
        offs = [Q.off - base, K.off - base, V.off - base]
        if any(o % 4 for o in offs + [ld]) or any(o + H * HD > ld for o in offs):
            return False
        total = B * S * ld_out
        self.launches = self.launches[:-2]
        self.launch_src = self.launch_src[:-2]
        self._last_softmax = self._last_dot = None
        self.fused_counts["softmax"] -= 1
        if not self.fused_counts["softmax"]:
            del self.fused_counts["softmax"]
        span = (B * S - 1) * ld + max(offs) + H * HD  # elements the kernel reads from `base`
        self._launch("attention_fused", self.b.sub(Q.buf.handle, base, span),
                     self._h(mask) if mask is not None else None,
                     self.b.sub(out.buf.handle, out.off, total),
                     [B, H, S, HD, ld, *offs, ld_out, bits, total], out_elems=total)
        self._note("attention")
        return True

    def _out_layout(self, op: HloOp, shape: list[int]) -> View | None:
        """If the dot's only reader is a transpose (after identity transposes), a buffer in
        the transposed layout, viewed in the dot's output order."""
        cur = op.result
        while True:
            j = self._sole(cur)
            if j is None or j in self.absorbed:
                return None
            c = self.ops[j]
            perm = _ints(c.attrs.get("dimensions"))
            if c.opcode != "transpose":
                return None
            if perm == list(range(len(c.shape))):
                cur = c.result
                continue
            tshape = [shape[p] for p in perm]
            ts = _rm_strides(tshape)
            st = [0] * len(shape)
            for i, p in enumerate(perm):
                st[p] = ts[i]
            return View(self._alloc(_n(tshape)), 0, shape, tuple(st))

    # ---- fused groups
    def _lower_group(self, g: dict) -> View:
        temps: list = []
        try:
            kind = g["kind"]
            if kind == "epilogue":
                head = self.ops[g["head"]]
                out_shape = self._op(g["out"]).shape
                bias = self._vec(g["bias"], temps) if g["bias"] else None
                if head.opcode == "convolution":
                    x = self._get(g["inputs"][0]) if g["pad"] else self._get(head.operands[0])
                    res = self._contig(self._get(g["residual"]), temps) if g["residual"] else None
                    out = self._new(out_shape)
                    pt = g["pad"][1] if g["pad"] else 0
                    pl = g["pad"][2] if g["pad"] else 0
                    self._conv(head, x, pt, pl, bias, res, g["act"], out, temps)
                    self._note("conv")
                    return out
                res = self._contig(self._get(g["residual"]), temps) if g["residual"] else None
                out = self._new(out_shape)
                self._dot(head, bias, res, g["act"], temps,
                          View(out.buf, out.off, head.shape, _rm_strides(head.shape)))
                self._note("dot")
                return out
            if kind == "softmax":
                x = self._contig(self._get(g["x"]), temps)
                mask = self._vec(g["mask"], temps) if g["mask"] else None
                out = self._new(x.shape)
                bits = int(np.array([g["scale"]], np.float32).view(np.int32)[0])
                self._launch("softmax_rows", self._h(x), self._h(mask) if mask else None,
                             self._h(out), [g["rows"], g["cols"], bits], out_elems=out.n)
                self._last_softmax = (len(self.launches) - 1, x, out, mask, bits, g)
                self._note("softmax")
                return out
            if kind in ("layernorm", "rmsnorm"):
                x = self._contig(self._get(g["x"]), temps)
                D = g["cols"]
                if kind == "layernorm":
                    gm, bt = self._vec(g["gamma"], temps), self._vec(g["beta"], temps)
                    if gm.buf is bt.buf and bt.off == gm.off + D:
                        w = View(gm.buf, gm.off, [2 * D], (1,))
                    else:
                        w = self._new([2 * D])
                        w.buf.refs += 1
                        temps.append(w)
                        self._launch("reshape", self._h(gm), None, self._h(w, D), [D],
                                     out_elems=D)
                        self._launch("reshape", self._h(bt), None,
                                     self.b.sub(w.buf.handle, w.off + D, D), [D], out_elems=D)
                else:
                    w = self._vec(g["w"], temps)
                out = self._new(x.shape)
                bits = int(np.array([g["eps"]], np.float32).view(np.int32)[0])
                self._launch("layernorm_rows" if kind == "layernorm" else "rmsnorm_rows",
                             self._h(x), self._h(w), self._h(out), [g["rows"], D, bits],
                             out_elems=out.n)
                self._note(kind)
                return out
            if kind == "meanpool":
                x = self._contig(self._get(g["x"]), temps)
                n, h, w_, c = g["dims"]
                out = self._new(self.ops[g["anchor"]].shape)
                self._launch("global_avg_pool_nhwc", self._h(x), None, self._h(out),
                             [n, h, w_, c], out_elems=n * c)
                self._note("meanpool")
                return out
            raise AssertionError(kind)
        finally:
            for t in temps:
                self._drop(t)

    def _vec(self, name: str, temps: list) -> View:
        v = self._get(name)
        flat = _reshape_view(v, [v.n])
        if flat is None or not flat.contiguous():
            flat = self._contig(View(v.buf, v.off, v.shape, v.strides), temps)
            flat = View(flat.buf, flat.off, [v.n], (1,))
        return flat

    def _note(self, kind: str) -> None:
        self.fused_counts[kind] = self.fused_counts.get(kind, 0) + 1

    # ------------------------------------------------------------------ execution
    def run(self, graph: bool = False) -> list:
        """Execute the program; returns the output handles (see outputs())."""
        if graph and self._graph is None and self._warm and hasattr(self.b, "capture_begin"):
            self.b.capture_begin()
            try:
                self._replay()
            finally:
                self._graph = self.b.capture_end()
        if graph and self._graph is not None:
            self.b.graph_launch(self._graph)
        else:
            self._replay()
            self._warm = True
        return self.outputs()

    def _replay(self, after=None) -> None:
        launch = self.b.launch
        for i, (k, a, b, c, push, bias, res, act, alpha, oe) in enumerate(self.launches):
            launch(k, a, b, c, push, bias=bias, residual=res, act=act, alpha=alpha,
                   out_elems=oe)
            if after is not None:
                after(i)

    def run_traced(self, after) -> list:
        """One eager replay calling after(i) once launch i is enqueued (its output handle is
        self.launches[i][3]): per-launch checks such as the NaN trace, before a later launch
        reuses the buffer."""
        self._replay(after)
        self._warm = True
        return self.outputs()

    def steps(self) -> list[dict]:
        """The ENTRY ops in order with what became of each: the `steps` list of the HLO
        runner's report (compiler.rs:226-232 GraphStep).  `execution` names the lowering
        (a launch, a fused group, a strided view or an alias) and `spv_name` the first
        registry kernel launched for the op (None when it launches nothing)."""
        kernels: dict[str, list] = {}
        for (k, *_rest), src in zip(self.launches, self.launch_src):
            kernels.setdefault(src, []).append(k)
        anchor_of = {m: a for a, g in self.groups.items() for m in g["members"]}
        out = []
        for i, op in enumerate(self.ops):
            ks = kernels.get(op.result, [])
            if i in anchor_of and i not in self.groups:
                ex = f"fused_into {self.ops[anchor_of[i]].result}"
            elif i in self.groups:
                ex = f"hip_fused_{self.groups[i]['kind']}"
            elif op.opcode == "parameter":
                ex = "bound_parameter"
            elif op.opcode == "constant":
                ex = "materialized scalar constant"
            elif op.opcode in ("tuple", "get-tuple-element"):
                ex = "tuple_alias"
            elif ks:
                ex = "hip_" + "+".join(dict.fromkeys(ks))
            elif op.opcode in ("reshape", "convert"):
                ex = "metadata_reshape"
            else:
                ex = "strided_view"
            out.append({"result": op.result, "opcode": op.opcode, "execution": ex,
                        "elements": _n(op.shape), "spv_name": ks[0] if ks else None})
        return out

    def outputs(self) -> list:
        """(handle, shape) of each ROOT value, contiguous."""
        return [(self._h(v, v.n), list(v.shape)) for v in self._outputs]

    def read(self, k: int = 0) -> np.ndarray:
        h, shape = self.outputs()[k]
        return np.asarray(self.b.read(h))[:_n(shape)].reshape(shape)

    def close(self) -> None:
        if self._graph is not None:
            self.b.graph_destroy(self._graph)
            self._graph = None
        for buf in self.owned:
            self.b.free(buf.handle)
        self.owned = []
        self.launches = []
        self.launch_src = []


def _batch2(v: View, dims: Sequence[int]):
    """(outer stride, inner stride) of batch axes `dims` of `v` split as outer = all but the
    last axis, inner = the last axis; None if the outer axes are not one strided run."""
    if not dims:
        return (0, 0)
    inner = v.strides[dims[-1]] if v.shape[dims[-1]] != 1 else 0
    outer = [(v.shape[d], v.strides[d]) for d in dims[:-1] if v.shape[d] != 1]
    if not outer:
        return (0, inner)
    for (s0, t0), (s1, t1) in zip(outer, outer[1:]):
        if t0 != s1 * t1:
            return None
    return (outer[-1][1], inner)


def _run(v: View, dims: Sequence[int]):
    """Stride of axes `dims` of `v` merged into one (0 when they are all size 1), or None if
    they are not one strided run."""
    ds = [(v.shape[d], v.strides[d]) for d in dims if v.shape[d] != 1]
    if not ds:
        return 0
    for (s0, t0), (s1, t1) in zip(ds, ds[1:]):
        if t0 != s1 * t1:
            return None
    return ds[-1][1]


def _compare(direction: str, a, b):
    return {"LT": np.less, "LE": np.less_equal, "EQ": np.equal, "NE": np.not_equal,
            "GE": np.greater_equal, "GT": np.greater}[direction](a, b).astype(np.float64)


def _eval_elementwise(oc: str, a):
    x = a[0]
    y = a[1] if len(a) > 1 else None
    f = {"add": lambda: x + y, "subtract": lambda: x - y, "multiply": lambda: x * y,
         "divide": lambda: x / y, "maximum": lambda: np.maximum(x, y),
         "minimum": lambda: np.minimum(x, y), "power": lambda: np.power(x, y),
         "abs": lambda: np.abs(x), "exponential": lambda: np.exp(x), "log": lambda: np.log(x),
         "sqrt": lambda: np.sqrt(x), "rsqrt": lambda: 1.0 / np.sqrt(x),
         "negate": lambda: -x, "tanh": lambda: np.tanh(x),
         "logistic": lambda: 1.0 / (1.0 + np.exp(-x)), "sine": lambda: np.sin(x),
         "cosine": lambda: np.cos(x)}[oc]
    return f()
