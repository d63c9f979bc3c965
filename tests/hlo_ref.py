"""Test-side helpers for the HLO executor (spirv_inference_amd.hlo_exec).

* OracleBackend: the executor's backend interface on the CPU oracle (same kernel names and
  push vectors), so one HLO walk can be run on the device and on the checker.
* eval_numpy: an independent float64 interpreter of the same ENTRY op list with XLA's
  semantics written directly in numpy (no registry kernels), to pin the lowering itself.
* fixture_text / seeded_params: the reference's HLO fixtures (tests/golden/hlo) and
  seeded parameters of their declared shapes (their weights are not in the reference).
"""
import gzip
import pathlib
import re

import numpy as np

import oracle as orc
from spirv_inference_amd import hlo_exec as X

HLO_DIR = pathlib.Path(__file__).resolve().parent / "golden" / "hlo"


def fixture_text(model: str) -> str:
    with gzip.open(HLO_DIR / f"{model}.stablehlo.txt.gz", "rt") as f:
        return f.read()


class OracleBackend:
    """Values are float32 numpy arrays; launches run the oracle's kernels."""

    def upload(self, arr):
        return np.ascontiguousarray(arr, np.float32).reshape(-1).copy()

    def empty(self, n):
        return np.zeros(max(1, n), np.float32)

    def launch(self, kernel, in0, in1, out, push, bias=None, residual=None, act=0, alpha=0.0,
               out_elems=None):
        n = out.size if out_elems is None else out_elems
        out[:n] = orc.run(kernel, in0, in1, n, list(push), bias=bias, residual=residual,
                          act=act, alpha=alpha, out_init=out[:n])

    def sub(self, t, offset, n):
        return t[offset:offset + n]

    def write(self, t, offset, arr):
        t[offset:offset + arr.size] = arr

    def read(self, t):
        return t

    def free(self, t):
        pass


def seeded_params(ops, seed=11):
    """Parameters in parameter order: rank >= 2 tensors ~ N(0, 1/fan_in) (fan_in = all but
    the last axis; the first parameter, the network input, ~ N(0, 1)), rank-1 tensors
    ~ U[0.5, 1.5] (positive, so batch-norm variances stay valid)."""
    rng = np.random.default_rng(seed)
    shapes = {}
    for op in ops:
        if op.opcode == "parameter":
            idx = int(re.search(r"parameter\((\d+)\)", op.raw).group(1))
            shapes[idx] = op.shape
    out = []
    for i in range(len(shapes)):
        s = shapes[i]
        if i == 0 or len(s) < 2:
            a = rng.standard_normal(s) if i == 0 else rng.uniform(0.5, 1.5, s)
        else:
            a = rng.standard_normal(s) / np.sqrt(max(1, int(np.prod(s[:-1]))))
        out.append(np.asarray(a, np.float32))
    return out


def _conv_nhwc(x, w, stride, pads):
    (pt, pb), (pl, pr) = pads
    x = np.pad(x, ((0, 0), (pt, pb), (pl, pr), (0, 0)))
    kh, kw, ic, oc = w.shape
    n, h, wd, _ = x.shape
    oh, ow = (h - kh) // stride[0] + 1, (wd - kw) // stride[1] + 1
    y = np.zeros((n, oh, ow, oc))
    for i in range(kh):
        for j in range(kw):
            patch = x[:, i:i + stride[0] * (oh - 1) + 1:stride[0], j:j + stride[1] * (ow - 1) + 1:stride[1], :]
            y += patch @ w[i, j]
    return y


def eval_numpy(ops, params, all_values=False):
    """float64 evaluation with XLA semantics; returns the last op's value (all_values: the
    dict of every value; a tuple ROOT's elements are then looked up by name)."""
    v, last = {}, None
    for op in ops:
        a = [v[o] for o in op.operands if o in v]
        oc, shape = op.opcode, tuple(op.shape)
        if oc == "parameter":
            r = np.asarray(params[int(re.search(r"parameter\((\d+)\)", op.raw).group(1))], np.float64).reshape(shape)
        elif oc == "constant":
            r = np.full(shape, X._constant(op.raw), np.float64)
        elif oc in X.ALIASES:
            r = a[0].reshape(shape) if oc in ("reshape", "convert") else a[0]
        elif oc in ("broadcast", "broadcast_in_dim"):
            dims = X._ints(op.attrs.get("dimensions"))
            src = a[0]
            if src.size == 1:
                r = np.full(shape, src.reshape(-1)[0])
            else:
                order = np.argsort(dims)
                t = np.transpose(src, order)
                tgt = [1] * len(shape)
                for k, d in enumerate(np.array(dims)[order]):
                    tgt[d] = t.shape[k]
                r = np.broadcast_to(t.reshape(tgt), shape).copy()
        elif oc == "transpose":
            r = np.transpose(a[0], X._ints(op.attrs.get("dimensions")))
        elif oc == "slice":
            st, lim, sp = X._slice_spec(op.raw)
            r = a[0][tuple(slice(s, l, p) for s, l, p in zip(st, lim, sp))]
        elif oc == "concatenate":
            r = np.concatenate(a, axis=(X._ints(op.attrs.get("dimensions")) or [0])[0])
        elif oc == "compare":
            f = {"LT": np.less, "LE": np.less_equal, "EQ": np.equal, "NE": np.not_equal,
                 "GE": np.greater_equal}.get(op.attrs.get("direction"), np.greater)
            r = f(a[0], a[1]).astype(np.float64)
        elif oc == "select":
            r = np.where(a[0] != 0, a[1], a[2])
        elif oc == "pad":
            pads = X._pairs(op.attrs.get("padding"))
            r = np.pad(a[0], pads, constant_values=a[1].reshape(-1)[0])
        elif oc == "convolution":
            win = op.attrs.get("window")
            stride = X._window(win, "stride") or [1, 1]
            pads = X._pairs(win.split("pad=", 1)[1].split(" ")[0]) if "pad=" in win else [(0, 0), (0, 0)]
            r = _conv_nhwc(a[0], a[1], stride, pads)
        elif oc in ("dot", "dot_general"):
            lc, rc = X._ints(op.attrs.get("lhs_contracting_dims")), X._ints(op.attrs.get("rhs_contracting_dims"))
            lb, rb = X._ints(op.attrs.get("lhs_batch_dims")), X._ints(op.attrs.get("rhs_batch_dims"))
            lf = [d for d in range(a[0].ndim) if d not in lb + lc]
            rf = [d for d in range(a[1].ndim) if d not in rb + rc]
            L = np.transpose(a[0], lb + lf + lc)
            R = np.transpose(a[1], rb + rc + rf)
            B = int(np.prod([a[0].shape[d] for d in lb])) if lb else 1
            M = int(np.prod([a[0].shape[d] for d in lf])) if lf else 1
            N = int(np.prod([a[1].shape[d] for d in rf])) if rf else 1
            K = a[0].shape[lc[0]]
            r = np.matmul(L.reshape(B, M, K), R.reshape(B, K, N)).reshape(shape)
        elif oc == "reduce":
            dims = tuple(X._ints(op.attrs.get("dimensions")))
            init = a[1].reshape(-1)[0]
            is_max = "to_apply=%max" in op.raw or init == -np.inf
            r = (np.maximum(a[0].max(axis=dims), init) if is_max else a[0].sum(axis=dims) + init).reshape(shape)
        elif oc == "reduce-window":
            win = op.attrs.get("window")
            size, stride = X._window(win, "size"), X._window(win, "stride")
            pads = X._pairs(win.split("pad=", 1)[1].split(" ")[0]) if "pad=" in win else [(0, 0)] * 4
            x = np.pad(a[0], pads, constant_values=-np.inf)
            r = np.full(shape, -np.inf)
            for i in range(size[1]):
                for j in range(size[2]):
                    r = np.maximum(r, x[:, i:i + stride[1] * (shape[1] - 1) + 1:stride[1],
                                         j:j + stride[2] * (shape[2] - 1) + 1:stride[2], :])
        elif oc in X.ELEMENTWISE:
            f = {"add": np.add, "subtract": np.subtract, "multiply": np.multiply,
                 "divide": np.divide, "maximum": np.maximum, "minimum": np.minimum,
                 "power": np.power, "abs": np.abs, "exponential": np.exp, "log": np.log,
                 "sqrt": np.sqrt, "rsqrt": lambda x: 1.0 / np.sqrt(x), "negate": np.negative,
                 "tanh": np.tanh, "logistic": lambda x: 1.0 / (1.0 + np.exp(-x)),
                 "sine": np.sin}[oc]
            r = f(*[np.broadcast_to(t, shape) for t in a])
        else:
            raise NotImplementedError(oc)
        v[op.result] = np.asarray(r, np.float64)
        last = op.result
    return v if all_values else v[last]
