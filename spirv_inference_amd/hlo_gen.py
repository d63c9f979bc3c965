"""XLA HLO text modules of the benchmark configs, in the dialect of the reference's fixtures.

The reference's HLO path takes modules that TensorFlow / PyTorch exporters wrote
(source/xla_hlo/tools/export_tf_stablehlo.py:60-68, export_llama.py:269-375); its fixtures
are a Keras ResNet-50 v1 at batch 1, one simplified BERT block and a TinyLlama S=64 full
recompute.  None of them is a benchmark config, and the exporters need TensorFlow, torch and
network weights.  This module writes the configs' own modules directly, as text that
`parser.rs:86-170` (and `hlo_exec.parse_hlo_text`) reads: `%name = f32[dims]{layout}
opcode(f32[...] %operand, ...), attributes`, reducer computations before the ENTRY, one op
per line, scalar constants broadcast with `dimensions={}`, softmax as reduce(max) / subtract /
exponential / reduce(sum) / divide with the reshape-broadcast chains the fixtures have
(resnet50.stablehlo.txt:1714-1730), GELU as the erfc expansion of bert_base.stablehlo.txt:55-144.

* resnet50_v15(batch): ResNet-50 v1.5 (stride on the 3x3 conv), NHWC, HWIO weights, batch norm
  folded into each convolution as a bias add, ReLU as maximum with 0, max pool as
  reduce-window with -inf padding, mean pool as reduce(sum) / 49, dense + softmax.
* bert_base(batch, seq, layers): the encoder after the embedding LayerNorm: fused QKV dot,
  heads split by reshape + transpose, scaled scores + additive mask, softmax, context,
  output dot + bias + residual, LayerNorm (mean / variance / rsqrt chain), FFN with GELU.
* llama_decode_step(cfg, max_seq): one M=1 TinyLlama step against a KV cache: RMSNorm chain,
  one [q|k|v] dot, rotate-half RoPE from slices / negate / concatenate, GQA by broadcast, the
  new key / value concatenated behind the cached ones, additive mask, SwiGLU, lm_head.
  Outputs (tuple): logits and every layer's new key and value rows.

Each function returns (text, params): params lists (label, shape) in parameter order, so a
caller can bind the same weights the C++ graphs (shp_model_*) or the decoder (shp_llama_*) hold.
"""
from __future__ import annotations

import math
from typing import Sequence

import numpy as np

# erfc(z) as XLA expands it for f32 (the constants and the branch structure of
# bert_base.stablehlo.txt:64-137): |z| > 1 uses exp(-z^2) * P(1/z^2) / (|z| * Q(1/z^2)),
# reflected for z < 0; |z| <= 1 uses 1 - z * R(z^2).
_ERFC_P = (0.102081165, 0.429206669, 0.323790789, 0.053971976)
_ERFC_Q = (0.0172516778, 0.391371638, 1.0, 0.621732414, 0.0956628621)
_ERF_R = (0.000561802299, -0.00491381669, 0.0267075151, -0.112800106, 0.376122952,
          -1.12837911)


class Val:
    __slots__ = ("name", "shape")

    def __init__(self, name: str, shape: Sequence[int]):
        self.name, self.shape = name, list(shape)


def _t(shape: Sequence[int], pred: bool = False) -> str:
    ty = "pred" if pred else "f32"
    if not shape:
        return f"{ty}[]"
    layout = ",".join(str(i) for i in reversed(range(len(shape))))
    return f"{ty}[{','.join(str(d) for d in shape)}]{{{layout}}}"


def _c(v: float) -> str:
    if v == -np.inf:
        return "-inf"
    if v == np.inf:
        return "inf"
    return repr(float(np.float32(v))) if v != int(v) else str(int(v))


class HloBuilder:
    """Writes one HLO module op by op; every method returns the new value."""

    def __init__(self, module: str):
        self.module = module
        self.lines: list[str] = []
        self.params: list[tuple[str, list[int]]] = []
        self.param_names: list[str] = []
        self.count = 0
        self.preds: set[str] = set()

    def _emit(self, base: str, shape, rhs: str, pred: bool = False) -> Val:
        self.count += 1
        name = f"%{base}.{self.count}"
        self.lines.append(f"  {name} = {_t(shape, pred)} {rhs}")
        if pred:
            self.preds.add(name)
        return Val(name, shape)

    def _ref(self, v: Val) -> str:
        return f"{_t(v.shape, v.name in self.preds)} {v.name}"

    # ---- leaves
    def param(self, shape: Sequence[int], label: str) -> Val:
        idx = len(self.params)
        self.params.append((label, list(shape)))
        v = self._emit(f"arg{idx}", shape, f"parameter({idx}), parameter_replication={{false}}")
        self.param_names.append(v.name)
        return v

    def const(self, value: float) -> Val:
        return self._emit("constant", [], f"constant({_c(value)})")

    def splat(self, value: float, shape: Sequence[int]) -> Val:
        return self.bcast(self.const(value), shape, [])

    # ---- shape ops
    def bcast(self, v: Val, shape: Sequence[int], dims: Sequence[int]) -> Val:
        d = ",".join(str(x) for x in dims)
        return self._emit("broadcast", shape, f"broadcast({self._ref(v)}), dimensions={{{d}}}")

    def reshape(self, v: Val, shape: Sequence[int]) -> Val:
        return self._emit("reshape", shape, f"reshape({self._ref(v)})")

    def transpose(self, v: Val, perm: Sequence[int]) -> Val:
        shape = [v.shape[p] for p in perm]
        d = ",".join(str(x) for x in perm)
        return self._emit("transpose", shape, f"transpose({self._ref(v)}), dimensions={{{d}}}")

    def slice(self, v: Val, starts: Sequence[int], limits: Sequence[int]) -> Val:
        shape = [l - s for s, l in zip(starts, limits)]
        spec = ", ".join(f"[{s}:{l}]" for s, l in zip(starts, limits))
        return self._emit("slice", shape, f"slice({self._ref(v)}), slice={{{spec}}}")

    def concat(self, vals: Sequence[Val], dim: int) -> Val:
        shape = list(vals[0].shape)
        shape[dim] = sum(v.shape[dim] for v in vals)
        ops = ", ".join(self._ref(v) for v in vals)
        return self._emit("concatenate", shape, f"concatenate({ops}), dimensions={{{dim}}}")

    def tuple(self, vals: Sequence[Val]) -> Val:
        self.count += 1
        name = f"%tuple.{self.count}"
        ty = "(" + ", ".join(_t(v.shape) for v in vals) + ")"
        ops = ", ".join(self._ref(v) for v in vals)
        self.lines.append(f"  {name} = {ty} tuple({ops})")
        return Val(name, [])

    # ---- elementwise
    def binary(self, op: str, a: Val, b: Val) -> Val:
        return self._emit(op, a.shape, f"{op}({self._ref(a)}, {self._ref(b)})")

    def unary(self, op: str, a: Val) -> Val:
        return self._emit(op, a.shape, f"{op}({self._ref(a)})")

    def compare(self, a: Val, b: Val, direction: str) -> Val:
        return self._emit("compare", a.shape, f"compare({self._ref(a)}, {self._ref(b)}), "
                          f"direction={direction}", pred=True)

    def select(self, p: Val, a: Val, b: Val) -> Val:
        return self._emit("select", a.shape,
                          f"select({self._ref(p)}, {self._ref(a)}, {self._ref(b)})")

    def scalar_op(self, op: str, a: Val, value: float) -> Val:
        return self.binary(op, a, self.splat(value, a.shape))

    def relu(self, a: Val) -> Val:
        return self.binary("maximum", a, self.splat(0.0, a.shape))

    def add_vec(self, a: Val, vec: Val) -> Val:
        """a + vec broadcast along the last axis (a BiasAdd)."""
        return self.binary("add", a, self.bcast(vec, a.shape, [len(a.shape) - 1]))

    def mul_vec(self, a: Val, vec: Val) -> Val:
        return self.binary("multiply", a, self.bcast(vec, a.shape, [len(a.shape) - 1]))

    # ---- reductions
    def reduce(self, v: Val, dims: Sequence[int], kind: str) -> Val:
        init = self.const(-np.inf if kind == "max" else 0.0)
        shape = [d for k, d in enumerate(v.shape) if k not in dims]
        d = ",".join(str(x) for x in dims)
        comp = "%max_F32" if kind == "max" else "%add_F32"
        return self._emit("reduce", shape, f"reduce({self._ref(v)}, {self._ref(init)}), "
                          f"dimensions={{{d}}}, to_apply={comp}")

    def row_bcast(self, r: Val, shape: Sequence[int]) -> Val:
        """A per-row value (shape[:-1]) broadcast along the last axis, through the
        reshape / broadcast / reshape chain the fixtures write."""
        lead = list(shape[:-1])
        t = self.reshape(r, lead + [1])
        t = self.bcast(t, lead + [1], list(range(len(lead) + 1)))
        t = self.reshape(t, lead)
        return self.bcast(t, shape, list(range(len(lead))))

    def reduce_window_max(self, v: Val, k: int, s: int, pad: int) -> Val:
        n, h, w, c = v.shape
        oh, ow = (h + 2 * pad - k) // s + 1, (w + 2 * pad - k) // s + 1
        init = self.const(-np.inf)
        return self._emit("reduce-window", [n, oh, ow, c],
                          f"reduce-window({self._ref(v)}, {self._ref(init)}), "
                          f"window={{size=1x{k}x{k}x1 stride=1x{s}x{s}x1 "
                          f"pad=0_0x{pad}_{pad}x{pad}_{pad}x0_0}}, to_apply=%max_F32")

    # ---- dense
    def conv(self, x: Val, w: Val, stride: int, pad: int) -> Val:
        n, h, wd, _ = x.shape
        kh, kw, _, oc = w.shape
        oh, ow = (h + 2 * pad - kh) // stride + 1, (wd + 2 * pad - kw) // stride + 1
        return self._emit("convolution", [n, oh, ow, oc],
                          f"convolution({self._ref(x)}, {self._ref(w)}), window={{size={kh}x{kw} "
                          f"stride={stride}x{stride} pad={pad}_{pad}x{pad}_{pad}}}, "
                          f"dim_labels=b01f_01io->b01f")

    def dot(self, a: Val, b: Val, lc: Sequence[int], rc: Sequence[int],
            lb: Sequence[int] = (), rb: Sequence[int] = ()) -> Val:
        lf = [d for d in range(len(a.shape)) if d not in lb and d not in lc]
        rf = [d for d in range(len(b.shape)) if d not in rb and d not in rc]
        shape = [a.shape[d] for d in lb] + [a.shape[d] for d in lf] + [b.shape[d] for d in rf]
        j = lambda xs: ",".join(str(x) for x in xs)
        attrs = ""
        if lb:
            attrs += f", lhs_batch_dims={{{j(lb)}}}"
        attrs += f", lhs_contracting_dims={{{j(lc)}}}"
        if rb:
            attrs += f", rhs_batch_dims={{{j(rb)}}}"
        attrs += f", rhs_contracting_dims={{{j(rc)}}}"
        return self._emit("dot", shape, f"dot({self._ref(a)}, {self._ref(b)}){attrs}")

    # ---- composite forms of the fixtures
    def softmax(self, x: Val) -> Val:
        r = len(x.shape)
        m = self.reduce(x, [r - 1], "max")
        e = self.unary("exponential", self.binary("subtract", x, self.row_bcast(m, x.shape)))
        z = self.reduce(e, [r - 1], "sum")
        return self.binary("divide", e, self.row_bcast(z, x.shape))

    def layernorm(self, x: Val, gamma: Val, beta: Val, eps: float) -> Val:
        D = x.shape[-1]
        r = len(x.shape)
        mean = self.binary("divide", self.reduce(x, [r - 1], "sum"),
                           self.splat(float(D), x.shape[:-1]))
        d = self.binary("subtract", x, self.row_bcast(mean, x.shape))
        var = self.binary("divide", self.reduce(self.binary("multiply", d, d), [r - 1], "sum"),
                          self.splat(float(D), x.shape[:-1]))
        rs = self.unary("rsqrt", self.binary("add", var, self.splat(eps, x.shape[:-1])))
        y = self.binary("multiply", d, self.row_bcast(rs, x.shape))
        return self.add_vec(self.mul_vec(y, gamma), beta)

    def rmsnorm(self, x: Val, w: Val, eps: float) -> Val:
        D = x.shape[-1]
        r = len(x.shape)
        ms = self.binary("divide", self.reduce(self.binary("multiply", x, x), [r - 1], "sum"),
                         self.splat(float(D), x.shape[:-1]))
        rs = self.unary("rsqrt", self.binary("add", ms, self.splat(eps, x.shape[:-1])))
        return self.mul_vec(self.binary("multiply", x, self.row_bcast(rs, x.shape)), w)

    def gelu_erf(self, x: Val) -> Val:
        """0.5 * x * erfc(-x / sqrt(2)) with XLA's f32 erfc expansion."""
        sh = x.shape
        half = self.binary("multiply", self.splat(0.5, sh), x)
        z = self.binary("multiply", self.unary("negate", x), self.splat(0.707106769, sh))
        az = self.unary("abs", z)
        big = self.compare(az, self.splat(1.0, sh), "GT")
        neg = self.compare(z, self.splat(0.0, sh), "LT")
        z2 = self.binary("multiply", z, z)
        ez = self.unary("exponential", self.unary("negate", z2))
        iz2 = self.binary("divide", self.splat(1.0, sh), z2)

        def horner(coefs, t):
            acc = self.binary("multiply", self.splat(coefs[0], sh), t)
            for c in coefs[1:-1]:
                acc = self.binary("multiply", self.binary("add", acc, self.splat(c, sh)), t)
            return self.binary("add", acc, self.splat(coefs[-1], sh))

        p = horner(_ERFC_P, iz2)
        amin = self.binary("minimum", self.unary("abs", z), self.splat(10.06, sh))
        q = horner(_ERFC_Q, iz2)
        tail = self.binary("multiply", ez, self.binary("divide", p,
                                                         self.binary("multiply", amin, q)))
        refl = self.select(neg, self.binary("subtract", self.splat(2.0, sh), tail), tail)
        zz = self.binary("multiply", z, z)
        rr = horner(_ERF_R, zz)
        small = self.binary("add", self.binary("multiply", z, rr), self.splat(1.0, sh))
        erfc = self.select(big, refl, small)
        return self.binary("multiply", half, erfc)

    # ---- module text
    def text(self, root: Val, root_shapes: Sequence[Sequence[int]] | None = None) -> str:
        args = ", ".join(f"{nm[1:]}: {_t(s).split('{')[0]}"
                         for nm, (_, s) in zip(self.param_names, self.params))
        out_ty = ("(" + ", ".join(_t(s) for s in root_shapes) + ")") if root_shapes \
            else _t(root.shape)
        layout = ", ".join(_t(s) for _, s in self.params)
        lines = [f"HloModule {self.module}, entry_computation_layout={{({layout})->{out_ty}}}",
                 "",
                 "%max_F32 (lhs: f32[], rhs: f32[]) -> f32[] {",
                 "  %lhs = f32[] parameter(0)",
                 "  %rhs = f32[] parameter(1)",
                 "  ROOT %maximum = f32[] maximum(f32[] %lhs, f32[] %rhs)",
                 "}",
                 "",
                 "%add_F32 (x: f32[], y: f32[]) -> f32[] {",
                 "  %x = f32[] parameter(0)",
                 "  %y = f32[] parameter(1)",
                 "  ROOT %add = f32[] add(f32[] %x, f32[] %y)",
                 "}",
                 "",
                 f"ENTRY %main.{self.module} ({args}) -> {out_ty} {{"]
        body = list(self.lines)
        for k in range(len(body) - 1, -1, -1):
            if body[k].lstrip().startswith(root.name + " "):
                body[k] = body[k].replace("  %", "  ROOT %", 1)
                break
        lines += body + ["}", ""]
        return "\n".join(lines)


def resnet50_v15(batch: int = 32, image: int = 224, classes: int = 1000):
    """ResNet-50 v1.5 inference module; params in the order the C++
    graph (models.cpp build_resnet50) creates its weights: input, then per convolution
    (stem; per bottleneck the projection shortcut first, then 1x1, 3x3, 1x1) the HWIO
    weight and the folded-BN bias, then the dense weight [2048, classes] and bias."""
    b = HloBuilder(f"resnet50_v1_5_b{batch}")
    x = b.param([batch, image, image, 3], "input")

    def conv(x: Val, oc: int, k: int, s: int, label: str, relu: bool,
             residual: Val | None = None) -> Val:
        w = b.param([k, k, x.shape[3], oc], f"{label}/w")
        bias = b.param([oc], f"{label}/b")
        y = b.add_vec(b.conv(x, w, s, (k - 1) // 2), bias)
        if residual is not None:
            y = b.binary("add", y, residual)
        return b.relu(y) if relu else y

    x = conv(x, 64, 7, 2, "conv1", True)
    x = b.reduce_window_max(x, 3, 2, 1)
    for st, nblocks in enumerate((3, 4, 6, 3)):
        width = 64 << st
        for blk in range(nblocks):
            s = 2 if (blk == 0 and st > 0) else 1
            pre = f"conv{st + 2}_block{blk + 1}"
            shortcut = conv(x, 4 * width, 1, s, f"{pre}_0", False) if blk == 0 else x
            t = conv(x, width, 1, 1, f"{pre}_1", True)
            t = conv(t, width, 3, s, f"{pre}_2", True)
            x = conv(t, 4 * width, 1, 1, f"{pre}_3", True, residual=shortcut)
    n, h, w, c = x.shape
    pooled = b.binary("divide", b.reduce(x, [1, 2], "sum"), b.splat(float(h * w), [n, c]))
    fw = b.param([c, classes], "predictions/w")
    fb = b.param([classes], "predictions/b")
    logits = b.add_vec(b.dot(pooled, fw, [1], [0]), fb)
    probs = b.softmax(logits)
    return b.text(probs), b.params


def bert_base(batch: int = 8, seq: int = 128, layers: int = 12, hidden: int = 768,
              heads: int = 12, ffn: int = 3072, eps: float = 1e-12):
    """BERT-base encoder module from the embedding LayerNorm's output:
    params x [batch, seq, hidden], the additive attention mask [seq], then per layer
    wqkv [hidden, 3*hidden], bqkv, wo, bo, ln1 gamma/beta, w1, b1, w2, b2, ln2 gamma/beta."""
    b = HloBuilder(f"bert_base_b{batch}_s{seq}_l{layers}")
    hd = hidden // heads
    x = b.param([batch, seq, hidden], "embeddings_ln")
    mask = b.param([seq], "mask")
    for l in range(layers):
        p = f"layer{l}"
        wqkv = b.param([hidden, 3 * hidden], f"{p}_qkv/w")
        bqkv = b.param([3 * hidden], f"{p}_qkv/b")
        qkv = b.add_vec(b.dot(x, wqkv, [2], [0]), bqkv)

        def heads_of(k):
            t = b.slice(qkv, [0, 0, k * hidden], [batch, seq, (k + 1) * hidden])
            t = b.reshape(t, [batch, seq, heads, hd])
            return b.transpose(t, [0, 2, 1, 3])

        q, k, v = heads_of(0), heads_of(1), heads_of(2)
        scores = b.dot(q, k, [3], [3], [0, 1], [0, 1])
        scores = b.binary("multiply", scores, b.splat(1.0 / math.sqrt(hd), scores.shape))
        scores = b.binary("add", scores, b.bcast(mask, scores.shape, [3]))
        probs = b.softmax(scores)
        ctxv = b.dot(probs, v, [3], [2], [0, 1], [0, 1])
        ctxv = b.reshape(b.transpose(ctxv, [0, 2, 1, 3]), [batch, seq, hidden])
        wo = b.param([hidden, hidden], f"{p}_attn_out/w")
        bo = b.param([hidden], f"{p}_attn_out/b")
        t1 = b.binary("add", b.add_vec(b.dot(ctxv, wo, [2], [0]), bo), x)
        g1 = b.param([hidden], f"{p}_attn_ln/gamma")
        be1 = b.param([hidden], f"{p}_attn_ln/beta")
        x1 = b.layernorm(t1, g1, be1, eps)
        w1 = b.param([hidden, ffn], f"{p}_ffn1/w")
        b1 = b.param([ffn], f"{p}_ffn1/b")
        hdn = b.gelu_erf(b.add_vec(b.dot(x1, w1, [2], [0]), b1))
        w2 = b.param([ffn, hidden], f"{p}_ffn2/w")
        b2 = b.param([hidden], f"{p}_ffn2/b")
        t2 = b.binary("add", b.add_vec(b.dot(hdn, w2, [2], [0]), b2), x1)
        g2 = b.param([hidden], f"{p}_out_ln/gamma")
        be2 = b.param([hidden], f"{p}_out_ln/beta")
        x = b.layernorm(t2, g2, be2, eps)
    return b.text(x), b.params


def llama_decode_step(n_layers: int = 22, hidden: int = 2048, n_heads: int = 32,
                      n_kv_heads: int = 4, head_dim: int = 64, ffn: int = 5632,
                      vocab: int = 32000, max_seq: int = 64, rms_eps: float = 1e-5):
    """One M=1 decode step of the TinyLlama graph (export_llama.py:284-375) against a KV
    cache.  Params: h [1, hidden] (the token's embedding row), cos / sin [1, head_dim] of the
    position (run_llama_spirv.py:87-97), mask [max_seq + 1] (0 for cached positions < pos
    and for the last entry, the new token; -1e9 elsewhere), then per layer attn_norm,
    wqkv [(n_heads + 2 n_kv) * head_dim, hidden] ([out, in] rows: q | k | v), wo
    [hidden, n_heads * head_dim], ffn_norm, w_gate_up [2 ffn, hidden] (gate / up rows
    interleaved), w_down [hidden, ffn], k_cache / v_cache [n_kv, max_seq, head_dim]; then
    final_norm and lm_head [vocab, hidden].  The weights are the decoder's own layout, read
    with rhs_contracting_dims={1}.  Output tuple: logits [1, vocab], then per layer the new
    key and value [n_kv, 1, head_dim] (rotated key) for the caller to store at `pos`.
    Masked cache rows still enter the score and context products (times a zero weight), so
    every cache row must hold finite values: zero-initialise the caches."""
    b = HloBuilder(f"llama_decode_l{n_layers}_h{hidden}")
    qd, kvd, g = n_heads * head_dim, n_kv_heads * head_dim, n_heads // n_kv_heads
    T = max_seq + 1
    half = head_dim // 2
    h = b.param([1, hidden], "h")
    cos = b.param([1, head_dim], "rope_cos")
    sin = b.param([1, head_dim], "rope_sin")
    mask = b.param([T], "mask")
    outs = []

    def rope(t: Val, nh: int) -> Val:  # t [nh, 1, head_dim], rotate-half (export_llama.py:288-296)
        x1 = b.slice(t, [0, 0, 0], [nh, 1, half])
        x2 = b.slice(t, [0, 0, half], [nh, 1, head_dim])
        rot = b.concat([b.unary("negate", x2), x1], 2)
        c = b.bcast(b.reshape(cos, [head_dim]), t.shape, [2])
        s = b.bcast(b.reshape(sin, [head_dim]), t.shape, [2])
        return b.binary("add", b.binary("multiply", t, c), b.binary("multiply", rot, s))

    for l in range(n_layers):
        p = f"layer{l}"
        an = b.param([hidden], f"{p}/attn_norm")
        wqkv = b.param([qd + 2 * kvd, hidden], f"{p}/wqkv")
        wo = b.param([hidden, qd], f"{p}/wo")
        fn = b.param([hidden], f"{p}/ffn_norm")
        wgu = b.param([2 * ffn, hidden], f"{p}/w_gate_up")
        wd = b.param([hidden, ffn], f"{p}/w_down")
        kc = b.param([n_kv_heads, max_seq, head_dim], f"{p}/k_cache")
        vc = b.param([n_kv_heads, max_seq, head_dim], f"{p}/v_cache")
        xn = b.rmsnorm(h, an, rms_eps)
        qkv = b.dot(xn, wqkv, [1], [1])                              # [1, qd + 2 kvd]
        q = b.transpose(b.reshape(b.slice(qkv, [0, 0], [1, qd]), [1, n_heads, head_dim]),
                        [1, 0, 2])                                   # [n_heads, 1, hd]
        k = b.transpose(b.reshape(b.slice(qkv, [0, qd], [1, qd + kvd]),
                                  [1, n_kv_heads, head_dim]), [1, 0, 2])
        v = b.transpose(b.reshape(b.slice(qkv, [0, qd + kvd], [1, qd + 2 * kvd]),
                                  [1, n_kv_heads, head_dim]), [1, 0, 2])
        q, k = rope(q, n_heads), rope(k, n_kv_heads)
        outs += [k, v]
        keys = b.concat([kc, k], 1)                                  # [n_kv, T, hd]
        vals = b.concat([vc, v], 1)
        # GQA: query head hh reads kv head hh // g (export_llama.py:333-343 tiles x g)
        qg = b.reshape(q, [n_kv_heads, g, head_dim])
        sc = b.dot(qg, keys, [2], [2], [0], [0])                     # [n_kv, g, T]
        sc = b.binary("multiply", sc, b.splat(1.0 / math.sqrt(head_dim), sc.shape))
        sc = b.binary("add", sc, b.bcast(mask, sc.shape, [2]))
        pr = b.softmax(sc)
        att = b.dot(pr, vals, [2], [1], [0], [0])                    # [n_kv, g, hd]
        att = b.reshape(att, [1, qd])
        h = b.binary("add", b.dot(att, wo, [1], [1]), h)
        xn = b.rmsnorm(h, fn, rms_eps)
        gu = b.reshape(b.dot(xn, wgu, [1], [1]), [1, ffn, 2])
        gate = b.reshape(b.slice(gu, [0, 0, 0], [1, ffn, 1]), [1, ffn])
        up = b.reshape(b.slice(gu, [0, 0, 1], [1, ffn, 2]), [1, ffn])
        act = b.binary("multiply", b.binary("multiply", gate, b.unary("logistic", gate)), up)
        h = b.binary("add", b.dot(act, wd, [1], [1]), h)
    fnorm = b.param([hidden], "final_norm")
    lm = b.param([vocab, hidden], "lm_head")
    logits = b.dot(b.rmsnorm(h, fnorm, rms_eps), lm, [1], [1])
    root = b.tuple([logits] + outs)
    shapes = [logits.shape] + [o.shape for o in outs]
    return b.text(root, shapes), b.params


def model_bindings(model, spec):
    """Bind a generated module's parameters (resnet50_v15 / bert_base) to the tensors of the
    resident C++ graph of the same config (models.Model, shp_model_*), read in place: the
    HLO path and the graph then run on the same weights and inputs."""
    from .runtime import DeviceTensor
    by_label = {op.label: op for op in model.ops()}

    def tensor(tid: int, need: int) -> DeviceTensor:
        info = model.tensor_info(tid)
        if info.elems < need:
            raise ValueError(f"model tensor {tid} has {info.elems} elements, need {need}")
        return DeviceTensor(model.ctx, info.elems, ptr=info.ptr, owned=False)

    out = []
    for label, shape in spec:
        n = int(np.prod(shape))
        if label == "input":
            out.append(model.input(0))
        elif label == "embeddings_ln":
            out.append(tensor(by_label["embeddings_ln"].out, n))
        elif label == "mask":  # the softmax's, or the fused attention's at sequence 128
            op = by_label.get("layer0_softmax") or by_label["layer0_attention"]
            out.append(tensor(op.in1, n))
        else:
            name, part = label.rsplit("/", 1)
            op = by_label[name]
            if part == "w":
                out.append(tensor(op.in1, n))
            elif part == "b":
                out.append(tensor(op.bias, n))
            elif part == "gamma":   # layernorm_rows weights are [gamma | beta] in one tensor
                out.append((tensor(op.in1, 2 * n), 0))
            elif part == "beta":
                out.append((tensor(op.in1, 2 * n), n))
            else:
                raise KeyError(label)
    return out


def llama_bindings(lm, spec):
    """Bind llama_decode_step's weight and cache parameters to a decoder's resident tensors
    (models.Llama, shp_llama_weight); the per-step inputs h / rope_cos / rope_sin / mask get
    zero arrays for the caller to set (HloProgram.set_param)."""
    from .runtime import DeviceTensor
    out = []
    for label, shape in spec:
        n = int(np.prod(shape))
        if label in ("h", "rope_cos", "rope_sin", "mask"):
            out.append(np.zeros(shape, np.float32))
            continue
        if "/" in label:
            layer, which = label.split("/")
            ptr, elems = lm.weight_ptr(int(layer[len("layer"):]), which)
        else:
            ptr, elems = lm.weight_ptr(0, label)
        if elems != n:
            raise ValueError(f"{label}: decoder tensor has {elems} elements, module needs {n}")
        out.append(DeviceTensor(lm.ctx, elems, ptr=ptr, owned=False))
    return out


def main(argv=None) -> int:
    """Write a config's module: python -m spirv_inference_amd.hlo_gen --model resnet50_v15
    --batch 32 --output resnet50_b32.hlo.txt (plus a .params.json of labels and shapes)."""
    import argparse
    import json
    import pathlib
    ap = argparse.ArgumentParser(description="HLO text modules of the benchmark configs")
    ap.add_argument("--model", required=True,
                    choices=["resnet50_v15", "bert_base", "llama_decode_step"])
    ap.add_argument("--batch", type=int, default=None)
    ap.add_argument("--seq", type=int, default=128)
    ap.add_argument("--layers", type=int, default=None)
    ap.add_argument("--max-seq", type=int, default=64)
    ap.add_argument("--output", required=True, type=pathlib.Path)
    a = ap.parse_args(argv)
    if a.model == "resnet50_v15":
        text, spec = resnet50_v15(a.batch or 32)
    elif a.model == "bert_base":
        text, spec = bert_base(a.batch or 8, a.seq, a.layers or 12)
    else:
        text, spec = llama_decode_step(n_layers=a.layers or 22, max_seq=a.max_seq)
    a.output.write_text(text)
    a.output.with_suffix(".params.json").write_text(
        json.dumps([{"label": l, "shape": s} for l, s in spec], indent=1) + "\n")
    print(f"{a.output}: {len(text.splitlines())} lines, {len(spec)} parameters")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
