"""TFLite front end on the GPU: TFL3 models run by TfliteExecutor on the registry kernels,
against a float64 numpy restatement of the TFLite ops (small graphs) and against the resident
model graph the file was exported from.

Gates: per-graph outputs within 1e-4 abs + 1e-4 rel (BASELINE.json per-op tolerance); the
exported MobileNetV2 and EfficientNet-Lite0 bit-identical to the graphs they came from,
eagerly and from the executor's hipGraph.
"""
import json
import subprocess
import sys

import numpy as np
import pytest

from conftest import ROOT, assert_close
from spirv_inference_amd import tflite as T

pytestmark = pytest.mark.gpu
RNG = np.random.default_rng(7)


def rnd(*shape, scale=1.0):
    return (RNG.standard_normal(shape) * scale).astype(np.float32)


def test_logistic_model(ctx):
    """The reference's synthetic loader smoke model: LOGISTIC over the deterministic ramp."""
    w = T.TfliteWriter("synthetic float32 logistic model")
    i, o = w.tensor("input", [1, 8]), w.tensor("output", [1, 8])
    w.inputs, w.outputs = [i], [o]
    w.op("LOGISTIC", [i], [o])
    m = T.parse_model(w.finish())
    print("[gpu] tflite logistic", flush=True)
    rep, y = T.run_model(ctx, m)
    x = T.default_input(8).astype(np.float64)
    assert_close(y, 1.0 / (1.0 + np.exp(-x)), 1e-6, 1e-6, "logistic")
    assert rep["status"] == "pass" and rep["ops"][0]["dispatches"][0]["kernel"] == "sigmoid"


# ---- float64 numpy restatement of the TFLite ops used below --------------------------------
def ref_conv(x, w, b, stride, same, act):
    n, ih, iw, ic = x.shape
    oc, kh, kw, _ = w.shape
    if same:
        oh, ow = -(-ih // stride), -(-iw // stride)
        ph = max((oh - 1) * stride + kh - ih, 0)
        pw = max((ow - 1) * stride + kw - iw, 0)
        x = np.pad(x, ((0, 0), (ph // 2, ph - ph // 2), (pw // 2, pw - pw // 2), (0, 0)))
    else:
        oh, ow = (ih - kh) // stride + 1, (iw - kw) // stride + 1
    y = np.zeros((n, oh, ow, oc))
    for dy in range(kh):
        for dx in range(kw):
            patch = x[:, dy:dy + stride * oh:stride, dx:dx + stride * ow:stride, :]
            y += patch @ w[:, dy, dx, :].T.astype(np.float64)
    return act(y + b)


def ref_depthwise(x, w, b, stride, act):
    n, ih, iw, c = x.shape
    _, kh, kw, _ = w.shape
    oh, ow = -(-ih // stride), -(-iw // stride)
    ph, pw = max((oh - 1) * stride + kh - ih, 0), max((ow - 1) * stride + kw - iw, 0)
    x = np.pad(x, ((0, 0), (ph // 2, ph - ph // 2), (pw // 2, pw - pw // 2), (0, 0)))
    y = np.zeros((n, oh, ow, c))
    for dy in range(kh):
        for dx in range(kw):
            y += x[:, dy:dy + stride * oh:stride, dx:dx + stride * ow:stride, :] * w[0, dy, dx]
    return act(y + b)


relu6 = lambda v: np.clip(v, 0.0, 6.0)
ident = lambda v: v


def test_small_cnn_graph(ctx):
    """CONV_2D (SAME, stride 2, RELU6) -> DEPTHWISE 3x3 (RELU6) -> CONV 1x1 -> ADD ->
    MAX_POOL 2x2 VALID -> CONCATENATION(axis 3) -> MEAN(H,W) -> FULLY_CONNECTED -> SOFTMAX,
    operators stored out of order so the executor must sort them."""
    n, hw, c0, c1 = 2, 11, 3, 8
    x = rnd(n, hw, hw, c0)
    w1, b1 = rnd(c1, 3, 3, c0, scale=0.3), rnd(c1, scale=0.1)
    wd, bd = rnd(1, 3, 3, c1, scale=0.3), rnd(c1, scale=0.1)
    w2, b2 = rnd(c1, 1, 1, c1, scale=0.3), rnd(c1, scale=0.1)
    wf, bf = rnd(10, 2 * c1, scale=0.3), rnd(10, scale=0.1)

    w = T.TfliteWriter("small cnn")
    tx = w.tensor("x", [n, hw, hw, c0])
    h1 = w.tensor("h1", [n, 6, 6, c1])
    h2 = w.tensor("h2", [n, 6, 6, c1])
    h3 = w.tensor("h3", [n, 6, 6, c1])
    h4 = w.tensor("h4", [n, 6, 6, c1])
    h5 = w.tensor("h5", [n, 3, 3, c1])
    h6 = w.tensor("h6", [n, 3, 3, 2 * c1])
    h7 = w.tensor("h7", [n, 2 * c1])
    h8 = w.tensor("h8", [n, 10])
    y = w.tensor("y", [n, 10])
    ax = w.tensor("axes", [2], np.array([1, 2], np.int32).view(np.float32), ttype=2)
    cw = [w.tensor(nm, a.shape, a) for nm, a in
          (("w1", w1), ("b1", b1), ("wd", wd), ("bd", bd), ("w2", w2), ("b2", b2),
           ("wf", wf), ("bf", bf))]
    w.inputs, w.outputs = [tx], [y]
    w.op("SOFTMAX", [h8], [y], "SoftmaxOptions", {0: ("f", 1.0)})
    w.op("FULLY_CONNECTED", [h7, cw[6], cw[7]], [h8], "FullyConnectedOptions", {})
    w.op("CONV_2D", [tx, cw[0], cw[1]], [h1], "Conv2DOptions",
         {0: ("b", 0), 1: ("i", 2), 2: ("i", 2), 3: ("b", 3)})
    w.op("DEPTHWISE_CONV_2D", [h1, cw[2], cw[3]], [h2], "DepthwiseConv2DOptions",
         {0: ("b", 0), 1: ("i", 1), 2: ("i", 1), 3: ("i", 1), 4: ("b", 3)})
    w.op("CONV_2D", [h2, cw[4], cw[5]], [h3], "Conv2DOptions", {0: ("b", 0)})
    w.op("ADD", [h3, h1], [h4], "AddOptions", {})
    w.op("MAX_POOL_2D", [h4], [h5], "Pool2DOptions",
         {0: ("b", 1), 1: ("i", 2), 2: ("i", 2), 3: ("i", 2), 4: ("i", 2)})
    w.op("CONCATENATION", [h5, h5], [h6], "ConcatenationOptions", {0: ("i", 3)})
    w.op("MEAN", [h6, ax], [h7], "ReducerOptions", {})
    m = T.parse_model(w.finish())
    assert T.topological_order(m)[-2:] == [1, 0]
    print("[gpu] tflite small cnn", flush=True)
    rep, got = T.run_model(ctx, m, x)

    xd = x.astype(np.float64)
    r1 = ref_conv(xd, w1, b1, 2, True, relu6)
    r2 = ref_depthwise(r1, wd, bd, 1, relu6)
    r4 = ref_conv(r2, w2, b2, 1, True, ident) + r1
    r5 = r4.reshape(n, 3, 2, 3, 2, c1).max(axis=(2, 4))
    r7 = np.concatenate([r5, r5], axis=3).mean(axis=(1, 2))
    r8 = r7 @ wf.T.astype(np.float64) + bf
    e = np.exp(r8 - r8.max())
    ref = e / e.sum()  # softmax1000 over every element of the output, as the reference
    assert_close(got, ref.reshape(-1), 1e-4, 1e-4, "small cnn probs")
    kernels = [d["kernel"] for op in rep["ops"] for d in op["dispatches"]]
    # the residual ADD runs in the second convolution's epilogue
    assert kernels == ["conv2d_nhwc", "depthwise_conv2d_nhwc", "conv2d_nhwc",
                       "hlo_reduce_window_rank4", "hlo_concatenate_into", "hlo_concatenate_into",
                       "global_avg_pool_nhwc", "fully_connected", "softmax1000"]
    add = next(op for op in rep["ops"] if op["op"] == "ADD")
    assert add["dispatches"] == [] and "fused_into" in add
    # one executor over several inputs: every tensor keeps its buffer, results repeat
    ex = T.TfliteExecutor(ctx, m)
    try:
        ex.set_input(x)
        ex.run()
        first = ex.output()
        owned = len(ex.owned)
        ex.set_input(rnd(n, hw, hw, c0))
        ex.run()
        ex.set_input(x)
        ex.run()
        assert len(ex.owned) == owned, "run() allocated new buffers"
        assert len(ex.op_log) == len(m.operators)
        assert ex.output().tobytes() == first.tobytes()
        assert_close(first, ref.reshape(-1), 1e-4, 1e-4, "small cnn probs (executor reuse)")
    finally:
        ex.close()


@pytest.mark.parametrize("arch,batch,adds", [("mobilenet_v2", 1, 10),
                                             ("efficientnet_lite0", 8, 9)])
def test_export_roundtrip_and_graph_replay(ctx, arch, batch, adds):
    """A resident model graph exported to TFL3, parsed back and run by the executor equals
    the graph's own run bit for bit: every op is the same kernel with the same push vector
    on the same weights (the executor folds each CONV_2D + ADD residual back into one
    epilogue launch, as the graph has it).  Replays of the executor's hipGraph equal its
    eager run, with a new input set between replays."""
    from spirv_inference_amd.models import Model
    with Model(ctx, arch, batch, seed=2) as mdl:
        mdl.run()
        ctx.sync()
        probs = mdl.output(0).download()
        x = mdl.input(0).download()
        n_graph_ops = len(mdl.ops())
        data = T.model_to_tflite(mdl)
    m = T.parse_model(data)
    assert not m.unsupported_ops and not m.quantized_tensors
    assert m.op_histogram["ADD"] == adds
    print(f"[gpu] tflite {arch} b{batch} export: {len(data)} bytes, {len(m.operators)} ops",
          flush=True)
    ex = T.TfliteExecutor(ctx, m)
    try:
        assert len(ex.residual_adds) == adds
        ex.set_input(x)
        ex.run()
        ctx.sync()
        eager = ex.output()
        assert sum(len(o["dispatches"]) for o in ex.op_log) == n_graph_ops
        assert eager.tobytes() == probs.tobytes(), np.abs(eager - probs).max()
        x2 = (x[::-1] * 0.5).astype(np.float32).copy()
        for rep in range(3):
            ex.set_input(x if rep % 2 == 0 else x2)
            ex.run(graph=True)
            ctx.sync()
            got = ex.output()
            if rep % 2 == 0:
                assert got.tobytes() == eager.tobytes(), f"replay {rep}"
            else:
                other = got
        ex.set_input(x2)
        ex.run()  # eager on the second input equals its replay
        ctx.sync()
        assert ex.output().tobytes() == other.tobytes()
    finally:
        ex.close()
    rep, got = T.run_model(ctx, m, x)
    assert got.tobytes() == probs.tobytes()
    assert rep["top1"] == T.top1(probs)


def test_tflite_run_cli(tmp_path):
    """The CLI (main.rs's flags): kernel self-test, then a model with a report and dumps."""
    w = T.TfliteWriter("cli")
    i, o = w.tensor("input", [1, 16]), w.tensor("output", [1, 16])
    w.inputs, w.outputs = [i], [o]
    w.op("TANH", [i], [o])
    path = tmp_path / "tanh.tflite"
    path.write_bytes(w.finish())
    report = tmp_path / "report.json"
    print("[gpu] tflite_run CLI", flush=True)
    r = subprocess.run([sys.executable, "-m", "spirv_inference_amd.tflite_run", "--model",
                        str(path), "--report", str(report), "--dump-dir", str(tmp_path / "d"),
                        "--self-test-kernels"], cwd=ROOT, capture_output=True, text=True,
                       timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    rep = json.loads(report.read_text())
    assert rep["status"] == "pass"
    st = rep["sections"]["kernel_self_test"]
    assert st["status"] == "pass" and len(st["cases"]) == 15
    assert all(c["mismatch_count"] == 0 for c in st["cases"])
    dumped = np.fromfile(tmp_path / "d" / "output.raw.f32", "<f4")
    np.testing.assert_allclose(dumped, np.tanh(T.default_input(16)), rtol=1e-5, atol=1e-6)


def test_elementwise_graph(ctx):
    """Every binary and unary lowering, fused activations on ADD and AVERAGE_POOL_2D, RESHAPE
    views, L2_NORMALIZATION and the 10-class SOFTMAX, chained, against float64 numpy."""
    shape = [1, 4, 4, 10]
    x = RNG.uniform(0.5, 2.0, shape).astype(np.float32)
    c = RNG.uniform(0.5, 2.0, shape).astype(np.float32)
    ten = np.full(shape, 10.0, np.float32)
    w = T.TfliteWriter("elementwise")
    tx = w.tensor("x", shape)
    tc, tten = w.tensor("c", shape, c), w.tensor("ten", shape, ten)
    w.inputs = [tx]
    d = {}

    def op(name, builtin, ins, out_shape=shape, kind=None, opts=None):
        d[name] = w.tensor(name, out_shape)
        w.op(builtin, ins, [d[name]], kind, opts or {})
        return d[name]

    op("t1", "SUB", [tx, tc])
    op("t2", "MUL", [d["t1"], tc])
    op("t3", "DIV", [d["t2"], tc])
    op("t4", "POW", [tx, tc])
    op("t5", "MINIMUM", [d["t3"], d["t4"]])
    op("t6", "MAXIMUM", [d["t5"], d["t1"]])
    op("t7", "ABS", [d["t6"]])
    op("t8", "NEG", [d["t7"]])
    op("t9", "EXP", [d["t8"]])
    op("t10", "LOG", [d["t9"]])
    op("t11", "SQRT", [d["t4"]])
    op("t12", "RSQRT", [d["t4"]])
    op("t13", "TANH", [d["t1"]])
    op("t14", "LOGISTIC", [d["t13"]])
    op("t15", "LEAKY_RELU", [d["t1"]], kind="LeakyReluOptions", opts={0: ("f", 0.1)})
    op("t16", "MUL", [d["t15"], tten])
    op("t17", "RELU6", [d["t16"]])
    op("t18", "ADD", [d["t17"], d["t12"]], kind="AddOptions", opts={0: ("b", 3)})
    op("t19", "ADD", [d["t18"], d["t10"]])
    op("t20", "ADD", [d["t19"], d["t11"]])
    op("t21", "ADD", [d["t20"], d["t14"]])
    op("flat", "RESHAPE", [d["t21"]], [1, 160])
    op("l2", "L2_NORMALIZATION", [d["flat"]], [1, 160])
    op("back", "RESHAPE", [d["l2"]])
    op("pool", "AVERAGE_POOL_2D", [d["back"]], [1, 1, 1, 10], "Pool2DOptions",
       {0: ("b", 1), 1: ("i", 4), 2: ("i", 4), 3: ("i", 4), 4: ("i", 4), 5: ("b", 1)})
    op("y", "SOFTMAX", [d["pool"]], [1, 10], "SoftmaxOptions", {0: ("f", 1.0)})
    w.outputs = [d["y"]]
    m = T.parse_model(w.finish())
    print("[gpu] tflite elementwise graph", flush=True)
    rep, got = T.run_model(ctx, m, x)

    X, Cc = x.astype(np.float64), c.astype(np.float64)
    t1 = X - Cc
    t3 = t1 * Cc / Cc
    t4 = X ** Cc
    t6 = np.maximum(np.minimum(t3, t4), t1)
    t10 = np.log(np.exp(-np.abs(t6)))
    t11, t12 = np.sqrt(t4), 1.0 / np.sqrt(t4)
    t14 = 1.0 / (1.0 + np.exp(-np.tanh(t1)))
    t17 = np.clip(np.where(t1 >= 0, t1, 0.1 * t1) * 10.0, 0.0, 6.0)
    t18 = np.clip(t17 + t12, 0.0, 6.0)
    t21 = t18 + t10 + t11 + t14
    l2 = t21 / np.sqrt((t21 ** 2).sum())
    pool = np.maximum(l2.reshape(16, 10).mean(axis=0), 0.0)
    e = np.exp(pool - pool.max())
    assert_close(got, e / e.sum(), 1e-4, 1e-4, "elementwise graph")
    kernels = {d_["kernel"] for o in rep["ops"] for d_ in o["dispatches"]}
    assert {"sub", "mul", "div", "pow", "min", "max", "abs", "neg", "exp", "log", "sqrt",
            "rsqrt", "tanh", "sigmoid", "leaky_relu", "relu6", "add", "l2_normalization",
            "global_avg_pool_nhwc", "relu", "softmax10"} <= kernels
