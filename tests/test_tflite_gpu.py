"""TFLite front end on the GPU: TFL3 models run by TfliteExecutor on the registry kernels,
against a float64 numpy restatement of the TFLite ops (small graphs) and against the resident
model graph the file was exported from.

Gates: per-graph outputs within 1e-4 abs + 1e-4 rel (BASELINE.json per-op tolerance), the
exported MobileNetV2 bit-identical to the graph it came from except for the residual adds
(one rounding apart), identical top-1.
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
    assert kernels == ["conv2d_nhwc", "depthwise_conv2d_nhwc", "conv2d_nhwc", "add",
                       "hlo_reduce_window_rank4", "hlo_concatenate_into", "hlo_concatenate_into",
                       "global_avg_pool_nhwc", "fully_connected", "softmax1000"]


def test_mobilenet_v2_export_roundtrip(ctx):
    """A resident MobileNetV2 graph exported to TFL3, parsed back and run by the executor
    equals the graph's own run: every op is the same kernel on the same weights, except that
    a residual the graph fuses into the projection convolution becomes CONV_2D + ADD."""
    from spirv_inference_amd.models import Model
    with Model(ctx, "mobilenet_v2", 1, seed=2) as mdl:
        mdl.run()
        ctx.sync()
        probs = mdl.output(0).download()
        logits = mdl.output(1).download()
        x = mdl.input(0).download()
        data = T.model_to_tflite(mdl)
    m = T.parse_model(data)
    assert not m.unsupported_ops and not m.quantized_tensors
    assert m.op_histogram["ADD"] == 10 and m.op_histogram["DEPTHWISE_CONV_2D"] == 17
    print(f"[gpu] tflite mobilenet_v2 export: {len(data)} bytes, {len(m.operators)} ops",
          flush=True)
    rep, got = T.run_model(ctx, m, x)
    assert_close(got, probs, 1e-6, 1e-4, "exported mobilenet_v2 probs")
    assert int(np.argmax(got)) == int(np.argmax(probs)) == int(np.argmax(logits))
    assert rep["top1"]["model_class"] == int(np.argmax(probs))


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
