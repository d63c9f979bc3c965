"""TFLite front end on the CPU: FlatBuffer reading / writing, option decoding with the
reference's defaults, topological order, unsupported-op and quantized-tensor detection
(source/tflite_loader/src/{model,op_decoder,graph,scheduler}.rs)."""
import struct

import numpy as np
import pytest

from spirv_inference_amd import tflite as T


def logistic_model() -> bytes:
    """The model fixtures/make_synthetic_logistic_tflite.py:20-83 writes: tensors input /
    output [1, 8], one LOGISTIC operator (deprecated and new builtin code 14), version 3."""
    w = T.TfliteWriter("synthetic float32 logistic model for cuda-spirv loader smoke test")
    i = w.tensor("input", [1, 8])
    o = w.tensor("output", [1, 8])
    w.inputs, w.outputs = [i], [o]
    w.op("LOGISTIC", [i], [o])
    return w.finish()


def test_logistic_fixture_fields():
    data = logistic_model()
    assert data[4:8] == b"TFL3"
    m = T.parse_model(data, "logistic.tflite")
    assert m.version == 3
    assert m.description.startswith("synthetic float32 logistic model")
    assert [(t.name, t.shape, t.tensor_type) for t in m.tensors] == [
        ("input", [1, 8], "Float32"), ("output", [1, 8], "Float32")]
    assert (m.inputs, m.outputs) == ([0], [1])
    assert [(o.builtin, o.code, o.inputs, o.outputs) for o in m.operators] == [
        ("LOGISTIC", 14, [0], [1])]
    assert m.op_histogram == {"LOGISTIC": 1} and not m.unsupported_ops
    assert T.validate_supported_graph(m)["status"] == "pass"
    assert T.topological_order(m) == [0]
    s = m.summary()
    assert s["buffers"][0]["data_len"] == 0 and s["operators"][0]["builtin_options_table_pos"] is None


def test_identifier_and_size_checks():
    with pytest.raises(ValueError, match="too small"):
        T.parse_model(b"TFL3")
    bad = bytearray(logistic_model())
    bad[4:8] = b"XXXX"
    with pytest.raises(ValueError, match="TFL3"):
        T.parse_model(bytes(bad))
    truncated = logistic_model()[:40]
    with pytest.raises(ValueError):
        T.parse_model(truncated)


def test_constant_buffers_roundtrip():
    w = T.TfliteWriter()
    x = w.tensor("x", [1, 4, 4, 3])
    data = np.arange(2 * 3 * 3 * 3, dtype=np.float32) * 0.5
    k = w.tensor("k", [2, 3, 3, 3], data)
    y = w.tensor("y", [1, 4, 4, 2])
    w.inputs, w.outputs = [x], [y]
    w.op("CONV_2D", [x, k, -1], [y], "Conv2DOptions",
         {0: ("b", 1), 1: ("i", 2), 2: ("i", 3), 3: ("b", 3), 4: ("i", 1), 5: ("i", 1)})
    m = T.parse_model(w.finish())
    buf = m.buffers[m.tensors[1].buffer]
    np.testing.assert_array_equal(np.frombuffer(buf.data, "<f4"), data)
    assert buf.data_offset % 16 == 0
    o = T.decode_options(m.operators[0])
    assert o == {"kind": "conv2d", "padding": "valid", "stride_w": 2, "stride_h": 3,
                 "fused_activation": "relu6", "dilation_w_factor": 1, "dilation_h_factor": 1}
    assert m.operators[0].options_type == T.OPTIONS_TYPE["Conv2DOptions"]
    assert m.operators[0].inputs == [0, 1, -1]


@pytest.mark.parametrize("builtin,kind,expected", [
    ("CONV_2D", "Conv2DOptions", {"padding": "same", "stride_w": 1, "stride_h": 1,
                                  "fused_activation": "none", "dilation_w_factor": 1,
                                  "dilation_h_factor": 1}),
    ("DEPTHWISE_CONV_2D", "DepthwiseConv2DOptions", {"depth_multiplier": 1, "stride_w": 1}),
    ("MAX_POOL_2D", "Pool2DOptions", {"filter_w": 1, "filter_h": 1, "padding": "same"}),
    ("SOFTMAX", "SoftmaxOptions", {"beta": 1.0}),
    ("LEAKY_RELU", "LeakyReluOptions", {"alpha": pytest.approx(0.2)}),
    ("CONCATENATION", "ConcatenationOptions", {"axis": 0, "fused_activation": "none"}),
    ("MEAN", "ReducerOptions", {"keep_dims": False}),
])
def test_option_defaults(builtin, kind, expected):
    """Absent option fields take op_decoder.rs's defaults (stride 1, dilation 1, beta 1.0,
    leaky alpha 0.2, SAME padding, no activation)."""
    w = T.TfliteWriter()
    a = w.tensor("a", [1, 2, 2, 2])
    b = w.tensor("b", [1, 2, 2, 2])
    w.inputs, w.outputs = [a], [b]
    w.op(builtin, [a], [b], kind, {})
    o = T.decode_options(T.parse_model(w.finish()).operators[0])
    for k, v in expected.items():
        assert o[k] == v, (k, o)


def test_resize_bilinear_reads_schema_fields():
    w = T.TfliteWriter()
    a = w.tensor("a", [1, 2, 2, 1])
    b = w.tensor("b", [1, 4, 4, 1])
    w.inputs, w.outputs = [a], [b]
    w.op("RESIZE_BILINEAR", [a], [b], "ResizeBilinearOptions", {2: ("B", 1), 3: ("B", 0)})
    o = T.decode_options(T.parse_model(w.finish()).operators[0])
    assert o == {"kind": "resize", "align_corners": True, "half_pixel_centers": False}


def _two_op_model(first_consumer: bool) -> T.TfliteModel:
    w = T.TfliteWriter()
    x = w.tensor("x", [4])
    h = w.tensor("h", [4])
    y = w.tensor("y", [4])
    w.inputs, w.outputs = [x], [y]
    if first_consumer:
        w.op("EXP", [h], [y])
        w.op("ABS", [x], [h])
    else:
        w.op("ABS", [x], [h])
        w.op("EXP", [h], [y])
    return T.parse_model(w.finish())


def test_topological_order():
    """scheduler.rs:1684-1730: a model already in ready order keeps it; otherwise producers
    come first; two producers of one tensor are an error."""
    assert T.topological_order(_two_op_model(False)) == [0, 1]
    assert T.topological_order(_two_op_model(True)) == [1, 0]
    w = T.TfliteWriter()
    x = w.tensor("x", [4])
    y = w.tensor("y", [4])
    w.inputs, w.outputs = [x], [y]
    w.op("ABS", [x], [y])
    w.op("EXP", [x], [y])
    with pytest.raises(ValueError, match="multiple producers"):
        T.topological_order(T.parse_model(w.finish()))


def test_unsupported_and_quantized_detection():
    """model.rs:334-350 / graph.rs:5-21: an operator code outside the recognised table and a
    non-float, non-int32 tensor each block the graph."""
    w = T.TfliteWriter()
    x = w.tensor("x", [4])
    y = w.tensor("y", [4], ttype=3)  # UInt8
    w.inputs, w.outputs = [x], [y]
    w.op("ABS", [x], [y])
    data = bytearray(w.finish())
    m = T.parse_model(bytes(data))
    assert m.quantized_tensors == ["y:UInt8"]
    with pytest.raises(ValueError, match="quantized"):
        T.validate_supported_graph(m)
    # RELU (code 19) is not in the reference's operator table
    w = T.TfliteWriter()
    x = w.tensor("x", [4])
    y = w.tensor("y", [4])
    w.inputs, w.outputs = [x], [y]
    w.op("ABS", [x], [y])
    w.opcodes[0] = 19
    m = T.parse_model(w.finish())
    assert m.unsupported_ops == ["operator 0: UNKNOWN_19"]
    with pytest.raises(ValueError, match="unsupported TFLite ops"):
        T.validate_supported_graph(m)


def test_default_input_and_top1():
    v = T.default_input(8)
    np.testing.assert_array_equal(v, (np.arange(8) - 4.0) * 0.25)
    # the last maximum wins (Rust max_by), and a 1001-class head drops its background class
    assert T.top1(np.array([1.0, 3.0, 3.0, 2.0]))["model_class"] == 2
    h = np.zeros(1001, np.float32)
    h[0], h[7] = 9.0, 5.0
    t = T.top1(h)
    assert (t["model_class"], t["class"]) == (7, 6)


def _alias_model(builtin, in_shape, out_shape, in_type=0, out_type=0):
    w = T.TfliteWriter("alias check")
    i = w.tensor("input", in_shape, ttype=in_type)
    o = w.tensor("output", out_shape, ttype=out_type)
    w.inputs, w.outputs = [i], [o]
    w.op(builtin, [i], [o])
    return T.parse_model(w.finish(), "alias.tflite")


@pytest.mark.parametrize("builtin", ["RESHAPE", "SQUEEZE", "EXPAND_DIMS", "CAST"])
def test_view_ops_reject_element_count_change(builtin):
    """scheduler.rs:241-249: a view op may not change the element count.  The executor checks
    it when it is built, before any device call (no context is touched here)."""
    m = _alias_model(builtin, [1, 8], [1, 9])
    with pytest.raises(ValueError, match="element count changed from 8 to 9"):
        T.TfliteExecutor(None, m)
    T.TfliteExecutor(None, _alias_model(builtin, [1, 8], [2, 4]))  # same count: accepted


def test_cast_only_float32_to_float32():
    """scheduler.rs:230-240: Cast must be Float32 -> Float32."""
    m = _alias_model("CAST", [1, 8], [1, 8], in_type=2)  # Int32 -> Float32
    with pytest.raises(ValueError, match="Cast only supports Float32->Float32, got Int32->Float32"):
        T.TfliteExecutor(None, m)


def _residual_model(conv_act=0, add_act=0, extra_reader=False, late_residual=False):
    """x -> CONV_2D (1x1) -> y; ADD(y, x) -> z (a residual connection), with variants that
    must not fuse: an activation on the convolution, a second reader of y, a residual that
    is computed after the convolution."""
    w = T.TfliteWriter()
    x = w.tensor("x", [1, 4, 4, 3])
    k = w.tensor("k", [3, 1, 1, 3], np.ones(9, np.float32))
    y = w.tensor("y", [1, 4, 4, 3])
    z = w.tensor("z", [1, 4, 4, 3])
    w.inputs, w.outputs = [x], [z]
    conv_opts = {0: ("b", 0), 1: ("i", 1), 2: ("i", 1), 3: ("b", conv_act)}
    if late_residual:
        r = w.tensor("r", [1, 4, 4, 3])
        w.op("CONV_2D", [x, k, -1], [y], "Conv2DOptions", conv_opts)
        w.op("ABS", [x], [r])
        w.op("ADD", [y, r], [z], "AddOptions", {0: ("b", add_act)})
    else:
        w.op("CONV_2D", [x, k, -1], [y], "Conv2DOptions", conv_opts)
        w.op("ADD", [y, x], [z], "AddOptions", {0: ("b", add_act)})
    if extra_reader:
        q = w.tensor("q", [1, 4, 4, 3])
        w.op("NEG", [y], [q])
        w.outputs.append(q)
    return T.parse_model(w.finish())


class _NoDevice:
    """TfliteExecutor's constructor touches no device; its fusion analysis is host logic."""


@pytest.mark.parametrize("variant,fused", [({}, True), ({"add_act": 3}, True),
                                           ({"conv_act": 1}, False),
                                           ({"extra_reader": True}, False)])
def test_executor_fuses_residual_add_into_conv(variant, fused):
    m = _residual_model(**variant)
    ex = T.TfliteExecutor(_NoDevice(), m)
    conv = next(o.index for o in m.operators if o.builtin == "CONV_2D")
    add = next(o.index for o in m.operators if o.builtin == "ADD")
    if fused:
        assert ex.residual_adds == {conv: (add, 0)}
    else:
        assert ex.residual_adds == {}


def test_executor_keeps_add_when_residual_comes_later():
    m = _residual_model(late_residual=True)
    order = T.topological_order(m)
    ex = T.TfliteExecutor(_NoDevice(), m)
    conv = next(o.index for o in m.operators if o.builtin == "CONV_2D")
    absop = next(o.index for o in m.operators if o.builtin == "ABS")
    if order.index(absop) > order.index(conv):
        assert ex.residual_adds == {}
    else:
        assert conv in ex.residual_adds


def _mbconv_model(cin=8, ce=32, cout=8, k=3, s=1, expand=True, residual=True, extra=None):
    """x -> [1x1 CONV_2D relu6] -> DEPTHWISE k x k relu6 -> 1x1 CONV_2D -> [ADD x] with
    variants that must not fuse (extra: 'expand_reader' reads the expanded tensor elsewhere,
    'dw_output' makes the depthwise output a model output, 'dilated' dilates the depthwise,
    'strided_expand' gives the expand stride 2)."""
    rng = np.random.default_rng(0)
    w = T.TfliteWriter()
    h = 6
    oh = (h + s - 1) // s
    x = w.tensor("x", [1, h, h, cin])
    w.inputs = [x]
    src = x
    ops = {}
    if expand:
        we = w.tensor("we", [ce, 1, 1, cin], rng.standard_normal(ce * cin).astype(np.float32))
        be = w.tensor("be", [ce], rng.standard_normal(ce).astype(np.float32))
        es = 2 if extra == "strided_expand" else 1
        eh = (h + es - 1) // es
        e = w.tensor("e", [1, eh, eh, ce])
        ops["expand"] = w.op("CONV_2D", [x, we, be], [e], "Conv2DOptions",
                             {0: ("b", 0), 1: ("i", es), 2: ("i", es), 3: ("b", 3)})
        src, h = e, eh
        oh = (h + s - 1) // s
    else:
        ce = cin
    wd = w.tensor("wd", [1, k, k, ce], rng.standard_normal(k * k * ce).astype(np.float32))
    bd = w.tensor("bd", [ce], rng.standard_normal(ce).astype(np.float32))
    d = w.tensor("d", [1, oh, oh, ce])
    dil = 2 if extra == "dilated" else 1
    ops["dw"] = w.op("DEPTHWISE_CONV_2D", [src, wd, bd], [d], "DepthwiseConv2DOptions",
                     {0: ("b", 0), 1: ("i", s), 2: ("i", s), 3: ("i", 1), 4: ("b", 3),
                      5: ("i", dil), 6: ("i", dil)})
    wp = w.tensor("wp", [cout, 1, 1, ce], rng.standard_normal(cout * ce).astype(np.float32))
    y = w.tensor("y", [1, oh, oh, cout])
    ops["project"] = w.op("CONV_2D", [d, wp, -1], [y], "Conv2DOptions",
                          {0: ("b", 0), 1: ("i", 1), 2: ("i", 1), 3: ("b", 0)})
    out = y
    if residual and s == 1 and cin == cout and not (expand and extra == "strided_expand"):
        z = w.tensor("z", [1, oh, oh, cout])
        ops["add"] = w.op("ADD", [y, x], [z], "AddOptions", {0: ("b", 0)})
        out = z
    w.outputs = [out]
    if extra == "expand_reader":
        q = w.tensor("q", [1, h, h, ce])
        w.op("NEG", [src], [q])
        w.outputs.append(q)
    if extra == "dw_output":
        w.outputs.append(d)
    return T.parse_model(w.finish()), ops


@pytest.mark.parametrize("kw", [{}, {"expand": False, "cin": 16, "cout": 16},
                                {"k": 5, "s": 2, "residual": False},
                                {"cout": 12, "residual": False}])
def test_executor_fuses_inverted_residual_chain(kw):
    m, ops = _mbconv_model(**kw)
    want = {"expand": ops.get("expand"), "dw": ops["dw"], "src": 0}
    ex = T.TfliteExecutor(_NoDevice(), m, fuse_blocks=True)  # every chain the kernel takes
    assert ex.blocks == {ops["project"]: want}
    if "add" in ops:  # the projection still takes its residual ADD
        assert ex.residual_adds == {ops["project"]: (ops["add"], 0)}
    # by default where the plan query expects one launch to pay: blocks with an expand at
    # this size (36 output pixels), not a depthwise + projection pair alone
    auto = T.TfliteExecutor(_NoDevice(), m).blocks
    assert auto == ({ops["project"]: want} if kw.get("expand", True) else {})
    assert T.TfliteExecutor(_NoDevice(), m, fuse_blocks=False).blocks == {}


@pytest.mark.parametrize("extra", ["expand_reader", "dw_output", "dilated", "strided_expand"])
def test_executor_keeps_chains_it_cannot_fuse(extra):
    m, ops = _mbconv_model(extra=extra)
    ex = T.TfliteExecutor(_NoDevice(), m, fuse_blocks=True)
    if extra in ("expand_reader", "strided_expand"):
        # the depthwise and projection still fuse, reading the expanded tensor as the input
        e_out = m.operators[ops["expand"]].outputs[0]
        assert ex.blocks == {ops["project"]: {"expand": None, "dw": ops["dw"], "src": e_out}}
    else:
        assert ex.blocks == {}


def test_executor_needs_channel_multiples_for_a_block():
    m, _ = _mbconv_model(cin=6, ce=24, cout=6)  # cin % 4 != 0, ce % 16 != 0
    assert T.TfliteExecutor(_NoDevice(), m, fuse_blocks=True).blocks == {}


def _head_model(cin=8, cout=12, k=1, pool="MEAN", axes=(1, 2), conv_out=False, act=3,
                pool_act=0):
    """x -> CONV_2D k x k (act) -> global pool (MEAN over axes, or AVERAGE_POOL_2D over the
    whole map with pool_act) -> FULLY_CONNECTED; conv_out also makes the convolution's output
    a model output."""
    rng = np.random.default_rng(1)
    w = T.TfliteWriter()
    h = 5
    x = w.tensor("x", [1, h, h, cin])
    w.inputs = [x]
    wc = w.tensor("wc", [cout, k, k, cin], rng.standard_normal(cout * k * k * cin).astype(np.float32))
    bc = w.tensor("bc", [cout], rng.standard_normal(cout).astype(np.float32))
    c = w.tensor("c", [1, h, h, cout])
    ops = {"conv": w.op("CONV_2D", [x, wc, bc], [c], "Conv2DOptions",
                        {0: ("b", 0), 1: ("i", 1), 2: ("i", 1), 3: ("b", act)})}
    p = w.tensor("p", [1, cout])
    if pool == "MEAN":
        ax = w.tensor("axes", [len(axes)], np.array(axes, np.int32).view(np.float32), ttype=2)
        ops["pool"] = w.op("MEAN", [c, ax], [p], "ReducerOptions", {0: ("B", 0)})
    else:
        ops["pool"] = w.op("AVERAGE_POOL_2D", [c], [p], "Pool2DOptions",
                           {0: ("b", 1), 1: ("i", 1), 2: ("i", 1), 3: ("i", h), 4: ("i", h),
                            5: ("b", pool_act)})
    wf = w.tensor("wf", [3, cout], rng.standard_normal(3 * cout).astype(np.float32))
    f = w.tensor("f", [1, 3])
    w.op("FULLY_CONNECTED", [p, wf, -1], [f], "FullyConnectedOptions", {0: ("b", 0)})
    w.outputs = [f] + ([c] if conv_out else [])
    return T.parse_model(w.finish()), ops


@pytest.mark.parametrize("kw,fuses", [({}, True), ({"pool": "AVERAGE_POOL_2D"}, True),
                                      ({"act": 0}, True), ({"k": 3}, False),
                                      ({"conv_out": True}, False), ({"axes": (1,)}, False),
                                      ({"cin": 6}, False),
                                      ({"pool": "AVERAGE_POOL_2D", "pool_act": 1}, False)])
def test_executor_fuses_the_classifier_head(kw, fuses):
    """A 1x1 CONV_2D read only by a global pool runs as one conv1x1_gap_nhwc launch (by
    default, and not with fuse_blocks=False); 3x3 kernels, a convolution output that is a
    model output, a MEAN over H only, a channel count off the multiple of 4 and a pool with
    an activation of its own keep the two operators."""
    try:
        m, ops = _head_model(**kw)
    except ValueError:
        assert not fuses  # a MEAN over one axis may not even describe a [1, C] output
        return
    want = {ops["pool"]: ops["conv"]} if fuses else {}
    assert T.TfliteExecutor(_NoDevice(), m).heads == want
    assert T.TfliteExecutor(_NoDevice(), m, fuse_blocks=False).heads == {}
