"""HIP kernels vs the CPU oracle, through the C ABI, on seeded inputs (GPU).

Gate: per-op |hip - oracle| <= 1e-4 + 1e-4*|oracle| in fp32;
data movement (copy/transpose/pad/concat) and max-reductions bit-exact.  The reference's
golden vectors go through the host-to-host drop-in (shp_run_kernel) with the reference's
own thresholds (tests/parity_test/generate_fixtures.py:108-113).
"""
import numpy as np
import pytest

from conftest import GOLDEN, assert_close, raw_f32, ulp_diff

pytestmark = pytest.mark.gpu
PARITY = GOLDEN / "parity"
RNG = np.random.default_rng(20261201)


def rnd(*shape, scale=1.0):
    return (RNG.standard_normal(shape) * scale).astype(np.float32)


def f32bits(v):
    return int(np.array([v], np.float32).view(np.int32)[0])


def hip(ctx, name, in0, in1, n_out, push, bias=None, residual=None, act=0, alpha=0.0,
        out_dtype=np.float32):
    # an absent binding is a null pointer, as in the model graphs
    t0 = ctx.tensor(in0) if in0 is not None else None
    t1 = ctx.tensor(in1) if in1 is not None else None
    tb = ctx.tensor(bias) if bias is not None else None
    tr = ctx.tensor(residual) if residual is not None else None
    out = ctx.empty(n_out, out_dtype)
    print(f"[gpu] {name} push={list(push)[:16]} n_out={n_out}", flush=True)
    ctx.launch(name, t0, t1, out, push, bias=tb, residual=tr, act=act, alpha=alpha)
    ctx.sync()
    y = out.download()
    for t in (t0, t1, tb, tr, out):
        if t is not None:
            t.free()
    return y


def both(ctx, orc, name, in0, in1, n_out, push, **kw):
    return hip(ctx, name, in0, in1, n_out, push, **kw), orc.run(name, in0, in1, n_out, push, **kw)


# ---- golden vectors through the drop-in host-to-host entry -------------------------------
def test_golden_relu_bit_exact(ctx):
    from spirv_inference_amd import KernelRun
    x = raw_f32(PARITY / "relu_input.raw.f32")
    out = ctx.run_kernel(KernelRun("relu", "relu", x, np.zeros(1, np.float32), x.size,
                                   (x.size + 127) // 128, [x.size]))
    assert out.vendor_id == 0x1002
    assert out.values.tobytes() == raw_f32(PARITY / "relu_ref.raw.f32").tobytes()


def test_golden_softmax(ctx):
    from spirv_inference_amd import KernelRun
    x = raw_f32(PARITY / "softmax_input.raw.f32")
    out = ctx.run_kernel(KernelRun("softmax", "softmax1000", x, np.zeros(1, np.float32), 128, 1,
                                   [128]))
    ref = raw_f32(PARITY / "softmax_ref.raw.f32")
    assert ulp_diff(out.values, ref).max() <= 8 and np.abs(out.values - ref).max() <= 1e-6


def test_golden_conv1d(ctx):
    from spirv_inference_amd import KernelRun
    x = raw_f32(PARITY / "conv1d_input.raw.f32")
    w = raw_f32(PARITY / "conv1d_filter.raw.f32")
    push = [1, 16, 1, 64, 3, 1, 32, 16, 1, 1, 1, 1, 0, 512]
    out = ctx.run_kernel(KernelRun("conv1d", "hlo_conv_nhwc_hwio", x, w, 512, 8, push))
    ref = raw_f32(PARITY / "conv1d_ref.raw.f32")
    rel = np.abs(out.values - ref) / np.maximum(np.abs(ref), 1e-30)
    assert ulp_diff(out.values, ref).max() <= 16 or rel.max() <= 1e-5


def test_golden_batchnorm(ctx, orc):
    from spirv_inference_amd import KernelRun
    x = raw_f32(PARITY / "batchnorm_input.raw.f32")
    mean, var, gamma, beta, eps = raw_f32(PARITY / "batchnorm_params.raw.f32")
    n = x.size
    full = lambda v: np.full(n, v, np.float32)
    run = lambda k, a, b: ctx.run_kernel(KernelRun(k, k, a, b, n, 2, [n])).values
    inv = run("rsqrt", run("add", full(var), full(eps)), np.zeros(1, np.float32))
    y = run("add", run("mul", run("mul", run("sub", x, full(mean)), inv), full(gamma)),
            full(beta))
    ref = raw_f32(PARITY / "batchnorm_ref.raw.f32")
    assert ulp_diff(y, ref).max() <= 8 and np.abs(y - ref).max() <= 1e-6


# ---- elementwise ---------------------------------------------------------------------------
UNARY = ["abs", "exp", "log", "neg", "sqrt", "rsqrt", "sigmoid", "logistic", "tanh", "relu",
         "relu6", "sine", "reshape", "silu", "gelu_erf", "cosine", "floor", "ceil"]


@pytest.mark.parametrize("name", UNARY)
@pytest.mark.parametrize("n", [1, 7, 4099, 1 << 20])
def test_unary(ctx, orc, name, n):
    x = rnd(n, scale=3.0)
    if name in ("log", "sqrt", "rsqrt"):
        x = np.abs(x) + 0.01
    y, r = both(ctx, orc, name, x, None, n, [n])
    if name in ("reshape", "abs", "neg", "relu", "relu6", "floor", "ceil"):
        assert y.tobytes() == r.tobytes()
    else:
        assert_close(y, r, 1e-4, 1e-4, name)


def test_leaky_relu(ctx, orc):
    x = rnd(1000)
    y, r = both(ctx, orc, "leaky_relu", x, None, 1000, [1000, f32bits(0.2)])
    assert y.tobytes() == r.tobytes()


@pytest.mark.parametrize("name", ["add", "sub", "mul", "div", "pow", "min", "max"])
@pytest.mark.parametrize("n", [5, 65537])
def test_binary(ctx, orc, name, n):
    a, b = rnd(n), rnd(n)
    if name == "pow":
        a = np.abs(a) + 0.1
    if name == "div":
        b = np.where(np.abs(b) < 0.1, 0.5, b).astype(np.float32)
    y, r = both(ctx, orc, name, a, b, n, [n])
    if name in ("add", "sub", "mul", "div", "min", "max"):
        assert y.tobytes() == r.tobytes()
    else:
        assert_close(y, r, 1e-4, 1e-4, name)


def test_data_movement_bit_exact(ctx, orc):
    a, b = rnd(1000), rnd(37)
    y, r = both(ctx, orc, "concat", a, b, 1037, [1000, 1037])
    assert y.tobytes() == r.tobytes()
    x = rnd(2, 5, 6, 7)
    for perm in [(0, 2, 3, 1), (0, 3, 1, 2), (0, 1, 3, 2), (1, 0, 2, 3), (3, 1, 2, 0)]:
        out_shape = [x.shape[p] for p in perm]
        push = [*x.shape, *out_shape, *perm, x.size]
        y, r = both(ctx, orc, "transpose", x, None, x.size, push)
        assert y.tobytes() == r.tobytes(), perm
    big = rnd(32, 112, 112, 64)[:1]  # NHWC -> NCHW at a ResNet stage-1 shape
    push = [1, 112, 112, 64, 1, 64, 112, 112, 0, 3, 1, 2, big.size]
    y, r = both(ctx, orc, "transpose", big, None, big.size, push)
    assert y.tobytes() == r.tobytes()
    push = [32, 230, 230, 3, 32, 224, 224, 3, 0, 3, 3, 0, 32 * 230 * 230 * 3]
    x = rnd(32, 224, 224, 3)
    y, r = both(ctx, orc, "pad", x, np.array([0.0], np.float32), push[12], push)
    assert y.tobytes() == r.tobytes()


def test_l2_and_broadcast(ctx, orc):
    x = rnd(5000)
    y, r = both(ctx, orc, "l2_normalization", x, None, 5000, [5000])
    assert_close(y, r, 1e-6, 1e-4, "l2_normalization")
    nb = f32bits(float(np.linalg.norm(x)))
    y, r = both(ctx, orc, "l2norm", x, None, 5000, [5000, nb])
    assert y.tobytes() == r.tobytes()
    a, b = rnd(3, 1, 4), rnd(1, 5, 4)
    for op in range(7):
        aa = np.abs(a) + 0.1 if op == 4 else a
        push = [op, 60, 1, 3, 5, 4, 0, 4, 0, 1, 0, 0, 4, 1]
        y, r = both(ctx, orc, "broadcast_binary", aa, b, 60, push)
        assert_close(y, r, 1e-5, 1e-5, f"broadcast op {op}")


def test_bias_act(ctx, orc):
    x, b, res = rnd(4, 100), rnd(100), rnd(4, 100)
    for act in range(8):
        y, r = both(ctx, orc, "bias_act", x, None, 400, [400, 100], bias=b, residual=res, act=act,
                    alpha=0.1)
        assert_close(y, r, 1e-5, 1e-5, f"bias_act {act}")


# ---- reductions / pools / softmax / norms ------------------------------------------------
def test_reduce_rank4(ctx, orc):
    x = rnd(8, 12, 128, 128)
    for axes in [(3,), (1, 2), (0,), (2,), (0, 1, 2, 3)]:
        flags = [1 if a in axes else 0 for a in range(4)]
        od = [1 if f else d for d, f in zip(x.shape, flags)]
        n_out = int(np.prod([d for d, f in zip(x.shape, flags) if not f]))
        for kind in (0, 1):
            push = [4, *x.shape, *od, *flags, kind, n_out]
            y, r = both(ctx, orc, "hlo_reduce_rank4", x, None, n_out, push)
            if kind == 1:
                assert y.tobytes() == r.tobytes()
            else:
                assert_close(y, r, 1e-4, 1e-4, f"reduce sum {axes}")


def test_resnet_pools(ctx, orc):
    x = np.abs(rnd(32, 112, 112, 64))
    # maxpool 3x3 s2 over the padded [32,114,114,64] (resnet50.stablehlo.txt:64-66)
    push = [32, 112, 112, 64, 56, 56, 3, 3, 2, 2, 1, 1, 1, 32 * 56 * 56 * 64]
    y, r = both(ctx, orc, "hlo_reduce_window_rank4", x, None, push[13], push)
    assert y.tobytes() == r.tobytes()
    # sum windows with C % 4 == 0 (four-channel path) and a C % 4 != 0 max (per-channel path)
    for shape, win, kind in (((3, 9, 10, 12), (2, 3, 2, 1, 0, 1), 0), ((2, 9, 9, 6), (3, 3, 2, 2, 1, 1), 1)):
        n, ih, iw, c = shape
        wh, ww, sh, sw, pt, pl = win
        oh, ow = (ih + 2 * pt - wh) // sh + 1, (iw + 2 * pl - ww) // sw + 1
        push = [n, ih, iw, c, oh, ow, wh, ww, sh, sw, pt, pl, kind, n * oh * ow * c]
        y, r = both(ctx, orc, "hlo_reduce_window_rank4", rnd(*shape), None, push[13], push)
        assert y.tobytes() == r.tobytes(), shape
    x = rnd(2, 16, 21, 21)
    push = [2, 16, 21, 21, 11, 11, 3, 3, 2, 2, 1, 1, 1, 2 * 16 * 11 * 11]
    y, r = both(ctx, orc, "max_pool2d", x, None, push[13], push)
    assert y.tobytes() == r.tobytes()
    x = rnd(32, 7, 7, 2048)
    y, r = both(ctx, orc, "global_avg_pool_nhwc", x, None, 32 * 2048, [32, 7, 7, 2048])
    assert_close(y, r, 1e-5, 1e-4, "gap nhwc")
    xc = rnd(8, 1280, 7, 7)
    y, r = both(ctx, orc, "global_avg_pool_sum", xc, None, 8 * 1280, [8, 1280, 7, 7])
    assert_close(y, r, 1e-4, 1e-4, "gap sum")
    y2, r2 = both(ctx, orc, "global_avg_pool_finalize", r, None, 8 * 1280, [8, 1280, 7, 7])
    assert y2.tobytes() == r2.tobytes()


def test_softmax_kernels(ctx, orc):
    x = rnd(10)
    y, r = both(ctx, orc, "softmax10", x, None, 10, [])
    assert_close(y, r, 1e-7, 1e-5, "softmax10")
    x = rnd(8, 1000, scale=4.0)  # EffNet-Lite0 head: whole-tensor semantics at batch 8
    y, r = both(ctx, orc, "softmax1000", x, None, 8000, [8000])
    assert_close(y, r, 1e-7, 1e-4, "softmax1000")
    for n in (1000, 1500, 9000):  # one, two and (past 8192) the three-pass kernel's elements
        x = rnd(n, scale=4.0)
        y, r = both(ctx, orc, "softmax1000", x, None, n, [n])
        assert_close(y, r, 1e-7, 1e-4, f"softmax1000 n={n}")
    for rows, cols in [(96 * 128, 128), (3, 32000), (7, 1)]:
        x = rnd(rows, cols, scale=3.0)
        mask = rnd(cols)
        push = [rows, cols, f32bits(0.125)]
        y, r = both(ctx, orc, "softmax_rows", x, mask, rows * cols, push)
        assert_close(y, r, 1e-6, 1e-4, f"softmax_rows {rows}x{cols}")


def test_row_norms(ctx, orc):
    x = rnd(1024, 768, scale=2.0)
    gb = np.concatenate([rnd(768), rnd(768)])
    push = [1024, 768, f32bits(1e-12)]
    y, r = both(ctx, orc, "layernorm_rows", x, gb, x.size, push)
    assert_close(y, r, 1e-4, 1e-4, "layernorm")
    x = rnd(4, 2048)
    push = [4, 2048, f32bits(1e-5)]
    y, r = both(ctx, orc, "rmsnorm_rows", x, np.ones(2048, np.float32), x.size, push)
    assert_close(y, r, 1e-5, 1e-4, "rmsnorm")


# ---- spatial -------------------------------------------------------------------------------
@pytest.mark.parametrize("k,s,c,n,hw", [(3, 1, 32, 1, 112), (3, 2, 96, 1, 112),
                                        (5, 2, 144, 8, 56), (5, 1, 1152, 8, 7), (3, 1, 6, 2, 9)])
def test_depthwise(ctx, orc, k, s, c, n, hw):
    pt = pl = (k - 1) // 2
    oh = (hw + 2 * pt - k) // s + 1
    total = n * c * oh * oh
    push = [n, c, hw, hw, oh, oh, k, k, s, s, 1, pt, pl, 1, 1, total]
    x = rnd(n, hw, hw, c)
    w = np.concatenate([rnd(k * k * c, scale=0.3), rnd(c)])
    res = rnd(total)
    y, r = both(ctx, orc, "depthwise_conv2d_nhwc", x, w, total, push, act="relu6")
    assert_close(y, r, 1e-4, 1e-4, "dw nhwc")
    y, r = both(ctx, orc, "depthwise_conv2d", x, w, total, push, residual=res)
    assert_close(y, r, 1e-4, 1e-4, "dw nchw")


@pytest.mark.parametrize("k,s,dil,c,n,h,w", [(3, 1, 2, 20, 2, 15, 13), (5, 2, 1, 100, 3, 17, 30),
                                             (3, 2, 1, 36, 1, 7, 7), (5, 1, 1, 4, 1, 9, 11),
                                             (3, 1, 1, 64, 1, 8, 8)])
def test_depthwise_nhwc_lds_tiles(ctx, orc, k, s, dil, c, n, h, w):
    """The LDS-tiled NHWC kernel on ragged tiles (output sizes not multiples of 8, channel
    counts not multiples of 32), dilation, stride 2 and a 5x5 window, with residual + ReLU6:
    against the oracle, and bit for bit against the untiled kernel."""
    from spirv_inference_amd._lib import check, lib
    oh, ow = -(-h // s), -(-w // s)
    pt = max((oh - 1) * s + (k - 1) * dil + 1 - h, 0) // 2
    pl = max((ow - 1) * s + (k - 1) * dil + 1 - w, 0) // 2
    total = n * oh * ow * c
    push = [n, c, h, w, oh, ow, k, k, s, s, 1, pt, pl, dil, dil, total]
    x = rnd(n, h, w, c)
    wt = np.concatenate([rnd(k * k * c, scale=0.3), rnd(c)])
    res = rnd(total)
    r = orc.run("depthwise_conv2d_nhwc", x, wt, total, push, residual=res, act="relu6")
    ys = {}
    try:
        for mode in (1, -1):  # forced tiled / untiled
            check(lib().shp_tune(ctx.handle, b"dw_tile", mode), "tune")
            ys[mode] = hip(ctx, "depthwise_conv2d_nhwc", x, wt, total, push, residual=res,
                           act="relu6")
    finally:
        check(lib().shp_tune(ctx.handle, b"dw_tile", 0), "tune")
    assert_close(ys[1], r, 1e-4, 1e-4, "dw nhwc tiles")
    np.testing.assert_array_equal(ys[1], ys[-1])


@pytest.mark.parametrize("k,s,c,n,h,w", [(3, 1, 20, 2, 15, 13), (5, 2, 100, 3, 17, 30),
                                         (5, 1, 8, 1, 9, 11), (3, 2, 36, 1, 7, 7),
                                         (5, 1, 240, 2, 28, 28)])
def test_depthwise_nhwc_wblocked(ctx, orc, k, s, c, n, h, w):
    """The W-blocked NHWC kernel (4 outputs per thread along W) on output widths that are not
    multiples of 4, stride 1 and 2, 3x3 and 5x5, with residual + ReLU6: against the oracle,
    bit for bit against the fixed-size kernel, and the automatic choice (the W-blocked kernel
    for 5x5 with output width >= 14) bit for bit the same."""
    from spirv_inference_amd._lib import check, lib
    oh, ow = -(-h // s), -(-w // s)
    pt = max((oh - 1) * s + k - h, 0) // 2
    pl = max((ow - 1) * s + k - w, 0) // 2
    total = n * oh * ow * c
    push = [n, c, h, w, oh, ow, k, k, s, s, 1, pt, pl, 1, 1, total]
    x = rnd(n, h, w, c)
    wt = np.concatenate([rnd(k * k * c, scale=0.3), rnd(c)])
    res = rnd(total)
    r = orc.run("depthwise_conv2d_nhwc", x, wt, total, push, residual=res, act="relu6")
    ys = {}
    try:
        for mode in (2, -1, 0):  # forced W-blocked / fixed, automatic
            check(lib().shp_tune(ctx.handle, b"dw_tile", mode), "tune")
            ys[mode] = hip(ctx, "depthwise_conv2d_nhwc", x, wt, total, push, residual=res,
                           act="relu6")
    finally:
        check(lib().shp_tune(ctx.handle, b"dw_tile", 0), "tune")
    assert_close(ys[2], r, 1e-4, 1e-4, "dw nhwc W-blocked")
    np.testing.assert_array_equal(ys[2], ys[-1])
    if k == 5 and ow >= 14:
        np.testing.assert_array_equal(ys[0], ys[2])


def test_resize_bilinear(ctx, orc):
    x = rnd(2, 3, 17, 13)
    for ac, hp in [(1, 0), (0, 1), (0, 0)]:
        push = [2, 3, 17, 13, 33, 29, ac, hp, 2 * 3 * 33 * 29]
        y, r = both(ctx, orc, "resize_bilinear", x, None, push[8], push)
        assert_close(y, r, 1e-5, 1e-5, f"resize {ac}{hp}")


# ---- dense contractions on MFMA -----------------------------------------------------------
# ResNet-50 v1.5 conv shapes (HLO path, NHWC/HWIO): (ih, ic, k, oc, stride)
RESNET_CONVS = [(224, 3, 7, 64, 2), (56, 64, 1, 64, 1), (56, 64, 3, 64, 1), (56, 64, 1, 256, 1),
                (56, 256, 1, 64, 1), (56, 256, 1, 128, 1), (56, 128, 3, 128, 2),
                (28, 128, 1, 512, 1), (56, 256, 1, 512, 2), (28, 512, 1, 256, 1),
                (28, 256, 3, 256, 2), (14, 256, 1, 1024, 1), (14, 1024, 1, 512, 1),
                (14, 512, 3, 512, 2), (7, 512, 1, 2048, 1), (14, 1024, 1, 2048, 2)]


@pytest.mark.parametrize("ih,ic,k,oc,s", RESNET_CONVS)
def test_hlo_conv_resnet_shapes(ctx, orc, ih, ic, k, oc, s):
    n = 2
    pad = (k - 1) // 2 if k > 1 else 0
    oh = (ih + 2 * pad - k) // s + 1
    x = rnd(n, ih, ih, ic)
    w = rnd(k, k, ic, oc, scale=float(np.sqrt(2.0 / (k * k * ic))))
    b, res = rnd(oc, scale=0.01), rnd(n * oh * oh * oc)
    push = [n, ih, ih, ic, k, k, oc, oh, oh, s, s, pad, pad, n * oh * oh * oc]
    y, r = both(ctx, orc, "hlo_conv_nhwc_hwio", x, w, push[13], push, bias=b, residual=res,
                act="relu")
    assert_close(y, r, 1e-4, 1e-4, f"conv {ih}x{ic} k{k} oc{oc} s{s}")


@pytest.mark.parametrize("ih,ic,k,oc,s", [(7, 512, 3, 512, 1), (56, 64, 3, 64, 1)])
def test_hlo_conv_full_batch(ctx, orc, ih, ic, k, oc, s):
    """b32 shapes: the late 3x3 layer exercises split-K, the early one the big tile grid."""
    n, pad = 32, 1
    oh = ih
    x = rnd(n, ih, ih, ic)
    w = rnd(k, k, ic, oc, scale=float(np.sqrt(2.0 / (k * k * ic))))
    push = [n, ih, ih, ic, k, k, oc, oh, oh, s, s, pad, pad, n * oh * oh * oc]
    y, r = both(ctx, orc, "hlo_conv_nhwc_hwio", x, w, push[13], push)
    assert_close(y, r, 1e-4, 1e-4, "conv b32")


# ---- the pipelined GEMM kernel (operand tiles DMA'd straight into LDS) --------------------
def _tune(ctx, key, value):
    """Planner override of one context (shp_tune, internal: not in the C ABI header)."""
    from spirv_inference_amd._lib import lib
    assert lib().shp_tune(ctx.handle, key.encode(), int(value)) == 0


@pytest.fixture
def gemm_workspace(ctx):
    """Split-K partials live in the context workspace, which a model graph sizes."""
    from spirv_inference_amd.models import Model
    Model(ctx, "resnet50_v1_5", 32, seed=2).close()


# (n, ih, ic, k, oc, stride, split-K): padding taps, M and N tails (oc 20, 132), a strided
# 1x1, split-K over a long and a short K
DMA_CONVS = [(2, 5, 16, 3, 20, 1, 0), (1, 9, 32, 3, 132, 2, 0), (3, 14, 48, 1, 72, 2, 0),
             (2, 7, 512, 3, 64, 1, 2), (1, 7, 64, 3, 64, 1, 3)]


@pytest.mark.parametrize("tile", [1, 2], ids=["128x128", "128x64"])
@pytest.mark.parametrize("n,ih,ic,k,oc,s,splits", DMA_CONVS)
def test_hlo_conv_dma_pipeline(ctx, orc, gemm_workspace, tile, n, ih, ic, k, oc, s, splits):
    pad = (k - 1) // 2
    oh = (ih + 2 * pad - k) // s + 1
    x = rnd(n, ih, ih, ic)
    w = rnd(k, k, ic, oc, scale=float(np.sqrt(2.0 / (k * k * ic))))
    b, res = rnd(oc, scale=0.01), rnd(n * oh * oh * oc)
    push = [n, ih, ih, ic, k, k, oc, oh, oh, s, s, pad, pad, n * oh * oh * oc]
    try:
        _tune(ctx, "gemm_dma", tile)
        _tune(ctx, "gemm_splits", splits)
        y = hip(ctx, "hlo_conv_nhwc_hwio", x, w, push[13], push, bias=b, residual=res,
                act="relu")
    finally:
        _tune(ctx, "gemm_dma", 0)
        _tune(ctx, "gemm_splits", 0)
    r = orc.run("hlo_conv_nhwc_hwio", x, w, push[13], push, bias=b, residual=res, act="relu")
    assert_close(y, r, 1e-4, 1e-4, f"dma conv {push[:13]} splits {splits}")


@pytest.mark.parametrize("tile", [1, 2], ids=["128x128", "128x64"])
@pytest.mark.parametrize("bt,m,k,n", [(1, 130, 36, 72), (1, 40, 100, 12), (96, 128, 64, 128)])
def test_dot_dma_pipeline(ctx, orc, tile, bt, m, k, n):
    """Row-major A through the pipelined kernel: K tails, M/N tails, strided batches."""
    a, b = rnd(bt, m, k), rnd(bt, k, n, scale=0.1)
    bias = rnd(n)
    try:
        _tune(ctx, "gemm_dma", tile)
        if bt == 1:
            y = hip(ctx, "hlo_dot_rank2", a[0], b[0], m * n, [m, k, n, m * n], bias=bias,
                    act="gelu_erf")
        else:
            y = hip(ctx, "hlo_dot_batched", a, b, bt * m * n, [bt, m, k, n, bt * m * n])
    finally:
        _tune(ctx, "gemm_dma", 0)
    if bt == 1:
        r = orc.run("hlo_dot_rank2", a[0], b[0], m * n, [m, k, n, m * n], bias=bias,
                    act="gelu_erf")
    else:
        r = orc.run("hlo_dot_batched", a, b, bt * m * n, [bt, m, k, n, bt * m * n])
    assert_close(y, r, 1e-4, 1e-4, f"dma dot {bt}x{m}x{k}x{n}")


@pytest.mark.parametrize("pg", [1, 2], ids=["prefetch1", "prefetch2"])
@pytest.mark.parametrize("tile,bk", [(1, 32), (1, 16), (2, 32), (2, 16), (3, 32), (3, 16)],
                         ids=["128x128k32", "128x128k16", "128x64k32", "128x64k16", "64x64k32",
                              "64x64k16"])
def test_gemm_tile_variants(ctx, orc, gemm_workspace, tile, bk, pg):
    """Every double-buffered tile the planner can choose, at both global prefetch depths, on
    a padded 3x3 conv with M/N tails and a residual (odd K-tile count), 1x1 convs with one and
    two K tiles, split-K, and a row-major product with a K tail."""
    cases = [((2, 9, 32, 3, 20, 1), 0), ((3, 8, 64, 1, 72, 1), 0), ((2, 6, 16, 1, 24, 1), 0),
             ((2, 7, 128, 3, 64, 1), 3)]
    try:
        _tune(ctx, "gemm_dma", -1)
        _tune(ctx, "gemm_tile", tile)
        _tune(ctx, "gemm_bk", bk)
        _tune(ctx, "gemm_pg", pg)
        for (n, ih, ic, k, oc, s), splits in cases:
            _tune(ctx, "gemm_splits", splits)
            pad = (k - 1) // 2
            oh = (ih + 2 * pad - k) // s + 1
            x = rnd(n, ih, ih, ic)
            w = rnd(k, k, ic, oc, scale=float(np.sqrt(2.0 / (k * k * ic))))
            b, res = rnd(oc, scale=0.01), rnd(n * oh * oh * oc)
            push = [n, ih, ih, ic, k, k, oc, oh, oh, s, s, pad, pad, n * oh * oh * oc]
            y, r = both(ctx, orc, "hlo_conv_nhwc_hwio", x, w, push[13], push, bias=b,
                        residual=res, act="relu")
            assert_close(y, r, 1e-4, 1e-4, f"conv {push[:13]} splits {splits}")
        _tune(ctx, "gemm_splits", 0)
        a, bm = rnd(1, 70, 100), rnd(1, 100, 36, scale=0.1)
        y, r = both(ctx, orc, "hlo_dot_batched", a, bm, 70 * 36, [1, 70, 100, 36, 70 * 36])
        assert_close(y, r, 1e-4, 1e-4, "dot 70x100x36")
    finally:
        for key in ("gemm_dma", "gemm_tile", "gemm_bk", "gemm_splits", "gemm_pg"):
            _tune(ctx, key, 0)


@pytest.mark.parametrize("splits", [2, 3, 6])
def test_splitk_in_kernel_fixup(ctx, orc, gemm_workspace, splits):
    """Split-K where the last split of each tile reduces the partials and applies the
    epilogue: three launches in a row (the tile counters must be back at zero after each),
    a batched product (one counter per batch and tile), and N % 4 != 0, which takes the
    separate reduction pass."""
    n, ih, ic, oc = 2, 7, 128, 64
    x = rnd(n, ih, ih, ic)
    w = rnd(3, 3, ic, oc, scale=float(np.sqrt(2.0 / (9 * ic))))
    b, res = rnd(oc, scale=0.01), rnd(n * ih * ih * oc)
    push = [n, ih, ih, ic, 3, 3, oc, ih, ih, 1, 1, 1, 1, n * ih * ih * oc]
    r = orc.run("hlo_conv_nhwc_hwio", x, w, push[13], push, bias=b, residual=res, act="relu")
    try:
        _tune(ctx, "gemm_splits", splits)
        for rep in range(3):
            y = hip(ctx, "hlo_conv_nhwc_hwio", x, w, push[13], push, bias=b, residual=res,
                    act="relu")
            assert_close(y, r, 1e-4, 1e-4, f"split-K conv, launch {rep}")
        for bt, m, nn in ((3, 40, 36), (1, 40, 30)):
            a, bm = rnd(bt, m, 768), rnd(bt, 768, nn, scale=0.1)
            q = [bt, m, 768, nn, bt * m * nn]
            y = hip(ctx, "hlo_dot_batched", a, bm, bt * m * nn, q)
            assert_close(y, orc.run("hlo_dot_batched", a, bm, bt * m * nn, q), 1e-4, 1e-4,
                         f"split-K dot {bt}x{m}x768x{nn}")
    finally:
        _tune(ctx, "gemm_splits", 0)


# (n, ih, ic, k, oc, stride, split-K): padding taps with an M tail and N % 64 != 0, a strided
# 1x1 (fixed tap, scalar channel advance), a 1x1 with an M tail, a strided 3x3 with N 132,
# split-K with the in-kernel fixup (3) and with the reduction pass (6)
BL_CONVS = [(2, 9, 64, 3, 20, 1, 0), (3, 14, 64, 1, 72, 2, 0), (2, 6, 128, 1, 24, 1, 0),
            (1, 9, 64, 3, 132, 2, 0), (2, 7, 128, 3, 64, 1, 3), (2, 7, 128, 3, 64, 1, 6)]


@pytest.mark.parametrize("tile,bk", [(1, 32), (2, 32), (3, 32), (3, 16), (3, 64)],
                         ids=["128x128k32", "128x64k32", "64x64k32", "64x64k16", "64x64k64"])
def test_gemm_buffer_loaded_kernel(ctx, orc, gemm_workspace, tile, bk):
    """The buffer-loaded kernel on each of its tiles: NHWC convolutions (padding taps read as
    zeros, strided 1x1, M and N tails, split-K both ways), a row-major product with bias and
    GELU, a batched product, the [out][in] fully-connected and the OHWI conv2d_nhwc operands.
    Each result is checked against the oracle and, where the double-buffered kernel has the
    same tile and K tile, bit for bit against it with the same split: both assign the K of a
    tile to MFMA k-pairs alike, so their sums are the same."""
    def conv_case(n, ih, ic, k, oc, s):
        pad = (k - 1) // 2
        oh = (ih + 2 * pad - k) // s + 1
        x = rnd(n, ih, ih, ic)
        w = rnd(k, k, ic, oc, scale=float(np.sqrt(2.0 / (k * k * ic))))
        b, res = rnd(oc, scale=0.01), rnd(n * oh * oh * oc)
        push = [n, ih, ih, ic, k, k, oc, oh, oh, s, s, pad, pad, n * oh * oh * oc]
        return ("hlo_conv_nhwc_hwio", x, w, push[13], push,
                dict(bias=b, residual=res, act="relu"))

    cases = [(conv_case(*c[:6]), c[6]) for c in BL_CONVS]
    a, bm = rnd(70, 128), rnd(128, 36, scale=0.1)
    cases.append((("hlo_dot_rank2", a, bm, 70 * 36, [70, 128, 36, 70 * 36],
                   dict(bias=rnd(36), act="gelu_erf")), 0))
    a, bm = rnd(3, 40, 256), rnd(3, 256, 36, scale=0.1)
    cases.append((("hlo_dot_batched", a, bm, 3 * 40 * 36, [3, 40, 256, 36, 3 * 40 * 36], {}), 2))
    w = np.concatenate([rnd(1000 * 2048, scale=0.05), rnd(1000)])
    cases.append((("fully_connected", rnd(32, 2048), w, 32 * 1000, [32, 2048, 1000, 32 * 1000],
                   {}), 0))
    w = np.concatenate([rnd(20 * 64 * 9, scale=0.1), rnd(20)])
    cases.append((("conv2d_nhwc", rnd(2, 9, 9, 64), w, 2 * 20 * 81,
                   [2, 64, 9, 9, 20, 9, 9, 3, 3, 1, 1, 1, 1, 1, 2 * 20 * 81], dict(act="relu6")),
                  0))
    try:
        _tune(ctx, "gemm_tile", tile)
        _tune(ctx, "gemm_bk", bk)
        for (name, x, w, n_out, push, kw), splits in cases:
            _tune(ctx, "gemm_splits", splits)
            _tune(ctx, "gemm_bl", 1)
            y = hip(ctx, name, x, w, n_out, push, **kw)
            r = orc.run(name, x, w, n_out, push, **kw)
            assert_close(y, r, 1e-4, 1e-4, f"buffer-loaded {name} {push[:13]} splits {splits}")
            if bk != 64:
                _tune(ctx, "gemm_bl", -1)
                _tune(ctx, "gemm_dma", -1)
                y0 = hip(ctx, name, x, w, n_out, push, **kw)
                _tune(ctx, "gemm_dma", 0)
                assert np.array_equal(y, y0), (name, push[:13], splits)
    finally:
        for key in ("gemm_bl", "gemm_dma", "gemm_tile", "gemm_bk", "gemm_splits"):
            _tune(ctx, key, 0)


@pytest.mark.parametrize("n,ih,oc,res,act", [(8, 48, 256, True, "relu"), (8, 48, 256, False, None),
                                             (6, 56, 64, True, "relu"), (6, 56, 64, False, "relu"),
                                             (4, 64, 512, True, None)],
                         ids=["n256-res-relu", "n256", "n64-res-relu", "n64-relu", "n512-res"])
def test_gemm_smallk_kernel(ctx, orc, n, ih, oc, res, act):
    """The persistent K = 64 kernel on 1x1 NHWC convolutions (M = 16384..18816: 32-row tiles
    that do not divide evenly over the CUs' row ranges; N 64, one 256-column slab, two slabs),
    with and without the residual and the ReLU.  Checked against the oracle, run twice (bit
    for bit the same), and against the planner's kernel with the persistent one switched off:
    both agree with the oracle, and some outputs differ in the last bits because the two pair
    the K terms differently, which shows that the persistent kernel ran."""
    ic = 64
    x = rnd(n, ih, ih, ic)
    w = rnd(1, 1, ic, oc, scale=float(np.sqrt(2.0 / ic)))
    kw = dict(bias=rnd(oc, scale=0.01))
    if res:
        kw["residual"] = rnd(n * ih * ih * oc)
    if act:
        kw["act"] = act
    push = [n, ih, ih, ic, 1, 1, oc, ih, ih, 1, 1, 0, 0, n * ih * ih * oc]
    r = orc.run("hlo_conv_nhwc_hwio", x, w, push[13], push, **kw)
    y = hip(ctx, "hlo_conv_nhwc_hwio", x, w, push[13], push, **kw)
    assert_close(y, r, 1e-4, 1e-4, f"small-K conv {push[:7]}")
    assert np.array_equal(y, hip(ctx, "hlo_conv_nhwc_hwio", x, w, push[13], push, **kw))
    try:
        _tune(ctx, "gemm_sk", -1)
        y0 = hip(ctx, "hlo_conv_nhwc_hwio", x, w, push[13], push, **kw)
    finally:
        _tune(ctx, "gemm_sk", 0)
    assert_close(y0, r, 1e-4, 1e-4, f"tiled conv {push[:7]}")
    assert not np.array_equal(y, y0), "the persistent small-K kernel did not run"


@pytest.mark.parametrize("n,ih,oc,act", [(2, 224, 64, "relu"), (8, 96, 128, None),
                                         (32, 113, 64, "relu")],
                         ids=["resnet-stem", "two-slabs", "odd-width"])
def test_conv_stem_kernel(ctx, orc, n, ih, oc, act):
    """The 7x7 stride-2 3-channel convolution kernel (kernel rows padded to 24 operands,
    padding taps read as zeros): the ResNet stem shape, two 64-column slabs, and an odd image
    width (the window overhangs the right border on every output row).  Checked against the
    oracle and against the planner's kernel with the stem kernel switched off (both agree with
    the oracle; some outputs differ in the last bits because the two order K differently, which
    shows that the stem kernel ran)."""
    ic, k, s, pad = 3, 7, 2, 3
    oh = (ih + 2 * pad - k) // s + 1
    x = rnd(n, ih, ih, ic)
    w = rnd(k, k, ic, oc, scale=float(np.sqrt(2.0 / (k * k * ic))))
    kw = dict(bias=rnd(oc, scale=0.01))
    if act:
        kw["act"] = act
    push = [n, ih, ih, ic, k, k, oc, oh, oh, s, s, pad, pad, n * oh * oh * oc]
    r = orc.run("hlo_conv_nhwc_hwio", x, w, push[13], push, **kw)
    y = hip(ctx, "hlo_conv_nhwc_hwio", x, w, push[13], push, **kw)
    assert_close(y, r, 1e-4, 1e-4, f"stem conv {push[:13]}")
    try:
        _tune(ctx, "gemm_stem", -1)
        y0 = hip(ctx, "hlo_conv_nhwc_hwio", x, w, push[13], push, **kw)
    finally:
        _tune(ctx, "gemm_stem", 0)
    assert_close(y0, r, 1e-4, 1e-4, f"tiled conv {push[:13]}")
    assert not np.array_equal(y, y0), "the stem kernel did not run"


@pytest.mark.parametrize("B,H,masked,pad_out", [(2, 3, True, 0), (1, 12, False, 32), (8, 12, True, 0)],
                         ids=["b2h3-mask", "b1h12-padded-out", "bert-b8"])
def test_attention_fused(ctx, orc, B, H, masked, pad_out):
    """The fused attention kernel (sequence 128, head dim 64) against the oracle: Q, K and V
    read in place from fused QKV rows, an additive key mask, context rows wider than H*64."""
    S, HD = 128, 64
    D = H * HD
    qkv = rnd(B * S, 3 * D)
    mask = rnd(S, scale=0.5) if masked else None
    ld_out = D + pad_out
    sb = int(np.array([0.125], np.float32).view(np.int32)[0])
    push = [B, H, S, HD, 3 * D, 0, D, 2 * D, ld_out, sb, B * S * ld_out]
    y, r = both(ctx, orc, "attention_fused", qkv, mask, B * S * ld_out, push)
    cols = np.arange(B * S * ld_out) % ld_out < D  # the padding columns are not written
    assert_close(y[cols], r[cols], 1e-4, 1e-4, f"attention_fused {push[:9]}")


def test_attention_fused_rejects_other_sequence_lengths(ctx):
    from spirv_inference_amd import ShpError
    S, HD, B, H = 64, 64, 1, 2
    qkv = rnd(B * S, 3 * H * HD)
    with pytest.raises(ShpError, match="sequence 128"):
        hip(ctx, "attention_fused", qkv, None, B * S * H * HD,
            [B, H, S, HD, 3 * H * HD, 0, H * HD, 2 * H * HD, H * HD, 1065353216, B * S * H * HD])


def test_hlo_conv_dma_by_planner(ctx, orc):
    """A shape the planner sends to the pipelined kernel on its own (K 512, 196 tiles)."""
    n, ih, ic, oc = 8, 28, 512, 256
    x = rnd(n, ih, ih, ic)
    w = rnd(1, 1, ic, oc, scale=float(np.sqrt(2.0 / ic)))
    b = rnd(oc, scale=0.01)
    push = [n, ih, ih, ic, 1, 1, oc, ih, ih, 1, 1, 0, 0, n * ih * ih * oc]
    y, r = both(ctx, orc, "hlo_conv_nhwc_hwio", x, w, push[13], push, bias=b, act="relu")
    assert_close(y, r, 1e-4, 1e-4, "conv 6272x256x512")


@pytest.mark.parametrize("n,ic,hw,oc,k,s,pad", [(1, 3, 224, 32, 3, 2, 0), (2, 6, 13, 10, 3, 1, 1),
                                                (1, 32, 28, 64, 1, 1, 0), (2, 5, 9, 7, 5, 2, 2)])
def test_conv2d_reference_and_nhwc(ctx, orc, n, ic, hw, oc, k, s, pad):
    oh = (hw + 2 * pad - k) // s + 1
    total = n * oc * oh * oh
    push = [n, ic, hw, hw, oc, oh, oh, k, k, s, s, 1, pad, pad, total]
    w = np.concatenate([rnd(oc * ic * k * k, scale=0.3), rnd(oc)])
    x = rnd(n, ic, hw, hw)
    y, r = both(ctx, orc, "conv2d", x, w, total, push)
    assert_close(y, r, 1e-4, 1e-4, "conv2d nchw")
    y, r = both(ctx, orc, "conv2d_nhwc", np.transpose(x, (0, 2, 3, 1)), w, total, push,
                act="relu6")
    assert_close(y, r, 1e-4, 1e-4, "conv2d nhwc")


@pytest.mark.parametrize("n,ic,h,w,oc,s,act,res", [
    (1, 3, 224, 224, 32, 2, "relu6", False),   # MobileNetV2 / EfficientNet-Lite0 stem
    (8, 3, 224, 224, 32, 2, "relu6", False),
    (2, 1, 17, 13, 16, 1, "relu", True),
    (3, 4, 9, 11, 8, 2, None, False),
    (2, 2, 10, 7, 24, 1, "relu6", True),
    (4, 2, 160, 160, 40, 1, "relu", False)],  # four channel groups per lane, five groups
    ids=["stem-b1", "stem-b8", "ic1-res", "ic4-odd", "ic2-res", "ic2-wide"])
def test_conv2d_nhwc_direct_small_channels(ctx, orc, n, ic, h, w, oc, s, act, res):
    """3x3 conv2d_nhwc with 1-4 input channels (SAME padding) runs the direct kernel (one
    thread: 8 output channels of one pixel, taps in the padding read as zeros): against the
    oracle, and against the implicit-GEMM kernels with the direct kernel switched off (both
    agree with the oracle; the two sum in different orders, so some outputs differ in the
    last bits, which shows the direct kernel ran)."""
    k = 3
    oh, ow = (h + s - 1) // s, (w + s - 1) // s
    pt = max((oh - 1) * s + k - h, 0) // 2
    pl = max((ow - 1) * s + k - w, 0) // 2
    total = n * oh * ow * oc
    push = [n, ic, h, w, oc, oh, ow, k, k, s, s, 1, pt, pl, total]
    wt = np.concatenate([rnd(oc * k * k * ic, scale=float(np.sqrt(2.0 / (k * k * ic)))),
                         rnd(oc, scale=0.1)])
    x = rnd(n, h, w, ic)
    kw = {"act": act} if act else {}
    if res:
        kw["residual"] = rnd(total)
    y, r = both(ctx, orc, "conv2d_nhwc", x, wt, total, push, **kw)
    assert_close(y, r, 1e-4, 1e-4, f"direct conv {push[:14]}")
    try:
        _tune(ctx, "conv_direct", -1)
        y0 = hip(ctx, "conv2d_nhwc", x, wt, total, push, **kw)
    finally:
        _tune(ctx, "conv_direct", 0)
    assert_close(y0, r, 1e-4, 1e-4, f"implicit-GEMM conv {push[:14]}")
    if n * oh * ow >= 1000:
        assert not np.array_equal(y, y0), "the direct kernel did not run"


@pytest.mark.parametrize("n,ic,h,w,oc,act,res,force", [
    (8, 112, 14, 14, 672, "relu6", False, 1),   # EfficientNet-Lite0 b8 block 9 expand
    (8, 192, 7, 7, 1152, "relu6", False, 1),    # block 12 expand
    (3, 20, 5, 7, 36, None, True, 1),           # partial 32x32 tiles, residual
    (2, 4, 9, 9, 8, "relu", False, 1),          # one K quarter
    (2, 24, 11, 13, 144, "relu6", False, 1),    # two chunks, the second partly past K
    (1, 80, 14, 14, 480, "relu6", True, 1),     # five chunks of the eight-chunk variant
    (1, 240, 3, 5, 70, None, True, 1),          # fifteen chunks
    (1, 256, 6, 6, 40, None, True, 1),          # one split's limit (LDS beyond 64 KiB)
    (8, 1152, 7, 7, 320, None, False, 0),       # EfficientNet-Lite0 b8 block 15 projection: K split
    (1, 960, 7, 7, 160, None, True, 0),         # MobileNetV2 b1 block 14 projection, residual
    (2, 300, 5, 5, 37, "relu", False, 1),       # K 300: 19 chunks in two runs, ragged tiles
    (2, 2048, 3, 3, 24, None, True, 1),         # K at the limit: 8 runs of 16 chunks
    (3, 80, 6, 5, 40, "relu6", True, 3)],       # a short K forced into three runs
    ids=["effnet-b9-expand", "effnet-b12-expand", "odd-res", "k4", "k24", "k80", "k240",
         "k256", "effnet-b15-project", "mbv2-b14-project", "k300", "k2048", "k80-split3"])
def test_conv2d_nhwc_1x1_small_kernel(ctx, orc, n, ic, h, w, oc, act, res, force):
    """1x1 conv2d_nhwc on the small-product kernel (32x32 tiles, operands staged through LDS in
    16-wide K chunks, each multiplied as it lands; past 256, K cut into runs whose partial tiles
    the last-arriving workgroup sums): against the oracle, and against the tiled GEMM with the
    small kernel switched off (both agree with the oracle; their K orders differ, so some
    outputs differ in the last bits, which shows the small kernel ran).  Two launches in a row
    check that the split-K tile counters are left at zero."""
    total = n * h * w * oc
    push = [n, ic, h, w, oc, h, w, 1, 1, 1, 1, 1, 0, 0, total]
    wt = np.concatenate([rnd(oc * ic, scale=float(np.sqrt(2.0 / ic))), rnd(oc, scale=0.1)])
    x = rnd(n, h, w, ic)
    kw = {"act": act} if act else {}
    if res:
        kw["residual"] = rnd(total)
    try:
        _tune(ctx, "gemm_small", force)
        y2 = hip(ctx, "conv2d_nhwc", x, wt, total, push, **kw)
        y, r = both(ctx, orc, "conv2d_nhwc", x, wt, total, push, **kw)
        _tune(ctx, "gemm_small", -1)
        y0 = hip(ctx, "conv2d_nhwc", x, wt, total, push, **kw)
    finally:
        _tune(ctx, "gemm_small", 0)
    assert_close(y, r, 1e-4, 1e-4, f"small 1x1 conv {push[:7]}")
    assert y.tobytes() == y2.tobytes(), "repeat launch differs"
    assert_close(y0, r, 1e-4, 1e-4, f"tiled 1x1 conv {push[:7]}")
    if total >= 4096:
        assert not np.array_equal(y, y0), "the small kernel did not run"


@pytest.mark.parametrize("b,k,n", [(1, 1280, 1000), (8, 1280, 1000), (32, 2048, 1000),
                                   (3, 37, 5), (5, 64, 13), (2, 4096, 9)])
def test_fully_connected(ctx, orc, b, k, n):
    w = np.concatenate([rnd(n * k, scale=0.05), rnd(n)])
    x = rnd(b, k)
    y, r = both(ctx, orc, "fully_connected", x, w, b * n, [b, k, n, b * n])
    assert_close(y, r, 1e-4, 1e-4, "fc")


@pytest.mark.parametrize("m,k,n,act,res", [
    (8, 1280, 1000, None, False),   # EfficientNet-Lite0 b8 classifier
    (2, 1280, 1000, "relu", False),
    (16, 768, 77, None, True),      # 16 rows, column tail, residual
    (5, 20, 13, "relu6", False),    # fewer chunks than wavefronts
    (3, 2048, 40, None, False)],    # eight chunks per wavefront
    ids=["b8-classifier", "m2-relu", "m16-res", "short-k", "k2048"])
def test_fully_connected_mfma(ctx, orc, m, k, n, act, res):
    """fully_connected with 2-16 rows on the split-K MFMA kernel: against the oracle, and
    against the wavefront-per-column / tiled kernels with it switched off (both agree with the
    oracle; their K orders differ, so some outputs differ in the last bits, which shows the
    MFMA kernel ran)."""
    w = np.concatenate([rnd(n * k, scale=float(np.sqrt(1.0 / k))), rnd(n)])
    x = rnd(m, k)
    kw = {"act": act} if act else {}
    if res:
        kw["residual"] = rnd(m * n)
    push = [m, k, n, m * n]
    y, r = both(ctx, orc, "fully_connected", x, w, m * n, push, **kw)
    try:
        _tune(ctx, "fc_mfma", -1)
        y0 = hip(ctx, "fully_connected", x, w, m * n, push, **kw)
    finally:
        _tune(ctx, "fc_mfma", 0)
    assert_close(y, r, 1e-4, 1e-4, f"fc mfma {push}")
    assert_close(y0, r, 1e-4, 1e-4, f"fc other {push}")
    if m * n >= 2000:
        assert not np.array_equal(y, y0), "the MFMA kernel did not run"


@pytest.mark.parametrize("bt,m,k,n", [(1, 32, 2048, 1000), (96, 128, 64, 128), (96, 128, 128, 64),
                                      (1, 1024, 768, 3072), (2, 33, 17, 65), (1, 64, 2048, 256)])
def test_dot_batched(ctx, orc, bt, m, k, n):
    a, b = rnd(bt, m, k), rnd(bt, k, n, scale=0.1)
    y, r = both(ctx, orc, "hlo_dot_batched", a, b, bt * m * n, [bt, m, k, n, bt * m * n])
    assert_close(y, r, 1e-4, 1e-4, "dot_batched")
    if bt == 1:
        y, r = both(ctx, orc, "hlo_dot_rank2", a[0], b[0], m * n, [m, k, n, m * n],
                    bias=rnd(n), act="gelu_erf")
        assert_close(y, r, 1e-4, 1e-4, "dot_rank2")


def test_dot_general_in_place_attention(ctx, orc):
    """BERT b8 s128: scores = Q K^T and P V read straight from [B, S, H, D]."""
    B, S, H, D = 8, 128, 12, 64
    q, k, v = rnd(B, S, H, D), rnd(B, S, H, D), rnd(B, S, H, D)
    push = [B, H, S, S, D, S * H * D, D, H * D, 1, S * H * D, D, 1, H * D, H * S * S, S * S, S, 1]
    y, r = both(ctx, orc, "dot_general_strided", q, k, B * H * S * S, push)
    assert_close(y, r, 1e-4, 1e-4, "QK^T")
    p = rnd(B, H, S, S, scale=0.1)
    push = [B, H, S, D, S, H * S * S, S * S, S, 1, S * H * D, D, H * D, 1, S * H * D, D, H * D, 1]
    y, r = both(ctx, orc, "dot_general_strided", p, v, B * S * H * D, push)
    assert_close(y, r, 1e-4, 1e-4, "PV")


def test_gemv_and_argmax(ctx, orc):
    x, w = rnd(2048), rnd(2560, 2048, scale=0.02)
    y, r = both(ctx, orc, "gemv_nt", x, w, 2560, [2560, 2048])
    assert_close(y, r, 1e-5, 1e-4, "gemv_nt")
    res = rnd(2560)
    y, r = both(ctx, orc, "gemv_nt", x, w, 2560, [2560, 2048], residual=res)
    assert_close(y, r, 1e-5, 1e-4, "gemv_nt residual")
    y, r = both(ctx, orc, "gemv_nt", x[:37], rnd(5, 37), 5, [5, 37], bias=rnd(5), act="silu")
    assert_close(y, r, 1e-5, 1e-4, "gemv_nt generic")
    logits = rnd(3, 32000)
    logits[1, 77] = logits[1, 4000] = 99.0  # tie -> lowest index
    y = hip(ctx, "argmax_rows", logits, None, 3, [3, 32000], out_dtype=np.int32)
    assert list(y) == [int(np.argmax(l)) for l in logits] and y[1] == 77


def test_errors_fail_closed(ctx):
    from spirv_inference_amd import ShpError
    t = ctx.tensor(np.zeros(8, np.float32))
    with pytest.raises(ShpError, match="UNKNOWN_KERNEL"):
        ctx.launch("no_such_kernel", t, t, t, [8])
    with pytest.raises(ShpError, match="PUSH"):
        ctx.launch("conv2d", t, t, t, [1, 2, 3])
    with pytest.raises(ShpError, match="SHAPE"):
        ctx.launch("add", t, t, t, [9])
    with pytest.raises(ShpError, match="UNSUPPORTED"):
        ctx.launch("add", t, t, t, [8], act="relu")
    t.free()


# ---- the HLO path's host shape ops, on the device (compiler.rs:336-586) --------------------
def _dev(ctx, name, x, y, n_out, push, init=None):
    tx = ctx.tensor(np.atleast_1d(x)) if x is not None else None
    ty = ctx.tensor(np.atleast_1d(y)) if y is not None else None
    out = ctx.tensor(init) if init is not None else ctx.empty(n_out)
    print(f"[gpu] {name} push={list(push)[:12]} n_out={n_out}", flush=True)
    ctx.launch(name, tx, ty, out, push)
    ctx.sync()
    r = out.download()
    for t in (tx, ty, out):
        if t is not None:
            t.free()
    return r


@pytest.mark.parametrize("src,out,dims", [((4, 1, 64, 64), (4, 8, 64, 64), (0, 1, 2, 3)),
                                          ((3, 5), (5, 2, 3), (2, 0)), ((1,), (2, 3, 4), (1,)),
                                          ((2048,), (8, 128, 2048), (2,)),
                                          ((1, 4, 1, 64, 64), (1, 4, 8, 64, 64), (0, 1, 2, 3, 4))])
def test_hlo_broadcast(ctx, orc, src, out, dims):
    from spirv_inference_amd import hlo_ops as H
    x, n, push = rnd(*src), int(np.prod(out)), H.broadcast_push(src, out, dims)
    np.testing.assert_array_equal(_dev(ctx, "hlo_broadcast", x, None, n, push),
                                  orc.run("hlo_broadcast", x, None, n, push))


@pytest.mark.parametrize("shape,perm", [((1, 64, 32, 64), (0, 2, 1, 3)), ((8, 128, 12, 64), (0, 2, 3, 1)),
                                        ((2, 3, 4, 5, 6), (4, 0, 3, 1, 2))])
def test_hlo_transpose(ctx, orc, shape, perm):
    from spirv_inference_amd import hlo_ops as H
    x, push = rnd(*shape), H.transpose_push(shape, perm)
    np.testing.assert_array_equal(_dev(ctx, "hlo_transpose", x, None, x.size, push),
                                  orc.run("hlo_transpose", x, None, x.size, push))


@pytest.mark.parametrize("shape,starts,limits,strides", [
    ((1, 32, 64, 64), (0, 0, 0, 0), (1, 32, 64, 32), (1, 1, 1, 1)),
    ((1, 32, 64, 64), (0, 0, 0, 32), (1, 32, 64, 64), (1, 1, 1, 1)),
    ((5, 9, 7), (1, 0, 2), (5, 9, 7), (2, 3, 2)), ((4, 6), (0, 2), (4, 9), (1, 1)),
    ((4, 6), (0, 7), (4, 9), (1, 1))])
def test_hlo_slice(ctx, orc, shape, starts, limits, strides):
    from spirv_inference_amd import hlo_ops as H
    x, push = rnd(*shape), H.slice_push(shape, starts, limits, strides)
    n = int(np.prod(H.slice_shape(starts, limits, strides)))
    np.testing.assert_array_equal(_dev(ctx, "hlo_slice", x, None, n, push),
                                  orc.run("hlo_slice", x, None, n, push))


@pytest.mark.parametrize("base,offset,shape,strides", [
    (2 * 3 * 4 * 5, 0, (2, 4, 3, 5), (60, 5, 20, 1)),
    (8 * 128 * 2304, 768, (8, 12, 128, 64), (128 * 2304, 64, 2304, 1)),
    (4 * 64, 0, (4, 8, 64), (64, 0, 1)), (30, 3, (4, 3), (6, 2))])
def test_hlo_strided_copy(ctx, orc, base, offset, shape, strides):
    x = rnd(base)
    n, push = int(np.prod(shape)), [len(shape), int(np.prod(shape)), *shape, *strides]
    np.testing.assert_array_equal(_dev(ctx, "hlo_strided_copy", x[offset:], None, n, push),
                                  orc.run("hlo_strided_copy", x[offset:], None, n, push))


def test_hlo_concatenate(ctx, orc):
    """Rotate-half's concatenate (two halves on the last axis) and a three-way axis-1 join."""
    from spirv_inference_amd import hlo_ops as H
    for shapes, dim in (([(1, 32, 64, 32), (1, 32, 64, 32)], 3), ([(2, 3, 5), (2, 4, 5), (2, 1, 5)], 1)):
        xs = [rnd(*s) for s in shapes]
        out_shape = list(shapes[0])
        out_shape[dim] = sum(s[dim] for s in shapes)
        n = int(np.prod(out_shape))
        ts = [ctx.tensor(x) for x in xs]
        out = ctx.tensor(np.zeros(n, np.float32))
        H.concatenate(ctx, list(zip(ts, shapes)), dim, out, out_shape)
        ctx.sync()
        y = out.download()
        for t in ts + [out]:
            t.free()
        r, off = np.zeros(n, np.float32), 0
        for x, s in zip(xs, shapes):
            r = orc.run("hlo_concatenate_into", x, None, n,
                        H.concatenate_into_push(out_shape, s, dim, off), out_init=r)
            off += s[dim]
        np.testing.assert_array_equal(y, r)
        np.testing.assert_array_equal(y, np.concatenate(xs, axis=dim).reshape(-1))


@pytest.mark.parametrize("direction", ["LT", "LE", "EQ", "NE", "GE", "GT"])
def test_hlo_compare(ctx, orc, direction):
    from spirv_inference_amd import hlo_ops as H
    for out, a, b in (((8, 128, 3072), (8, 128, 3072), (1,)), ((4, 5, 6), (5, 6), (4, 1, 6))):
        x, z = np.round(rnd(*a) * 2) / 2, np.round(rnd(*b) * 2) / 2
        n, push = int(np.prod(out)), H.compare_push(direction, out, a, b)
        np.testing.assert_array_equal(_dev(ctx, "hlo_compare", x, z, n, push),
                                      orc.run("hlo_compare", x, z, n, push))


def test_hlo_select(ctx, orc):
    """select_tensor on the device: on_false broadcast into the output, then hlo_select."""
    from spirv_inference_amd import hlo_ops as H
    for out, p, t, f in (((8, 128, 3072), (8, 128, 3072), (8, 128, 3072), (1,)),
                         ((4, 5, 6), (5, 6), (1, 6), (4, 5, 6))):
        pred, on_t, on_f = (rnd(*p) > 0).astype(np.float32), rnd(*t), rnd(*f)
        n = int(np.prod(out))
        tp, tt, tf, to = ctx.tensor(pred), ctx.tensor(on_t), ctx.tensor(on_f), ctx.empty(n)
        H.select(ctx, tp, p, tt, t, tf, f, to, out)
        ctx.sync()
        y = to.download()
        for x in (tp, tt, tf, to):
            x.free()
        fill = np.broadcast_to(on_f.reshape(f), out).astype(np.float32).reshape(-1)
        r = orc.run("hlo_select", pred, on_t, n, H.select_push(out, p, t), out_init=fill)
        np.testing.assert_array_equal(y, r)


@pytest.mark.parametrize("shape,dims", [((1, 4, 8, 64, 64), (4,)), ((1, 4, 8, 64, 64), (0, 2)),
                                        ((3, 5, 7, 2, 3, 4), (1, 2, 5)), ((32, 7, 7, 2048), (1, 2))])
def test_hlo_reduce(ctx, orc, shape, dims):
    """Sum folds in source order on both sides, so it is bit-exact like max."""
    from spirv_inference_amd import hlo_ops as H
    x = rnd(*shape)
    kept = int(np.prod([d for k, d in enumerate(shape) if k not in dims]))
    for kind, init in (("sum", 0.0), ("max", -np.inf)):
        push = H.reduce_push(kind, shape, dims, init)
        np.testing.assert_array_equal(_dev(ctx, "hlo_reduce", x, None, kept, push),
                                      orc.run("hlo_reduce", x, None, kept, push))


def test_hlo_shape_ops_fail_closed(ctx):
    from spirv_inference_amd import hlo_ops as H
    with pytest.raises(RuntimeError):  # not a permutation
        _dev(ctx, "hlo_transpose", rnd(4), None, 4, [2, 4, 2, 2, 0, 0])
    with pytest.raises(RuntimeError):  # total does not match the output
        _dev(ctx, "hlo_slice", rnd(4, 6), None, 5, H.slice_push((4, 6), (0, 0), (2, 6)))


@pytest.mark.parametrize("n,nan_at", [(0, []), (7, []), (7, [3]), (4099, [4098, 17, 2000]),
                                      (1 << 22, [(1 << 22) - 1, 123457, 1 << 21])])
def test_nan_count(ctx, orc, n, nan_at):
    """The HLO runner's NaN trace kernel: count and first index, bit-exact (inf is not NaN)."""
    x = rnd(max(n, 1))[:n].copy() if n else np.zeros(1, np.float32)
    if n:
        x[::97] = np.inf
    for i in nan_at:
        x[i] = np.nan
    y, r = both(ctx, orc, "nan_count", x, None, 2, [n])
    assert y.tobytes() == r.tobytes()
    c = y.view(np.int32)
    assert c[0] == len(nan_at) and c[1] == (min(nan_at) if nan_at else -1)
