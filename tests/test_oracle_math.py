"""Pins the oracle kernels that no reference golden vector covers, against independent
implementations (numpy / torch CPU in float64, closed forms and invariants).  CPU only."""
import numpy as np
import pytest
import torch

from conftest import assert_close, ulp_diff

RNG = np.random.default_rng(1234)


def rnd(*shape, scale=1.0):
    return (RNG.standard_normal(shape) * scale).astype(np.float32)


def conv_nhwc_ref(x, w, stride, pad):
    """float64 brute force: x [N,H,W,C], w [KH,KW,C,O], pads (top,left) with zero fill."""
    n, ih, iw, c = x.shape
    kh, kw, _, o = w.shape
    sh, sw = stride
    pt, pl = pad
    oh = (ih + 2 * pt - kh) // sh + 1
    ow = (iw + 2 * pl - kw) // sw + 1
    xp = np.zeros((n, ih + 2 * pt + kh, iw + 2 * pl + kw, c))
    xp[:, pt:pt + ih, pl:pl + iw] = x
    out = np.zeros((n, oh, ow, o))
    for ky in range(kh):
        for kx in range(kw):
            patch = xp[:, ky:ky + sh * oh:sh, kx:kx + sw * ow:sw, :]
            out += np.einsum("nhwc,co->nhwo", patch, w[ky, kx].astype(np.float64))
    return out


@pytest.mark.parametrize("shape", [(2, 9, 11, 5, 3, 3, 7, 1, 1, 1), (1, 16, 16, 8, 3, 3, 12, 2, 1, 1),
                                   (2, 15, 13, 3, 7, 7, 16, 2, 3, 3), (1, 7, 7, 32, 1, 1, 20, 1, 0, 0)])
def test_hlo_conv_vs_float64(orc, shape):
    n, ih, iw, ic, kh, kw, oc, s, pt, pl = shape
    x, w = rnd(n, ih, iw, ic), rnd(kh, kw, ic, oc, scale=0.2)
    ref = conv_nhwc_ref(x, w, (s, s), (pt, pl))
    oh, ow = ref.shape[1:3]
    push = [n, ih, iw, ic, kh, kw, oc, oh, ow, s, s, pt, pl, ref.size]
    y = orc.run("hlo_conv_nhwc_hwio", x, w, ref.size, push)
    assert_close(y, ref, 1e-5, 1e-5, "hlo_conv")


def test_conv2d_nchw_and_nhwc_conjugate(orc):
    n, ic, ih, iw, oc, kh, kw, s = 2, 6, 10, 9, 5, 3, 3, 2
    pt, pl = orc.same_padding(True, ih, iw, 5, 5, kh, kw, s, s)
    x = rnd(n, ih, iw, ic)
    w_ohwi, b = rnd(oc, kh, kw, ic, scale=0.3), rnd(oc)
    ref = conv_nhwc_ref(x, np.transpose(w_ohwi, (1, 2, 3, 0)), (s, s), (pt, pl))
    oh, ow = ref.shape[1:3]
    ref = ref + b
    total = n * oc * oh * ow
    push = [n, ic, ih, iw, oc, oh, ow, kh, kw, s, s, 1, pt, pl, total]
    y = orc.run("conv2d", np.transpose(x, (0, 3, 1, 2)), orc.pack_conv_weight(w_ohwi, b), total,
                push)
    assert_close(np.transpose(y.reshape(n, oc, oh, ow), (0, 2, 3, 1)), ref, 1e-5, 1e-5, "conv2d")
    packed_nhwc = np.concatenate([w_ohwi.reshape(-1), b])
    y2 = orc.run("conv2d_nhwc", x, packed_nhwc, total, push)
    assert_close(y2, ref, 1e-5, 1e-5, "conv2d_nhwc")


def test_same_padding_matches_tf_rule(orc):
    # TF SAME: total = max((out-1)*s + k - in, 0); top = total // 2 (scheduler.rs:1597-1614)
    assert orc.same_padding(True, 224, 224, 112, 112, 3, 3, 2, 2) == (0, 0)
    assert orc.same_padding(True, 112, 112, 112, 112, 3, 3, 1, 1) == (1, 1)
    assert orc.same_padding(True, 14, 14, 7, 7, 5, 5, 2, 2) == (1, 1)
    assert orc.same_padding(False, 14, 14, 7, 7, 5, 5, 2, 2) == (0, 0)


@pytest.mark.parametrize("nhwc", [False, True])
def test_depthwise_vs_float64(orc, nhwc):
    n, c, ih, iw, k, s, dil = 2, 8, 11, 10, 5, 2, 1
    pt, pl = 2, 2
    x = rnd(n, ih, iw, c)
    w, b = rnd(k, k, c, scale=0.3), rnd(c)
    oh, ow = (ih + 2 * pt - k) // s + 1, (iw + 2 * pl - k) // s + 1
    xp = np.zeros((n, ih + 2 * pt + k, iw + 2 * pl + k, c))
    xp[:, pt:pt + ih, pl:pl + iw] = x
    ref = np.zeros((n, oh, ow, c)) + b
    for ky in range(k):
        for kx in range(k):
            ref += xp[:, ky:ky + s * oh:s, kx:kx + s * ow:s, :] * w[ky, kx]
    total = n * c * oh * ow
    push = [n, c, ih, iw, oh, ow, k, k, s, s, 1, pt, pl, dil, dil, total]
    if nhwc:
        y = orc.run("depthwise_conv2d_nhwc", x, np.concatenate([w.reshape(-1), b]), total, push)
        assert_close(y, ref, 1e-5, 1e-5, "dw nhwc")
    else:
        y = orc.run("depthwise_conv2d", np.transpose(x, (0, 3, 1, 2)),
                    orc.pack_depthwise_weight(w, b), total, push)
        assert_close(np.transpose(y.reshape(n, c, oh, ow), (0, 2, 3, 1)), ref, 1e-5, 1e-5, "dw")


def test_fully_connected_and_dots_vs_matmul(orc):
    x, w, b = rnd(3, 40), rnd(17, 40), rnd(17)
    y = orc.run("fully_connected", x, orc.pack_fc_weight(w, b), 51, [3, 40, 17, 51])
    assert_close(y, x.astype(np.float64) @ w.T.astype(np.float64) + b, 1e-5, 1e-5, "fc")
    a, bb = rnd(4, 5, 33), rnd(4, 33, 7)
    y = orc.run("hlo_dot_batched", a, bb, 140, [4, 5, 33, 7, 140])
    assert_close(y, np.matmul(a.astype(np.float64), bb), 1e-5, 1e-5, "dot_batched")
    y = orc.run("hlo_dot_rank2", a[0], bb[0], 35, [5, 33, 7, 35])
    assert_close(y, a[0].astype(np.float64) @ bb[0], 1e-5, 1e-5, "dot_rank2")
    # dot_general in place: scores = Q K^T for Q,K in [B, S, H, D] (BERT layout)
    B, S, H, D = 2, 6, 3, 8
    q, k = rnd(B, S, H, D), rnd(B, S, H, D)
    push = [B, H, S, S, D, S * H * D, D, H * D, 1, S * H * D, D, 1, H * D, H * S * S, S * S, S, 1]
    y = orc.run("dot_general_strided", q, k, B * H * S * S, push)
    ref = np.einsum("bshd,bthd->bhst", q.astype(np.float64), k)
    assert_close(y, ref, 1e-5, 1e-5, "dot_general")


def test_reductions_vs_numpy(orc):
    x = rnd(3, 4, 5, 6)
    for axes in [(3,), (1, 2), (0,), (0, 1, 2, 3)]:
        flags = [1 if a in axes else 0 for a in range(4)]
        od = [1 if f else d for d, f in zip(x.shape, flags)]
        for kind, fn in [(0, np.sum), (1, np.max)]:
            ref = fn(x.astype(np.float64), axis=axes)
            push = [4, *x.shape, *od, *flags, kind, ref.size]
            y = orc.run("hlo_reduce_rank4", x, None, ref.size, push)
            assert_close(y, ref, 1e-5, 1e-5, f"reduce {axes} {kind}")


def test_pools_vs_numpy(orc):
    x = rnd(2, 9, 9, 4)
    t = torch.from_numpy(np.transpose(x, (0, 3, 1, 2)).astype(np.float64))
    ref = torch.nn.functional.max_pool2d(t, 3, 2, padding=1).numpy()
    oh, ow = ref.shape[2:]
    push = [2, 9, 9, 4, oh, ow, 3, 3, 2, 2, 1, 1, 1, ref.size]
    y = orc.run("hlo_reduce_window_rank4", x, None, ref.size, push)
    assert_close(y, np.transpose(ref, (0, 2, 3, 1)), 0, 0, "reduce_window max")
    push = [2, 4, 9, 9, oh, ow, 3, 3, 2, 2, 1, 1, 1, ref.size]
    y = orc.run("max_pool2d", np.transpose(x, (0, 3, 1, 2)), None, ref.size, push)
    assert_close(y, ref, 0, 0, "max_pool2d")
    s = orc.run("global_avg_pool_sum", np.transpose(x, (0, 3, 1, 2)), None, 8, [2, 4, 9, 9])
    m = orc.run("global_avg_pool_finalize", s, None, 8, [2, 4, 9, 9])
    assert_close(m, x.astype(np.float64).mean(axis=(1, 2)), 1e-6, 1e-5, "gap")
    m2 = orc.run("global_avg_pool_nhwc", x, None, 8, [2, 9, 9, 4])
    assert_close(m2, x.astype(np.float64).mean(axis=(1, 2)), 1e-6, 1e-5, "gap nhwc")


def test_softmax_and_norms_vs_float64(orc):
    x = rnd(5, 37)
    mask = rnd(37)
    scale = np.float32(0.125)
    ref = torch.softmax(torch.from_numpy(x.astype(np.float64) * scale + mask), -1).numpy()
    bits = int(np.array([scale], np.float32).view(np.int32)[0])
    y = orc.run("softmax_rows", x, mask, x.size, [5, 37, bits])
    assert_close(y, ref, 1e-6, 1e-5, "softmax_rows")
    assert np.allclose(y.reshape(5, 37).sum(-1), 1.0, atol=1e-6)
    g, b = rnd(37), rnd(37)
    eps = np.float32(1e-5)
    eb = int(np.array([eps], np.float32).view(np.int32)[0])
    ref = torch.nn.functional.layer_norm(torch.from_numpy(x.astype(np.float64)), (37,),
                                         torch.from_numpy(g.astype(np.float64)),
                                         torch.from_numpy(b.astype(np.float64)), eps=1e-5).numpy()
    y = orc.run("layernorm_rows", x, np.concatenate([g, b]), x.size, [5, 37, eb])
    assert_close(y, ref, 1e-5, 1e-5, "layernorm")
    xd = x.astype(np.float64)
    ref = xd / np.sqrt((xd * xd).mean(-1, keepdims=True) + 1e-5) * g
    y = orc.run("rmsnorm_rows", x, g, x.size, [5, 37, eb])
    assert_close(y, ref, 1e-5, 1e-5, "rmsnorm")


def test_softmax_rows_without_mask(orc):
    """An absent mask binding (NULL) means no mask — regression for the optional in1."""
    x = rnd(2, 1000, scale=5.0)
    y = orc.run("softmax_rows", x, None, x.size, [2, 1000, 1065353216])  # scale 1.0
    ref = torch.softmax(torch.from_numpy(x.astype(np.float64)), -1).numpy()
    assert_close(y, ref, 1e-6, 1e-5, "softmax_rows no mask")


@pytest.mark.parametrize("B,H,S,HD,masked", [(2, 3, 20, 8, True), (1, 2, 128, 64, False),
                                              (2, 1, 7, 5, True)])
def test_attention_fused_is_the_three_op_chain(orc, B, H, S, HD, masked):
    """attention_fused restates the scores dot_general, softmax_rows and the context
    dot_general on the fused QKV rows: bit for bit the same as running those three oracle ops
    (same float arithmetic and order), and within 1e-5 of a float64 softmax(QK^T s + m) V."""
    D = H * HD
    qkv = rnd(B * S, 3 * D)
    mask = rnd(S, scale=0.5) if masked else None
    sb = int(np.array([0.3], np.float32).view(np.int32)[0])
    y = orc.run("attention_fused", qkv, mask, B * S * D, [B, H, S, HD, 3 * D, 0, D, 2 * D, D, sb, B * S * D])
    flat = qkv.ravel()
    sc = orc.run("dot_general_strided", flat, flat[D:], B * H * S * S,
                 [B, H, S, S, HD, S * 3 * D, HD, 3 * D, 1, S * 3 * D, HD, 1, 3 * D, H * S * S, S * S, S, 1])
    pr = orc.run("softmax_rows", sc, mask, B * H * S * S, [B * H * S, S, sb])
    cx = orc.run("dot_general_strided", pr, flat[2 * D:], B * S * D,
                 [B, H, S, HD, S, H * S * S, S * S, S, 1, S * 3 * D, HD, 3 * D, 1, S * D, HD, D, 1])
    assert np.array_equal(y, cx)
    t = torch.from_numpy(qkv.astype(np.float64)).reshape(B, S, 3, H, HD)
    q, k, v = (t[:, :, i].permute(0, 2, 1, 3) for i in range(3))  # [B, H, S, HD]
    att = q @ k.transpose(-1, -2) * float(np.float32(0.3))
    if masked:
        att = att + torch.from_numpy(mask.astype(np.float64))
    ref = (torch.softmax(att, -1) @ v).permute(0, 2, 1, 3).reshape(-1).numpy()
    assert_close(y, ref, 1e-5, 1e-5, "attention_fused vs float64")


def test_gelu_erfc_expansion_vs_exact(orc):
    from scipy.special import erfc
    x = np.linspace(-12, 12, 4001).astype(np.float32)
    y = orc.run("gelu_erf", x, None, x.size, [x.size])
    xd = x.astype(np.float64)
    ref = 0.5 * xd * erfc(-xd / np.sqrt(2.0))
    assert_close(y, ref, 2e-6, 2e-6, "gelu (XLA erfc expansion)")


def test_data_movement_bit_exact(orc):
    x = rnd(2, 3, 4, 5)
    for perm in [(0, 2, 3, 1), (0, 3, 1, 2), (1, 0, 3, 2), (3, 2, 1, 0)]:
        ref = np.transpose(x, perm)
        push = [*x.shape, *ref.shape, *perm, x.size]
        y = orc.run("transpose", x, None, x.size, push)
        assert y.tobytes() == np.ascontiguousarray(ref).tobytes()
    ref = np.pad(x, [(0, 0), (1, 2), (3, 0), (0, 1)], constant_values=-2.5)
    push = [*ref.shape, *x.shape, 0, 1, 3, 0, ref.size]
    y = orc.run("pad", x, np.array([-2.5], np.float32), ref.size, push)
    # pad.comp only honours low pads; the high side is whatever remains of the output
    assert y.tobytes() == np.ascontiguousarray(ref).tobytes()
    a, b = rnd(7), rnd(5)
    y = orc.run("concat", a, b, 12, [7, 12])
    assert y.tobytes() == np.concatenate([a, b]).tobytes()
    y = orc.run("reshape", a, None, 7, [7])
    assert y.tobytes() == a.tobytes()


def test_broadcast_binary_and_l2(orc):
    a, b = rnd(3, 1, 4), rnd(1, 5, 4)
    ref = a * b  # float32 product: one rounding, bit-exact
    push = [2, ref.size, 1, 3, 5, 4, 0, 4, 0, 1, 0, 0, 4, 1]
    y = orc.run("broadcast_binary", a, b, ref.size, push)
    assert_close(y, ref, 0, 0, "broadcast mul")
    x = rnd(100)
    y = orc.run("l2_normalization", x, None, 100, [100])
    assert_close(y, x / np.linalg.norm(x.astype(np.float64)), 1e-6, 1e-5, "l2")
    nb = int(np.array([np.linalg.norm(x)], np.float32).view(np.int32)[0])
    y = orc.run("l2norm", x, None, 100, [100, nb])
    assert_close(y, x / np.linalg.norm(x.astype(np.float64)), 1e-6, 1e-5, "l2norm")


def test_resize_bilinear_vs_torch(orc):
    x = rnd(1, 3, 6, 7)
    for ac, hp in [(1, 0), (0, 1)]:
        ref = torch.nn.functional.interpolate(torch.from_numpy(x.astype(np.float64)),
                                              size=(11, 9), mode="bilinear",
                                              align_corners=bool(ac)).numpy()
        push = [1, 3, 6, 7, 11, 9, ac, hp, ref.size]
        y = orc.run("resize_bilinear", x, None, ref.size, push)
        assert_close(y, ref, 1e-5, 1e-5, f"resize ac={ac} hp={hp}")


def test_argmax_tie_rules(orc):
    v = np.array([1, 5, 2, 5, 0], np.float32)
    assert orc.argmax_first(v) == 1               # numpy argmax (run_llama_spirv.py:252-254)
    assert orc.top1_reference(v)[0] == 3          # Rust max_by keeps the last maximum
    v1001 = np.zeros(1001, np.float32)
    v1001[0] = 9.0
    v1001[10] = 3.0
    assert orc.top1_reference(v1001)[0] == 9      # background class skipped, offset by one


def _act_ref(v, act, alpha):
    """float64 activation formulas, written from their definitions (relu.comp, relu6.comp,
    leaky_relu.comp:17 max(alpha*x, x), sigmoid.comp, tanh.comp, SiLU x*sigmoid(x), GELU
    0.5*x*erfc(-x/sqrt(2)))."""
    from scipy.special import erfc
    return {"none": v, "relu": np.maximum(v, 0.0), "relu6": np.clip(v, 0.0, 6.0),
            "leaky": np.maximum(alpha * v, v), "sigmoid": 1.0 / (1.0 + np.exp(-v)),
            "tanh": np.tanh(v), "silu": v / (1.0 + np.exp(-v)),
            "gelu_erf": 0.5 * v * erfc(-v / np.sqrt(2.0))}[act]


@pytest.mark.parametrize("act", ["none", "relu", "relu6", "leaky", "sigmoid", "tanh", "silu",
                                 "gelu_erf"])
def test_gemv_nt_with_epilogue_vs_float64(orc, act):
    """gemv_nt (the decode GEMV: y[n] = sum_k x[k] W[n][k]) with bias, residual and each
    activation against float64 numpy."""
    N, K = 300, 517
    x, W = rnd(K), rnd(N, K, scale=0.1)
    bias, res = rnd(N), rnd(N)
    lin = W.astype(np.float64) @ x.astype(np.float64)
    y = orc.run("gemv_nt", x, W, N, [N, K], bias=bias, residual=res, act=act, alpha=0.2)
    assert_close(y, _act_ref(lin + bias + res, act, 0.2), 1e-5, 1e-5, f"gemv_nt {act}")
    y0 = orc.run("gemv_nt", x, W, N, [N, K])
    assert_close(y0, lin, 1e-5, 1e-5, "gemv_nt plain")


@pytest.mark.parametrize("act", ["relu", "relu6", "gelu_erf"])
def test_conv_epilogue_bias_per_channel_vs_float64(orc, act):
    """The fused epilogue on a convolution: bias indexed by the output channel (last NHWC
    dim), the residual in the output's layout, then the activation."""
    n, ih, ic, oc = 2, 6, 8, 12
    x, w = rnd(n, ih, ih, ic), rnd(3, 3, ic, oc, scale=0.3)
    bias = rnd(oc)
    lin = conv_nhwc_ref(x, w, (1, 1), (1, 1))
    res = rnd(*lin.shape)
    push = [n, ih, ih, ic, 3, 3, oc, ih, ih, 1, 1, 1, 1, lin.size]
    y = orc.run("hlo_conv_nhwc_hwio", x, w, lin.size, push, bias=bias, residual=res, act=act)
    assert_close(y, _act_ref(lin + bias + res, act, 0.0), 1e-5, 1e-5, f"conv epilogue {act}")


def test_gather_rows_vs_numpy_take(orc):
    """gather_rows: embed_table[ids] (run_llama_spirv.py:203), ids stored as int32 bits; an
    id outside [0, rows) gives a zero row."""
    rows, length = 50, 33
    table = rnd(rows, length)
    ids = np.array([3, 0, 49, 7, 3, -1, 50], np.int32)
    y = orc.run("gather_rows", ids.view(np.float32), table, ids.size * length,
                [ids.size, length, rows]).reshape(ids.size, length)
    ok = (ids >= 0) & (ids < rows)
    assert y[ok].tobytes() == np.take(table, ids[ok], axis=0).tobytes()
    assert not y[~ok].any()


def _rounding_probe_inputs():
    """Inputs that separate floor/ceil/sin/cos from plausible mistakes: a dense random sweep
    over +-1e4, exact integers and half-integers, +-0, the float32 neighbours just below and
    above integers, and large magnitudes where sin's argument reduction and the 2^23 limit
    (every float32 at or above it is an integer) matter."""
    rng = np.random.default_rng(77)
    sweep = rng.uniform(-1e4, 1e4, 100_000)
    ints = np.arange(-1000, 1001, dtype=np.float64)
    halves = ints + 0.5
    f_ints = ints.astype(np.float32)
    below = np.nextafter(f_ints, np.float32(-np.inf))
    above = np.nextafter(f_ints, np.float32(np.inf))
    big = np.concatenate([2.0 ** np.arange(20, 100), -(2.0 ** np.arange(20, 100)),
                          rng.uniform(1e5, 1e30, 2000) * rng.choice([-1, 1], 2000),
                          [8388607.5, -8388607.5, 8388608.0, 16777217.0, 3.4e38, -3.4e38]])
    # multiples of pi/2 in float32: sin/cos results near zero, where a wrong reduction fails
    near_pi = (np.arange(-2000, 2001) * (np.pi / 2)).astype(np.float32)
    return np.concatenate([sweep.astype(np.float32), f_ints, halves.astype(np.float32), below,
                           above, np.float32([0.0, -0.0, 1e-45, -1e-45, 1e-30, -1e-30]),
                           big.astype(np.float32), near_pi]).astype(np.float32)


@pytest.mark.parametrize("name,ref", [("floor", np.floor), ("ceil", np.ceil)])
def test_floor_ceil_bit_exact_vs_float64(orc, name, ref):
    """floor/ceil (`compiler.rs:1495-1499` f32::floor/ceil in cpu_elementwise) are exact in
    float32: the float64 result of a float32 input is representable, so the oracle must equal
    it bit for bit, signed zeros included (ceil(-0.5) = -0.0)."""
    x = _rounding_probe_inputs()
    y = orc.run(name, x, None, x.size, [x.size])
    want = ref(x.astype(np.float64)).astype(np.float32)
    assert y.tobytes() == want.tobytes(), name
    # signed zero and infinity handling spelled out
    s = orc.run(name, np.float32([-0.5, 0.5, -0.0, np.inf, -np.inf]), None, 5, [5])
    exp = {"floor": [-1.0, 0.0, -0.0, np.inf, -np.inf], "ceil": [-0.0, 1.0, -0.0, np.inf, -np.inf]}
    assert s.tobytes() == np.float32(exp[name]).tobytes()


@pytest.mark.parametrize("name,ref", [("sine", np.sin), ("cosine", np.cos)])
def test_sin_cos_within_one_ulp_of_float64(orc, name, ref):
    """sine (`kernels/sine/glsl/sine.comp:10`, o[i] = sin(a[i])) and the HLO path's
    f32::sin/cos (`compiler.rs:1495-1499`) against float64 numpy of the same float32 input:
    at most 1 ULP of the correctly rounded result everywhere, including the float32 multiples
    of pi/2 (results near zero) and magnitudes up to 3.4e38 (full argument reduction).  A
    reduction done in float32, a swapped sin/cos or a dropped sign fails this by many ULP."""
    x = _rounding_probe_inputs()
    y = orc.run(name, x, None, x.size, [x.size])
    exact = ref(x.astype(np.float64))
    want = exact.astype(np.float32)
    assert ulp_diff(y, want).max() <= 1, f"{name}: max ulp {ulp_diff(y, want).max()}"
    # identities that fix the sign and the phase: sin(-x) = -sin(x), cos(-x) = cos(x)
    yn = orc.run(name, -x, None, x.size, [x.size])
    if name == "sine":
        assert yn.tobytes() == (-y).tobytes()
    else:
        assert yn.tobytes() == y.tobytes()
    # special values: sin(+-0) keeps the sign, cos(0) = 1, non-finite inputs give NaN
    sp = orc.run(name, np.float32([0.0, -0.0, np.inf, -np.inf, np.nan]), None, 5, [5])
    if name == "sine":
        assert sp[:2].tobytes() == np.float32([0.0, -0.0]).tobytes()
    else:
        assert (sp[:2] == 1.0).all()
    assert np.isnan(sp[2:]).all()


@pytest.mark.parametrize("act", ["none", "relu", "relu6", "leaky", "sigmoid", "tanh", "silu",
                                 "gelu_erf"])
def test_bias_act_vs_float64(orc, act):
    """bias_act (the standalone epilogue: x + bias[i % period] + residual, then the
    activation) against float64 numpy."""
    x, b, r = rnd(4, 100), rnd(100), rnd(4, 100)
    y = orc.run("bias_act", x, None, 400, [400, 100], bias=b, residual=r, act=act, alpha=0.2)
    ref = _act_ref(x.astype(np.float64) + b + r, act, 0.2)
    assert_close(y, ref, 1e-6, 1e-6, f"bias_act {act}")


@pytest.mark.parametrize("name,ref", [("logistic", lambda v: 1.0 / (1.0 + np.exp(-v))),
                                      ("silu", lambda v: v / (1.0 + np.exp(-v)))])
def test_logistic_and_silu_kernels_vs_float64(orc, name, ref):
    """The unary kernels `logistic` (TFLite's name for sigmoid.comp) and `silu` over a wide
    range, including the saturated tails."""
    x = np.concatenate([rnd(1000, scale=4.0), np.float32([-90, -30, -1e-3, 0, 1e-3, 30, 90])])
    y = orc.run(name, x, None, x.size, [x.size])
    assert_close(y, ref(x.astype(np.float64)), 1e-6, 1e-6, name)


def test_argmax_rows_first_maximum(orc):
    """argmax_rows: per row the index of the first maximum (numpy's rule, lowest index on
    ties), stored as int32 bits."""
    rows, cols = 6, 1000
    x = rnd(rows, cols)
    x[1, [10, 500, 999]] = 9.0    # a three-way tie: the first index wins
    x[2, :] = -1.0                # every column tied
    x[3, 999] = 50.0              # maximum in the last column
    x[4, 0] = 50.0                # and in the first
    y = orc.run("argmax_rows", x, None, rows, [rows, cols]).view(np.int32)
    assert list(y) == list(np.argmax(x, axis=1))
    assert list(y[1:5]) == [10, 0, 999, 0]


def test_compare_is_tensor_rs_comparator(orc):
    """orc_compare restates tflite_loader/src/tensor.rs:28-54: a mismatch is |a - e| > eps (a
    difference equal to eps is not one), the relative error divides by max(|e|, 1e-30), and
    a length difference counts as that many mismatches; the maxima cover the common prefix."""
    e = np.float32([1.0, -2.0, 0.0, 4.0, 5.0])
    a = np.float32([1.0, -2.5, 1e-3, 4.0 + 0.25, 5.0])
    mm, ma, mr = orc.compare(a, e, 0.25)
    assert mm == 1                                    # only -2.5 (0.5 > eps); 4.25 sits at eps
    assert ma == np.float32(0.5)
    assert mr == np.float32(np.float32(1e-3) / np.float32(1e-30))
    mm2, _, _ = orc.compare(a[:3], e, 0.25)           # two missing values
    assert mm2 == 1 + 2
    assert orc.compare(e, e, 0.0)[0] == 0


@pytest.mark.parametrize("expand,k,s,res", [(True, 3, 2, False), (True, 5, 1, True),
                                            (False, 3, 1, False), (True, 3, 1, True)])
def test_inverted_residual_vs_float64(orc, expand, k, s, res):
    """inverted_residual_nhwc (the three MBConv operators in one call) against a float64
    numpy restatement of 1x1 conv + ReLU6, SAME-padded depthwise + ReLU6, 1x1 conv +
    residual: closed-form einsums and an explicit tap loop, not the oracle's loops."""
    rng = np.random.default_rng(3)
    n, cin, h, w, cout = 2, 8, 9, 7, 8
    ce = 32 if expand else cin
    oh, ow = (h + s - 1) // s, (w + s - 1) // s
    pt = max((oh - 1) * s + k - h, 0) // 2
    pl = max((ow - 1) * s + k - w, 0) // 2
    x = rng.standard_normal(n * h * w * cin).astype(np.float32)
    parts = []
    if expand:
        we, be = rng.standard_normal((ce, cin)) * 0.3, rng.standard_normal(ce) * 0.1
        parts += [we, be]
    wd, bd = rng.standard_normal((k, k, ce)) * 0.3, rng.standard_normal(ce) * 0.1
    wp, bp = rng.standard_normal((cout, ce)) * 0.2, rng.standard_normal(cout) * 0.1
    parts += [wd, bd, wp, bp]
    packed = np.concatenate([np.asarray(q, np.float32).reshape(-1) for q in parts])
    total = n * oh * ow * cout
    push = [n, cin, h, w, ce, cout, oh, ow, k, s, pt, pl, int(expand), 2, 2, total]
    got = orc.run("inverted_residual_nhwc", x, packed, total, push,
                  residual=x if res else None)
    X = x.reshape(n, h, w, cin).astype(np.float64)
    E = np.clip(np.einsum("nhwc,ec->nhwe", X, we) + be, 0, 6) if expand else X
    Ep = np.zeros((n, h + 2 * k, w + 2 * k, ce))
    Ep[:, pt:pt + h, pl:pl + w] = E
    D = np.zeros((n, oh, ow, ce))
    for ky in range(k):
        for kx in range(k):
            D += Ep[:, ky:ky + (oh - 1) * s + 1:s, kx:kx + (ow - 1) * s + 1:s] * wd[ky, kx]
    D = np.clip(D + bd, 0, 6)
    Y = np.einsum("nhwe,oe->nhwo", D, wp) + bp
    if res:
        Y = Y + X
    assert_close(got, Y.reshape(-1), 2e-6, 2e-6, "inverted_residual_nhwc")


@pytest.mark.parametrize("act,h,w", [("relu6", 7, 7), ("none", 3, 5), ("relu", 1, 1)])
def test_conv1x1_gap_vs_float64(orc, act, h, w):
    """conv1x1_gap_nhwc (the head's 1x1 convolution, its activation and the global average
    pool in one call) against a float64 einsum, clip and mean; relu6 with values spread past
    6 so the clamp matters, and a 1x1 map where the mean is the pixel itself."""
    rng = np.random.default_rng(5)
    n, cin, cout = 2, 12, 20
    x = (rng.standard_normal(n * h * w * cin) * 2).astype(np.float32)
    wt = (rng.standard_normal((cout, cin)) * 0.8).astype(np.float32)
    b = (rng.standard_normal(cout) * 0.5).astype(np.float32)
    got = orc.run("conv1x1_gap_nhwc", x, np.concatenate([wt.reshape(-1), b]), n * cout,
                  [n, cin, h, w, cout, n * cout], act=act)
    C = np.einsum("npc,oc->npo", x.reshape(n, h * w, cin).astype(np.float64), wt) + b
    if act == "relu6":
        assert (C > 6).any() and (C < 0).any()
    C = {"relu6": np.clip(C, 0, 6), "relu": np.maximum(C, 0), "none": C}[act]
    assert_close(got, C.mean(axis=1).reshape(-1), 2e-6, 2e-6, "conv1x1_gap_nhwc")
