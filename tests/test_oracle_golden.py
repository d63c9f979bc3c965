"""Pins the CPU oracle against the reference's own golden data (CPU only).

Sources of truth, all reference-held or independent of the oracle's code:
  * tests/parity_test/out/fixtures/*.raw.f32 + manifest.json (generate_fixtures.py:21-113),
    with the reference's thresholds (relu bit-exact; softmax/batchnorm ULP<=8 & abs<=1e-6;
    conv1d ULP<=16 & rel<=1e-5) and the committed CUDA/Intel outputs;
  * source/inference_poc/fixtures/manifest.json: SHA-256 of every edge of the closed-form
    conv1d -> batchnorm -> relu -> fc -> softmax fixture (fixture.rs:28-195);
  * the kernel self-test KAT of source/tflite_loader/src/engine.rs:21-174 (eps 1e-5).
"""
import hashlib
import json

import numpy as np
import pytest

from conftest import GOLDEN, raw_f32, ulp_diff

PARITY = GOLDEN / "parity"


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a, "<f4").tobytes()).hexdigest()


def manifest():
    return json.loads((PARITY / "manifest.json").read_text())


# ---- generator closed forms reproduce the reference's fixture bytes --------------------
@pytest.mark.parametrize("which,name,n", [
    (0, "relu_input", 4096), (1, "softmax_input", 128), (2, "batchnorm_input", 256),
    (3, "batchnorm_params", 5), (4, "conv1d_input", 1024), (5, "conv1d_filter", 6144)])
def test_parity_fixture_generator_matches_reference_bytes(orc, which, name, n):
    gen = orc.parity_fixture(which, n)
    ref = raw_f32(PARITY / f"{name}.raw.f32")
    assert gen.tobytes() == ref.tobytes()
    assert sha(gen) == manifest()["files"][name]["sha256"]


# ---- reference kernels against the golden outputs ---------------------------------------
def test_relu_bit_exact(orc):
    x = raw_f32(PARITY / "relu_input.raw.f32")
    y = orc.run("relu", x, None, x.size, [x.size])
    ref = raw_f32(PARITY / "relu_ref.raw.f32")
    assert y.tobytes() == ref.tobytes()
    # the reference's CUDA and Intel outputs agree bit-exactly too (advanced parity report)
    assert y.tobytes() == raw_f32(PARITY / "cuda_relu.raw.f32").tobytes()


def test_softmax_matches_golden(orc):
    x = raw_f32(PARITY / "softmax_input.raw.f32")
    y = orc.run("softmax1000", x, None, x.size, [x.size])
    ref = raw_f32(PARITY / "softmax_ref.raw.f32")
    assert ulp_diff(y, ref).max() <= 8
    assert np.abs(y - ref).max() <= 1e-6
    for dev in ("cuda", "intel"):
        other = raw_f32(PARITY / f"{dev}_softmax.raw.f32")
        assert ulp_diff(y, other).max() <= 8


def test_batchnorm_as_elementwise_chain(orc):
    """batchnorm = (x - mean) * rsqrt(var + eps) * gamma + beta through the oracle's
    sub/add/rsqrt/mul kernels (generate_fixtures.py:36-39)."""
    x = raw_f32(PARITY / "batchnorm_input.raw.f32")
    mean, var, gamma, beta, eps = raw_f32(PARITY / "batchnorm_params.raw.f32")
    n = x.size
    full = lambda v: np.full(n, v, np.float32)
    ve = orc.run("add", full(var), full(eps), n, [n])
    inv = orc.run("rsqrt", ve, None, n, [n])
    d = orc.run("sub", x, full(mean), n, [n])
    t = orc.run("mul", d, inv, n, [n])
    t = orc.run("mul", t, full(gamma), n, [n])
    y = orc.run("add", t, full(beta), n, [n])
    ref = raw_f32(PARITY / "batchnorm_ref.raw.f32")
    assert ulp_diff(y, ref).max() <= 8
    assert np.abs(y - ref).max() <= 1e-6


def conv1d_push_nhwc():
    # [16,64] * [3,64,32] pad 1 -> [16,32] as NHWC H=16 W=1 with HWIO KH=3 KW=1
    n, ih, iw, ic, kh, kw, oc, oh, ow = 1, 16, 1, 64, 3, 1, 32, 16, 1
    return [n, ih, iw, ic, kh, kw, oc, oh, ow, 1, 1, 1, 0, n * oh * ow * oc]


def test_conv1d_hlo_conv_bit_exact(orc):
    """hlo_conv_nhwc_hwio.comp accumulates ky -> kx -> ic exactly like conv1d_ref
    (generate_fixtures.py:42-58), so the result is bit-identical."""
    x = raw_f32(PARITY / "conv1d_input.raw.f32")
    w = raw_f32(PARITY / "conv1d_filter.raw.f32")
    y = orc.run("hlo_conv_nhwc_hwio", x, w, 512, conv1d_push_nhwc())
    ref = raw_f32(PARITY / "conv1d_ref.raw.f32")
    assert y.tobytes() == ref.tobytes()
    assert ulp_diff(y, raw_f32(PARITY / "cuda_conv1d.raw.f32")).max() <= 16


def test_conv1d_through_nchw_conv2d(orc):
    """conv2d.comp (NCHW, OIHW + bias tail, loop ic -> kh -> kw) on the transposed
    problem: NCHW/NHWC conjugation, within the reference's conv1d threshold."""
    x = raw_f32(PARITY / "conv1d_input.raw.f32").reshape(16, 64)
    w = raw_f32(PARITY / "conv1d_filter.raw.f32").reshape(3, 64, 32)
    x_nchw = x.T.reshape(1, 64, 16, 1)
    w_ohwi = np.transpose(w, (2, 0, 1))[:, :, None, :]  # [oc][kh][kw=1][ic]
    packed = orc.pack_conv_weight(w_ohwi, np.zeros(32, np.float32))
    push = [1, 64, 16, 1, 32, 16, 1, 3, 1, 1, 1, 0, 1, 0, 512]
    y = orc.run("conv2d", x_nchw, packed, 512, push).reshape(32, 16).T.reshape(-1)
    ref = raw_f32(PARITY / "conv1d_ref.raw.f32")
    rel = np.abs(y - ref) / np.maximum(np.abs(ref), 1e-30)
    assert ulp_diff(y, ref).max() <= 16 or rel.max() <= 1e-5


# ---- inference_poc closed-form graph: SHA-256 of every edge -----------------------------
def test_inference_poc_edges_sha256(orc):
    man = json.loads((GOLDEN / "inference_poc_manifest.json").read_text())["files"]
    x = orc.poc_fixture(0, 64)
    cw = orc.poc_fixture(1, 12)
    bn = orc.poc_fixture(2, 16)
    fc = orc.poc_fixture(3, 250)
    assert sha(x) == man["input"]["sha256"]
    assert sha(cw) == man["conv_weight"]["sha256"]
    assert sha(bn) == man["batchnorm_param"]["sha256"]
    assert sha(fc) == man["fc_param"]["sha256"]
    # conv1d: first column of the 8x8 input as an H=8 signal, valid width 3, 4 channels
    sig = x.reshape(8, 8)[:, 0].copy()
    conv = orc.run("hlo_conv_nhwc_hwio", sig, cw, 24,
                   [1, 8, 1, 1, 3, 1, 4, 6, 1, 1, 1, 0, 0, 24])
    assert sha(conv) == man["conv_output_ref"]["sha256"]
    # batchnorm: (x - mean) / sqrt(var + eps) * scale + bias, per channel c = i % 4
    p = bn.reshape(4, 4)
    rep = lambda col: np.tile(p[:, col], 6).astype(np.float32)
    eps = np.full(24, np.float32(1.0e-5), np.float32)
    d = orc.run("sub", conv, rep(2), 24, [24])
    s = orc.run("sqrt", orc.run("add", rep(3), eps, 24, [24]), None, 24, [24])
    t = orc.run("mul", orc.run("div", d, s, 24, [24]), rep(0), 24, [24])
    bno = orc.run("add", t, rep(1), 24, [24])
    assert sha(bno) == man["batchnorm_output_ref"]["sha256"]
    relu = orc.run("relu", bno, None, 24, [24])
    assert sha(relu) == man["relu_output_ref"]["sha256"]
    # fc: acc = bias[cls] + sum_i in[i] * W[i][cls] -> fully_connected with W transposed
    w_out_in = fc[:240].reshape(24, 10).T
    packed = orc.pack_fc_weight(w_out_in, fc[240:])
    logits = orc.run("fully_connected", relu, packed, 10, [1, 24, 10, 10])
    assert sha(logits) == man["logits_ref"]["sha256"]
    sm = orc.run("softmax10", logits, None, 10, [])
    assert sha(sm) == man["softmax_output_ref"]["sha256"]


# ---- engine.rs kernel self-test KAT -----------------------------------------------------
KAT_IN = np.array([0.25, 0.5, 0.75, 1.0, 1.25, 2.0, 3.0, 4.0], np.float32)
KAT_RHS = np.full(8, 2.0, np.float32)


def kat_cases():
    x, r = KAT_IN, KAT_RHS
    f = np.float32
    return [
        ("abs", None, np.abs(x), []), ("exp", None, np.exp(x), []), ("log", None, np.log(x), []),
        ("neg", None, -x, []), ("sqrt", None, np.sqrt(x), []),
        ("rsqrt", None, (f(1) / np.sqrt(x)).astype(f), []),
        ("sub", r, x - r, []), ("mul", r, x * r, []), ("div", r, x / r, []),
        ("pow", r, np.power(x, r), []), ("min", r, np.minimum(x, r), []),
        ("max", r, np.maximum(x, r), []),
        ("leaky_relu", None, np.maximum(x, f(0.1) * x), [f32bits(0.1)]),
        ("sigmoid", None, (f(1) / (f(1) + np.exp(-x))).astype(f), []),
        ("tanh", None, np.tanh(x), []),
    ]


def f32bits(v):
    return int(np.array([v], np.float32).view(np.int32)[0])


@pytest.mark.parametrize("case", kat_cases(), ids=lambda c: c[0])
def test_engine_self_test_kat(orc, case):
    name, rhs, expected, extra = case
    y = orc.run(name, KAT_IN, rhs, 8, [8] + extra)
    mism, max_abs, _ = orc.compare(y, expected, 1e-5)
    assert mism == 0, (name, max_abs)
