"""inverted_residual_nhwc (one launch per MBConv block) against the oracle's three-operator
chain: 1x1 conv2d_nhwc + act, depthwise_conv2d_nhwc + act, 1x1 conv2d_nhwc + residual + act
(source/tflite_loader/src/scheduler.rs:321-548), per block at the build's 1e-4 gate.

Cases: the MobileNetV2 b1 and EfficientNet-Lite0 blocks whose plans differ (a tile per
workgroup, expanded channels split over workgroups, output channels split), the block
without expand, 5x5 and stride 2, odd maps with partial edge tiles, channel counts that are
not multiples of 16, and plans forced through the context's tune keys so every code path
(split-channel fixup, several output-channel slices, small and large tiles) runs.
"""
import numpy as np
import pytest

from spirv_inference_amd import ShpError

pytestmark = pytest.mark.gpu

RELU6 = 2


def same(i, k, s):
    o = (i + s - 1) // s
    pad = max((o - 1) * s + k - i, 0)
    return o, pad // 2


def block(seed, n, cin, h, w, ce, cout, k, s, expand=True):
    rng = np.random.default_rng(seed)
    oh, pt = same(h, k, s)
    ow, pl = same(w, k, s)
    parts = []
    if expand:
        parts += [rng.standard_normal(ce * cin) * np.sqrt(2.0 / cin), rng.standard_normal(ce) * 0.1]
    parts += [rng.standard_normal(k * k * ce) * np.sqrt(2.0 / (k * k)), rng.standard_normal(ce) * 0.1,
              rng.standard_normal(cout * ce) * np.sqrt(1.0 / ce), rng.standard_normal(cout) * 0.1]
    packed = np.concatenate(parts).astype(np.float32)
    x = rng.uniform(-1, 1, n * h * w * cin).astype(np.float32)
    total = n * oh * ow * cout
    push = [n, cin, h, w, ce, cout, oh, ow, k, s, pt, pl, int(expand), RELU6, RELU6, total]
    return x, packed, push


def run_block(ctx, x, packed, push, residual=False, act=0):
    dx, dw, dy = ctx.tensor(x), ctx.tensor(packed), ctx.empty(push[15])
    try:
        ctx.launch("inverted_residual_nhwc", dx, dw, dy, push, residual=dx if residual else None,
                   act=act)
        ctx.sync()
        return dy.download()
    finally:
        for t in (dx, dw, dy):
            t.free()


def want(orc, x, packed, push, residual=False, act=0):
    return orc.run("inverted_residual_nhwc", x, packed, push[15], push,
                   residual=x if residual else None, act=act)


CASES = [  # (label, n, cin, h, w, ce, cout, k, s, expand, residual)
    ("mbv2_block2_b1", 1, 24, 56, 56, 144, 24, 3, 1, True, True),
    ("mbv2_block1_b1", 1, 16, 112, 112, 96, 24, 3, 2, True, False),
    ("mbv2_block14_b1", 1, 160, 7, 7, 960, 160, 3, 1, True, True),
    ("mbv2_block16_b1", 1, 160, 7, 7, 960, 320, 3, 1, True, False),
    ("mbv2_block0_b1", 1, 32, 112, 112, 32, 16, 3, 1, False, False),
    ("mbv2_block11_b1", 1, 96, 14, 14, 576, 96, 3, 1, True, True),
    ("effnet_block3_b2", 2, 24, 56, 56, 144, 40, 5, 2, True, False),
    ("effnet_block9_b2", 2, 112, 14, 14, 672, 112, 5, 1, True, True),
    ("effnet_block11_b2", 2, 112, 14, 14, 672, 192, 5, 2, True, False),
    ("odd_s2", 3, 20, 13, 11, 48, 28, 3, 2, True, False),
    ("odd_k5_res", 2, 36, 10, 9, 64, 36, 5, 1, True, True),
    # without expand, many input channels (staged 32 at a time over the halo)
    ("effnet_block12_dwproj_b2", 2, 1152, 7, 7, 1152, 192, 5, 1, False, False),
    ("effnet_block9_dwproj_b2", 2, 672, 14, 14, 672, 112, 5, 1, False, False),
    ("dwproj_s2_odd", 3, 48, 9, 11, 48, 24, 3, 2, False, False),
]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_block_matches_three_operator_chain(ctx, orc, case):
    label, n, cin, h, w, ce, cout, k, s, expand, res = case
    print(f"[block] {label}", flush=True)
    x, packed, push = block(7, n, cin, h, w, ce, cout, k, s, expand)
    got = run_block(ctx, x, packed, push, residual=res)
    ref = want(orc, x, packed, push, residual=res)
    from conftest import assert_close
    assert_close(got, ref, what=label)


FORCED = [  # (th, tw, expanded-channel splits, output-channel splits)
    (4, 4, 3, 2), (2, 8, 5, 3), (8, 8, 1, 1), (7, 7, 2, 1), (1, 4, 12, 2)]


@pytest.mark.parametrize("plan", FORCED, ids=[f"t{a}x{b}_s{c}_j{d}" for a, b, c, d in FORCED])
@pytest.mark.parametrize("case", [CASES[2], CASES[9], CASES[10], CASES[13]], ids=lambda c: c[0])
def test_forced_plans(ctx, orc, case, plan):
    label, n, cin, h, w, ce, cout, k, s, expand, res = case
    th, tw, S, J = plan
    print(f"[block] {label} plan {plan}", flush=True)
    x, packed, push = block(11, n, cin, h, w, ce, cout, k, s, expand)
    ref = want(orc, x, packed, push, residual=res, act=RELU6)
    for key, v in (("ir_th", th), ("ir_tw", tw), ("ir_splits", S), ("ir_cout_splits", J)):
        ctx.tune(key, v)
    try:
        got = run_block(ctx, x, packed, push, residual=res, act=RELU6)
        again = run_block(ctx, x, packed, push, residual=res, act=RELU6)
    finally:
        for key in ("ir_th", "ir_tw", "ir_splits", "ir_cout_splits"):
            ctx.tune(key, 0)
    from conftest import assert_close
    assert_close(got, ref, what=f"{label} {plan}")
    # the split partials are summed in split order: repeat launches agree bit for bit
    assert np.array_equal(got, again)


def test_graph_replay_resets_the_split_counters(ctx, orc):
    """A split plan captured into a graph and replayed: every replay equals the eager run
    (the last arrival of each tile leaves its counter at zero for the next launch)."""
    label, n, cin, h, w, ce, cout, k, s, expand, res = CASES[2]
    x, packed, push = block(5, n, cin, h, w, ce, cout, k, s, expand)
    dx, dw, dy = ctx.tensor(x), ctx.tensor(packed), ctx.empty(push[15])
    try:
        ctx.launch("inverted_residual_nhwc", dx, dw, dy, push, residual=dx)  # sizes the workspace
        ctx.sync()
        eager = dy.download()
        ctx.capture_begin()
        ctx.launch("inverted_residual_nhwc", dx, dw, dy, push, residual=dx)
        g = ctx.capture_end()
        try:
            for _ in range(4):
                dy.upload(np.zeros(push[15], np.float32))
                g.launch()
                ctx.sync()
                assert np.array_equal(dy.download(), eager)
        finally:
            g.destroy()
    finally:
        for t in (dx, dw, dy):
            t.free()
    from conftest import assert_close
    assert_close(eager, want(orc, x, packed, push, residual=True), what="eager")


def test_rejects_what_it_does_not_handle(ctx):
    x, packed, push = block(1, 1, 8, 8, 8, 32, 8, 3, 1)
    bad = list(push)
    bad[1] = 6  # cin not a multiple of 4
    with pytest.raises(ShpError, match="multiple of 4"):
        run_block(ctx, np.zeros(8 * 8 * 6, np.float32), packed, bad)
    bad = list(push)
    bad[4] = 40  # ce not a multiple of 16
    with pytest.raises(ShpError, match="multiple of 4, ce of 16"):
        run_block(ctx, x, packed, bad)
    bad = list(push)
    bad[15] += 1
    with pytest.raises(ShpError, match="total"):
        run_block(ctx, x, packed, bad)


HEADS = [  # (label, n, cin, h, w, cout, act)
    ("mbv2_head_b1", 1, 320, 7, 7, 1280, RELU6),
    ("effnet_head_b8", 8, 320, 7, 7, 1280, RELU6),
    ("odd", 3, 20, 5, 3, 40, 1),
    ("one_pixel", 2, 8, 1, 1, 16, 0),
    ("two_rounds", 1, 36, 12, 11, 24, RELU6),  # 132 pixels: wavefronts take two row blocks
    ("b16_two_col_blocks", 16, 320, 7, 7, 1280, RELU6),  # 640 workgroups of 32 channels
    ("k_past_512", 2, 516, 3, 3, 32, RELU6),  # the row-block kernel: cin > 512
]


@pytest.mark.parametrize("case", HEADS, ids=[c[0] for c in HEADS])
def test_conv1x1_gap_matches_conv_then_pool(ctx, orc, case):
    """conv1x1_gap_nhwc (1x1 conv + activation + global average pool in one launch) against
    the oracle's conv2d_nhwc + global_avg_pool_nhwc chain at the build's 1e-4 gate: maps of
    at most 64 pixels with K split over the wavefronts (one or two 16-channel column blocks
    per workgroup), and larger maps or more than 512 input channels on the row-block kernel."""
    label, n, cin, h, w, cout, act = case
    print(f"[head] {label}", flush=True)
    rng = np.random.default_rng(9)
    x = rng.uniform(-1, 1, n * h * w * cin).astype(np.float32)
    wt = np.concatenate([rng.standard_normal(cout * cin) * np.sqrt(2.0 / cin),
                         rng.standard_normal(cout) * 0.1]).astype(np.float32)
    push = [n, cin, h, w, cout, n * cout]
    dx, dw, dy = ctx.tensor(x), ctx.tensor(wt), ctx.empty(n * cout)
    try:
        ctx.launch("conv1x1_gap_nhwc", dx, dw, dy, push, act=act)
        ctx.sync()
        got = dy.download()
    finally:
        for t in (dx, dw, dy):
            t.free()
    ref = orc.run("conv1x1_gap_nhwc", x, wt, n * cout, push, act=act)
    from conftest import assert_close
    assert_close(got, ref, what=label)


def test_conv1x1_gap_rejects(ctx):
    x = np.zeros(2 * 7 * 7 * 6, np.float32)
    with pytest.raises(ShpError, match="multiple of 4"):
        ctx_run = ctx.tensor(x), ctx.tensor(np.zeros(16 * 6 + 16, np.float32)), ctx.empty(32)
        try:
            ctx.launch("conv1x1_gap_nhwc", *ctx_run, [2, 6, 7, 7, 16, 32])
        finally:
            for t in ctx_run:
                t.free()
