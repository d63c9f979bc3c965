"""shp_launch_static (split-K scratch in a fixed device array, no allocation) against
shp_launch_ex (split-K scratch in the context's hipMalloc'd workspace).

Both plan the same tiles and split counts and sum the partials in the same order, so the
outputs must be bit-identical.  Two calls in a row, the second on a smaller problem, show
that the shared array's leftover contents (partials and tile counters of the first call)
do not leak into the next one.  The context used for the static calls must end with no
workspace of its own: nothing was allocated for them.
"""
import ctypes as C

import numpy as np
import pytest

from spirv_inference_amd import Context, ShpError
from spirv_inference_amd._lib import Epilogue, check, lib

pytestmark = pytest.mark.gpu

# ResNet-50 b32 3x3 convolutions whose plans split K (18.4 MiB and 15.4 MiB of scratch).
CONV4 = dict(n=32, ih=14, ic=256, oc=256, oh=14, stride=1)
CONV5 = dict(n=32, ih=7, ic=512, oc=512, oh=7, stride=1)


def _push(n, ih, ic, oc, oh, stride):
    return [n, ih, ih, ic, 3, 3, oc, oh, oh, stride, stride, 1, 1, n * oh * oh * oc]


def _workspace_bytes(ctx):
    p, b = C.c_void_p(), C.c_uint64()
    check(lib().shp_workspace_info(ctx.handle, C.byref(p), C.byref(b)), "shp_workspace_info")
    return b.value


def _conv(ctx, entry, shape, seed):
    """One 3x3 convolution with bias + residual + ReLU through `entry`; returns the output."""
    push = _push(**shape)
    n, ih, ic, oc = shape["n"], shape["ih"], shape["ic"], shape["oc"]
    x = ctx.fill_random(ctx.empty(n * ih * ih * ic), seed, 1)
    w = ctx.fill_random(ctx.empty(9 * ic * oc), seed, 2, "normal", 0.0, float(np.sqrt(2 / (9 * ic))))
    b = ctx.fill_random(ctx.empty(oc), seed, 3, "normal", 0.0, 0.01)
    r = ctx.fill_random(ctx.empty(push[13]), seed, 4)
    y = ctx.empty(push[13])
    arr = (C.c_int32 * len(push))(*push)
    epi = Epilogue(b.ptr, r.ptr, 1, 0.0)
    rc = entry(ctx.handle, b"hlo_conv_nhwc_hwio", x.ptr, w.ptr, y.ptr, arr, len(push), push[13],
               C.byref(epi))
    check(rc, "conv launch")
    ctx.sync()
    out = y.download()
    for t in (x, w, b, r, y):
        t.free()
    return out


def test_static_scratch_matches_workspace_launch_twice():
    with Context("any") as ctx_static, Context("any") as ctx_ws:
        print("[no_alloc] static scratch vs workspace: conv4 b32, then conv5 b32", flush=True)
        for i, shape in enumerate((CONV4, CONV5)):
            got = _conv(ctx_static, lib().shp_launch_static, shape, seed=11 + i)
            want = _conv(ctx_ws, lib().shp_launch_ex, shape, seed=11 + i)
            assert np.isfinite(want).all() and np.abs(want).max() > 0
            assert np.array_equal(got, want), (
                f"call {i}: max |static - workspace| = {np.abs(got - want).max():.3e}")
        # the workspace entry point did split K (it grew its workspace); the static one
        # allocated nothing
        assert _workspace_bytes(ctx_ws) > 0
        assert _workspace_bytes(ctx_static) == 0


def test_static_scratch_rejects_plans_beyond_its_size():
    """A dot whose plan wants 64.06 MiB of split-K scratch is refused before any launch."""
    m, k, n = 4096, 16384, 1024
    with Context("any") as ctx:
        a, b, c = ctx.empty(m * k), ctx.empty(k * n), ctx.empty(m * n)
        push = [m, k, n, m * n]
        arr = (C.c_int32 * 4)(*push)
        rc = lib().shp_launch_static(ctx.handle, b"hlo_dot_rank2", a.ptr, b.ptr, c.ptr, arr, 4,
                                     m * n, None)
        assert rc != 0
        with pytest.raises(ShpError, match="static scratch"):
            check(rc, "shp_launch_static")
        ctx.sync()
        for t in (a, b, c):
            t.free()


def test_static_scratch_orders_launches_from_two_streams():
    """Two contexts (two streams) issue static launches back to back with no host wait in
    between: the second waits on the device for the first (the array is shared per GPU), so
    both equal their workspace-launched results bit for bit."""
    with Context("any") as ca, Context("any") as cb, Context("any") as cw:
        print("[no_alloc] two streams on the static scratch: conv4 on A, conv5 on B", flush=True)
        want = [_conv(cw, lib().shp_launch_ex, s, seed=21 + i) for i, s in enumerate((CONV4, CONV5))]
        bufs = []
        for i, (c, shape) in enumerate(((ca, CONV4), (cb, CONV5))):
            push = _push(**shape)
            n, ih, ic, oc = shape["n"], shape["ih"], shape["ic"], shape["oc"]
            x = c.fill_random(c.empty(n * ih * ih * ic), 21 + i, 1)
            w = c.fill_random(c.empty(9 * ic * oc), 21 + i, 2, "normal", 0.0,
                              float(np.sqrt(2 / (9 * ic))))
            b = c.fill_random(c.empty(oc), 21 + i, 3, "normal", 0.0, 0.01)
            r = c.fill_random(c.empty(push[13]), 21 + i, 4)
            y = c.empty(push[13])
            bufs.append((c, x, w, b, r, y, push))
        for c, x, w, b, r, y, push in bufs:  # inputs ready before either launch
            c.sync()
        for c, x, w, b, r, y, push in bufs:
            arr = (C.c_int32 * len(push))(*push)
            epi = Epilogue(b.ptr, r.ptr, 1, 0.0)
            check(lib().shp_launch_static(c.handle, b"hlo_conv_nhwc_hwio", x.ptr, w.ptr, y.ptr,
                                          arr, len(push), push[13], C.byref(epi)), "static")
        for (c, x, w, b, r, y, push), ref in zip(bufs, want):
            c.sync()
            assert np.array_equal(y.download(), ref)
            for t in (x, w, b, r, y):
                t.free()
