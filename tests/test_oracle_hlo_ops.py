"""Pins of the oracle's HLO shape ops (compiler.rs host helpers) against numpy (CPU).

broadcast_in_dim / transpose / slice / concatenate / compare / select are pure data
movement or predicates: they must equal numpy's own implementation bit for bit.  The
rank > 4 reduce folds in source-index order (reduce_tensor, compiler.rs:1730-1759): its
sum is checked bit-exactly against a sequential float32 loop on a small tensor and to
rounding against numpy's float64 sum on a larger one; max against np.fmax.reduce (the
NaN-ignoring maximum of Rust's f32::max).
"""
import numpy as np
import pytest

import oracle as orc
from spirv_inference_amd import hlo_ops as H

RNG = np.random.default_rng(7)


def r32(*shape):
    return RNG.standard_normal(shape).astype(np.float32)


def np_broadcast_in_dim(x, out_shape, dims):
    # move source axes into output order, then insert size-1 axes and broadcast
    order = np.argsort(dims)
    xt = np.transpose(x, order) if x.ndim else x
    shape = [1] * len(out_shape)
    for a, d in enumerate(np.array(dims)[order]):
        shape[d] = xt.shape[a]
    return np.broadcast_to(xt.reshape(shape), out_shape)


@pytest.mark.parametrize("src,out,dims", [
    ((4, 1, 64, 64), (4, 8, 64, 64), (0, 1, 2, 3)),          # GQA head tile (size-1 axis)
    ((2048,), (1, 64, 2048), (2,)),                          # bias row over tokens
    ((3, 5), (5, 2, 3), (2, 0)),                             # unsorted dimensions
    ((1,), (2, 3, 4), (1,)),                                 # one element -> splat
    ((), (7, 3), ()),                                        # scalar
    ((6, 7), (6, 7), (0, 1)),                                # same shape -> copy
    ((1, 4, 1, 64, 64), (1, 4, 8, 64, 64), (0, 1, 2, 3, 4)),  # rank 5
])
def test_broadcast(src, out, dims):
    x = r32(*src) if src else np.float32(RNG.standard_normal())
    y = orc.run("hlo_broadcast", np.atleast_1d(x), None, int(np.prod(out)),
                H.broadcast_push(src, out, dims))
    np.testing.assert_array_equal(y, np_broadcast_in_dim(np.asarray(x), out, dims).reshape(-1))


@pytest.mark.parametrize("shape,perm", [((1, 64, 32, 64), (0, 2, 1, 3)), ((2, 3, 4, 5, 6), (4, 0, 3, 1, 2)),
                                        ((8, 9), (1, 0)), ((3, 4, 5), (0, 1, 2))])
def test_transpose(shape, perm):
    x = r32(*shape)
    y = orc.run("hlo_transpose", x, None, x.size, H.transpose_push(shape, perm))
    np.testing.assert_array_equal(y, np.transpose(x, perm).reshape(-1))


@pytest.mark.parametrize("shape,starts,limits,strides", [
    ((1, 32, 64, 64), (0, 0, 0, 0), (1, 32, 64, 32), None),   # rotate-half, first half
    ((1, 32, 64, 64), (0, 0, 0, 32), (1, 32, 64, 64), None),  # second half
    ((5, 9, 7), (1, 0, 2), (5, 9, 7), (2, 3, 2)),             # strided
    ((4, 6), (0, 2), (4, 9), (1, 1)),                         # limit past the end -> zeros
])
def test_slice(shape, starts, limits, strides):
    x = r32(*shape)
    sp = strides or [1] * len(shape)
    out = H.slice_shape(starts, limits, sp)
    y = orc.run("hlo_slice", x, None, int(np.prod(out)), H.slice_push(shape, starts, limits, sp))
    ref = np.zeros(out, np.float32)
    view = x[tuple(slice(s, l, p) for s, l, p in zip(starts, limits, sp))]
    ref[tuple(slice(0, n) for n in view.shape)] = view
    np.testing.assert_array_equal(y, ref.reshape(-1))


@pytest.mark.parametrize("shapes,dim", [([(1, 32, 64, 32), (1, 32, 64, 32)], 3),
                                        ([(2, 3, 5), (2, 4, 5), (2, 1, 5)], 1),
                                        ([(3, 2), (1, 2)], 0)])
def test_concatenate(shapes, dim):
    xs = [r32(*s) for s in shapes]
    ref = np.concatenate(xs, axis=dim)
    y, off = np.zeros(ref.size, np.float32), 0
    for x, s in zip(xs, shapes):
        y = orc.run("hlo_concatenate_into", x, None, ref.size,
                    H.concatenate_into_push(ref.shape, s, dim, off), out_init=y)
        off += s[dim]
    np.testing.assert_array_equal(y, ref.reshape(-1))


OPS = {"LT": np.less, "LE": np.less_equal, "EQ": np.equal, "NE": np.not_equal,
       "GE": np.greater_equal, "GT": np.greater}


@pytest.mark.parametrize("direction", list(OPS))
@pytest.mark.parametrize("out,a,b", [((8, 128, 3072), (8, 128, 3072), ()),
                                     ((4, 5, 6), (5, 6), (4, 1, 6)),
                                     ((3, 7), (3, 7), (3, 7))])
def test_compare(direction, out, a, b):
    x = np.round(r32(*a) * 2) / 2 if a else np.float32(0.5)
    z = np.round(r32(*b) * 2) / 2 if b else np.float32(0.0)  # rounded: many equal pairs
    y = orc.run("hlo_compare", np.atleast_1d(x), np.atleast_1d(z), int(np.prod(out)),
                H.compare_push(direction, out, a, b))
    ref = OPS[direction](np.broadcast_to(x, out), np.broadcast_to(z, out)).astype(np.float32)
    np.testing.assert_array_equal(y, ref.reshape(-1))


def test_compare_flat_operand():
    # binary_tensor takes an operand with the output's element count flat, whatever its shape
    a, b = r32(6, 4), r32(4, 6)
    y = orc.run("hlo_compare", a, b, 24, H.compare_push("GT", (4, 6), (6, 4), (4, 6)))
    np.testing.assert_array_equal(y, (a.reshape(-1) > b.reshape(-1)).astype(np.float32))


@pytest.mark.parametrize("out,p,t,f", [((8, 128, 64), (8, 128, 64), (8, 128, 64), ()),
                                       ((4, 5, 6), (5, 6), (1, 6), (4, 5, 6))])
def test_select(out, p, t, f):
    pred = (r32(*p) > 0).astype(np.float32)
    on_t = r32(*t)
    on_f = r32(*f) if f else np.float32(-3.0)
    fill = np.broadcast_to(on_f, out).astype(np.float32)
    y = orc.run("hlo_select", pred, on_t, int(np.prod(out)), H.select_push(out, p, t),
                out_init=fill)
    ref = np.where(np.broadcast_to(pred, out) != 0, np.broadcast_to(on_t, out), fill)
    np.testing.assert_array_equal(y, ref.reshape(-1))


def test_reduce_sum_order_bit_exact():
    x = r32(2, 3, 4, 5, 6)
    dims = (1, 3)
    y = orc.run("hlo_reduce", x, None, 2 * 4 * 6, H.reduce_push("sum", x.shape, dims, 0.0))
    ref = np.zeros((2, 4, 6), np.float32)
    for a in range(2):  # source order: axis 1 outer, axis 3 inner, one fp32 add at a time
        for c in range(4):
            for e in range(6):
                acc = np.float32(0.0)
                for b in range(3):
                    for d in range(5):
                        acc = np.float32(acc + x[a, b, c, d, e])
                ref[a, c, e] = acc
    np.testing.assert_array_equal(y, ref.reshape(-1))


@pytest.mark.parametrize("shape,dims", [((1, 4, 8, 64, 64), (4,)), ((1, 4, 8, 64, 64), (0, 2)),
                                        ((3, 5, 7, 2, 3, 4), (1, 2, 5))])
def test_reduce_sum_and_max(shape, dims):
    x = r32(*shape)
    kept = int(np.prod([d for k, d in enumerate(shape) if k not in dims]))
    s = orc.run("hlo_reduce", x, None, kept, H.reduce_push("sum", shape, dims, 0.0))
    ref = x.astype(np.float64).sum(axis=dims).reshape(-1)
    np.testing.assert_allclose(s, ref, rtol=1e-5, atol=1e-4)
    m = orc.run("hlo_reduce", x, None, kept, H.reduce_push("max", shape, dims, -np.inf))
    np.testing.assert_array_equal(m, x.max(axis=dims).reshape(-1))


def test_reduce_max_ignores_nan():
    x = r32(2, 3, 4, 5, 6)
    x[0, 1, 2, 3, 4] = np.nan
    m = orc.run("hlo_reduce", x, None, 2 * 6, H.reduce_push("max", x.shape, (1, 2, 3), -np.inf))
    np.testing.assert_array_equal(m, np.fmax.reduce(x, axis=(1, 2, 3)).reshape(-1))


def test_errors_fail_closed():
    with pytest.raises(RuntimeError):  # perm not a permutation
        orc.run("hlo_transpose", r32(4), None, 4, [2, 4, 2, 2, 0, 0])
    with pytest.raises(RuntimeError):  # source dim does not match its output axis
        orc.run("hlo_broadcast", r32(3), None, 8, H.broadcast_push((3,), (2, 4), (1,)))


@pytest.mark.parametrize("base_shape,offset,shape,strides", [
    ((2, 3, 4, 5), 0, (2, 4, 3, 5), (60, 5, 20, 1)),          # transpose {0,2,1,3}
    ((8, 16, 2304), 768, (8, 12, 16, 64), (16 * 2304, 64, 2304, 1)),  # BERT head view of k
    ((4, 64), 0, (4, 8, 64), (64, 0, 1)),                      # broadcast axis (stride 0)
    ((30,), 3, (4, 3), (6, 2)),                                # offset + stepped slice
])
def test_oracle_strided_copy_is_numpy_as_strided(base_shape, offset, shape, strides):
    base = r32(*base_shape).reshape(-1)
    view = np.lib.stride_tricks.as_strided(base[offset:], shape, [s * 4 for s in strides])
    push = [len(shape), int(np.prod(shape)), *shape, *strides]
    got = orc.run("hlo_strided_copy", base[offset:], None, int(np.prod(shape)), push)
    np.testing.assert_array_equal(got, view.reshape(-1))


def test_oracle_strided_copy_rejects_a_view_past_its_input():
    with pytest.raises(RuntimeError, match="exceeds"):
        orc.run("hlo_strided_copy", r32(10), None, 12, [2, 12, 3, 4, 4, 1])
