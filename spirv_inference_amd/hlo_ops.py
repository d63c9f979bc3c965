"""Device counterparts of the HLO path's host-side shape ops (push builders + launches).

The reference's HLO executor runs `broadcast`, `transpose`, `slice`, `concatenate`,
`compare`, `select` and rank > 4 `reduce` on the CPU between its Vulkan dispatches
(source/xla_hlo/src/compiler.rs:336-586, helpers :1361-1418, :1521-1620, :1730-1759,
:1879-1952).  Here they are registry kernels on resident tensors (hlo_broadcast,
hlo_transpose, hlo_slice, hlo_concatenate_into, hlo_compare, hlo_select, hlo_reduce); the
functions below turn the HLO attributes a lowering parses into their i32 push vectors, and
`concatenate` / `select` add the multi-launch sequences the three-binding ABI needs.
"""
from __future__ import annotations

from typing import Sequence

import numpy as np

from .runtime import Context, DeviceTensor

DIRECTIONS = {"LT": 0, "LE": 1, "EQ": 2, "NE": 3, "GE": 4, "GT": 5}
MAX_RANK = 8


def _n(shape: Sequence[int]) -> int:
    return int(np.prod(shape, dtype=np.int64)) if len(shape) else 1


def _rank(shape: Sequence[int], lo: int = 1) -> int:
    r = len(shape)
    if not lo <= r <= MAX_RANK:
        raise ValueError(f"rank {r} outside {lo}..{MAX_RANK}")
    return r


def broadcast_push(src_shape: Sequence[int], out_shape: Sequence[int],
                   dimensions: Sequence[int]) -> list[int]:
    """broadcast_in_dim: source axis a lands on output axis dimensions[a]."""
    rs, ro = _rank(src_shape, 0), _rank(out_shape)
    if len(dimensions) != rs:
        raise ValueError("broadcast: one `dimensions` entry per source axis")
    return [rs, ro, _n(out_shape), *src_shape, *out_shape, *dimensions]


def transpose_push(src_shape: Sequence[int], perm: Sequence[int]) -> list[int]:
    """transpose: output axis i is source axis perm[i] (HLO `dimensions`)."""
    r = _rank(src_shape)
    return [r, _n(src_shape), *src_shape, *perm]


def slice_shape(starts, limits, strides) -> list[int]:
    return [(lim - st + sp - 1) // sp for st, lim, sp in zip(starts, limits, strides)]


def slice_push(src_shape: Sequence[int], starts: Sequence[int], limits: Sequence[int],
               strides: Sequence[int] | None = None) -> list[int]:
    """slice={[start:limit:stride], ...} (parse_slice_spec's triples; stride defaults to 1)."""
    r = _rank(src_shape)
    strides = list(strides) if strides is not None else [1] * r
    return [r, _n(slice_shape(starts, limits, strides)), *src_shape, *starts, *limits, *strides]


def concatenate_into_push(out_shape: Sequence[int], in_shape: Sequence[int], dim: int,
                          offset: int) -> list[int]:
    r = _rank(out_shape)
    return [r, dim, offset, *out_shape, *in_shape]


def compare_push(direction: str | int, out_shape: Sequence[int], a_shape: Sequence[int],
                 b_shape: Sequence[int]) -> list[int]:
    d = DIRECTIONS.get(direction, 5) if isinstance(direction, str) else int(direction)
    return [d, _n(out_shape), _rank(out_shape), len(a_shape), len(b_shape), *out_shape,
            *a_shape, *b_shape]


def select_push(out_shape: Sequence[int], pred_shape: Sequence[int],
                true_shape: Sequence[int]) -> list[int]:
    return [_n(out_shape), _rank(out_shape), len(pred_shape), len(true_shape), *out_shape,
            *pred_shape, *true_shape]


def reduce_push(kind: str, src_shape: Sequence[int], dims: Sequence[int],
                init: float) -> list[int]:
    """kind 'sum' or 'max' (reduce_kind); dims = the reduced axes."""
    r = _rank(src_shape)
    red = [1 if k in set(dims) else 0 for k in range(r)]
    kept = [d for d, f in zip(src_shape, red) if not f]
    bits = int(np.array([init], np.float32).view(np.int32)[0])
    return [1 if kind == "max" else 0, r, _n(kept), bits, *src_shape, *red]


def concatenate(ctx: Context, inputs: Sequence[tuple[DeviceTensor, Sequence[int]]], dim: int,
                out: DeviceTensor, out_shape: Sequence[int]) -> None:
    """cpu_concatenate on the device: one hlo_concatenate_into launch per operand."""
    offset = 0
    for t, shape in inputs:
        ctx.launch("hlo_concatenate_into", t, None, out,
                   concatenate_into_push(out_shape, shape, dim, offset))
        offset += shape[dim]


def select(ctx: Context, pred: DeviceTensor, pred_shape: Sequence[int], on_true: DeviceTensor,
           true_shape: Sequence[int], on_false: DeviceTensor, false_shape: Sequence[int],
           out: DeviceTensor, out_shape: Sequence[int]) -> None:
    """select_tensor on the device: on_false is broadcast into `out` (binary_tensor's
    operand rule), then hlo_select overwrites where pred != 0."""
    n = _n(out_shape)
    if _n(false_shape) == n:
        ctx.launch("reshape", on_false, None, out, [n])
    else:
        rf = len(false_shape)
        dims = list(range(len(out_shape) - rf, len(out_shape)))
        ctx.launch("hlo_broadcast", on_false, None, out, broadcast_push(false_shape, out_shape, dims))
    ctx.launch("hlo_select", pred, on_true, out, select_push(out_shape, pred_shape, true_shape))
