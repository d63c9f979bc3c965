"""Replays a resident model graph on the CPU oracle (TEST INFRASTRUCTURE).

Two modes over the op list the product library exposes (shp_model_op):
  per_op  — every op runs on the oracle with the GPU's own inputs (downloaded), and its
            output is compared with the GPU's: isolates each kernel's error.
  chained — the oracle runs the whole graph from the same weights and model inputs on
            its own outputs: the end-to-end CPU reference (and the bench's CPU baseline).
Views (kind 3) alias a slice of their parent tensor in both modes.
"""
from __future__ import annotations

import time

import numpy as np

from . import run


def _host_views(model, host: dict, tid: int):
    info = model.tensor_info(tid)
    if info.kind == 3:
        parent = _host_views(model, host, info.parent)
        return parent[info.offset: info.offset + info.elems]
    return host[tid]


def load_constants(model) -> dict:
    host = {}
    for tid in range(model.num_tensors()):
        info = model.tensor_info(tid)
        if info.kind in (1, 2):
            host[tid] = model.download(tid)
    return host


def per_op(model, atol=1e-4, rtol=1e-4, on_op=None) -> list[dict]:
    """Runs each op on the oracle with the GPU's inputs; returns per-op error records."""
    out = []
    for i, op in enumerate(model.ops()):
        get = lambda t: model.download(t) if t >= 0 else None
        t0 = time.perf_counter()
        want = run(op.kernel, get(op.in0), get(op.in1), op.out_elems, op.push, bias=get(op.bias),
                   residual=get(op.residual), act=op.act, alpha=op.alpha)
        got = model.download(op.out)
        err = np.abs(got.astype(np.float64) - want)
        excess = err - (atol + rtol * np.abs(want.astype(np.float64)))
        rec = dict(index=i, kernel=op.kernel, label=op.label, max_abs=float(err.max()),
                   worst_excess=float(excess.max()), finite=bool(np.isfinite(got).all()),
                   oracle_s=time.perf_counter() - t0)
        out.append(rec)
        if on_op:
            on_op(rec)
    return out


def chained(model, host: dict | None = None) -> dict:
    """The whole graph on the oracle; returns host arrays by tensor id."""
    host = dict(host) if host is not None else load_constants(model)
    for op in model.ops():
        get = lambda t: _host_views(model, host, t) if t >= 0 else None
        host[op.out] = run(op.kernel, get(op.in0), get(op.in1), op.out_elems, op.push,
                           bias=get(op.bias), residual=get(op.residual), act=op.act,
                           alpha=op.alpha)
    return host
