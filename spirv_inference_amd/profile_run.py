"""Run one benchmark config's resident graph a few times, for an external profiler.

    rocprofv3 --kernel-trace --stats -d out -- python3 -m spirv_inference_amd.profile_run \\
        --arch bert_base --batch 8 --seq 128 --steps 3

Every pass launches the graph eagerly (one dispatch per op, in graph order), so a kernel trace
or a counter collection sees each op as its own dispatch; `--graph` replays a hipGraph
capture instead.  `--copy-calibration-mb N` ends with one N MiB `reshape` copy (N MiB read and
N MiB written), against which HBM byte counters are scaled.  `--tune KEY=VALUE` applies a
planner override (shp_tune) to the run's context.  The op list (kernel, label,
algorithmic bytes and FLOPs per op) is written as JSON with `--ops-json`, so a trace can be
matched op by op.
"""
from __future__ import annotations

import argparse
import json
import sys
import time

from .models import Model
from .runtime import Context


def op_work(op, elems) -> tuple[float, float]:
    """(FLOPs, algorithmic HBM bytes) of one op: 2*MAC for the dense ops; bytes = every
    distinct input element read once + the output written once (+ bias and residual)."""
    q, k = op.push, op.kernel
    ins = [elems(op.in0), elems(op.in1)]
    extra = elems(op.bias) + elems(op.residual)
    flops = 0.0
    if k == "hlo_conv_nhwc_hwio":
        flops = 2.0 * q[0] * q[7] * q[8] * q[6] * q[4] * q[5] * q[3]
    elif k in ("conv2d", "conv2d_nhwc"):
        flops = 2.0 * q[0] * q[5] * q[6] * q[4] * q[1] * q[7] * q[8]
    elif k == "hlo_dot_rank2":
        flops = 2.0 * q[0] * q[1] * q[2]
    elif k == "hlo_dot_batched":
        flops = 2.0 * q[0] * q[1] * q[2] * q[3]
    elif k == "dot_general_strided":
        flops = 2.0 * q[0] * q[1] * q[2] * q[3] * q[4]
    elif k == "fully_connected":
        flops = 2.0 * q[0] * q[1] * q[2]
    elif k == "attention_fused":  # push {B, H, S, HD, ...}: two S x S x HD products per head
        flops = 4.0 * q[0] * q[1] * q[2] * q[2] * q[3]
    elif k in ("depthwise_conv2d", "depthwise_conv2d_nhwc"):
        flops = 2.0 * op.out_elems * q[6] * q[7]  # push {n, c, ih, iw, oh, ow, kh, kw, ...}
    elif k == "inverted_residual_nhwc":  # {n, cin, h, w, ce, cout, oh, ow, k, s, .., expand}
        px_in, px_out = q[0] * q[2] * q[3], q[0] * q[6] * q[7]
        flops = 2.0 * (px_in * q[1] * q[4] * q[12] + px_out * q[4] * q[8] * q[8] +
                       px_out * q[4] * q[5])
    elif k == "conv1x1_gap_nhwc":  # {n, cin, h, w, cout, total}
        flops = 2.0 * q[0] * q[2] * q[3] * q[1] * q[4]
    nbytes = 4.0 * (sum(ins) + op.out_elems + extra)
    return flops, nbytes


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--arch", required=True,
                    choices=["resnet50_v1_5", "mobilenet_v2", "efficientnet_lite0", "bert_base"])
    ap.add_argument("--batch", type=int, required=True)
    ap.add_argument("--seq", type=int, default=0)
    ap.add_argument("--steps", type=int, default=3)
    ap.add_argument("--graph", action="store_true")
    ap.add_argument("--copy-calibration-mb", type=int, default=0)
    ap.add_argument("--ops-json")
    ap.add_argument("--tune", action="append", default=[], metavar="KEY=VALUE",
                    help="planner override for this run's context (shp_tune), e.g. gemm_group=-1")
    a = ap.parse_args(argv)
    with Context("any") as ctx:
        for kv in a.tune:
            k, v = kv.split("=", 1)
            ctx.tune(k, int(v))
        with Model(ctx, a.arch, a.batch, a.seq, seed=2) as m:
            ops = m.ops()
            info = {}

            def elems(tid):
                if tid < 0:
                    return 0
                if tid not in info:
                    info[tid] = m.tensor_info(tid).elems
                return info[tid]

            if a.ops_json:
                rows = []
                for o in ops:
                    fl, by = op_work(o, elems)
                    rows.append({"kernel": o.kernel, "label": o.label, "flops": fl,
                                 "bytes": by, "push": list(o.push)})
                with open(a.ops_json, "w") as f:
                    json.dump(rows, f)
            m.use_graph(a.graph)
            m.run()  # warm (and capture, with --graph)
            ctx.sync()
            t0 = time.perf_counter()
            for _ in range(a.steps):
                m.run()
            ctx.sync()
            dt = (time.perf_counter() - t0) / max(a.steps, 1)
            print(f"[profile_run] {a.arch} b{a.batch}"
                  f"{' s' + str(a.seq) if a.seq else ''}: {len(ops)} ops per pass, "
                  f"{dt * 1e3:.3f} ms per pass ({'graph' if a.graph else 'eager'})", flush=True)
        if a.copy_calibration_mb > 0:
            n = a.copy_calibration_mb * (1 << 20) // 4
            src, dst = ctx.empty(n), ctx.empty(n)
            ctx.fill_random(src, 1, 1, "uniform", -1.0, 1.0)
            ctx.launch("reshape", src, None, dst, [n])
            ctx.sync()
            print(f"[profile_run] calibration copy of {a.copy_calibration_mb} MiB", flush=True)
            src.free()
            dst.free()
    return 0


if __name__ == "__main__":
    sys.exit(main())
