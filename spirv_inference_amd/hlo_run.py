"""Command-line runner for XLA HLO text modules on the device (the reference's xla_hlo CLI).

Same flags as source/xla_hlo/src/main.rs:14-70 and a report of the same shape
(:95-114: status, op_histogram, validation, execution, validate_only), but the module runs
on resident device tensors: compiled by spirv_inference_amd.hlo_program (views, fused
epilogues and row kernels, one launch list) by default, or op by op through
spirv_inference_amd.hlo_exec with --op-by-op (the reference's own lowering, one kernel per op).

    python -m spirv_inference_amd.hlo_run --input model.txt --run \\
        --inputs-f32 p0.raw.f32,p1.raw.f32 --output-f32 out.raw.f32 \\
        --expected-f32 want.raw.f32 --epsilon 1e-4 --report report.json

Parity uses the reference's comparator (tflite_loader/src/tensor.rs:28-54): a value is a
mismatch when |actual - expected| > epsilon; the relative error divides by
max(|expected|, 1e-30); a length difference counts as that many mismatches.
`--kernel-dir` is accepted for compatibility and ignored (the kernels are compiled in).
"""
from __future__ import annotations

import argparse
import hashlib
import json
import pathlib
import sys
import time
from collections import Counter

import numpy as np

from . import hlo_exec as X
from .weights import read_raw_f32

SUPPORTED = set(X.ELEMENTWISE) | set(X.ALIASES) | {
    "parameter", "constant", "broadcast", "broadcast_in_dim", "transpose", "slice",
    "concatenate", "compare", "select", "pad", "convolution", "dot", "dot_general", "reduce",
    "reduce-window"}


def compare(actual: np.ndarray, expected: np.ndarray, epsilon: float) -> dict:
    """tensor.rs:28-54 compare."""
    n = min(actual.size, expected.size)
    a, e = actual[:n].astype(np.float32), expected[:n].astype(np.float32)
    ab = np.abs(a - e)
    rel = ab / np.maximum(np.abs(e), np.float32(1e-30))
    return {"mismatch_count": int((ab > epsilon).sum()) + abs(actual.size - expected.size),
            "max_abs_error": float(ab.max()) if n else 0.0,
            "max_rel_error": float(rel.max()) if n else 0.0}


def validate(ops) -> dict:
    bad = sorted({op.opcode for op in ops if op.opcode not in SUPPORTED})
    if bad:
        return {"status": "blocked_unsupported_feature",
                "reason": "unsupported HLO ops: " + ", ".join(bad)}
    return {"status": "pass"}


def run(ops, inputs: list[pathlib.Path], output: pathlib.Path | None,
        expected: pathlib.Path | None, epsilon: float, device: str,
        op_by_op: bool = False) -> dict:
    from .hlo_program import HloProgram
    from .runtime import Context
    params = [np.asarray(read_raw_f32(p)) for p in inputs]
    with Context(device) as ctx:
        t0 = time.perf_counter()
        if op_by_op:
            ex = X.HloExecutor(X.DeviceBackend(ctx), ops)
            out, shape = ex.run(params)
            ctx.sync()
            y = out.download()
            steps = len(ex.record)
        else:
            prog = HloProgram(X.DeviceBackend(ctx), ops, params)
            prog.run()
            ctx.sync()
            y = prog.read(0).reshape(-1)
            shape = prog.outputs()[0][1]
            steps = len(prog.launches)
            prog.close()
        ms = (time.perf_counter() - t0) * 1e3
        dev = {"name": ctx.device_name, "vendor_id": ctx.vendor_id, "device_id": ctx.device_id}
    if output is not None:
        output.parent.mkdir(parents=True, exist_ok=True)
        y.astype("<f4").tofile(output)
    res = {"status": "pass", "steps": steps, "mode": "op_by_op" if op_by_op else "compiled",
           "output_shape": list(shape),
           "output": {"path": str(output) if output else None, "elements": int(y.size),
                      "sha256": hashlib.sha256(y.astype("<f4").tobytes()).hexdigest()},
           "device": dev, "elapsed_ms": ms}
    if expected is not None:
        cmp = compare(y, np.asarray(read_raw_f32(expected)), epsilon)
        res["parity"] = {"status": "pass" if cmp["mismatch_count"] == 0 else "fail",
                         "epsilon": epsilon, **cmp}
        if cmp["mismatch_count"]:
            res["status"] = "fail"
    else:
        res["parity"] = {"status": "not_requested"}
    return res


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--input", required=True, type=pathlib.Path)
    ap.add_argument("--report", type=pathlib.Path)
    ap.add_argument("--validate-only", action="store_true")
    ap.add_argument("--run", action="store_true")
    ap.add_argument("--kernel-dir")
    ap.add_argument("--device", default="any")
    ap.add_argument("--input-f32", type=pathlib.Path)
    ap.add_argument("--input1-f32", type=pathlib.Path)
    ap.add_argument("--inputs-f32", default="")
    ap.add_argument("--output-f32", type=pathlib.Path)
    ap.add_argument("--expected-f32", type=pathlib.Path)
    ap.add_argument("--epsilon", type=float, default=1e-4)
    ap.add_argument("--op-by-op", action="store_true",
                    help="one kernel per HLO op (the reference's lowering) instead of compiling")
    a = ap.parse_args(argv)
    ops = X.parse_hlo_text(a.input.read_text())
    validation = validate(ops)
    execution = {"status": "not_requested"}
    if a.run and not a.validate_only:
        inputs = [pathlib.Path(p) for p in a.inputs_f32.split(",") if p]
        if not inputs:
            if a.input_f32 is None:
                ap.error("--run requires --input-f32 or --inputs-f32")
            inputs = [a.input_f32] + ([a.input1_f32] if a.input1_f32 else [])
        if validation["status"] != "pass":
            execution = {"status": "blocked", "reason": validation["reason"]}
        else:
            execution = run(ops, inputs, a.output_f32, a.expected_f32, a.epsilon, a.device,
                            a.op_by_op)
    status = execution["status"] if execution["status"] in ("pass", "fail") else validation["status"]
    report = {"status": status, "input": str(a.input), "op_histogram": dict(Counter(o.opcode for o in ops)),
              "validation": validation, "execution": execution, "validate_only": a.validate_only}
    text = json.dumps(report, indent=2)
    if a.report:
        a.report.parent.mkdir(parents=True, exist_ok=True)
        a.report.write_text(text + "\n")
    print(text)
    return 0 if status != "fail" else 1


if __name__ == "__main__":
    sys.exit(main())
