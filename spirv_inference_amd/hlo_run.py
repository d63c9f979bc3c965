"""Command-line runner for XLA HLO text modules on the device (the reference's xla_hlo CLI).

Same flags and defaults as source/xla_hlo/src/main.rs:6-70 (`--report` defaults to
xla_hlo/reports/hlo_report.json and is always written, `--epsilon` defaults to 1e-6) and a
report of the same shape (main.rs:95-114: status, input, module, op_histogram, validation,
execution, validate_only; compiler.rs:652-667 for `execution`: mode, final_result, steps,
dispatch_count, dispatches with per-launch elapsed_ms, device, output, parity with
expected_sha256).  The module runs on resident device tensors: compiled by
spirv_inference_amd.hlo_program (views, fused epilogues and row kernels, one launch list)
by default, or op by op through spirv_inference_amd.hlo_exec with --op-by-op (the
reference's own lowering, one kernel per op).

    python -m spirv_inference_amd.hlo_run --input model.txt --run \\
        --inputs-f32 p0.raw.f32,p1.raw.f32 --output-f32 out.raw.f32 \\
        --expected-f32 want.raw.f32 --epsilon 1e-4 --report report.json

Where the report differs from the reference's, it is because the work differs:
* a dispatch is one registry-kernel launch on the HIP stream; `spv_name` holds the kernel's
  registry name (the stem of the reference's `<kernel>.spv`), `elapsed_ms` the hipEvent
  time of that launch;
* a step's `execution` names the device lowering ("hip_<kernel>", "hip_fused_<kind>",
  "fused_into <anchor>", "strided_view", ...) where the reference names a Vulkan or CPU one;
* `execution.engine` says which of the two lowerings ran ("compiled" or "op_by_op").

NaN trace (compiler.rs:613-623): after every op that produces a value on the device, a
`nan_count` launch counts its NaN values on the device; each op with NaN values gets the
reference's `NaN TRACE:` line on stderr.  The counts are untimed.

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
import re
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

DEFAULT_REPORT = pathlib.Path("xla_hlo/reports/hlo_report.json")  # main.rs:8
DEFAULT_EPSILON = 1.0e-6                                            # main.rs:18

# parser.rs:226-244: the attribute keys a module dump lists
_REF_ATTR_KEYS = ("window", "dim_labels", "dimensions", "padding", "lhs_batch_dims",
                  "rhs_batch_dims", "lhs_contracting_dims", "rhs_contracting_dims",
                  "feature_group_count", "batch_group_count", "to_apply", "direction", "index")


def compare(actual: np.ndarray, expected: np.ndarray, epsilon: float) -> dict:
    """tensor.rs:28-54 compare."""
    n = min(actual.size, expected.size)
    a, e = actual[:n].astype(np.float32), expected[:n].astype(np.float32)
    ab = np.abs(a - e)
    rel = ab / np.maximum(np.abs(e), np.float32(1e-30))
    return {"mismatch_count": int((ab > np.float32(epsilon)).sum()) + abs(actual.size - expected.size),
            "max_abs_error": float(ab.max()) if n else 0.0,
            "max_rel_error": float(rel.max()) if n else 0.0}


def validate(ops) -> dict:
    bad = sorted({op.opcode for op in ops if op.opcode not in SUPPORTED})
    if bad:
        return {"status": "blocked_unsupported_feature",
                "reason": "unsupported HLO ops: " + ", ".join(bad)}
    return {"status": "pass"}


# ---- the module dump (main.rs:108 "module": the parsed HloModule, ir.rs HloModule/HloOp) ----
def _attr_value(line: str, key: str) -> str | None:
    """parser.rs:246-256: `{...}`, `"..."`, else up to the first ',' of the rest of the line
    (or its first ' ' when it has no ',')."""
    i = line.find(key + "=")
    if i < 0:
        return None
    rest = line[i + len(key) + 1:]
    if rest.startswith("{"):
        j = rest.find("}", 1)
        return rest[1:j] if j >= 0 else None
    if rest.startswith('"'):
        j = rest.find('"', 1)
        return rest[1:j] if j >= 0 else None
    j = rest.find(",")
    if j < 0:
        j = rest.find(" ")
    return (rest[:j] if j >= 0 else rest).strip()


def _quoted(line: str, key: str) -> str | None:
    """parser.rs:258-264 parse_quoted_attr."""
    i = line.find(key + '="')
    if i < 0:
        return None
    rest = line[i + len(key) + 2:]
    j = rest.find('"')
    return rest[:j] if j >= 0 else None


def ref_attributes(line: str) -> dict:
    """parser.rs:226-244 parse_attributes, including the metadata op_type / op_name."""
    out = {}
    for k in _REF_ATTR_KEYS:
        v = _attr_value(line, k)
        if v is not None:
            out[k] = v
    if "metadata={" in line:
        for k in ("op_type", "op_name"):
            v = _quoted(line, k)
            if v is not None:
                out["metadata." + k] = v
    return dict(sorted(out.items()))


def _element_type(rtype: str | None) -> str | None:
    """parser.rs:196-205: the text before '[' unless empty or a tuple type."""
    if not rtype:
        return None
    et = rtype.strip().split("[", 1)[0].strip()
    return et if et and not et.startswith("(") else None


def module_json(text: str, ops) -> dict:
    return {"name": X.module_name(text),
            "ops": [{"attributes": ref_attributes(op.raw),
                     "element_type": _element_type(op.result_type),
                     "opcode": op.opcode, "operands": list(op.operands), "raw": op.raw,
                     "result": op.result, "result_type": op.result_type,
                     "shape": list(op.shape)} for op in ops]}


# ---- execution ----------------------------------------------------------------------------
def _count_nan(backend, slots, k: int, tensor, n: int) -> None:
    """Enqueue the NaN count of tensor[0, n) into slot k (two int32 words)."""
    backend.launch("nan_count", tensor, None, backend.sub(slots, 2 * k, 2), [int(n)],
                   out_elems=2)


def _nan_lines(counts: np.ndarray, traced: list) -> list[str]:
    """compiler.rs:613-623's message for every traced value that holds NaN values."""
    c = np.asarray(counts, np.float32).view(np.int32).reshape(-1, 2)
    lines = []
    for k, (result, opcode, n, shape) in enumerate(traced):
        if c[k, 0] > 0:
            lines.append(f"NaN TRACE: {result} ({opcode}) produced {int(c[k, 0])}/{n} NaN "
                         f"values (first at index {int(c[k, 1])}), shape={list(shape)}")
    return lines


def execute(backend, ops, params, op_by_op: bool = False, trace_nan: bool = True) -> dict:
    """Runs the module once on `backend` (DeviceBackend, or any object with its interface);
    returns the output, its shape, the steps, the launches attributed to their HLO results
    and the NaN-trace lines.  When the backend can time launches (timing / timing_reset /
    timing_launches), each dispatch carries its elapsed_ms."""
    timed = all(hasattr(backend, a) for a in ("timing", "timing_reset", "timing_launches"))
    traced: list = []
    slots = backend.empty(2 * (len(ops) + 1))

    def count(result, opcode, tensor, n, shape):
        if not trace_nan:
            return
        if timed:
            backend.timing(False)
        _count_nan(backend, slots, len(traced), tensor, n)
        if timed:
            backend.timing(True)
        traced.append((result, opcode, n, shape))

    if timed:
        backend.timing_reset()
        backend.timing(True)
    t0 = time.perf_counter()
    prog = None
    try:
        if op_by_op:
            ex = X.HloExecutor(backend, ops)

            def on_value(op, tensor, shape):
                count(op.result, op.opcode, tensor, X._n(shape), shape)

            out, shape = ex.run(params, on_value=on_value)
            y = np.asarray(backend.read(out))[:X._n(shape)].copy()
            launched = {r: ks for (r, _oc, ks) in ex.record}
            launches = [(r, k, n) for (r, _oc, ks) in ex.record for (k, n) in ks]
            steps = _executor_steps(ops, launched)
        else:
            from .hlo_program import HloProgram
            prog = HloProgram(backend, ops, params)
            last = {}
            for i, src in enumerate(prog.launch_src):
                last[src] = i
            ends = {i: src for src, i in last.items()}
            opcode_of = {op.result: op.opcode for op in ops}
            shape_of = {op.result: op.shape for op in ops}

            def after(i):
                if i in ends:
                    src = ends[i]
                    l = prog.launches[i]
                    n = l[9] if l[9] is not None else X._n(shape_of.get(src, [1]))
                    count(src, opcode_of.get(src, "?"), l[3], n, shape_of.get(src, [n]))

            prog.run_traced(after)
            y = np.asarray(prog.read(0)).reshape(-1).copy()
            shape = prog.outputs()[0][1]
            launches = [(src, l[0], l[9]) for l, src in zip(prog.launches, prog.launch_src)]
            steps = prog.steps()
        counts = np.asarray(backend.read(slots)).copy()
    finally:
        if prog is not None:
            prog.close()
        backend.free(slots)
    wall_ms = (time.perf_counter() - t0) * 1e3
    times = backend.timing_launches() if timed else []
    if timed:
        backend.timing(False)
    return {"output": y, "shape": list(shape), "steps": steps, "launches": launches,
            "times": times, "nan": _nan_lines(counts, traced), "wall_ms": wall_ms}


_EXEC_NAMES = {"broadcast": "hip_shaped_broadcast", "broadcast_in_dim": "hip_shaped_broadcast",
               "transpose": "hip_transpose", "pad": "hip_pad",
               "convolution": "hip_convolution_nhwc_hwio", "reduce-window": "hip_reduce_window",
               "dot": "hip_dot_general", "dot_general": "hip_dot_general",
               "compare": "hip_compare_predicate_as_f32", "select": "hip_select",
               "concatenate": "hip_concatenate", "slice": "hip_slice"}


def _executor_steps(ops, launched: dict) -> list[dict]:
    """Steps of the op-by-op walk, named like compiler.rs:267-611's with the device in place
    of Vulkan / the host CPU."""
    out = []
    for op in ops:
        ks = launched.get(op.result, [])
        oc = op.opcode
        if oc == "parameter":
            ex = "uploaded parameter"
        elif oc == "constant":
            ex = "materialized scalar constant"
        elif oc in ("reshape", "convert"):
            ex = "metadata_reshape"
        elif oc in ("tuple", "get-tuple-element"):
            ex = "tuple_alias"
        elif oc == "reduce":
            ex = "hip_reduce_rank5" if ks and ks[-1][0] == "hlo_reduce" else "hip_reduce"
        elif oc in _EXEC_NAMES:
            ex = _EXEC_NAMES[oc]
        else:
            ex = "hip_elementwise"
        out.append({"result": op.result, "opcode": oc, "execution": ex,
                    "elements": X._n(op.shape), "spv_name": ks[-1][0] if ks else None})
    return out


def run(ops, inputs: list[pathlib.Path], output: pathlib.Path | None,
        expected: pathlib.Path | None, epsilon: float, device: str,
        op_by_op: bool = False, backend=None, device_info: dict | None = None) -> dict:
    """compiler.rs:267-668 run_graph's report on this build's device.  `backend` and
    `device_info` replace the HIP context (a test passes a checker backend here)."""
    params = [np.asarray(read_raw_f32(p)) for p in inputs]
    n_params = sum(1 for op in ops if op.opcode == "parameter")
    if len(params) < n_params:
        raise ValueError(f"missing --inputs-f32 entry for parameter({len(params)}): "
                         f"{n_params} parameters, {len(params)} inputs")
    ctx = None
    if backend is None:
        from .runtime import Context
        ctx = Context(device)
        backend = _TimedDeviceBackend(ctx)
        device_info = probe_device(ctx)
    try:
        r = execute(backend, ops, params, op_by_op=op_by_op)
    finally:
        if ctx is not None:
            ctx.close()
    dev = device_info or {}
    for s in r["steps"]:
        if s["opcode"] == "parameter":
            m = re.search(r"parameter\((\d+)\)", next(o.raw for o in ops if o.result == s["result"]))
            if m and int(m.group(1)) < len(inputs):
                s["execution"] = f"loaded parameter({m.group(1)}) from {inputs[int(m.group(1))]}"
    for line in r["nan"]:
        print(line, file=sys.stderr)
    times = r["times"]
    if times and len(times) != len(r["launches"]):
        raise RuntimeError(f"{len(times)} timed launches for {len(r['launches'])} recorded")
    opcode_of = {op.result: op.opcode for op in ops}
    dispatches = []
    for k, (src, kernel, n) in enumerate(r["launches"]):
        dispatches.append({"device_id": dev.get("device_id"), "device_name": dev.get("name"),
                           "elapsed_ms": times[k][1] if times else None,
                           "elements": n, "opcode": opcode_of.get(src), "result": src,
                           "spv_name": kernel, "vendor_id": dev.get("vendor_id")})
    y = r["output"]
    if output is not None:
        output.parent.mkdir(parents=True, exist_ok=True)
        y.astype("<f4").tofile(output)
    res = {"status": "pass", "mode": "shaped_hlo_graph",
           "engine": "op_by_op" if op_by_op else "compiled",
           "final_result": ops[-1].result if ops else None,
           "steps": r["steps"], "dispatch_count": len(dispatches), "dispatches": dispatches,
           "device": dev,
           "output": {"path": str(output) if output else None, "elements": int(y.size),
                      "shape": r["shape"],
                      "sha256": hashlib.sha256(y.astype("<f4").tobytes()).hexdigest()},
           "elapsed_ms": r["wall_ms"]}
    if expected is not None:
        raw = pathlib.Path(expected).read_bytes()
        cmp = compare(y, np.asarray(read_raw_f32(expected)), epsilon)
        res["parity"] = {"status": "pass" if cmp["mismatch_count"] == 0 else "fail",
                         "epsilon": epsilon, **cmp,
                         "expected_sha256": hashlib.sha256(raw).hexdigest()}
        if cmp["mismatch_count"]:
            res["status"] = "fail"
    else:
        res["parity"] = {"status": "not_requested"}
    return res


def probe_device(ctx) -> dict:
    """compiler.rs:1954-1977 probe_vulkan_device: one `add` of [1] + [2] through the
    host-to-host drop-in (shp_run_kernel), reported with the device identity."""
    from .runtime import KernelRun
    out = ctx.run_kernel(KernelRun("xla_hlo_device_probe_add", "add", np.float32([1.0]),
                                   np.float32([2.0]), 1, 1, [1]))
    return {"name": out.device_name, "vendor_id": out.vendor_id, "device_id": out.device_id,
            "probe_elapsed_ms": out.elapsed_ms, "probe_output": [float(v) for v in out.values]}


class _TimedDeviceBackend(X.DeviceBackend):
    """DeviceBackend with the context's per-launch hipEvent timing exposed to execute()."""

    def timing(self, enable: bool) -> None:
        self.ctx.timing(enable)

    def timing_reset(self) -> None:
        self.ctx.timing_reset()

    def timing_launches(self) -> list:
        return self.ctx.timing_launches()


def build_report(input_path, text: str, ops, validation: dict, execution: dict,
                 validate_only: bool) -> dict:
    """main.rs:95-114: the top level of the report."""
    status = execution["status"] if execution["status"] in ("pass", "fail") else validation["status"]
    return {"status": status, "input": str(input_path), "module": module_json(text, ops),
            "op_histogram": dict(sorted(Counter(o.opcode for o in ops).items())),
            "validation": validation, "execution": execution, "validate_only": validate_only}


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--input", required=True, type=pathlib.Path)
    ap.add_argument("--report", type=pathlib.Path, default=DEFAULT_REPORT)
    ap.add_argument("--validate-only", action="store_true")
    ap.add_argument("--run", action="store_true")
    ap.add_argument("--kernel-dir")
    ap.add_argument("--device", default="any")
    ap.add_argument("--input-f32", type=pathlib.Path)
    ap.add_argument("--input1-f32", type=pathlib.Path)
    ap.add_argument("--inputs-f32", default="")
    ap.add_argument("--output-f32", type=pathlib.Path)
    ap.add_argument("--expected-f32", type=pathlib.Path)
    ap.add_argument("--epsilon", type=float, default=DEFAULT_EPSILON)
    ap.add_argument("--op-by-op", action="store_true",
                    help="one kernel per HLO op (the reference's lowering) instead of compiling")
    a = ap.parse_args(argv)
    text = a.input.read_text()
    ops = X.parse_hlo_text(text)
    validation = validate(ops)
    execution = {"status": "not_requested"}
    # main.rs:88-104: --run executes even with --validate-only (which is only recorded)
    if a.run:
        inputs = [pathlib.Path(p) for p in a.inputs_f32.split(",") if p]
        if not inputs:
            if a.input_f32 is None:
                ap.error("--run requires --input-f32 or --inputs-f32")
            inputs = [a.input_f32] + ([a.input1_f32] if a.input1_f32 else [])
        if validation["status"] != "pass":
            # run_graph starts with validate_supported (compiler.rs:276) and fails there
            print(f"error: {validation['reason']}", file=sys.stderr)
            return 1
        execution = run(ops, inputs, a.output_f32, a.expected_f32, a.epsilon, a.device,
                        a.op_by_op)
    report = build_report(a.input, text, ops, validation, execution, a.validate_only)
    out = json.dumps(report, indent=2)
    a.report.parent.mkdir(parents=True, exist_ok=True)
    a.report.write_text(out + "\n")
    print(out)
    # main.rs:112-114 returns Ok(()) once the report is written, a failed parity included:
    # callers read the status from the report
    return 0


if __name__ == "__main__":
    sys.exit(main())
