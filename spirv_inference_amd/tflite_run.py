"""tflite_run: the tflite_loader command line (source/tflite_loader/src/main.rs) on the device.

    python -m spirv_inference_amd.tflite_run [--self-test-kernels] [--model MODEL.tflite]
        [--input-f32 input.raw.f32] [--inspect-only] [--device any|amd|<ordinal>]
        [--report out.json] [--dump-dir dir]

Same flags and report shape as main.rs:18-138: `status` pass / fail /
blocked_unsupported_feature, `sections` {kernel_self_test, model, graph_validation,
execution}, `non_claims`.  `--kernel-dir` is accepted and ignored (kernels are compiled into
the library, chosen by the reference's names).  The kernel self-test is engine.rs:15-200's
eight-element known-answer test, through the host-to-host `run_kernel` entry; the model run
keeps every tensor on the device (TfliteExecutor) and writes the output tensors to --dump-dir.
"""
from __future__ import annotations

import argparse
import hashlib
import json
import os
import sys

import numpy as np

from . import tflite
from .runtime import Context, KernelRun, f32_bits

KAT_INPUT = np.array([0.25, 0.5, 0.75, 1.0, 1.25, 2.0, 3.0, 4.0], np.float32)


def _kat_cases():
    x, r, f = KAT_INPUT, np.full(8, 2.0, np.float32), np.float32
    ep, en = np.exp(x), np.exp(-x)
    return [
        ("abs", [8], None, np.abs(x)), ("exp", [8], None, np.exp(x)),
        ("log", [8], None, np.log(x)), ("neg", [8], None, -x), ("sqrt", [8], None, np.sqrt(x)),
        ("rsqrt", [8], None, (f(1) / np.sqrt(x)).astype(f)),
        ("sub", [8], r, x - r), ("mul", [8], r, x * r), ("div", [8], r, x / r),
        ("pow", [8], r, np.power(x, r)), ("min", [8], r, np.minimum(x, r)),
        ("max", [8], r, np.maximum(x, r)),
        ("leaky_relu", [8, f32_bits(0.1)], None, np.maximum(x, f(0.1) * x)),
        ("sigmoid", [8], None, (f(1) / (f(1) + np.exp(-x))).astype(f)),
        ("tanh", [8], None, ((ep - en) / (ep + en)).astype(f)),
    ]


def compare(actual, expected, eps):
    """tensor.rs:28-54: mismatch iff |a - e| > eps; relative error against max(|e|, 1e-30)."""
    a = np.asarray(actual, np.float32).reshape(-1)
    e = np.asarray(expected, np.float32).reshape(-1)
    n = min(a.size, e.size)
    d = np.abs(a[:n].astype(np.float64) - e[:n])
    rel = d / np.maximum(np.abs(e[:n].astype(np.float64)), 1e-30)
    return {"mismatch_count": int((d > eps).sum()) + abs(a.size - e.size),
            "max_abs_error": float(d.max()) if n else 0.0,
            "max_rel_error": float(rel.max()) if n else 0.0, "epsilon": eps}


def kernel_self_test(ctx: Context, dump_dir: str) -> dict:
    os.makedirs(dump_dir, exist_ok=True)
    cases, mism = [], 0
    for name, push, rhs, expected in _kat_cases():
        out = ctx.run_kernel(KernelRun(name, name, KAT_INPUT,
                                       rhs if rhs is not None else np.zeros(8, np.float32), 8,
                                       1, push))
        out.values.astype("<f4").tofile(os.path.join(dump_dir, f"{name}.raw.f32"))
        c = compare(out.values, expected, 1e-5)
        mism += c["mismatch_count"]
        cases.append({"name": name, "kernel": name, "elapsed_ms": out.elapsed_ms, **c})
    return {"status": "pass" if mism == 0 else "fail", "mismatch_count": mism,
            "device": {"name": ctx.device_name}, "cases": cases}


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--model")
    ap.add_argument("--input-f32")
    ap.add_argument("--kernel-dir", default="kernels", help="accepted for compatibility; unused")
    ap.add_argument("--report", default="tflite_loader/out/tflite_report.json")
    ap.add_argument("--dump-dir", default="tflite_loader/out/tensors")
    ap.add_argument("--device", default="any")
    ap.add_argument("--self-test-kernels", action="store_true")
    ap.add_argument("--inspect-only", action="store_true")
    args = ap.parse_args(argv)
    if not args.self_test_kernels and not args.model:
        ap.error("nothing to do; pass --self-test-kernels and/or --model <path>")
    sections, status = {}, "pass"
    with Context(args.device) as ctx:
        if args.self_test_kernels:
            r = kernel_self_test(ctx, args.dump_dir)
            if r["status"] != "pass":
                status = "fail"
            sections["kernel_self_test"] = r
        if args.model:
            m = tflite.load_model(args.model)
            try:
                gv = tflite.validate_supported_graph(m)
            except ValueError as e:
                status = "blocked_unsupported_feature"
                gv = {"status": "blocked_unsupported_feature", "reason": str(e)}
            sections["model"] = m.summary()
            sections["graph_validation"] = gv
            if not args.inspect_only and status == "pass":
                values, source = None, None
                if args.input_f32:
                    raw = open(args.input_f32, "rb").read()
                    values = np.frombuffer(raw, "<f4")
                    source = {"kind": "cli_input_f32", "path": args.input_f32,
                              "bytes": len(raw), "sha256": hashlib.sha256(raw).hexdigest()}
                try:
                    rep, out = tflite.run_model(ctx, m, values, source)
                    os.makedirs(args.dump_dir, exist_ok=True)
                    out.astype("<f4").tofile(os.path.join(args.dump_dir, "output.raw.f32"))
                    rep["device"] = {"name": ctx.device_name, "vendor_id": 0x1002}
                    sections["execution"] = rep
                except ValueError as e:
                    status = "blocked_unsupported_feature"
                    sections["execution"] = {"status": "blocked_unsupported_feature",
                                             "reason": str(e)}
    report = {"status": status, "crate": "tflite_loader (spirv_inference_amd.tflite_run)",
              "kernel_dir": args.kernel_dir, "input_f32": args.input_f32,
              "dump_dir": args.dump_dir, "sections": sections,
              "non_claims": {"uses_cuda": False, "uses_cublas": False, "uses_cudnn": False,
                             "claims_full_tensorflow_runtime": False}}
    os.makedirs(os.path.dirname(os.path.abspath(args.report)), exist_ok=True)
    with open(args.report, "w") as f:
        json.dump(report, f, indent=2)
    print(json.dumps(report, indent=2))
    return 0 if status == "pass" else 1


if __name__ == "__main__":
    sys.exit(main())
