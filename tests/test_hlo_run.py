"""The HLO runner's report against the reference's own (CPU: the walk runs on the oracle
backend, so no GPU is needed).

Pins, from source/xla_hlo/reports/resnet50_local_c6_report.json (extracted to
tests/golden/hlo/resnet50_report.json.gz by tests/golden/collect_hlo_fixtures.py):
* the report's key layout (main.rs:95-114, compiler.rs:652-667) is contained in ours;
* the `module` dump of resnet50.stablehlo.txt equals the reference's op for op (parser.rs
  result / opcode / operands / result_type / element_type / shape / attributes / raw);
* the op histogram, the final result, and the op-by-op walk's steps as (result, opcode,
  elements) equal the reference's;
* every reference dispatch has a launch of the same kernel for the same result.
Also: main.rs's defaults (epsilon 1e-6, report path), the NaN trace line of
compiler.rs:613-623, and parity.expected_sha256.
"""
import gzip
import hashlib
import json
import pathlib

import numpy as np
import pytest

from hlo_ref import HLO_DIR, OracleBackend, fixture_text, seeded_params
from spirv_inference_amd import hlo_exec as X
from spirv_inference_amd import hlo_run


@pytest.fixture(scope="module")
def ref_report():
    with gzip.open(HLO_DIR / "resnet50_report.json.gz", "rt") as f:
        return json.load(f)


class TimedOracle(OracleBackend):
    """The oracle backend with host-clock launch timing, standing in for the device's
    hipEvent timing."""

    def __init__(self):
        self._on, self._log = False, []

    def timing(self, enable):
        self._on = enable

    def timing_reset(self):
        self._log = []

    def timing_launches(self):
        return list(self._log)

    def launch(self, kernel, *a, **kw):
        import time
        t0 = time.perf_counter()
        super().launch(kernel, *a, **kw)
        if self._on:
            self._log.append((kernel, (time.perf_counter() - t0) * 1e3))


DEV = {"name": "oracle", "vendor_id": 0, "device_id": 0, "probe_elapsed_ms": 0.0,
       "probe_output": [3.0]}


def _contains(ours, ref, path="report"):
    """Every key of the reference layout exists in ours, recursively."""
    if isinstance(ref, dict):
        assert isinstance(ours, dict), path
        for k, v in ref.items():
            assert k in ours, f"{path}.{k} missing"
            _contains(ours[k], v, f"{path}.{k}")
    elif isinstance(ref, list) and ref:
        assert isinstance(ours, list) and ours, path
        _contains(ours[0], ref[0], f"{path}[0]")


def test_module_dump_equals_reference(ref_report):
    text = fixture_text("resnet50")
    ops = X.parse_hlo_text(text)
    mod = hlo_run.module_json(text, ops)
    ref = ref_report["module"]
    assert mod["name"] == ref["name"]
    assert len(mod["ops"]) == len(ref["ops"])
    for i, (a, b) in enumerate(zip(mod["ops"], ref["ops"])):
        assert a == b, f"op {i}: {a} != {b}"


@pytest.fixture(scope="module")
def resnet_run(tmp_path_factory, ref_report):
    tmp = tmp_path_factory.mktemp("hlo_run")
    text = fixture_text("resnet50")
    (tmp / "m.txt").write_text(text)
    ops = X.parse_hlo_text(text)
    params = seeded_params(ops)
    paths = []
    for i, p in enumerate(params):
        paths.append(tmp / f"p{i:03d}.raw.f32")
        p.astype("<f4").tofile(paths[-1])
    reports = {}
    for mode in ("op_by_op", "compiled"):
        reports[mode] = hlo_run.run(ops, paths, tmp / f"{mode}.raw.f32", None, 1e-6, "any",
                                    op_by_op=mode == "op_by_op", backend=TimedOracle(),
                                    device_info=DEV)
    return ops, paths, reports


def test_report_layout_contains_reference(resnet_run, ref_report):
    ops, _, reports = resnet_run
    text = fixture_text("resnet50")
    for mode, ex in reports.items():
        # the reference's run compared against an expected file: parity with
        # expected_sha256 is pinned in test_nan_trace_lines; here the rest of the layout
        ex = dict(ex, parity={"status": "pass", "epsilon": 0.0, "mismatch_count": 0,
                              "max_abs_error": 0.0, "max_rel_error": 0.0, "expected_sha256": ""})
        report = hlo_run.build_report("m.txt", text, ops, {"status": "pass"}, ex, False)
        _contains(report, ref_report["skeleton"])
        assert ex["mode"] == ref_report["mode"] and ex["final_result"] == ref_report["final_result"]
        assert ex["dispatch_count"] == len(ex["dispatches"]) > 0
        assert all(d["elapsed_ms"] is not None and d["elapsed_ms"] >= 0 for d in ex["dispatches"])


def test_histogram_and_steps_equal_reference(resnet_run, ref_report):
    ops, _, reports = resnet_run
    from collections import Counter
    assert dict(Counter(o.opcode for o in ops)) == ref_report["op_histogram"]
    for mode, ex in reports.items():
        steps = [[s["result"], s["opcode"], s["elements"]] for s in ex["steps"]]
        assert steps == ref_report["steps"], mode
    # the op-by-op walk launches every kernel the reference dispatched, for the same result
    launched = {}
    for d in reports["op_by_op"]["dispatches"]:
        launched.setdefault(d["result"], []).append(d["spv_name"])
    for result, opcode, spv, elements in ref_report["dispatches"]:
        assert spv.removesuffix(".spv") in launched.get(result, []), (result, spv)


def test_parameter_steps_name_their_files(resnet_run):
    ops, paths, reports = resnet_run
    for mode, ex in reports.items():
        s = next(s for s in ex["steps"] if s["opcode"] == "parameter")
        assert s["execution"].startswith("loaded parameter(") and str(paths[0].parent) in s["execution"]


def test_compiled_and_op_by_op_agree(resnet_run):
    _, _, reports = resnet_run
    a = reports["compiled"]["output"]
    b = reports["op_by_op"]["output"]
    assert a["elements"] == b["elements"] == 1000
    ya = np.fromfile(a["path"], "<f4")
    yb = np.fromfile(b["path"], "<f4")
    assert np.abs(ya - yb).max() <= 1e-4 * np.abs(yb).max() + 1e-6
    # the compiled program fuses: fewer launches than the op-by-op walk
    assert reports["compiled"]["dispatch_count"] < reports["op_by_op"]["dispatch_count"]


NAN_MOD = """HloModule nanmod
ENTRY %main (p0: f32[2,3]) -> f32[2,3] {
  %p0 = f32[2,3]{1,0} parameter(0)
  %l = f32[2,3]{1,0} log(f32[2,3]{1,0} %p0)
  %e = f32[2,3]{1,0} exponential(f32[2,3]{1,0} %l)
  ROOT %a = f32[2,3]{1,0} add(f32[2,3]{1,0} %e, f32[2,3]{1,0} %p0)
}
"""


@pytest.mark.parametrize("op_by_op", [True, False])
def test_nan_trace_lines(tmp_path, capsys, op_by_op):
    """compiler.rs:613-623: one stderr line per op whose result holds NaN values, with the
    count, the first index and the shape; log of a negative value is NaN and propagates."""
    x = np.float32([1.0, -2.0, 3.0, 4.0, -0.5, 6.0])
    x.tofile(tmp_path / "x.raw.f32")
    (x * 0 + 7).astype("<f4").tofile(tmp_path / "want.raw.f32")
    ops = X.parse_hlo_text(NAN_MOD)
    ex = hlo_run.run(ops, [tmp_path / "x.raw.f32"], None, tmp_path / "want.raw.f32", 1e-6,
                     "any", op_by_op=op_by_op, backend=TimedOracle(), device_info=DEV)
    err = capsys.readouterr().err.strip().splitlines()
    assert err == [
        "NaN TRACE: %l (log) produced 2/6 NaN values (first at index 1), shape=[2, 3]",
        "NaN TRACE: %e (exponential) produced 2/6 NaN values (first at index 1), shape=[2, 3]",
        "NaN TRACE: %a (add) produced 2/6 NaN values (first at index 1), shape=[2, 3]"]
    assert ex["status"] == "fail"
    assert ex["parity"]["expected_sha256"] == hashlib.sha256(
        (tmp_path / "want.raw.f32").read_bytes()).hexdigest()


def test_defaults_follow_main_rs():
    assert hlo_run.DEFAULT_EPSILON == np.float32(1e-6)
    assert str(hlo_run.DEFAULT_REPORT) == "xla_hlo/reports/hlo_report.json"


def test_oracle_nan_count(orc):
    x = np.float32([0, np.nan, 1, np.nan, np.inf])
    c = orc.run("nan_count", x, None, 2, [5]).view(np.int32)
    assert list(c) == [2, 1]
    c = orc.run("nan_count", np.float32([1, 2]), None, 2, [2]).view(np.int32)
    assert list(c) == [0, -1]
