"""The HLO executor's parser and lowering on the CPU (oracle backend vs float64 numpy).

The reference's own HLO fixtures (tests/golden/hlo) are parsed as parser.rs does and walked
with the executor's lowering on the oracle backend (the registry kernels' CPU restatement);
an independent float64 numpy interpreter with XLA semantics checks the result.  The same
walk on the device backend is checked op by op in test_hlo_exec_gpu.py.
"""
import json

import numpy as np
import pytest

from hlo_ref import HLO_DIR, OracleBackend, eval_numpy, fixture_text, seeded_params
from spirv_inference_amd import hlo_exec as X


def test_fixture_bytes_match_manifest():
    import gzip
    import hashlib
    man = json.loads((HLO_DIR / "manifest.json").read_text())
    for m, rec in man.items():
        data = gzip.open(HLO_DIR / f"{m}.stablehlo.txt.gz").read()
        assert len(data) == rec["bytes"] and hashlib.sha256(data).hexdigest() == rec["sha256"]


@pytest.mark.parametrize("model,n_params,n_conv,n_dot", [("resnet50", 321, 53, 1),
                                                         ("bert_base", 3, 0, 4),
                                                         ("tinyllama", 204, 0, 199)])
def test_parse_entry_like_parser_rs(model, n_params, n_conv, n_dot):
    # parameter counts = the fixtures' --inputs-f32 lists (resnet50_inputs.txt: 321 files,
    # bert_base_inputs.txt: 3, tinyllama_inputs.txt: 204); only the ENTRY computation counts
    ops = X.parse_hlo_text(fixture_text(model))
    assert sum(op.opcode == "parameter" for op in ops) == n_params
    assert sum(op.opcode == "convolution" for op in ops) == n_conv
    assert sum(op.opcode in ("dot", "dot_general") for op in ops) == n_dot
    assert all(op.result.startswith("%") for op in ops)


def run_both(text, params=None, seed=11):
    ops = X.parse_hlo_text(text)
    params = params if params is not None else seeded_params(ops, seed)
    got, shape = X.HloExecutor(OracleBackend(), ops).run(params)
    return got.reshape(shape), eval_numpy(ops, params)


def test_bert_block_fixture():
    got, ref = run_both(fixture_text("bert_base"))
    scale = np.abs(ref).max()
    assert np.isfinite(got).all()
    assert np.abs(got - ref).max() <= 1e-4 * scale + 1e-5, np.abs(got - ref).max() / scale


def test_resnet50_fixture_b1():
    got, ref = run_both(fixture_text("resnet50"))
    assert got.shape == ref.shape == (1, 1000)
    assert np.isfinite(got).all()
    assert int(np.argmax(got)) == int(np.argmax(ref))
    np.testing.assert_allclose(got, ref, rtol=1e-3, atol=1e-6)


SYNTH = """HloModule synth
ENTRY %main (p0: f32[2,3,4], p1: f32[4,5]) -> f32[2,3,5] {
  %p0 = f32[2,3,4]{2,1,0} parameter(0)
  %p1 = f32[4,5]{1,0} parameter(1)
  %s0 = f32[2,3,2]{2,1,0} slice(f32[2,3,4]{2,1,0} %p0), slice={[0:2], [0:3], [0:2]}
  %s1 = f32[2,3,2]{2,1,0} slice(f32[2,3,4]{2,1,0} %p0), slice={[0:2], [0:3], [2:4]}
  %n1 = f32[2,3,2]{2,1,0} negate(f32[2,3,2]{2,1,0} %s1)
  %c = f32[2,3,4]{2,1,0} concatenate(f32[2,3,2]{2,1,0} %n1, f32[2,3,2]{2,1,0} %s0), dimensions={2}
  %z = f32[] constant(0)
  %zb = f32[2,3,4]{2,1,0} broadcast(f32[] %z), dimensions={}
  %gt = pred[2,3,4]{2,1,0} compare(f32[2,3,4]{2,1,0} %c, f32[2,3,4]{2,1,0} %zb), direction=GT
  %sel = f32[2,3,4]{2,1,0} select(pred[2,3,4]{2,1,0} %gt, f32[2,3,4]{2,1,0} %c, f32[2,3,4]{2,1,0} %p0)
  %t = f32[3,2,4]{2,1,0} transpose(f32[2,3,4]{2,1,0} %sel), dimensions={1,0,2}
  %r5 = f32[3,2,1,4,1]{4,3,2,1,0} reshape(f32[3,2,4]{2,1,0} %t)
  %init = f32[] constant(0)
  %red = f32[3,4]{1,0} reduce(f32[3,2,1,4,1]{4,3,2,1,0} %r5, f32[] %init), dimensions={1,2,4}, to_apply=%add
  %d = f32[3,5]{1,0} dot(f32[3,4]{1,0} %red, f32[4,5]{1,0} %p1), lhs_contracting_dims={1}, rhs_contracting_dims={0}
  %b = f32[2,3,5]{2,1,0} broadcast(f32[3,5]{1,0} %d), dimensions={1,2}
  ROOT %e = f32[2,3,5]{2,1,0} exponential(f32[2,3,5]{2,1,0} %b)
}
"""


def test_synthetic_module_covers_host_ops():
    """slice / concatenate / compare / select / transpose / rank-5 reduce / dot / broadcast."""
    got, ref = run_both(SYNTH)
    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-6)


def test_batched_dot_general_with_permuted_operands():
    text = """HloModule d
ENTRY %main (a: f32[4,6,3], b: f32[3,4,5]) -> f32[4,6,5] {
  %a = f32[4,6,3]{2,1,0} parameter(0)
  %b = f32[3,4,5]{2,1,0} parameter(1)
  ROOT %d = f32[4,6,5]{2,1,0} dot(f32[4,6,3]{2,1,0} %a, f32[3,4,5]{2,1,0} %b), lhs_batch_dims={0}, lhs_contracting_dims={2}, rhs_batch_dims={1}, rhs_contracting_dims={0}
}
"""
    got, ref = run_both(text)
    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-6)


def test_cli_validate_only_and_unsupported(tmp_path, capsys, monkeypatch):
    from spirv_inference_amd import hlo_run
    p = tmp_path / "m.txt"
    p.write_text(fixture_text("bert_base"))
    assert hlo_run.main(["--input", str(p), "--validate-only", "--report", str(tmp_path / "r.json")]) == 0
    rep = json.loads((tmp_path / "r.json").read_text())
    assert rep["status"] == "pass" and rep["op_histogram"]["dot"] == 4
    capsys.readouterr()
    q = tmp_path / "g.txt"
    q.write_text(SYNTH.replace("exponential(", "gather("))
    # without --report the report still goes to main.rs:8's default path
    monkeypatch.chdir(tmp_path)
    assert hlo_run.main(["--input", str(q), "--validate-only"]) == 0
    rep = json.loads(capsys.readouterr().out)
    assert rep["status"] == "blocked_unsupported_feature" and "gather" in rep["validation"]["reason"]
    assert json.loads((tmp_path / "xla_hlo/reports/hlo_report.json").read_text()) == rep


def test_cli_compare_follows_tensor_rs():
    from spirv_inference_amd.hlo_run import compare
    c = compare(np.array([1.0, 2.0, 3.0], np.float32), np.array([1.0, 2.5, 3.0, 4.0], np.float32), 0.1)
    # one value off by 0.5 > eps, plus one missing value
    assert c["mismatch_count"] == 2 and c["max_abs_error"] == 0.5 and abs(c["max_rel_error"] - 0.2) < 1e-7
    assert compare(np.zeros(2, np.float32), np.zeros(2, np.float32), 0.0)["mismatch_count"] == 0
