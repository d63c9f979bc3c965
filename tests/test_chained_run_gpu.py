"""The chained-runtime counterpart on the device: main.rs's flags and report, the four stages on
resident tensors (eager and from one hipGraph), every edge within the fixture's epsilon of the
oracle's chain; a corrupted expected edge fails that edge only."""
import json

import numpy as np
import pytest

from chained_fixture import inputs, oracle_chain, write_manifest
from spirv_inference_amd import chained_run as CR

pytestmark = pytest.mark.gpu


def _cli(tmp_path, manifest, graph=False):
    # main.rs:109-120 reads the four shader files before running; their bytes are only
    # recorded here, so any readable file stands in for them
    spv = {}
    for k in ("conv2d", "batchnorm", "relu", "softmax"):
        spv[k] = tmp_path / f"{k}.spv"
        spv[k].write_bytes(k.encode())
    argv = ["--device", "any", "--conv2d-spv", str(spv["conv2d"]),
            "--batchnorm-spv", str(spv["batchnorm"]), "--relu-spv", str(spv["relu"]),
            "--softmax-spv", str(spv["softmax"]), "--fixture-manifest", str(manifest),
            "--report", str(tmp_path / "report.json"), "--dump-dir", str(tmp_path / "dump")]
    rc = CR.main(argv + (["--graph"] if graph else []))
    return rc, json.loads((tmp_path / "report.json").read_text())


@pytest.mark.parametrize("graph", [False, True])
def test_chained_cli_passes(tmp_path, graph):
    print(f"[chained] graph={graph}", flush=True)
    rc, rep = _cli(tmp_path, write_manifest(tmp_path), graph)
    assert rc == 0 and rep["status"] == "pass", rep["edges"]
    assert rep["device"]["vendor_id"] == "0x1002"
    assert set(rep["edges"]) == set(CR.EDGES)
    assert rep["max_abs_error"] <= 1e-4
    for e, r in rep["edges"].items():
        dumped = np.fromfile(r["dump_path"], "<f4")
        assert dumped.size == CR.ELEMENTS and r["mismatch_count"] == 0, e
    print(f"[chained] max abs {rep['max_abs_error']:.2e}, max ulp {rep['max_ulp_error']}",
          flush=True)


def test_chained_cli_reports_a_bad_edge(tmp_path):
    x, f, bn = inputs()
    edges = oracle_chain(x, f, bn)
    edges["relu_output"] = edges["relu_output"].copy()
    edges["relu_output"][[5, 200]] += np.float32(1e-2)
    rc, rep = _cli(tmp_path, write_manifest(tmp_path, edges=edges))
    assert rc == 1 and rep["status"] == "fail"
    assert rep["edges"]["relu_output"]["mismatch_count"] == 2
    assert rep["mismatch_count"] == 2
