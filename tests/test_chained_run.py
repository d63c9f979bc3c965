"""The chained-runtime counterpart on the CPU: its comparator and ULP distance against the
reference's definitions (runtime/chained_graph_runtime/src/main.rs:774-819), and the oracle's
restatement of the chain against float64 numpy, which pins the expected edges the GPU run is
checked against."""
import struct

import numpy as np
import pytest

from chained_fixture import inputs, numpy_chain, oracle_chain
from spirv_inference_amd import chained_run as CR


def rust_ulp(a: float, b: float) -> int:
    """main.rs:809-819 line by line on Python ints."""
    def ordered(v):
        bits = struct.unpack("<i", struct.pack("<f", v))[0]
        return -2 ** 31 - bits if bits < 0 else bits
    return abs(ordered(a) - ordered(b))


@pytest.mark.parametrize("a,b", [(0.0, -0.0), (1.0, np.nextafter(np.float32(1), np.float32(2))),
                                 (1.0, -1.0), (-2.5, -2.5000002), (1e-38, -1e-38),
                                 (3.4e38, 1.0), (0.1, 0.1)])
def test_ulp_distance_is_the_references(a, b):
    a32, b32 = np.float32(a), np.float32(b)
    assert int(CR.ulp_distance(np.array([a32]), np.array([b32]))[0]) == \
        rust_ulp(float(a32), float(b32))


def test_compare_edge_counts_and_fails_on_length():
    e = np.linspace(-1, 1, 256).astype(np.float32)
    a = e.copy()
    a[[3, 70]] += np.float32(2e-4)
    a[100] = np.nextafter(e[100], np.float32(9))
    r = CR.compare_edge(a, e, 1e-4, "x")
    assert r["mismatch_count"] == 2
    assert r["max_ulp_error"] >= 1 and abs(r["max_abs_error"] - 2e-4) < 1e-6
    with pytest.raises(ValueError, match="length"):
        CR.compare_edge(a[:-1], e, 1e-4, "x")


def test_oracle_chain_matches_float64():
    x, f, bn = inputs()
    o, n = oracle_chain(x, f, bn), numpy_chain(x, f, bn)
    for k in CR.EDGES:
        np.testing.assert_allclose(o[k], n[k], rtol=1e-5, atol=1e-6, err_msg=k)
    assert (o["relu_output"] == 0).any() and (o["relu_output"] > 0).any()
    assert abs(float(o["softmax_output"].sum()) - 1.0) < 1e-5


def test_cli_fails_on_an_unreadable_spv_path(tmp_path, capsys):
    """main.rs:109-120: a --*-spv path that cannot be read ends the run with an error naming
    it, before any device work and without a report."""
    from chained_fixture import write_manifest
    manifest = write_manifest(tmp_path)
    ok = tmp_path / "ok.spv"
    ok.write_bytes(b"\x03\x02\x23\x07")
    missing = tmp_path / "typo" / "relu.spv"
    argv = ["--device", "any", "--conv2d-spv", str(ok), "--batchnorm-spv", str(ok),
            "--relu-spv", str(missing), "--softmax-spv", str(ok),
            "--fixture-manifest", str(manifest), "--report", str(tmp_path / "r.json"),
            "--dump-dir", str(tmp_path / "dump")]
    assert CR.main(argv) == 1
    assert str(missing) in capsys.readouterr().err
    assert not (tmp_path / "r.json").exists()
    assert CR.spv_entry(str(ok))["sha256"] == __import__("hashlib").sha256(ok.read_bytes()).hexdigest()
