"""The reference's HLO fixtures executed on the device (GPU): every op a registry kernel on
resident tensors (spirv_inference_amd.hlo_exec), against the same lowering on the CPU oracle
and against float64 numpy.  Parameters are seeded (the fixtures' weights are not in the
reference).  Gates: the chained end-to-end outputs within 1e-4 * max|ref| (BERT block) /
1e-3 (ResNet-50 b1, TinyLlama S=64 logits), identical top-1; every intermediate of the BERT
block within 1e-4 of the oracle walk.
"""
import time

import numpy as np
import pytest

from hlo_ref import OracleBackend, eval_numpy, fixture_text, seeded_params
from spirv_inference_amd import hlo_exec as X

pytestmark = pytest.mark.gpu


def device_run(ctx, ops, params, keep=False):
    ex = X.HloExecutor(X.DeviceBackend(ctx), ops)
    t0 = time.perf_counter()
    out, shape = ex.run(params, keep=keep)
    ctx.sync()
    dt = time.perf_counter() - t0
    return ex, out, shape, dt


def test_bert_block_every_op_vs_oracle(ctx):
    ops = X.parse_hlo_text(fixture_text("bert_base"))
    params = seeded_params(ops)
    print(f"[hlo] bert_base block: {len(ops)} ops", flush=True)
    ex, out, shape, dt = device_run(ctx, ops, params, keep=True)
    ox = X.HloExecutor(OracleBackend(), ops)
    ref, _ = ox.run(params, keep=True)
    for name, (t, s) in ex.values.items():
        d, o = t.download(), ox.values[name][0]
        scale = max(np.abs(o).max(), 1e-30)
        assert np.isfinite(d).all(), name
        assert np.abs(d - o).max() <= 1e-4 * scale + 1e-6, (name, np.abs(d - o).max(), scale)
    y = out.download().reshape(shape)
    nref = eval_numpy(ops, params)
    assert np.abs(y - nref).max() <= 1e-4 * np.abs(nref).max() + 1e-5
    print(f"[hlo] bert_base block on device: {dt * 1e3:.1f} ms (host walk included)", flush=True)


def test_resnet50_fixture_b1(ctx):
    ops = X.parse_hlo_text(fixture_text("resnet50"))
    params = seeded_params(ops)
    print(f"[hlo] resnet50 fixture: {len(ops)} ops", flush=True)
    _, out, shape, dt = device_run(ctx, ops, params)
    y = out.download().reshape(shape)
    ref, _ = X.HloExecutor(OracleBackend(), ops).run(params)
    ref = ref.reshape(shape)
    nref = eval_numpy(ops, params)
    assert np.isfinite(y).all()
    assert int(np.argmax(y)) == int(np.argmax(ref)) == int(np.argmax(nref))
    np.testing.assert_allclose(y, ref, rtol=1e-3, atol=1e-6)
    np.testing.assert_allclose(y, nref, rtol=1e-3, atol=1e-6)
    print(f"[hlo] resnet50 fixture on device: {dt * 1e3:.1f} ms (host walk included)", flush=True)


def test_tinyllama_fixture_forward(ctx):
    """The S=64 full-recompute forward (export_llama.py:269-375 graph): 22 layers of
    dot / transpose / slice / concatenate (rotate-half) / reduce / broadcast on the device."""
    ops = X.parse_hlo_text(fixture_text("tinyllama"))
    params = seeded_params(ops)
    print(f"[hlo] tinyllama fixture: {len(ops)} ops, "
          f"{sum(p.size for p in params) * 4 / 1e9:.2f} GB of parameters", flush=True)
    _, out, shape, dt = device_run(ctx, ops, params)
    y = out.download().reshape(shape)
    nref = eval_numpy(ops, params)
    assert np.isfinite(y).all()
    assert (np.argmax(y.reshape(-1, shape[-1]), 1) == np.argmax(nref.reshape(-1, shape[-1]), 1)).mean() > 0.99
    np.testing.assert_allclose(y, nref, rtol=1e-3, atol=1e-3 * np.abs(nref).max())
    print(f"[hlo] tinyllama fixture on device: {dt * 1e3:.1f} ms (uploads + host walk included)",
          flush=True)


def test_cli_runs_fixture_with_reference_flags(tmp_path):
    """hlo_run with main.rs's flags: --inputs-f32 list, --output-f32, --expected-f32, --epsilon."""
    from spirv_inference_amd import hlo_run
    text = fixture_text("bert_base")
    (tmp_path / "m.txt").write_text(text)
    ops = X.parse_hlo_text(text)
    params = seeded_params(ops)
    paths = []
    for i, p in enumerate(params):
        paths.append(tmp_path / f"p{i:03d}.raw.f32")
        p.astype("<f4").tofile(paths[-1])
    eval_numpy(ops, params).astype("<f4").tofile(tmp_path / "want.raw.f32")
    rc = hlo_run.main(["--input", str(tmp_path / "m.txt"), "--run", "--inputs-f32",
                       ",".join(map(str, paths)), "--output-f32", str(tmp_path / "out.raw.f32"),
                       "--expected-f32", str(tmp_path / "want.raw.f32"), "--epsilon", "1e-3",
                       "--report", str(tmp_path / "r.json")])
    import json
    rep = json.loads((tmp_path / "r.json").read_text())
    assert rc == 0 and rep["status"] == "pass", rep["execution"]
    ex = rep["execution"]
    assert ex["device"]["vendor_id"] == 0x1002 and ex["device"]["probe_output"] == [3.0]
    assert (tmp_path / "out.raw.f32").stat().st_size == 4 * ex["output"]["elements"]
    # compiler.rs:652-667: one record per device launch, each with its own hipEvent time
    assert ex["dispatch_count"] == len(ex["dispatches"]) > 0
    assert all(d["elapsed_ms"] > 0 and d["device_name"] == ex["device"]["name"]
               for d in ex["dispatches"])
    assert len(ex["steps"]) == len(ops) and ex["final_result"] == ops[-1].result
    assert ex["parity"]["epsilon"] == np.float32(1e-3)
    assert rep["module"]["ops"][0]["result"] == ops[0].result
    print(f"[hlo_run] {ex['dispatch_count']} dispatches, "
          f"{sum(d['elapsed_ms'] for d in ex['dispatches']):.3f} ms of kernel time", flush=True)
