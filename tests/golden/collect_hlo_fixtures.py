"""Copy the reference's XLA HLO text fixtures into tests/golden/hlo/ (gzipped data).

Run in the build container, where the reference checkout exists:

    python tests/golden/collect_hlo_fixtures.py [/root/reference]

The files are the model graphs the reference's HLO runner executes
(source/xla_hlo/fixtures/<model>.stablehlo.txt: ResNet-50 Keras v1 b1, one BERT-base block,
the TinyLlama S=64 full-recompute forward).  Their weights are not in the reference (the
raw-f32 parameter files are not vendored), so tests feed seeded parameters of the declared
shapes.  The text is kept byte for byte (gzip only) with its SHA-256 in manifest.json.

It also extracts, from the reference's own HLO-runner report of the ResNet-50 fixture
(source/xla_hlo/reports/resnet50_local_c6_report.json), the data that pins this build's
runner report: the nested key layout, the parsed `module` (every op's result, opcode,
operands, types, shape, attributes and raw line), the op histogram, and per step / per
dispatch the (result, opcode, elements[, kernel]) lists.  Timings, paths and device names
are dropped.  Stored as hlo/resnet50_report.json.gz.
"""
import gzip
import hashlib
import json
import pathlib
import sys

MODELS = ("bert_base", "resnet50", "tinyllama")


def skeleton(v):
    """The key layout of a JSON value: dicts map each key to its child's layout, lists
    hold the layout of their first element (or nothing), leaves are None."""
    if isinstance(v, dict):
        return {k: skeleton(x) for k, x in sorted(v.items())}
    if isinstance(v, list):
        return [skeleton(v[0])] if v else []
    return None


def main() -> int:
    ref = pathlib.Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
    src = ref / "source" / "xla_hlo" / "fixtures"
    out = pathlib.Path(__file__).resolve().parent / "hlo"
    out.mkdir(exist_ok=True)
    manifest = {}
    for m in MODELS:
        data = (src / f"{m}.stablehlo.txt").read_bytes()
        with gzip.GzipFile(out / f"{m}.stablehlo.txt.gz", "wb", mtime=0) as f:
            f.write(data)
        manifest[m] = {"source": f"source/xla_hlo/fixtures/{m}.stablehlo.txt",
                       "bytes": len(data), "sha256": hashlib.sha256(data).hexdigest()}
    rep_path = ref / "source" / "xla_hlo" / "reports" / "resnet50_local_c6_report.json"
    rep = json.loads(rep_path.read_text())
    ex = rep["execution"]
    pinned = {"source": "source/xla_hlo/reports/resnet50_local_c6_report.json",
              "source_sha256": hashlib.sha256(rep_path.read_bytes()).hexdigest(),
              "skeleton": skeleton(rep), "module": rep["module"],
              "op_histogram": rep["op_histogram"],
              "steps": [[s["result"], s["opcode"], s["elements"]] for s in ex["steps"]],
              "dispatches": [[d["result"], d["opcode"], d["spv_name"], d["elements"]]
                             for d in ex["dispatches"]],
              "dispatch_count": ex["dispatch_count"], "final_result": ex["final_result"],
              "mode": ex["mode"]}
    blob = json.dumps(pinned, sort_keys=True).encode()
    with gzip.GzipFile(out / "resnet50_report.json.gz", "wb", mtime=0) as f:
        f.write(blob)
    (out / "manifest.json").write_text(json.dumps(manifest, indent=2) + "\n")
    print(json.dumps(manifest, indent=2))
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
