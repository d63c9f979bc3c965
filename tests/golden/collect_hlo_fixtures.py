"""Copy the reference's XLA HLO text fixtures into tests/golden/hlo/ (gzipped data).

Run in the build container, where the reference checkout exists:

    python tests/golden/collect_hlo_fixtures.py [/root/reference]

The files are the model graphs the reference's HLO runner executes
(source/xla_hlo/fixtures/<model>.stablehlo.txt: ResNet-50 Keras v1 b1, one BERT-base block,
the TinyLlama S=64 full-recompute forward).  Their weights are not in the reference (the
raw-f32 parameter files are not vendored), so tests feed seeded parameters of the declared
shapes.  The text is kept byte for byte (gzip only) with its SHA-256 in manifest.json.
"""
import gzip
import hashlib
import json
import pathlib
import sys

MODELS = ("bert_base", "resnet50", "tinyllama")


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
    (out / "manifest.json").write_text(json.dumps(manifest, indent=2) + "\n")
    print(json.dumps(manifest, indent=2))
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
