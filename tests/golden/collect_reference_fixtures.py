"""Copies the reference's own golden data files into tests/golden/ (run in the build
container only; /root/reference does not exist on the GPU box).

Only data is copied — raw little-endian float32 tensors and JSON manifests the reference's
tests hold — never source.  Provenance (destination <- reference path):
  parity/<name>.raw.f32        <- tests/parity_test/out/fixtures/<name>.raw.f32
  parity/manifest.json         <- tests/parity_test/out/fixtures/manifest.json
  parity/cuda_<k>.raw.f32      <- tests/parity_test/out/cuda/<k>/output.raw.f32
  parity/intel_<k>.raw.f32     <- tests/parity_test/out/intel/<k>/output.raw.f32
  parity/advanced_parity_result.json <- tests/parity_test/out/compare/advanced_parity_result.json
  inference_poc_manifest.json  <- source/inference_poc/fixtures/manifest.json
"""
import pathlib
import shutil
import sys

REF = pathlib.Path("/root/reference")
HERE = pathlib.Path(__file__).resolve().parent


def main() -> int:
    if not REF.is_dir():
        print("reference tree not present; nothing to collect", file=sys.stderr)
        return 1
    dst = HERE / "parity"
    dst.mkdir(exist_ok=True)
    fx = REF / "tests/parity_test/out/fixtures"
    for p in sorted(fx.glob("*.raw.f32")):
        shutil.copyfile(p, dst / p.name)
    shutil.copyfile(fx / "manifest.json", dst / "manifest.json")
    for dev in ("cuda", "intel"):
        for k in ("relu", "softmax", "batchnorm", "conv1d"):
            shutil.copyfile(REF / f"tests/parity_test/out/{dev}/{k}/output.raw.f32",
                            dst / f"{dev}_{k}.raw.f32")
    shutil.copyfile(REF / "tests/parity_test/out/compare/advanced_parity_result.json",
                    dst / "advanced_parity_result.json")
    shutil.copyfile(REF / "source/inference_poc/fixtures/manifest.json",
                    HERE / "inference_poc_manifest.json")
    return 0


if __name__ == "__main__":
    sys.exit(main())
