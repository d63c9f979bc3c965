"""Chained conv2d -> batchnorm -> relu -> softmax on resident device tensors, with a per-edge
parity report: the counterpart of runtime/chained_graph_runtime (src/main.rs).

The reference program creates a Vulkan device, four pipelines and host-visible storage buffers,
records the four dispatches with a memory barrier between them in one command buffer, reads
every edge back, and compares each with the fixture's expected tensor: a mismatch is
|actual - expected| > epsilon, and the maximum ULP distance is reported beside the maximum
absolute error (main.rs:81-258 run and report, :774-819 compare_edge / ulp_distance).

Here the edges are device tensors that stay in HBM between the stages; the stages are registry
kernels launched on one stream (optionally replayed from one hipGraph):

  conv2d     kernels/conv2d (conv2d.comp: NCHW, OIHW weight + bias tail), one 16x16 channel,
             3x3 filter (the fixture's 9 taps), SAME padding, bias 0
  batchnorm  inference_poc's batchnorm_infer form (source/inference_poc/shaders/
             batchnorm_infer.comp:10-15): params [scale, bias, mean, var],
             y = (x - mean) * inversesqrt(var + 1e-5) * scale + bias, as sub / mul / mul / add
             launches over per-tensor constants prepared once (rsqrt kernel for the factor)
  relu       relu.comp
  softmax    softmax1000.comp over the 256 elements

Flags are main.rs's (parse_args :821-852): --device, --conv2d-spv, --batchnorm-spv,
--relu-spv, --softmax-spv (recorded with their SHA-256 when the files exist; the kernels are
compiled in), --fixture-manifest, --report, --dump-dir.  The manifest has main.rs's layout:
{"epsilon", "inputs": {conv2d_input, conv2d_filter, batchnorm_params},
 "edges": {conv2d_output, batchnorm_output, relu_output, softmax_output}}, each {path, sha256}
pointing at a float32 .npy file.
"""
from __future__ import annotations

import argparse
import hashlib
import json
import pathlib
import sys

import numpy as np

ELEMENTS = 256
SIDE = 16
FILTER_ELEMENTS = 9
BATCHNORM_PARAM_ELEMENTS = 4
BN_EPS = 1e-5
EDGES = ("conv2d_output", "batchnorm_output", "relu_output", "softmax_output")


def sha256_bytes(b: bytes) -> str:
    return hashlib.sha256(b).hexdigest()


def f32_bytes(a: np.ndarray) -> bytes:
    return np.ascontiguousarray(a, dtype="<f4").tobytes()


def ulp_distance(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """main.rs:809-819: distance of the bit patterns mapped to a monotonic integer line."""
    def ordered(v):
        bits = np.ascontiguousarray(v, np.float32).view(np.int32).astype(np.int64)
        return np.where(bits < 0, np.int64(-2 ** 31) - bits, bits)
    return np.abs(ordered(a) - ordered(b)).astype(np.uint64)


def compare_edge(actual: np.ndarray, expected: np.ndarray, epsilon: float, dump: str) -> dict:
    """main.rs:774-807 compare_edge: a length difference is an error, not a mismatch."""
    if actual.size != expected.size:
        raise ValueError(f"edge length mismatch: actual={actual.size} expected={expected.size}")
    a, e = actual.astype(np.float32), expected.astype(np.float32)
    ab = np.abs(a - e)
    return {"tensor_sha256": sha256_bytes(f32_bytes(a)),
            "oracle_sha256": sha256_bytes(f32_bytes(e)),
            "mismatch_count": int((ab > np.float32(epsilon)).sum()),
            "max_abs_error": float(ab.max()) if a.size else 0.0,
            "max_ulp_error": int(ulp_distance(a, e).max()) if a.size else 0,
            "dump_path": dump}


def chain_launches():
    """(kernel, push) of each stage: the push vectors of the reference kernels' Params blocks."""
    return {
        "conv2d": ("conv2d", [1, 1, SIDE, SIDE, 1, SIDE, SIDE, 3, 3, 1, 1, 1, 1, 1, ELEMENTS]),
        "relu": ("relu", [ELEMENTS]),
        "softmax": ("softmax1000", [ELEMENTS]),
    }


class ChainedGraph:
    """The four-stage chain on one context: every tensor allocated once, inputs uploaded once,
    the stages launched back to back with no host round trip (run()), optionally captured
    into a hipGraph (graph=True)."""

    def __init__(self, ctx, conv_input: np.ndarray, conv_filter: np.ndarray,
                 bn_params: np.ndarray):
        if conv_input.size != ELEMENTS or conv_filter.size != FILTER_ELEMENTS or \
                bn_params.size != BATCHNORM_PARAM_ELEMENTS:
            raise ValueError("unexpected fixture sizes for 256-element Conv2D -> BatchNorm -> "
                             "ReLU -> Softmax harness")
        self.ctx = ctx
        w = np.concatenate([conv_filter.reshape(-1), [0.0]]).astype(np.float32)  # bias tail
        scale, bias, mean, var = [float(v) for v in bn_params.reshape(-1)]
        self.t = {
            "x": ctx.tensor(conv_input.reshape(-1)), "w": ctx.tensor(w),
            "mean": ctx.tensor(np.full(ELEMENTS, mean, np.float32)),
            "var_eps": ctx.tensor(np.full(ELEMENTS, np.float32(var) + np.float32(BN_EPS),
                                          np.float32)),
            "scale": ctx.tensor(np.full(ELEMENTS, scale, np.float32)),
            "bias": ctx.tensor(np.full(ELEMENTS, bias, np.float32)),
        }
        for k in ("inv", "conv2d_output", "bn_centred", "bn_normed", "bn_scaled",
                  "batchnorm_output", "relu_output", "softmax_output"):
            self.t[k] = ctx.empty(ELEMENTS)
        # inversesqrt(var + eps) once: a per-tensor constant of this graph
        ctx.launch("rsqrt", self.t["var_eps"], None, self.t["inv"], [ELEMENTS])
        self._graph = None
        self.stages = self._stage_list()

    def _stage_list(self):
        t, L = self.t, chain_launches()
        return [
            (L["conv2d"][0], t["x"], t["w"], t["conv2d_output"], L["conv2d"][1]),
            ("sub", t["conv2d_output"], t["mean"], t["bn_centred"], [ELEMENTS]),
            ("mul", t["bn_centred"], t["inv"], t["bn_normed"], [ELEMENTS]),
            ("mul", t["bn_normed"], t["scale"], t["bn_scaled"], [ELEMENTS]),
            ("add", t["bn_scaled"], t["bias"], t["batchnorm_output"], [ELEMENTS]),
            (L["relu"][0], t["batchnorm_output"], None, t["relu_output"], L["relu"][1]),
            (L["softmax"][0], t["relu_output"], None, t["softmax_output"], L["softmax"][1]),
        ]

    def _launch_all(self):
        for k, a, b, o, push in self.stages:
            self.ctx.launch(k, a, b, o, push)

    def run(self, graph: bool = False) -> dict:
        if graph:
            if self._graph is None:
                self._launch_all()  # eager once, then record
                self.ctx.sync()
                self.ctx.capture_begin()
                try:
                    self._launch_all()
                finally:
                    self._graph = self.ctx.capture_end()
            self._graph.launch()
        else:
            self._launch_all()
        self.ctx.sync()
        return {e: self.t[e].download() for e in EDGES}

    def close(self):
        if self._graph is not None:
            self._graph.destroy()
            self._graph = None
        for v in self.t.values():
            v.free()
        self.t = {}


def read_npy_f32(path: pathlib.Path) -> np.ndarray:
    """main.rs:854-897 read_npy_f32: a little-endian float32 .npy array (no pickles)."""
    a = np.load(path, allow_pickle=False)
    if a.dtype != np.dtype("<f4"):
        raise ValueError(f"{path}: expected little-endian float32, found {a.dtype}")
    return a.reshape(-1)


def spv_entry(path: str) -> dict:
    """main.rs:109-120: each --*-spv file is read (and hashed) before anything runs; an
    unreadable path is an error naming it.  The bytes are not used here (the kernels are
    compiled into the library), only recorded."""
    try:
        data = pathlib.Path(path).read_bytes()
    except OSError as e:
        raise OSError(f"reading {path}: {e.strerror or e}") from e
    return {"path": path, "sha256": sha256_bytes(data)}


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--device", required=True)
    for k in ("conv2d", "batchnorm", "relu", "softmax"):
        ap.add_argument(f"--{k}-spv", required=True)
    ap.add_argument("--fixture-manifest", required=True, type=pathlib.Path)
    ap.add_argument("--report", required=True, type=pathlib.Path)
    ap.add_argument("--dump-dir", required=True, type=pathlib.Path)
    ap.add_argument("--graph", action="store_true", help="replay the chain from one hipGraph")
    a = ap.parse_args(argv)
    man = json.loads(a.fixture_manifest.read_text())
    base = a.fixture_manifest.parent

    def load(ref):
        p = pathlib.Path(ref["path"])
        return read_npy_f32(p if p.is_absolute() else base / p)

    x = load(man["inputs"]["conv2d_input"])
    f = load(man["inputs"]["conv2d_filter"])
    bn = load(man["inputs"]["batchnorm_params"])
    want = {e: load(man["edges"][e]) for e in EDGES}
    if any(v.size != ELEMENTS for v in want.values()):
        raise ValueError("unexpected fixture sizes for 256-element Conv2D -> BatchNorm -> ReLU "
                         "-> Softmax harness")
    try:
        source_spv = {k: spv_entry(getattr(a, f"{k}_spv")) for k in
                      ("conv2d", "batchnorm", "relu", "softmax")}
    except OSError as e:
        print(f"error: {e}", file=sys.stderr)
        return 1
    from .runtime import Context
    a.dump_dir.mkdir(parents=True, exist_ok=True)
    with Context("any" if a.device in ("any", "amd") else a.device) as ctx:
        g = ChainedGraph(ctx, x, f, bn)
        try:
            got = g.run(graph=a.graph)
        finally:
            g.close()
        dev = {"role": a.device, "name": ctx.device_name, "vendor_id": f"0x{ctx.vendor_id:04x}",
               "device_id": f"0x{ctx.device_id:04x}"}
    eps = float(man["epsilon"])
    edges = {}
    for e in EDGES:
        dump = a.dump_dir / f"edge_{e}.raw.f32"
        dump.write_bytes(f32_bytes(got[e]))
        edges[e] = compare_edge(got[e], want[e], eps, str(dump))
    mismatches = sum(v["mismatch_count"] for v in edges.values())
    L = chain_launches()
    report = {
        "status": "pass" if mismatches == 0 else "fail",
        "device": dev,
        "graph": ["conv2d", "batchnorm", "relu", "softmax"],
        "graph_execution_kind": ("hipgraph_replay_resident_device_tensors" if a.graph else
                                 "multi-dispatch_chained_resident_device_tensors"),
        "single_dispatch_graph_runtime_claimed": False,
        "artificial_padding_used": False,
        "element_count": ELEMENTS,
        "epsilon": eps,
        "dispatch": {
            "conv2d": {"kernel": L["conv2d"][0], "push": L["conv2d"][1]},
            "batchnorm": {"kernels": ["sub", "mul", "mul", "add"],
                          "form": "(x - mean) * inversesqrt(var + 1e-5) * scale + bias",
                          "params": ["scale", "bias", "mean", "var"]},
            "relu": {"kernel": L["relu"][0], "push": L["relu"][1]},
            "softmax": {"kernel": L["softmax"][0], "push": L["softmax"][1]},
            "ordering": "one HIP stream: each stage reads the previous edge after it is written",
        },
        "source_spv": source_spv,
        "fixture_manifest": str(a.fixture_manifest),
        "fixture_hashes": {
            **{k: man["inputs"][k].get("sha256") for k in man["inputs"]},
            **{f"{k}_oracle": man["edges"][k].get("sha256") for k in EDGES},
        },
        "edges": edges,
        "mismatch_count": mismatches,
        "max_abs_error": max(v["max_abs_error"] for v in edges.values()),
        "max_ulp_error": max(v["max_ulp_error"] for v in edges.values()),
        "non_claims": {"claims_single_dispatch_graph_runtime": False,
                       "uses_vendor_blas_or_dnn": False, "uses_pad_to_1024": False,
                       "includes_softmax": True},
    }
    text = json.dumps(report, indent=2)
    a.report.parent.mkdir(parents=True, exist_ok=True)
    a.report.write_text(text + "\n")
    print(text)
    return 0 if mismatches == 0 else 1


if __name__ == "__main__":
    sys.exit(main())
