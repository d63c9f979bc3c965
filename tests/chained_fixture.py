"""A fixture manifest for spirv_inference_amd.chained_run in the layout of
runtime/chained_graph_runtime/src/main.rs:30-56 (epsilon, inputs, edges; float32 .npy files with
SHA-256), whose expected edges are the C oracle's restatement of the same chain.

The reference ships neither its chain's shaders nor its fixture, so the inputs are closed forms
in the style of tests/parity_test/generate_fixtures.py:67-82 (integer patterns scaled by powers
of two, exact in float32)."""
import hashlib
import json

import numpy as np

import oracle as orc
from spirv_inference_amd import chained_run as CR


def inputs():
    i = np.arange(256)
    x = (((i * 17) % 97 - 48) * 0.015625).astype(np.float32)
    f = (((np.arange(9) * 11) % 53 - 26) * 0.03125).astype(np.float32)
    bn = np.array([1.25, 0.125, 0.0625, 0.75], np.float32)  # scale, bias, mean, var
    return x, f, bn


def oracle_chain(x, f, bn):
    """The chain's launches on the oracle (same kernel names and push vectors)."""
    L = CR.chain_launches()
    n = CR.ELEMENTS
    w = np.concatenate([f, [0.0]]).astype(np.float32)
    scale, bias, mean, var = bn
    var_eps = np.full(n, np.float32(var) + np.float32(CR.BN_EPS), np.float32)
    inv = orc.run("rsqrt", var_eps, None, n, [n])
    conv = orc.run(L["conv2d"][0], x, w, n, L["conv2d"][1])
    t = orc.run("sub", conv, np.full(n, mean, np.float32), n, [n])
    t = orc.run("mul", t, inv, n, [n])
    t = orc.run("mul", t, np.full(n, scale, np.float32), n, [n])
    bnv = orc.run("add", t, np.full(n, bias, np.float32), n, [n])
    relu = orc.run(L["relu"][0], bnv, None, n, L["relu"][1])
    sm = orc.run(L["softmax"][0], relu, None, n, L["softmax"][1])
    return {"conv2d_output": conv, "batchnorm_output": bnv, "relu_output": relu,
            "softmax_output": sm}


def numpy_chain(x, f, bn):
    """Float64 restatement: 3x3 SAME conv of one 16x16 channel, inference batchnorm, ReLU,
    softmax over all 256 values."""
    img = np.pad(x.astype(np.float64).reshape(16, 16), 1)
    k = f.astype(np.float64).reshape(3, 3)
    conv = np.zeros((16, 16))
    for dy in range(3):
        for dx in range(3):
            conv += k[dy, dx] * img[dy:dy + 16, dx:dx + 16]
    scale, bias, mean, var = bn.astype(np.float64)
    b = (conv.reshape(-1) - mean) / np.sqrt(var + CR.BN_EPS) * scale + bias
    r = np.maximum(b, 0.0)
    e = np.exp(r - r.max())
    return {"conv2d_output": conv.reshape(-1), "batchnorm_output": b, "relu_output": r,
            "softmax_output": e / e.sum()}


def write_manifest(tmp, epsilon=1e-4, edges=None):
    x, f, bn = inputs()
    edges = edges or oracle_chain(x, f, bn)

    def save(name, arr):
        p = tmp / f"{name}.npy"
        np.save(p, np.asarray(arr, "<f4"), allow_pickle=False)
        return {"path": p.name, "sha256": hashlib.sha256(p.read_bytes()).hexdigest()}

    man = {"epsilon": epsilon,
           "inputs": {"conv2d_input": save("conv2d_input", x),
                      "conv2d_filter": save("conv2d_filter", f),
                      "batchnorm_params": save("batchnorm_params", bn)},
           "edges": {k: save(k, v) for k, v in edges.items()}}
    path = tmp / "manifest.json"
    path.write_text(json.dumps(man, indent=1))
    return path
