"""The benchmark configs through the HLO path on the device: the generated HLO text modules
(hlo_gen) compiled by hlo_program and run on the registry kernels, on the very weights of the
C++ graphs (shp_model_*) and of the decoder (shp_llama_*).

* ResNet-50 v1.5 b32 and BERT-base b8 s128 (12 layers): the compiled module issues the same
  launches as the C++ graph (kernel, push vector, epilogue), and its output is bit-identical
  to the graph's, eagerly and from hipGraph replays with host work in between.
* TinyLlama decode step (full 1.1B shape, KV cache): at several positions of a prompt the
  module's logits equal the decoder's own step within 1e-4 / 1e-4 with the same argmax, and
  its new key / value rows equal what the decoder wrote into its cache.
* The reference's ResNet-50 and TinyLlama fixtures compiled the same way, against float64 numpy.
"""
import time

import numpy as np
import pytest

from conftest import assert_close
from hlo_ref import eval_numpy, fixture_text, seeded_params
from llama_fixture import rope_tables
from spirv_inference_amd import hlo_exec as X
from spirv_inference_amd import hlo_gen as G
from spirv_inference_amd.hlo_program import HloProgram
from spirv_inference_amd.models import TINYLLAMA, Llama, Model

pytestmark = pytest.mark.gpu


def _launch_signature(prog):
    return [(k, list(p), bias is not None, res is not None, act)
            for (k, _a, _b, _c, p, bias, res, act, _al, _oe) in prog.launches]


def _model_signature(model, skip=()):
    return [(o.kernel, list(o.push), o.bias >= 0, o.residual >= 0, o.act)
            for o in model.ops() if o.label not in skip]


def _compare_graph_replays(ctx, prog, want, n=3):
    for r in range(n):
        prog.run(graph=True)
        ctx.sync()
        got = prog.read(0).reshape(-1)
        assert np.array_equal(got, want), f"graph replay {r} differs from the C++ graph"
        prog.read(0)  # host work between the replays


def test_resnet50_b32_hlo_module_equals_cpp_graph(ctx):
    text, spec = G.resnet50_v15(32)
    ops = X.parse_hlo_text(text)
    print(f"[hlo-gen] resnet50 v1.5 b32: {len(ops)} HLO ops, {len(spec)} parameters", flush=True)
    with Model(ctx, "resnet50_v1_5", 32) as m:
        m.run()
        ctx.sync()
        want = m.output(0).download()
        prog = HloProgram(X.DeviceBackend(ctx), ops, G.model_bindings(m, spec))
        assert _launch_signature(prog) == _model_signature(m)
        prog.run()
        ctx.sync()
        got = prog.read(0).reshape(-1)
        assert np.array_equal(got, want), np.abs(got - want).max()
        _compare_graph_replays(ctx, prog, want)
        t0 = time.perf_counter()
        for _ in range(10):
            prog.run(graph=True)
        ctx.sync()
        dt = (time.perf_counter() - t0) / 10
        print(f"[hlo-gen] resnet50 b32 via HLO module: {dt * 1e3:.3f} ms/step "
              f"({32 / dt:.0f} img/s), {len(prog.launches)} launches", flush=True)
        prog.close()


def test_bert_base_b8_s128_hlo_module_equals_cpp_graph(ctx):
    text, spec = G.bert_base(8, 128, 12)
    ops = X.parse_hlo_text(text)
    print(f"[hlo-gen] bert-base b8 s128: {len(ops)} HLO ops, {len(spec)} parameters", flush=True)
    with Model(ctx, "bert_base", 8, 128) as m:
        m.run()
        ctx.sync()
        want = m.output(0).download()
        prog = HloProgram(X.DeviceBackend(ctx), ops, G.model_bindings(m, spec))
        skip = ("word_embeddings", "add_position", "add_token_type", "embeddings_ln")
        assert _launch_signature(prog) == _model_signature(m, skip)
        prog.run()
        ctx.sync()
        got = prog.read(0).reshape(-1)
        assert np.array_equal(got, want), np.abs(got - want).max()
        _compare_graph_replays(ctx, prog, want)
        prog.close()


def test_tinyllama_decode_step_module_matches_decoder(ctx):
    cfg = dict(TINYLLAMA)
    text, spec = G.llama_decode_step(cfg["n_layers"], cfg["hidden"], cfg["n_heads"],
                                     cfg["n_kv_heads"], cfg["head_dim"], cfg["ffn"],
                                     cfg["vocab"], cfg["max_seq"], cfg["rms_eps"])
    ops = X.parse_hlo_text(text)
    print(f"[hlo-gen] tinyllama decode step: {len(ops)} HLO ops", flush=True)
    S, H, hd, nkv = cfg["max_seq"], cfg["hidden"], cfg["head_dim"], cfg["n_kv_heads"]
    cos, sin = rope_tables(S, hd, cfg["rope_theta"])
    rng = np.random.default_rng(3)
    prompt = [int(t) for t in rng.integers(0, cfg["vocab"], 12)]
    check_at = {0, 1, 5, 11}
    with Llama(ctx, seed=4) as lm:
        lm.set_engine("graph")
        prog = HloProgram(X.DeviceBackend(ctx), ops, G.llama_bindings(lm, spec))
        eptr, _ = lm.weight_ptr(0, "embed")
        from spirv_inference_amd.runtime import DeviceTensor
        lm.reset()
        # the module reads every cache row (masked ones too): they must hold finite values
        for layer in range(cfg["n_layers"]):
            for which in ("k_cache", "v_cache"):
                p, n = lm.weight_ptr(layer, which)
                ctx.fill_random(DeviceTensor(ctx, n, ptr=p, owned=False), 0, 0, "uniform", 0, 0)
        for pos, tok in enumerate(prompt):
            if pos in check_at:
                row = DeviceTensor(ctx, H, ptr=eptr + 4 * tok * H, owned=False).download()
                mask = np.zeros(S + 1, np.float32)
                mask[pos:S] = -1e9
                prog.set_param(0, row)
                prog.set_param(1, cos[0, 0, pos])
                prog.set_param(2, sin[0, 0, pos])
                prog.set_param(3, mask)
                prog.run(graph=pos > 1)
                ctx.sync()
                outs = [prog.read(k) for k in range(len(prog.outputs()))]
            lm.step(tok)
            if pos in check_at:
                want = lm.logits()
                assert_close(outs[0].reshape(-1), want, 1e-4, 1e-4, f"HLO step pos {pos}")
                assert int(np.argmax(outs[0])) == int(np.argmax(want)), pos
                for layer in (0, cfg["n_layers"] - 1):
                    kc = lm.weight(layer, "k_cache").reshape(nkv, S, hd)[:, pos]
                    vc = lm.weight(layer, "v_cache").reshape(nkv, S, hd)[:, pos]
                    assert_close(outs[1 + 2 * layer].reshape(nkv, hd), kc, 1e-5, 1e-4, "k row")
                    assert_close(outs[2 + 2 * layer].reshape(nkv, hd), vc, 1e-5, 1e-4, "v row")
                print(f"[hlo-gen] decode step pos {pos}: logits match, argmax "
                      f"{int(np.argmax(want))}", flush=True)
        prog.close()


def test_reference_fixtures_compiled(ctx):
    """The reference's ResNet-50 (Keras v1, b1: pad + VALID conv folds into the conv's padding)
    and TinyLlama S=64 fixtures through the compiled program, against float64 numpy."""
    for name, tol in (("resnet50", 1e-3), ("tinyllama", 1e-3)):
        ops = X.parse_hlo_text(fixture_text(name))
        params = seeded_params(ops)
        prog = HloProgram(X.DeviceBackend(ctx), ops, params)
        prog.run()
        ctx.sync()
        y = prog.read(0)
        ref = eval_numpy(ops, params).reshape(y.shape)
        rows = y.reshape(-1, y.shape[-1])
        assert (rows.argmax(1) == ref.reshape(rows.shape).argmax(1)).mean() > 0.99, name
        np.testing.assert_allclose(y, ref, rtol=tol, atol=tol * np.abs(ref).max())
        print(f"[hlo-gen] fixture {name}: {len(prog.launches)} launches for {len(ops)} ops, "
              f"fused {prog.fused_counts}", flush=True)
        prog.close()
