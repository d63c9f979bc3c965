"""The device decode engines against the reference's own TinyLlama graph (GPU).

One seeded weight set at the full TinyLlama-1.1B shape goes into a device decoder and, as
export_llama.py's [in, out] parameter list, into the reference's HLO module
(tests/golden/hlo/tinyllama.stablehlo.txt.gz, source/xla_hlo/tools/export_llama.py:269-375),
which hlo_ref.eval_numpy evaluates in float64 on the host.  At every prompt position the
persistent and graph engines' logits must be within |d - r| <= 1e-4 + 1e-4 |r| of the graph's,
with the same argmax.  tests/test_oracle_llama_graph.py holds the CPU oracle to the same graph.
"""
import numpy as np
import pytest

from conftest import assert_close
from hlo_ref import eval_numpy, fixture_text
from llama_fixture import S_FIXTURE, hlo_params, seeded_weights

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def graph_case():
    from spirv_inference_amd import hlo_exec as X
    from spirv_inference_amd.models import TINYLLAMA
    cfg = dict(TINYLLAMA)
    print("[llama graph] seeding weights and evaluating the reference graph in float64",
          flush=True)
    w = seeded_weights(cfg, seed=21)
    prompt = [int(t) for t in np.random.default_rng(3).integers(0, cfg["vocab"], 32)]
    ops = X.parse_hlo_text(fixture_text("tinyllama"))
    ref = eval_numpy(ops, hlo_params(cfg, w, prompt)).reshape(S_FIXTURE, cfg["vocab"])
    return cfg, w, prompt, ref[:len(prompt)]


@pytest.mark.parametrize("engine", ["persistent", "graph"])
def test_decode_engine_matches_reference_graph(ctx, graph_case, engine):
    from spirv_inference_amd import weights as W
    from spirv_inference_amd.models import Llama
    cfg, w, prompt, ref = graph_case
    print(f"[llama graph] engine={engine}", flush=True)
    with Llama(ctx, seed=2) as lm:
        P = W._Placer(lm)
        try:
            P.copy(-1, "embed", w["embed"])
            P.copy(-1, "final_norm", w["final_norm"])
            P.copy(-1, "lm_head", w["lm_head"])
            for l, tensors in enumerate(w["layers"]):
                for name, arr in zip(("attn_norm", "wqkv", "wo", "ffn_norm", "w_gate_up",
                                      "w_down"), tensors):
                    P.copy(l, name, arr)
        finally:
            P.close()
        lm.set_engine(engine)
        lm.reset()
        for pos, tok in enumerate(prompt):
            lm.step(tok)
            lg = lm.logits()
            assert_close(lg, ref[pos], 1e-4, 1e-4, f"{engine} logits at position {pos}")
            assert int(np.argmax(lg)) == int(np.argmax(ref[pos])), pos
