"""Pins the decode oracle (orc_llama_full, orc_llama_step) to the reference's own TinyLlama
graph: the HLO module exported by source/xla_hlo/tools/export_llama.py:269-375
(tests/golden/hlo/tinyllama.stablehlo.txt.gz), evaluated in float64 by an independent numpy
interpreter of its op list (hlo_ref.eval_numpy), on one seeded weight set at the full
TinyLlama-1.1B shape.  The prompt is padded to the graph's S = 64 and masked as
run_llama_spirv.py:100-107 builds it; rows of the prompt positions are compared.

What this holds in place that the oracle's own self-consistency (step vs full recompute)
cannot: the GQA head mapping (head h reads KV head h // 8: the graph's tile at :333-343),
rotate-half RoPE with the float32 tables (:288-296), RMSNorm with its weight (:284-286), the
1/8 score scale and the mask add (:346-348), SiLU gating (:298-299), the [in, out] weight
orientation, and the layer order.  CPU only; about 40 s and 14 GB of host memory.
"""
import numpy as np
import pytest

from conftest import assert_close
from hlo_ref import eval_numpy, fixture_text
from llama_fixture import S_FIXTURE, hlo_params, seeded_weights


@pytest.fixture(scope="module")
def graph_case(orc):
    from spirv_inference_amd import hlo_exec as X
    from spirv_inference_amd.models import TINYLLAMA
    cfg = dict(TINYLLAMA)
    w = seeded_weights(cfg, seed=21)
    prompt = [int(t) for t in np.random.default_rng(3).integers(0, cfg["vocab"], 32)]
    ops = X.parse_hlo_text(fixture_text("tinyllama"))
    ref = eval_numpy(ops, hlo_params(cfg, w, prompt)).reshape(S_FIXTURE, cfg["vocab"])
    return cfg, w, prompt, ref[:len(prompt)]


def test_llama_full_recompute_matches_reference_graph(orc, graph_case):
    cfg, w, prompt, ref = graph_case
    c = orc.LlamaCfg(**cfg)
    full = orc.llama_full(c, w["layers"], w["embed"], w["final_norm"], w["lm_head"], prompt)
    assert_close(full, ref, 1e-4, 1e-4, "orc_llama_full vs export_llama.py graph")
    assert (full.argmax(1) == ref.argmax(1)).all()


def test_llama_kv_cache_steps_match_reference_graph(orc, graph_case):
    cfg, w, prompt, ref = graph_case
    c = orc.LlamaCfg(**cfg)
    cache = cfg["n_layers"] * cfg["n_kv_heads"] * cfg["max_seq"] * cfg["head_dim"]
    kc, vc = np.zeros(cache, np.float32), np.zeros(cache, np.float32)
    for pos, tok in enumerate(prompt):
        lg = orc.llama_step(c, w["layers"], w["embed"], w["final_norm"], w["lm_head"], kc, vc,
                            pos, tok)
        assert_close(lg, ref[pos], 1e-4, 1e-4, f"orc_llama_step pos {pos} vs graph")
        assert int(np.argmax(lg)) == int(np.argmax(ref[pos])), pos


def test_graph_check_detects_a_gqa_mapping_error(orc, graph_case):
    """The comparison above is sharp enough to see the mistake a self-consistency check would
    share between both oracle paths: KV heads mapped h % 4 instead of h // 8.  The wrong
    mapping is emulated on the oracle's side by permuting the query heads' weight rows, so that
    head h is computed with the rows of head p(h), whose KV head under h // 8 equals h % 4."""
    cfg, w, prompt, ref = graph_case
    nh, nkv, hd = cfg["n_heads"], cfg["n_kv_heads"], cfg["head_dim"]
    group = nh // nkv
    # slot j of the permuted model carries original head perm[j], chosen so that
    # j // group == perm[j] % nkv
    slots = {}
    for h in range(nh):
        kv = h % nkv
        slots.setdefault(kv, []).append(h)
    perm = [slots[j // group][j % group] for j in range(nh)]
    layers = []
    for attn_norm, wqkv, wo, ffn_norm, w_gu, w_down in w["layers"]:
        q = wqkv[:nh * hd].reshape(nh, hd, -1)[perm].reshape(nh * hd, -1)
        o = wo.reshape(wo.shape[0], nh, hd)[:, perm].reshape(wo.shape[0], nh * hd)
        layers.append([attn_norm, np.concatenate([q, wqkv[nh * hd:]]), np.ascontiguousarray(o),
                       ffn_norm, w_gu, w_down])
    c = orc.LlamaCfg(**cfg)
    wrong = orc.llama_full(c, layers, w["embed"], w["final_norm"], w["lm_head"], prompt[:8])
    err = np.abs(wrong - ref[:8]) - (1e-4 + 1e-4 * np.abs(ref[:8]))
    assert err.max() > 0.01
