"""The HLO-text modules of the benchmark configs (spirv_inference_amd.hlo_gen) and their
compiled execution (spirv_inference_amd.hlo_program), on the CPU.

* Every generated module parses with the reference parser's rules and declares the
  parameters the generator lists.
* The compiled program (views, fused epilogues, fused softmax / LayerNorm / RMSNorm / mean
  pool, pooled buffers) on the oracle backend matches an independent float64 numpy
  interpreter of the same op list (hlo_ref.eval_numpy) and the op-by-op walk of
  hlo_exec.HloExecutor, at reduced sizes of the three configs and on the reference's own
  BERT block fixture (whose GELU is the erfc expansion bert_base.stablehlo.txt:55-144).
* The TinyLlama decode-step module against a KV cache equals the oracle's KV-cache step
  (orc_llama_step, itself pinned to export_llama.py's graph) at every position.
* The activation-region matcher fuses exactly the regions that are an epilogue activation.
"""
import collections

import numpy as np
import pytest

from conftest import assert_close
from hlo_ref import OracleBackend, eval_numpy, fixture_text, seeded_params
from llama_fixture import rope_tables, seeded_weights
from spirv_inference_amd import hlo_exec as X
from spirv_inference_amd import hlo_gen as G
from spirv_inference_amd.hlo_program import HloProgram, View, Buf, _reshape_view

SMALL_LLAMA = dict(n_layers=2, hidden=256, n_heads=8, n_kv_heads=2, head_dim=64, ffn=128,
                   vocab=50, max_seq=8, rms_eps=1e-5, rope_theta=10000.0)


def _modules():
    return {
        "resnet50_b2_64px": G.resnet50_v15(2, 64),
        "bert_b2_s16_l2": G.bert_base(2, 16, 2, 64, 4, 128),
        "llama_step_small": G.llama_decode_step(2, 256, 8, 2, 64, 128, 50, 8),
    }


def _run(text, params):
    ops = X.parse_hlo_text(text)
    prog = HloProgram(OracleBackend(), ops, params)
    prog.run()
    return ops, prog, [prog.read(k) for k in range(len(prog.outputs()))]


@pytest.mark.parametrize("name", list(_modules()))
def test_generated_module_parses_and_declares_its_params(name):
    text, params = _modules()[name]
    ops = X.parse_hlo_text(text)
    decl = {}
    for op in ops:
        if op.opcode == "parameter":
            decl[int(op.raw.split("parameter(")[1].split(")")[0])] = op.shape
    assert [decl[i] for i in range(len(decl))] == [s for _, s in params]
    assert len({lbl for lbl, _ in params}) == len(params)
    assert ops[-1].raw.startswith("ROOT ")
    # only opcodes the reference parser knows (parser.rs:113-160; concatenate via the fallback)
    assert {op.opcode for op in ops} <= set(X._OPCODES) | {"concatenate"}
    header = text.split("ENTRY ", 1)[1].split(")", 1)[0]
    assert header.count(":") == len(params)


def test_fused_resnet_matches_numpy_and_op_walk():
    text, _ = G.resnet50_v15(2, 64)
    ops = X.parse_hlo_text(text)
    params = seeded_params(ops, seed=5)
    _, prog, (y,) = _run(text, params)
    assert prog.fused_counts == {"conv": 53, "meanpool": 1, "dot": 1, "softmax": 1}
    kinds = collections.Counter(l[0] for l in prog.launches)
    assert kinds == {"hlo_conv_nhwc_hwio": 53, "hlo_reduce_window_rank4": 1,
                     "global_avg_pool_nhwc": 1, "hlo_dot_rank2": 1, "softmax_rows": 1}
    # every convolution carries its bias; 49 carry ReLU; 16 the residual (the block outputs)
    convs = [l for l in prog.launches if l[0] == "hlo_conv_nhwc_hwio"]
    assert all(l[5] is not None for l in convs)
    assert sum(l[7] == 1 for l in convs) == 49 and sum(l[6] is not None for l in convs) == 16
    ref = eval_numpy(ops, params)
    assert_close(y, ref, 1e-4, 1e-4, "fused ResNet-50 vs float64 numpy")
    walk, _ = X.HloExecutor(OracleBackend(), ops).run(params)
    assert_close(y, walk.reshape(y.shape), 1e-5, 1e-5, "fused vs op-by-op walk")
    assert (y.argmax(1) == ref.argmax(1)).all()


def test_fused_bert_matches_numpy_and_op_walk():
    text, _ = G.bert_base(2, 16, 2, 64, 4, 128)
    ops = X.parse_hlo_text(text)
    params = seeded_params(ops, seed=6)
    _, prog, (y,) = _run(text, params)
    assert prog.fused_counts == {"dot": 8, "softmax": 2, "layernorm": 4}
    acts = sorted(l[7] for l in prog.launches if l[0] == "hlo_dot_rank2")
    assert acts.count(7) == 2  # GELU-erfc in the two FFN1 epilogues
    kinds = collections.Counter(l[0] for l in prog.launches)
    assert kinds["dot_general_strided"] == 4 and "hlo_strided_copy" not in kinds
    assert "hlo_transpose" not in kinds  # head split and merge read / write in place
    ref = eval_numpy(ops, params)
    assert_close(y, ref, 1e-4, 1e-4, "fused BERT vs float64 numpy")
    walk, _ = X.HloExecutor(OracleBackend(), ops).run(params)
    assert_close(y, walk.reshape(y.shape), 1e-5, 1e-5, "fused vs op-by-op walk")


def test_attention_block_fuses_at_sequence_128():
    """At sequence 128 and head dim 64 the scores dot -> softmax -> context dot of each layer
    compile to one attention_fused launch reading the fused QKV rows in place (the C++
    graph's op), and the result still matches float64 numpy and the op-by-op walk."""
    text, _ = G.bert_base(1, 128, 1, 128, 2, 256)
    ops = X.parse_hlo_text(text)
    params = seeded_params(ops, seed=7)
    _, prog, (y,) = _run(text, params)
    assert prog.fused_counts.get("attention") == 1 and "softmax" not in prog.fused_counts
    kinds = collections.Counter(l[0] for l in prog.launches)
    assert kinds["attention_fused"] == 1 and "dot_general_strided" not in kinds
    push = next(l[4] for l in prog.launches if l[0] == "attention_fused")
    assert push[:9] == [1, 2, 128, 64, 3 * 128, 0, 128, 256, 128]
    ref = eval_numpy(ops, params)
    assert_close(y, ref, 1e-4, 1e-4, "fused-attention BERT vs float64 numpy")
    walk, _ = X.HloExecutor(OracleBackend(), ops).run(params)
    assert_close(y, walk.reshape(y.shape), 1e-5, 1e-5, "fused-attention vs op-by-op walk")


def test_fused_program_on_reference_bert_block():
    """The reference's own BERT block fixture: its erfc-expanded GELU (about 90 ops) is
    recognised as the GELU epilogue of the last dot."""
    text = fixture_text("bert_base")
    ops = X.parse_hlo_text(text)
    params = seeded_params(ops)
    _, prog, (y,) = _run(text, params)
    assert len(prog.launches) <= 6
    last_dot = [l for l in prog.launches if l[0] == "hlo_dot_rank2"][-1]
    assert last_dot[7] == 7 and last_dot[6] is not None  # GELU with the residual fused
    assert_close(y, eval_numpy(ops, params), 1e-4, 1e-4, "fused BERT block vs numpy")


def _llama_step_params(cfg, w, kc, vc, pos, token):
    """The decode-step module's parameters for `token` at `pos` (hlo_gen.llama_decode_step),
    the caches holding positions < pos in the decoder's [layer][kv][max_seq][hd] layout."""
    L, nkv, S, hd = cfg["n_layers"], cfg["n_kv_heads"], cfg["max_seq"], cfg["head_dim"]
    cos, sin = rope_tables(S, hd, cfg["rope_theta"])
    mask = np.zeros(S + 1, np.float32)
    mask[pos:S] = -1e9
    per = nkv * S * hd
    p = [w["embed"][token].reshape(1, -1), cos[0, 0, pos:pos + 1], sin[0, 0, pos:pos + 1], mask]
    for l, (an, wqkv, wo, fn, wgu, wd) in enumerate(w["layers"]):
        p += [an, wqkv, wo, fn, wgu, wd, kc[l * per:(l + 1) * per], vc[l * per:(l + 1) * per]]
    return p + [w["final_norm"], w["lm_head"]]


def test_llama_decode_step_module_matches_oracle_step(orc):
    cfg = dict(SMALL_LLAMA)
    w = seeded_weights(cfg, seed=9)
    c = orc.LlamaCfg(**cfg)
    text, _ = G.llama_decode_step(cfg["n_layers"], cfg["hidden"], cfg["n_heads"],
                                  cfg["n_kv_heads"], cfg["head_dim"], cfg["ffn"], cfg["vocab"],
                                  cfg["max_seq"], cfg["rms_eps"])
    ops = X.parse_hlo_text(text)
    L, nkv, S, hd = cfg["n_layers"], cfg["n_kv_heads"], cfg["max_seq"], cfg["head_dim"]
    kc = np.zeros(L * nkv * S * hd, np.float32)
    vc = np.zeros_like(kc)
    tokens = [3, 17, 42, 8, 8, 29, 1, 40]
    for pos, tok in enumerate(tokens):
        params = _llama_step_params(cfg, w, kc, vc, pos, tok)
        prog = HloProgram(OracleBackend(), ops, params)
        prog.run()
        outs = [prog.read(k) for k in range(len(prog.outputs()))]
        want = orc.llama_step(c, w["layers"], w["embed"], w["final_norm"], w["lm_head"], kc, vc,
                              pos, tok)
        assert_close(outs[0].reshape(-1), want, 1e-4, 1e-4, f"decode-step module pos {pos}")
        assert int(np.argmax(outs[0])) == int(np.argmax(want))
        # the new key / value rows are what the oracle's step wrote into its cache at pos
        for l in range(L):
            base = l * nkv * S * hd
            k_row = kc[base:base + nkv * S * hd].reshape(nkv, S, hd)[:, pos]
            v_row = vc[base:base + nkv * S * hd].reshape(nkv, S, hd)[:, pos]
            assert_close(outs[1 + 2 * l].reshape(nkv, hd), k_row, 1e-5, 1e-5, f"k l{l} p{pos}")
            assert_close(outs[2 + 2 * l].reshape(nkv, hd), v_row, 1e-5, 1e-5, f"v l{l} p{pos}")
        if pos == 0:
            allv = eval_numpy(ops, params, all_values=True)
            assert_close(outs[0], allv[prog._roots[0]], 1e-4, 1e-4, "step module vs numpy")


def _act_module(body):
    """A one-dot module whose result goes through `body(builder, value)`."""
    b = G.HloBuilder("act")
    x = b.param([4, 8], "x")
    w = b.param([8, 16], "w")
    y = body(b, b.dot(x, w, [1], [0]))
    return b.text(y)


@pytest.mark.parametrize("body,act", [
    (lambda b, v: b.relu(v), 1),
    (lambda b, v: b.binary("minimum", b.relu(v), b.splat(6.0, v.shape)), 2),
    (lambda b, v: b.unary("logistic", v), 4),
    (lambda b, v: b.unary("tanh", v), 5),
    (lambda b, v: b.binary("multiply", v, b.unary("logistic", v)), 6),
    (lambda b, v: b.gelu_erf(v), 7),
    (lambda b, v: b.binary("multiply", v, v), 0),                       # x^2: not an epilogue
    (lambda b, v: b.binary("maximum", v, b.splat(0.5, v.shape)), 0),     # max(x, 0.5)
    # ReLU only on [-12, 12]: clamps at 20 and 1e4 are not ReLU and must not fuse as it
    (lambda b, v: b.binary("minimum", b.relu(v), b.splat(20.0, v.shape)), 0),
    (lambda b, v: b.binary("minimum", b.relu(v), b.splat(1e4, v.shape)), 0),
    # tanh.comp's clamp to +-20 before tanh is tanh everywhere in float (tanh(20) rounds to 1)
    (lambda b, v: b.unary("tanh", b.binary("maximum", b.binary("minimum", v, b.splat(20.0, v.shape)),
                                          b.splat(-20.0, v.shape))), 5),
])
def test_activation_regions(body, act):
    text = _act_module(body)
    ops = X.parse_hlo_text(text)
    params = seeded_params(ops, seed=2)
    _, prog, (y,) = _run(text, params)
    dots = [l for l in prog.launches if l[0] == "hlo_dot_rank2"]
    assert len(dots) == 1 and dots[0][7] == act
    assert_close(y, eval_numpy(ops, params), 1e-5, 1e-5, f"act {act}")


def test_reshape_views_follow_numpy():
    base = np.arange(2 * 3 * 4 * 5, dtype=np.float32).reshape(2, 3, 4, 5)
    buf = Buf(None, base.size, True)
    cases = [((0, 2, 1, 3), (2, 4, 15)), ((0, 2, 1, 3), (8, 15)), ((0, 1, 2, 3), (6, 20)),
             ((1, 0, 2, 3), (3, 2, 20)), ((0, 2, 1, 3), (2, 4, 3, 5))]
    for perm, shape in cases:
        t = np.transpose(base, perm)
        v = View(buf, 0, t.shape, [base.strides[p] // 4 for p in perm])
        r = _reshape_view(v, shape)
        want = t.reshape(shape)
        if r is None:
            assert not np.shares_memory(want, base), (perm, shape)
            continue
        got = np.lib.stride_tricks.as_strided(base, r.shape, [s * 4 for s in r.strides])
        np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("extra", ["probs", "scores"])
def test_attention_not_fused_when_probs_or_scores_are_read_elsewhere(extra):
    """The fused attention launch writes neither the scores nor the probabilities: when a
    program output also reads either of them, the three launches stay, and every output
    (the probabilities' rows summing to 1) matches float64 numpy."""
    text, _ = G.bert_base(1, 128, 1, 128, 2, 256)
    ops = X.parse_hlo_text(text)
    root = next(o for o in ops if o.raw.lstrip().startswith("ROOT"))
    if extra == "probs":  # the softmax's divide
        other = next(o for o in ops if o.opcode == "divide")
    else:  # the scores dot, the first dot with batch dims
        other = next(o for o in ops if o.opcode == "dot" and "lhs_batch_dims" in o.raw)
    ty = lambda o: o.raw.split("=", 1)[1].split()[0]
    line = root.raw.strip()
    text2 = text.replace(line, line.replace("ROOT ", "", 1) + "\n  ROOT %out = (" + ty(root) +
                         ", " + ty(other) + ") tuple(" + ty(root) + " " + root.result + ", " +
                         ty(other) + " " + other.result + ")")
    ops2 = X.parse_hlo_text(text2)
    params = seeded_params(ops2, seed=7)
    _, prog, outs = _run(text2, params)
    assert "attention" not in prog.fused_counts and prog.fused_counts.get("softmax") == 1
    allv = eval_numpy(ops2, params, all_values=True)
    assert_close(outs[0], allv[root.result], 1e-4, 1e-4, "hidden output")
    assert_close(outs[1], allv[other.result], 1e-4, 1e-4, f"{extra} output")
    if extra == "probs":
        assert np.allclose(outs[1].sum(-1), 1.0, atol=1e-5)
