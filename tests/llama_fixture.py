"""Test-side helpers that tie the decode oracle and the device decoder to the reference's own
TinyLlama graph: tests/golden/hlo/tinyllama.stablehlo.txt.gz, the S=64 full-recompute
forward that source/xla_hlo/tools/export_llama.py:269-375 exports, evaluated in float64 by
hlo_ref.eval_numpy.

One weight set is held in the decoder's layout ([out, in] rows, q|k|v rows in one matrix,
gate/up rows interleaved) and handed to the graph as export_llama.py's parameter list
(token_emb, rope_cos, rope_sin, causal_mask, then per layer input_ln_w, q_w, k_w, v_w, o_w,
post_ln_w, gate_w, up_w, down_w, then final_ln_w, lm_head_w; projections [in, out],
export_llama.py:137-160,203-217,238) as transposed views, so both sides read the same bytes.
"""
from __future__ import annotations

import concurrent.futures as cf
import os

import numpy as np

S_FIXTURE = 64  # the graph's fixed sequence length (export_llama.py: S = 64)


def rope_tables(seq: int, head_dim: int = 64, theta: float = 10000.0):
    """cos/sin [1, 1, seq, head_dim] as precompute_rope builds them in float32
    (source/xla_hlo/tools/run_llama_spirv.py:87-97)."""
    inv = 1.0 / (theta ** (np.arange(0, head_dim, 2, dtype=np.float32) / head_dim))
    freqs = np.outer(np.arange(seq, dtype=np.float32), inv)
    emb = np.concatenate([freqs, freqs], axis=-1)
    return (np.cos(emb).reshape(1, 1, seq, head_dim).astype(np.float32),
            np.sin(emb).reshape(1, 1, seq, head_dim).astype(np.float32))


def causal_mask(seq: int, n_valid: int) -> np.ndarray:
    """0 where allowed, -1e9 where c > r or c >= n_valid (run_llama_spirv.py:100-107)."""
    r = np.arange(seq)[:, None]
    c = np.arange(seq)[None, :]
    return np.where((c > r) | (c >= n_valid), np.float32(-1e9),
                    np.float32(0.0)).reshape(1, 1, seq, seq).astype(np.float32)


def seeded_weights(cfg: dict, seed: int, norm_lo: float = 0.5, norm_hi: float = 1.5):
    """Weights in the decoder's layout: matrices N(0, 0.02), RMSNorm weights U[lo, hi) (not
    all ones, so a dropped norm-weight multiply shows), embedding table [vocab, hidden].
    Every tensor has its own child stream of SeedSequence(seed), filled on a thread pool
    (about a billion values at the TinyLlama shape)."""
    H, F, V, L = cfg["hidden"], cfg["ffn"], cfg["vocab"], cfg["n_layers"]
    qd = cfg["n_heads"] * cfg["head_dim"]
    kvd = cfg["n_kv_heads"] * cfg["head_dim"]
    shapes = []
    for _ in range(L):
        shapes += [(H,), (qd + 2 * kvd, H), (H, qd), (H,), (2 * F, H), (H, F)]
    shapes += [(V, H), (H,), (V, H)]
    children = np.random.SeedSequence(seed).spawn(len(shapes))

    def make(i):
        g = np.random.default_rng(children[i])
        s = shapes[i]
        if len(s) == 1:
            return g.uniform(norm_lo, norm_hi, s).astype(np.float32)
        a = np.empty(s, np.float32)
        g.standard_normal(out=a, dtype=np.float32)
        a *= np.float32(0.02)
        return a

    with cf.ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 1)) as ex:
        t = list(ex.map(make, range(len(shapes))))
    layers = [t[6 * l:6 * l + 6] for l in range(L)]
    return dict(layers=layers, embed=t[6 * L], final_norm=t[6 * L + 1], lm_head=t[6 * L + 2])


def hlo_params(cfg: dict, w: dict, prompt, seq: int = S_FIXTURE, pad_token: int = 0):
    """export_llama.py's parameter list for `prompt` padded to `seq` with `pad_token`
    (export_llama.py:165-175): projections as [in, out] views of the decoder-layout weights."""
    H = cfg["hidden"]
    qd = cfg["n_heads"] * cfg["head_dim"]
    kvd = cfg["n_kv_heads"] * cfg["head_dim"]
    padded = list(prompt) + [pad_token] * (seq - len(prompt))
    cos, sin = rope_tables(seq, cfg["head_dim"], cfg["rope_theta"])
    params = [w["embed"][padded].reshape(1, seq, H), cos, sin, causal_mask(seq, len(prompt))]
    for attn_norm, wqkv, wo, ffn_norm, w_gu, w_down in w["layers"]:
        params += [attn_norm, wqkv[:qd].T, wqkv[qd:qd + kvd].T, wqkv[qd + kvd:].T, wo.T,
                   ffn_norm, w_gu[0::2].T, w_gu[1::2].T, w_down.T]
    params += [w["final_norm"], w["lm_head"].T]
    return params
