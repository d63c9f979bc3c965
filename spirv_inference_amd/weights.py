"""Real-weight loaders for the resident TinyLlama-shape decoder (files supplied locally).

Two sources, both read without executing anything from the file:

* the reference's raw-f32 parameter files, as `export_llama.py` writes them and the HLO
  runner takes them (`--inputs-f32`, a comma-separated list, source/xla_hlo/src/main.rs:35-42;
  little-endian float32, no header).  Parameter order and shapes follow
  source/xla_hlo/tools/export_llama.py:137-160 (token_emb, rope_cos, rope_sin, causal_mask,
  then per layer input_ln_w, q_w, k_w, v_w, o_w, post_ln_w, gate_w, up_w, down_w, then
  final_ln_w, lm_head_w), projections stored [in, out] (`.T` at :203-217,238); the
  embedding table is the separate `<prefix>_token_embedding.raw.f32` [vocab, hidden]
  (:126-129, looked up on the host by run_llama_spirv.py:160-203);
* a Hugging Face `safetensors` checkpoint (the `state` names export_llama.py reads,
  [out, in] matrices), through the safetensors reader.

The decoder keeps projections [out, in] row-major, q|k|v rows in one matrix and gate/up
rows interleaved (2n = gate n, 2n+1 = up n).  Tensors are uploaded once into a staging
buffer and put in that layout on the device by hlo_transpose launches written straight into
the decoder's weight buffers.  The RoPE tables and the causal mask of the parameter list are
not weights: the decoder derives them from rope_theta and the position, and the loader
checks the tables against that instead of loading them.
"""
from __future__ import annotations

import pathlib
from typing import Sequence

import numpy as np

from .hlo_ops import transpose_push
from .models import Llama
from .runtime import DeviceTensor

LAYER_PARAMS = ("input_ln_w", "q_w", "k_w", "v_w", "o_w", "post_ln_w", "gate_w", "up_w", "down_w")
N_HEAD_PARAMS = 4  # token_emb, rope_cos, rope_sin, causal_mask


def read_input_list(list_file: str | pathlib.Path, base: str | pathlib.Path | None = None
                    ) -> list[pathlib.Path]:
    """Paths of an `--inputs-f32` list (comma-separated, empty entries skipped), resolved
    against `base` (default: the list file's directory)."""
    list_file = pathlib.Path(list_file)
    base = pathlib.Path(base) if base is not None else list_file.parent
    text = list_file.read_text()
    return [base / p.strip() for p in text.replace("\n", ",").split(",") if p.strip()]


def read_raw_f32(path: str | pathlib.Path, shape: Sequence[int] | None = None) -> np.ndarray:
    """A headerless little-endian float32 file, memory-mapped; its size must match `shape`."""
    path = pathlib.Path(path)
    n = path.stat().st_size
    if n % 4:
        raise ValueError(f"{path}: {n} bytes is not a whole number of float32 values")
    a = np.memmap(path, dtype="<f4", mode="r")
    if shape is not None:
        want = int(np.prod(shape))
        if a.size != want:
            raise ValueError(f"{path}: {a.size} values, expected {want} for shape {list(shape)}")
        a = a.reshape(shape)
    return a


class _Placer:
    """Uploads host tensors and writes them, permuted, into the decoder's weight buffers."""

    def __init__(self, lm: Llama):
        self.lm, self.ctx = lm, lm.ctx
        c = lm.cfg
        self.H, self.F, self.V = c["hidden"], c["ffn"], c["vocab"]
        self.qd = c["n_heads"] * c["head_dim"]
        self.kvd = c["n_kv_heads"] * c["head_dim"]
        biggest = max(self.V * self.H, 2 * self.F * self.H, (self.qd + 2 * self.kvd) * self.H)
        self.stage = self.ctx.empty(biggest)

    def close(self):
        self.stage.free()

    def _dst(self, layer: int, which: str, offset: int = 0, n: int | None = None) -> DeviceTensor:
        ptr, elems = self.lm.weight_ptr(layer, which)
        n = elems - offset if n is None else n
        if offset + n > elems:
            raise ValueError(f"{which}: {offset}+{n} values past a buffer of {elems}")
        return DeviceTensor(self.ctx, n, ptr=ptr + 4 * offset, owned=False)

    def _stage(self, arr: np.ndarray) -> DeviceTensor:
        a = np.ascontiguousarray(arr, dtype=np.float32).reshape(-1)
        view = DeviceTensor(self.ctx, a.size, ptr=self.stage.ptr, owned=False)
        return view.upload(a)

    def copy(self, layer: int, which: str, arr: np.ndarray, offset: int = 0):
        src = self._stage(arr)
        dst = self._dst(layer, which, offset, src.n)
        self.ctx.launch("reshape", src, None, dst, [src.n])
        self.ctx.sync()

    def permute(self, layer: int, which: str, arr: np.ndarray, perm: Sequence[int],
                offset: int = 0):
        src = self._stage(arr)
        dst = self._dst(layer, which, offset, src.n)
        self.ctx.launch("hlo_transpose", src, None, dst, transpose_push(arr.shape, perm))
        self.ctx.sync()

    def check(self, layer: int, which: str, want: int, got: Sequence[int]):
        if int(np.prod(got)) != want:
            raise ValueError(f"layer {layer} {which}: shape {list(got)} does not fit "
                             f"{want} values")


def _check_rope(cos: np.ndarray, sin: np.ndarray, head_dim: int, theta: float):
    """The list's RoPE tables must be the ones the decoder derives (export_llama.py:116-124)."""
    s = cos.size // head_dim
    inv = 1.0 / (theta ** (np.arange(0, head_dim, 2, dtype=np.float32) / head_dim))
    emb = np.concatenate([np.outer(np.arange(s, dtype=np.float32), inv)] * 2, axis=-1)
    if not (np.allclose(cos.reshape(s, head_dim), np.cos(emb), atol=1e-5)
            and np.allclose(sin.reshape(s, head_dim), np.sin(emb), atol=1e-5)):
        raise ValueError("rope_cos/rope_sin do not match rope_theta of the decoder config")


def load_llama_reference_params(lm: Llama, params: Sequence[str | pathlib.Path],
                                embedding: str | pathlib.Path) -> None:
    """Load the export_llama.py parameter files (in list order) and embedding table."""
    c = lm.cfg
    L, H, F, V = c["n_layers"], c["hidden"], c["ffn"], c["vocab"]
    qd, kvd = c["n_heads"] * c["head_dim"], c["n_kv_heads"] * c["head_dim"]
    if len(params) != N_HEAD_PARAMS + len(LAYER_PARAMS) * L + 2:
        raise ValueError(f"{len(params)} parameter files, expected "
                         f"{N_HEAD_PARAMS + len(LAYER_PARAMS) * L + 2} for {L} layers")
    _check_rope(read_raw_f32(params[1]), read_raw_f32(params[2]), c["head_dim"], c["rope_theta"])
    P = _Placer(lm)
    try:
        P.copy(-1, "embed", read_raw_f32(embedding, (V, H)))
        for layer in range(L):
            f = {name: params[N_HEAD_PARAMS + len(LAYER_PARAMS) * layer + j]
                 for j, name in enumerate(LAYER_PARAMS)}
            P.copy(layer, "attn_norm", read_raw_f32(f["input_ln_w"], (H,)))
            # [in, out] -> rows of wqkv: q | k | v
            P.permute(layer, "wqkv", read_raw_f32(f["q_w"], (H, qd)), (1, 0))
            P.permute(layer, "wqkv", read_raw_f32(f["k_w"], (H, kvd)), (1, 0), offset=qd * H)
            P.permute(layer, "wqkv", read_raw_f32(f["v_w"], (H, kvd)), (1, 0),
                      offset=(qd + kvd) * H)
            P.permute(layer, "wo", read_raw_f32(f["o_w"], (qd, H)), (1, 0))
            P.copy(layer, "ffn_norm", read_raw_f32(f["post_ln_w"], (H,)))
            # [2][in][out] -> [out][2][in]: row 2n + j = (gate, up)[j] column n
            gu = np.stack([read_raw_f32(f["gate_w"], (H, F)), read_raw_f32(f["up_w"], (H, F))])
            P.permute(layer, "w_gate_up", gu, (2, 0, 1))
            P.permute(layer, "w_down", read_raw_f32(f["down_w"], (F, H)), (1, 0))
        P.copy(-1, "final_norm", read_raw_f32(params[-2], (H,)))
        P.permute(-1, "lm_head", read_raw_f32(params[-1], (H, V)), (1, 0))
    finally:
        P.close()


def load_llama_reference_fixture(lm: Llama, fixture_dir: str | pathlib.Path,
                                 prefix: str = "tinyllama") -> None:
    """A directory as export_llama.py leaves it: <prefix>_param_NNN_<name>.raw.f32 files
    (sorted by NNN) and <prefix>_token_embedding.raw.f32."""
    d = pathlib.Path(fixture_dir)
    params = sorted(d.glob(f"{prefix}_param_*.raw.f32"))
    load_llama_reference_params(lm, params, d / f"{prefix}_token_embedding.raw.f32")


def load_llama_safetensors(lm: Llama, paths: str | pathlib.Path | Sequence) -> None:
    """A Hugging Face Llama checkpoint in safetensors form (one file or shards)."""
    from safetensors import safe_open

    if isinstance(paths, (str, pathlib.Path)):
        paths = [paths]
    where = {}
    for p in paths:
        with safe_open(str(p), framework="numpy") as f:
            for k in f.keys():
                where[k] = p

    def get(name, shape):
        if name not in where:
            raise KeyError(f"{name} not in the checkpoint")
        with safe_open(str(where[name]), framework="numpy") as f:
            a = f.get_tensor(name)
        if tuple(a.shape) != tuple(shape):
            raise ValueError(f"{name}: shape {list(a.shape)}, expected {list(shape)}")
        return a.astype(np.float32, copy=False)

    c = lm.cfg
    L, H, F, V = c["n_layers"], c["hidden"], c["ffn"], c["vocab"]
    qd, kvd = c["n_heads"] * c["head_dim"], c["n_kv_heads"] * c["head_dim"]
    P = _Placer(lm)
    try:
        P.copy(-1, "embed", get("model.embed_tokens.weight", (V, H)))
        for layer in range(L):
            pre = f"model.layers.{layer}."
            P.copy(layer, "attn_norm", get(pre + "input_layernorm.weight", (H,)))
            P.copy(layer, "wqkv", get(pre + "self_attn.q_proj.weight", (qd, H)))
            P.copy(layer, "wqkv", get(pre + "self_attn.k_proj.weight", (kvd, H)), offset=qd * H)
            P.copy(layer, "wqkv", get(pre + "self_attn.v_proj.weight", (kvd, H)),
                   offset=(qd + kvd) * H)
            P.copy(layer, "wo", get(pre + "self_attn.o_proj.weight", (H, qd)))
            P.copy(layer, "ffn_norm", get(pre + "post_attention_layernorm.weight", (H,)))
            gu = np.stack([get(pre + "mlp.gate_proj.weight", (F, H)),
                           get(pre + "mlp.up_proj.weight", (F, H))])
            P.permute(layer, "w_gate_up", gu, (1, 0, 2))  # [2][F][H] -> [F][2][H]
            P.copy(layer, "w_down", get(pre + "mlp.down_proj.weight", (H, F)))
        P.copy(-1, "final_norm", get("model.norm.weight", (H,)))
        head = "lm_head.weight" if "lm_head.weight" in where else "model.embed_tokens.weight"
        P.copy(-1, "lm_head", get(head, (V, H)))
    finally:
        P.close()
