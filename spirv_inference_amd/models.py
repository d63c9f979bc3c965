"""Resident model graphs (shp_model_*) and the KV-cache decoder (shp_llama_*).

The graphs replace the reference's two front-ends for the benchmark configs — the TFLite
scheduler (source/tflite_loader/src/scheduler.rs:29-1082) for MobileNetV2 and
EfficientNet-Lite0, the HLO interpreter (source/xla_hlo/src/compiler.rs:267-668) for
ResNet-50 and BERT — and TinyLlama's subprocess-per-token driver
(source/xla_hlo/tools/run_llama_spirv.py:194-295).
"""
from __future__ import annotations

import ctypes as C
import dataclasses

import numpy as np

from ._lib import LlamaConfig, OpDesc, check, lib
from .runtime import Context, DeviceTensor

ARCHS = ("resnet50_v1_5", "mobilenet_v2", "efficientnet_lite0", "bert_base")


@dataclasses.dataclass
class Op:
    kernel: str
    label: str
    push: list
    in0: int
    in1: int
    out: int
    bias: int
    residual: int
    act: int
    alpha: float
    out_elems: int


@dataclasses.dataclass
class TensorInfo:
    ptr: int
    elems: int
    kind: int      # 0 activation, 1 weight, 2 input, 3 view
    parent: int
    offset: int


class Model:
    def __init__(self, ctx: Context, arch: str, batch: int, seq_len: int = 0, seed: int = 2):
        self.ctx = ctx
        self.arch, self.batch, self.seq_len, self.seed = arch, batch, seq_len, seed
        h = C.c_void_p()
        check(lib().shp_model_create(ctx.handle, arch.encode(), batch, seq_len, seed,
                                     C.byref(h)), f"shp_model_create({arch})")
        self.handle = h.value

    def close(self):
        if self.handle:
            lib().shp_model_destroy(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def run(self) -> None:
        check(lib().shp_model_run(self.handle), f"shp_model_run({self.arch})")

    def use_graph(self, enable: bool) -> None:
        check(lib().shp_model_use_graph(self.handle, int(enable)), "shp_model_use_graph")

    def _io(self, fn, index: int) -> DeviceTensor:
        p, n = C.c_void_p(), C.c_uint64()
        check(fn(self.handle, index, C.byref(p), C.byref(n)), "model io")
        return DeviceTensor(self.ctx, n.value, ptr=p.value, owned=False)

    def input(self, index: int = 0) -> DeviceTensor:
        return self._io(lib().shp_model_input, index)

    def output(self, index: int = 0) -> DeviceTensor:
        return self._io(lib().shp_model_output, index)

    def work(self) -> tuple[float, float]:
        f, w = C.c_double(), C.c_double()
        check(lib().shp_model_work(self.handle, C.byref(f), C.byref(w)), "shp_model_work")
        return f.value, w.value

    def ops(self) -> list[Op]:
        out = []
        d = OpDesc()
        for i in range(lib().shp_model_num_ops(self.handle)):
            check(lib().shp_model_op(self.handle, i, C.byref(d)), "shp_model_op")
            out.append(Op(d.kernel.decode(), d.label.decode(), list(d.push[:d.n_push]), d.in0,
                          d.in1, d.out, d.bias, d.residual, d.act, d.alpha, d.out_elems))
        return out

    def tensor_info(self, tid: int) -> TensorInfo:
        p, n, k = C.c_void_p(), C.c_uint64(), C.c_int32()
        check(lib().shp_model_tensor(self.handle, tid, C.byref(p), C.byref(n), C.byref(k)),
              "shp_model_tensor")
        par, off = C.c_int32(), C.c_uint64()
        check(lib().shp_model_tensor_parent(self.handle, tid, C.byref(par), C.byref(off)),
              "shp_model_tensor_parent")
        return TensorInfo(p.value or 0, n.value, k.value, par.value, off.value)

    def num_tensors(self) -> int:
        return lib().shp_model_num_tensors(self.handle)

    def download(self, tid: int) -> np.ndarray:
        info = self.tensor_info(tid)
        return DeviceTensor(self.ctx, info.elems, ptr=info.ptr, owned=False).download()


TINYLLAMA = dict(n_layers=22, hidden=2048, n_heads=32, n_kv_heads=4, head_dim=64, ffn=5632,
                 vocab=32000, max_seq=64, rms_eps=1e-5, rope_theta=10000.0)


class Llama:
    """Greedy decode with a KV cache; weights row-major [out, in] in HBM."""

    def __init__(self, ctx: Context, seed: int = 2, **cfg):
        c = dict(TINYLLAMA)
        c.update(cfg)
        self.cfg = c
        self.ctx = ctx
        self._cfg = LlamaConfig(**c)
        h = C.c_void_p()
        check(lib().shp_llama_create(ctx.handle, C.byref(self._cfg), seed, C.byref(h)),
              "shp_llama_create")
        self.handle = h.value

    def close(self):
        if self.handle:
            lib().shp_llama_destroy(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def reset(self):
        check(lib().shp_llama_reset(self.handle), "shp_llama_reset")

    def use_graph(self, enable: bool):
        check(lib().shp_llama_use_graph(self.handle, int(enable)), "shp_llama_use_graph")

    ENGINES = {"kernels": 0, "graph": 1, "persistent": 2}

    def set_engine(self, name: str):
        """'kernels' (eager per-op launches), 'graph' (per-token hipGraph) or 'persistent'
        (one cooperative launch per step/decode call; the default where supported)."""
        check(lib().shp_llama_set_engine(self.handle, self.ENGINES[name]), "shp_llama_set_engine")

    @property
    def engine(self) -> str:
        e = C.c_int()
        check(lib().shp_llama_engine(self.handle, C.byref(e)), "shp_llama_engine")
        return {v: k for k, v in self.ENGINES.items()}[e.value]

    def set_wait_limit(self, polls: int = -1):
        """Bound of the persistent engine's grid waits in polls (-1: the default).  A wait
        that gives up ends the decode call with ShpError (SHP_ERR_HIP) and leaves the state
        undefined until reset()."""
        check(lib().shp_llama_set_wait_limit(self.handle, int(polls)), "shp_llama_set_wait_limit")

    def step(self, token: int):
        check(lib().shp_llama_step(self.handle, int(token)), "shp_llama_step")

    def decode(self, n_steps: int):
        check(lib().shp_llama_decode(self.handle, int(n_steps)), "shp_llama_decode")

    def tokens(self) -> list[int]:
        buf = (C.c_int32 * 4096)()
        n = C.c_int32()
        check(lib().shp_llama_tokens(self.handle, buf, 4096, C.byref(n)), "shp_llama_tokens")
        return list(buf[:n.value])

    def generate(self, prompt, n_new: int) -> list[int]:
        p = (C.c_int32 * len(prompt))(*[int(t) for t in prompt])
        out = (C.c_int32 * max(1, n_new))()
        n = C.c_int32()
        check(lib().shp_llama_generate(self.handle, p, len(prompt), n_new, out, C.byref(n)),
              "shp_llama_generate")
        return list(out[:n.value])

    def logits(self) -> np.ndarray:
        p, n = C.c_void_p(), C.c_uint64()
        check(lib().shp_llama_logits(self.handle, C.byref(p), C.byref(n)), "shp_llama_logits")
        return DeviceTensor(self.ctx, n.value, ptr=p.value, owned=False).download()

    def weight_ptr(self, layer: int, which: str) -> tuple[int, int]:
        """Device address and element count of a weight tensor (see shp_llama_weight)."""
        p, n = C.c_void_p(), C.c_uint64()
        check(lib().shp_llama_weight(self.handle, layer, which.encode(), C.byref(p), C.byref(n)),
              "shp_llama_weight")
        return p.value, n.value

    def weight(self, layer: int, which: str) -> np.ndarray:
        p, n = self.weight_ptr(layer, which)
        return DeviceTensor(self.ctx, n, ptr=p, owned=False).download()

    def weight_bytes(self) -> float:
        b = C.c_double()
        check(lib().shp_llama_weight_bytes(self.handle, C.byref(b)), "shp_llama_weight_bytes")
        return b.value
