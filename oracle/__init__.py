"""ctypes wrapper of liboracle.so — the CPU restatement of the reference kernels.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg, always as the checker or the CPU baseline, never as the product path.
"""
from __future__ import annotations

import ctypes as C
import os
import pathlib
import subprocess
from typing import Optional, Sequence

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
# SHP_ORACLE_LIB selects another build of the same source (the sanitizer build of `make asan`)
LIB_PATH = pathlib.Path(os.environ.get("SHP_ORACLE_LIB", HERE / "liboracle.so"))
_LIB = None

ACT = {"none": 0, "relu": 1, "relu6": 2, "leaky": 3, "sigmoid": 4, "tanh": 5, "silu": 6,
       "gelu_erf": 7}


class LlamaCfg(C.Structure):
    _fields_ = [("n_layers", C.c_int32), ("hidden", C.c_int32), ("n_heads", C.c_int32),
                ("n_kv_heads", C.c_int32), ("head_dim", C.c_int32), ("ffn", C.c_int32),
                ("vocab", C.c_int32), ("max_seq", C.c_int32), ("rms_eps", C.c_float),
                ("rope_theta", C.c_float)]


def build() -> pathlib.Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


def lib() -> C.CDLL:
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise ImportError(f"{LIB_PATH} missing: run `make -C oracle`")
        h = C.CDLL(str(LIB_PATH))
        fp = C.POINTER(C.c_float)
        h.orc_run_kernel.restype = C.c_int
        h.orc_run_kernel.argtypes = [C.c_char_p, C.c_void_p, C.c_size_t, C.c_void_p, C.c_size_t,
                                     C.c_void_p, C.c_size_t, C.POINTER(C.c_int32), C.c_size_t,
                                     C.c_void_p, C.c_void_p, C.c_int32, C.c_float]
        h.orc_last_error.restype = C.c_char_p
        h.orc_kernel_count.restype = C.c_int
        h.orc_kernel_name.restype = C.c_char_p
        h.orc_kernel_name.argtypes = [C.c_int]
        h.orc_set_threads.argtypes = [C.c_int]
        h.orc_same_padding.argtypes = [C.c_int] * 9 + [C.POINTER(C.c_int32)] * 2
        h.orc_pack_conv_weight.argtypes = [C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int,
                                           C.c_int, C.c_void_p]
        h.orc_pack_depthwise_weight.argtypes = [C.c_void_p, C.c_void_p, C.c_int, C.c_int,
                                                C.c_int, C.c_void_p]
        h.orc_pack_fc_weight.argtypes = [C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_void_p]
        h.orc_top1_reference.restype = C.c_int
        h.orc_top1_reference.argtypes = [C.c_void_p, C.c_size_t, fp]
        h.orc_argmax_first.restype = C.c_int
        h.orc_argmax_first.argtypes = [C.c_void_p, C.c_size_t]
        h.orc_compare.argtypes = [C.c_void_p, C.c_size_t, C.c_void_p, C.c_size_t, C.c_float,
                                  C.POINTER(C.c_uint64), fp, fp]
        h.orc_parity_fixture.restype = C.c_int
        h.orc_parity_fixture.argtypes = [C.c_int, C.c_void_p, C.c_size_t]
        h.orc_poc_fixture.restype = C.c_int
        h.orc_poc_fixture.argtypes = [C.c_int, C.c_void_p, C.c_size_t]
        h.orc_llama_step.restype = C.c_int
        h.orc_llama_step.argtypes = [C.POINTER(LlamaCfg), C.POINTER(C.c_void_p), C.c_void_p,
                                     C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int32,
                                     C.c_int32, C.c_void_p]
        h.orc_llama_full.restype = C.c_int
        h.orc_llama_full.argtypes = [C.POINTER(LlamaCfg), C.POINTER(C.c_void_p), C.c_void_p,
                                     C.c_void_p, C.c_void_p, C.c_void_p, C.c_int32, C.c_void_p]
        _LIB = h
    return _LIB


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32).reshape(-1)


def run(name: str, in0, in1, n_out: int, push: Sequence[int], bias=None, residual=None,
        act: str | int = 0, alpha: float = 0.0, out_init=None) -> np.ndarray:
    """Run one reference kernel on the CPU; returns the output as float32.

    `out_init` is the output buffer's content on entry (zeros by default), for the ops that
    keep part of it: hlo_select (on_false) and hlo_concatenate_into (the other slabs)."""
    # an absent binding is NULL (optional inputs such as softmax_rows' mask test for it)
    a0 = _f32(in0) if in0 is not None else None
    a1 = _f32(in1) if in1 is not None else None
    b = _f32(bias) if bias is not None else None
    r = _f32(residual) if residual is not None else None
    out = np.zeros(max(1, n_out), dtype=np.float32)
    if out_init is not None:
        out[:n_out] = _f32(out_init)[:n_out]
    parr = (C.c_int32 * max(1, len(push)))(*[int(p) for p in push])
    act_code = ACT[act] if isinstance(act, str) else int(act)
    rc = lib().orc_run_kernel(name.encode(), a0.ctypes.data if a0 is not None else None,
                              a0.size if a0 is not None else 0,
                              a1.ctypes.data if a1 is not None else None,
                              a1.size if a1 is not None else 0,
                              out.ctypes.data, n_out, parr, len(push),
                              b.ctypes.data if b is not None else None,
                              r.ctypes.data if r is not None else None, act_code, alpha)
    if rc != 0:
        raise RuntimeError(f"oracle {name}: {lib().orc_last_error().decode()}")
    return out[:n_out]


def kernel_names() -> list[str]:
    h = lib()
    return [h.orc_kernel_name(i).decode() for i in range(h.orc_kernel_count())]


def parity_fixture(which: int, n: int) -> np.ndarray:
    out = np.zeros(n, np.float32)
    if lib().orc_parity_fixture(which, out.ctypes.data, n) != 0:
        raise RuntimeError(lib().orc_last_error().decode())
    return out


def poc_fixture(which: int, n: int) -> np.ndarray:
    out = np.zeros(n, np.float32)
    if lib().orc_poc_fixture(which, out.ctypes.data, n) != 0:
        raise RuntimeError(lib().orc_last_error().decode())
    return out


def same_padding(same: bool, ih, iw, oh, ow, kh, kw, sh, sw) -> tuple[int, int]:
    pt, pl = C.c_int32(), C.c_int32()
    lib().orc_same_padding(int(same), ih, iw, oh, ow, kh, kw, sh, sw, C.byref(pt), C.byref(pl))
    return pt.value, pl.value


def pack_conv_weight(ohwi: np.ndarray, bias: np.ndarray) -> np.ndarray:
    oc, kh, kw, ic = ohwi.shape
    out = np.zeros(oc * kh * kw * ic + oc, np.float32)
    w, b = _f32(ohwi), _f32(bias)
    lib().orc_pack_conv_weight(w.ctypes.data, b.ctypes.data, oc, kh, kw, ic, out.ctypes.data)
    return out


def pack_depthwise_weight(hwc: np.ndarray, bias: np.ndarray) -> np.ndarray:
    kh, kw, c = hwc.shape[-3:]
    out = np.zeros(kh * kw * c + c, np.float32)
    w, b = _f32(hwc), _f32(bias)
    lib().orc_pack_depthwise_weight(w.ctypes.data, b.ctypes.data, kh, kw, c, out.ctypes.data)
    return out


def pack_fc_weight(w: np.ndarray, bias: np.ndarray) -> np.ndarray:
    o, i = w.shape
    out = np.zeros(o * i + o, np.float32)
    wf, b = _f32(w), _f32(bias)
    lib().orc_pack_fc_weight(wf.ctypes.data, b.ctypes.data, o, i, out.ctypes.data)
    return out


def top1_reference(v) -> tuple[int, float]:
    a = _f32(v)
    conf = C.c_float()
    cls = lib().orc_top1_reference(a.ctypes.data, a.size, C.byref(conf))
    return cls, conf.value


def argmax_first(v) -> int:
    a = _f32(v)
    return lib().orc_argmax_first(a.ctypes.data, a.size)


def compare(actual, expected, eps: float) -> tuple[int, float, float]:
    a, e = _f32(actual), _f32(expected)
    mm, ma, mr = C.c_uint64(), C.c_float(), C.c_float()
    lib().orc_compare(a.ctypes.data, a.size, e.ctypes.data, e.size, eps, C.byref(mm),
                      C.byref(ma), C.byref(mr))
    return mm.value, ma.value, mr.value


def set_threads(n: int) -> None:
    lib().orc_set_threads(int(n))


def _layer_ptrs(layers: Sequence[Sequence[np.ndarray]]):
    flat = [np.ascontiguousarray(a, dtype=np.float32) for L in layers for a in L]
    arr = (C.c_void_p * len(flat))(*[a.ctypes.data for a in flat])
    return arr, flat


def llama_step(cfg: LlamaCfg, layers, embed, final_norm, lm_head, k_cache: np.ndarray,
               v_cache: np.ndarray, pos: int, token: int) -> np.ndarray:
    arr, keep = _layer_ptrs(layers)
    e, fn, lm = _f32(embed), _f32(final_norm), _f32(lm_head)  # keep alive during the call
    logits = np.zeros(cfg.vocab, np.float32)
    rc = lib().orc_llama_step(C.byref(cfg), arr, e.ctypes.data, fn.ctypes.data, lm.ctypes.data,
                              k_cache.ctypes.data, v_cache.ctypes.data, pos, token,
                              logits.ctypes.data)
    if rc != 0:
        raise RuntimeError(lib().orc_last_error().decode())
    return logits


def llama_full(cfg: LlamaCfg, layers, embed, final_norm, lm_head, tokens) -> np.ndarray:
    arr, keep = _layer_ptrs(layers)
    e, fn, lm = _f32(embed), _f32(final_norm), _f32(lm_head)  # keep alive during the call
    t = np.ascontiguousarray(tokens, dtype=np.int32)
    logits = np.zeros((t.size, cfg.vocab), np.float32)
    rc = lib().orc_llama_full(C.byref(cfg), arr, e.ctypes.data, fn.ctypes.data, lm.ctypes.data,
                              t.ctypes.data, t.size, logits.ctypes.data)
    if rc != 0:
        raise RuntimeError(lib().orc_last_error().decode())
    return logits
