"""ctypes binding of libspirv_hip.so (the C ABI declared in include/spirv_hip.h).

The library is loaded from this package directory only.  There is no fallback: if the
shared object is missing, importing any runtime entry point raises ImportError.
"""
from __future__ import annotations

import ctypes as C
import pathlib

PKG = pathlib.Path(__file__).resolve().parent
LIB_PATH = PKG / "libspirv_hip.so"

SHP_OK = 0
ERRORS = {
    -1: "SHP_ERR_INVALID",
    -2: "SHP_ERR_UNKNOWN_KERNEL",
    -3: "SHP_ERR_PUSH",
    -4: "SHP_ERR_SHAPE",
    -5: "SHP_ERR_HIP",
    -6: "SHP_ERR_NO_DEVICE",
    -7: "SHP_ERR_UNSUPPORTED",
}

globals().update({name: code for code, name in ERRORS.items()})  # SHP_ERR_* constants

ACT = {"none": 0, "relu": 1, "relu6": 2, "leaky": 3, "sigmoid": 4, "tanh": 5, "silu": 6,
       "gelu_erf": 7}


class ShpError(RuntimeError):
    """A non-zero status from the C ABI (the anyhow::Error of the reference host)."""

    def __init__(self, code: int, where: str, message: str):
        super().__init__(f"{where}: {ERRORS.get(code, code)}: {message}")
        self.code = code


class RunInfo(C.Structure):
    _fields_ = [("device_name", C.c_char * 256), ("vendor_id", C.c_uint32),
                ("device_id", C.c_uint32), ("elapsed_ms", C.c_double)]


class Epilogue(C.Structure):
    _fields_ = [("bias", C.c_void_p), ("residual", C.c_void_p), ("act", C.c_int32),
                ("alpha", C.c_float)]


class OpDesc(C.Structure):
    _fields_ = [("kernel", C.c_char * 64), ("push", C.c_int32 * 40), ("n_push", C.c_int32),
                ("in0", C.c_int32), ("in1", C.c_int32), ("out", C.c_int32),
                ("bias", C.c_int32), ("residual", C.c_int32), ("act", C.c_int32),
                ("alpha", C.c_float), ("out_elems", C.c_uint64), ("label", C.c_char * 64)]


class LlamaConfig(C.Structure):
    _fields_ = [("n_layers", C.c_int32), ("hidden", C.c_int32), ("n_heads", C.c_int32),
                ("n_kv_heads", C.c_int32), ("head_dim", C.c_int32), ("ffn", C.c_int32),
                ("vocab", C.c_int32), ("max_seq", C.c_int32), ("rms_eps", C.c_float),
                ("rope_theta", C.c_float)]


# (name, restype, argtypes) of every exported entry point, in header order.
SIGNATURES = [
    ("shp_create", C.c_int, [C.c_char_p, C.POINTER(C.c_void_p)]),
    ("shp_destroy", None, [C.c_void_p]),
    ("shp_last_error", C.c_char_p, []),
    ("shp_device_info", C.c_int, [C.c_void_p, C.POINTER(RunInfo)]),
    ("shp_set_stream", C.c_int, [C.c_void_p, C.c_void_p]),
    ("shp_get_stream", C.c_void_p, [C.c_void_p]),
    ("shp_alloc", C.c_int, [C.c_void_p, C.c_size_t, C.POINTER(C.c_void_p)]),
    ("shp_free", C.c_int, [C.c_void_p, C.c_void_p]),
    ("shp_upload", C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_size_t]),
    ("shp_download", C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_size_t]),
    ("shp_sync", C.c_int, [C.c_void_p]),
    ("shp_fill_random", C.c_int, [C.c_void_p, C.c_void_p, C.c_uint64, C.c_uint64, C.c_uint64,
                                  C.c_int32, C.c_float, C.c_float]),
    ("shp_kernel_count", C.c_int, []),
    ("shp_kernel_name", C.c_char_p, [C.c_int]),
    ("shp_kernel_push_count", C.c_int, [C.c_char_p]),
    ("shp_launch", C.c_int, [C.c_void_p, C.c_char_p, C.c_void_p, C.c_void_p, C.c_void_p,
                             C.POINTER(C.c_int32), C.c_size_t, C.c_uint64]),
    ("shp_launch_ex", C.c_int, [C.c_void_p, C.c_char_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                C.POINTER(C.c_int32), C.c_size_t, C.c_uint64,
                                C.POINTER(Epilogue)]),
    ("shp_launch_static", C.c_int, [C.c_void_p, C.c_char_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                    C.POINTER(C.c_int32), C.c_size_t, C.c_uint64,
                                    C.POINTER(Epilogue)]),
    ("shp_block_plan", C.c_int, [C.POINTER(C.c_int32), C.c_size_t, C.POINTER(C.c_int32)]),
    ("shp_run_kernel", C.c_int, [C.c_void_p, C.c_char_p, C.c_void_p, C.c_size_t, C.c_void_p,
                                 C.c_size_t, C.c_void_p, C.c_size_t, C.POINTER(C.c_int32),
                                 C.c_size_t, C.c_uint32, C.POINTER(RunInfo)]),
    ("shp_capture_begin", C.c_int, [C.c_void_p]),
    ("shp_capture_end", C.c_int, [C.c_void_p, C.POINTER(C.c_void_p)]),
    ("shp_graph_launch", C.c_int, [C.c_void_p]),
    ("shp_graph_destroy", None, [C.c_void_p]),
    ("shp_timing_enable", C.c_int, [C.c_void_p, C.c_int]),
    ("shp_timing_reset", C.c_int, [C.c_void_p]),
    ("shp_timing_entry", C.c_int, [C.c_void_p, C.c_int, C.c_char_p, C.c_size_t,
                                   C.POINTER(C.c_double), C.POINTER(C.c_uint64)]),
    ("shp_timing_launch_count", C.c_int, [C.c_void_p, C.POINTER(C.c_uint64)]),
    ("shp_timing_launch", C.c_int, [C.c_void_p, C.c_uint64, C.c_char_p, C.c_size_t,
                                    C.POINTER(C.c_double)]),
    ("shp_model_create", C.c_int, [C.c_void_p, C.c_char_p, C.c_int32, C.c_int32, C.c_uint64,
                                   C.POINTER(C.c_void_p)]),
    ("shp_model_destroy", None, [C.c_void_p]),
    ("shp_model_run", C.c_int, [C.c_void_p]),
    ("shp_model_use_graph", C.c_int, [C.c_void_p, C.c_int]),
    ("shp_model_input", C.c_int, [C.c_void_p, C.c_int, C.POINTER(C.c_void_p),
                                  C.POINTER(C.c_uint64)]),
    ("shp_model_output", C.c_int, [C.c_void_p, C.c_int, C.POINTER(C.c_void_p),
                                   C.POINTER(C.c_uint64)]),
    ("shp_model_work", C.c_int, [C.c_void_p, C.POINTER(C.c_double), C.POINTER(C.c_double)]),
    ("shp_model_num_ops", C.c_int, [C.c_void_p]),
    ("shp_model_op", C.c_int, [C.c_void_p, C.c_int, C.POINTER(OpDesc)]),
    ("shp_model_num_tensors", C.c_int, [C.c_void_p]),
    ("shp_model_tensor", C.c_int, [C.c_void_p, C.c_int, C.POINTER(C.c_void_p),
                                   C.POINTER(C.c_uint64), C.POINTER(C.c_int32)]),
    ("shp_model_tensor_parent", C.c_int, [C.c_void_p, C.c_int, C.POINTER(C.c_int32),
                                          C.POINTER(C.c_uint64)]),
    ("shp_llama_create", C.c_int, [C.c_void_p, C.POINTER(LlamaConfig), C.c_uint64,
                                   C.POINTER(C.c_void_p)]),
    ("shp_llama_destroy", None, [C.c_void_p]),
    ("shp_llama_reset", C.c_int, [C.c_void_p]),
    ("shp_llama_step", C.c_int, [C.c_void_p, C.c_int32]),
    ("shp_llama_decode", C.c_int, [C.c_void_p, C.c_int32]),
    ("shp_llama_tokens", C.c_int, [C.c_void_p, C.POINTER(C.c_int32), C.c_int32,
                                   C.POINTER(C.c_int32)]),
    ("shp_llama_generate", C.c_int, [C.c_void_p, C.POINTER(C.c_int32), C.c_int32, C.c_int32,
                                     C.POINTER(C.c_int32), C.POINTER(C.c_int32)]),
    ("shp_llama_use_graph", C.c_int, [C.c_void_p, C.c_int]),
    ("shp_llama_set_engine", C.c_int, [C.c_void_p, C.c_int]),
    ("shp_llama_set_wait_limit", C.c_int, [C.c_void_p, C.c_int64]),
    ("shp_llama_engine", C.c_int, [C.c_void_p, C.POINTER(C.c_int)]),
    ("shp_llama_logits", C.c_int, [C.c_void_p, C.POINTER(C.c_void_p), C.POINTER(C.c_uint64)]),
    ("shp_llama_weight", C.c_int, [C.c_void_p, C.c_int32, C.c_char_p, C.POINTER(C.c_void_p),
                                   C.POINTER(C.c_uint64)]),
    ("shp_llama_weight_bytes", C.c_int, [C.c_void_p, C.POINTER(C.c_double)]),
]

# Internal hooks for tests and experiments, exported by the library but not declared in
# include/spirv_hip.h: per-context planner overrides and split-K workspace control.
INTERNAL = [
    ("shp_tune", C.c_int, [C.c_void_p, C.c_char_p, C.c_int]),
    ("shp_reserve_workspace", C.c_int, [C.c_void_p, C.c_uint64]),
    ("shp_workspace_info", C.c_int, [C.c_void_p, C.POINTER(C.c_void_p), C.POINTER(C.c_uint64)]),
]

_LIB = None


def lib() -> C.CDLL:
    """The loaded library with every signature bound; raises if it has not been built."""
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise ImportError(
                f"{LIB_PATH} is missing: build it with `python -c 'import __graft_entry__ as g; "
                "g.build()'` (there is no CPU fallback)")
        h = C.CDLL(str(LIB_PATH))
        for name, res, args in SIGNATURES + INTERNAL:
            fn = getattr(h, name, None)
            if fn is None:  # completeness is enforced by tests/test_abi.py
                continue
            fn.restype = res
            fn.argtypes = args
        _LIB = h
    return _LIB


def check(rc: int, where: str) -> None:
    if rc != SHP_OK:
        msg = lib().shp_last_error()
        raise ShpError(rc, where, msg.decode() if msg else "")
