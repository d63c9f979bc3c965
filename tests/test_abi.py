"""C-ABI boundary checks that need no GPU: the library loads, exports every symbol the
header declares, registers every reference kernel with the reference's push-vector
length, and fails closed without a device."""
import ctypes as C
import pathlib
import re

import pytest

ROOT = pathlib.Path(__file__).resolve().parent.parent

# Reference kernel names -> i32 count of the Params block of kernels/<op>/glsl/<op>.comp
# (the stems the host resolves, source/tflite_loader/src/kernels.rs:12-238 and the HLO
# binders in source/xla_hlo/src/compiler.rs:768-1135,1155-1228).
REFERENCE_PUSH = {
    "add": 1, "sub": 1, "mul": 1, "div": 1, "pow": 1, "min": 1, "max": 1, "exp": 1, "neg": 1,
    "abs": 1, "sqrt": 1, "rsqrt": 1, "log": 1, "leaky_relu": 2, "logistic": 1, "sigmoid": 1,
    "tanh": 1, "relu6": 1, "relu": 1, "reshape": 1, "concat": 2, "transpose": 13,
    "conv2d": 15, "depthwise_conv2d": 16, "global_avg_pool_sum": 4,
    "global_avg_pool_finalize": 4, "max_pool2d": 14, "l2norm": 2, "resize_bilinear": 9,
    "fully_connected": 4, "softmax10": 0, "softmax1000": 1, "sine": 1, "pad": 13,
    "hlo_conv_nhwc_hwio": 14, "hlo_dot_batched": 5, "hlo_dot_rank2": 4, "hlo_reduce_rank4": 15,
    "hlo_reduce_window_rank4": 14,
}


def header_symbols():
    text = (ROOT / "include" / "spirv_hip.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(shp_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_header_symbol():
    from spirv_inference_amd import _lib
    h = C.CDLL(str(_lib.LIB_PATH))
    missing = [s for s in header_symbols() if not hasattr(h, s)]
    assert not missing, f"declared in include/spirv_hip.h but not exported: {missing}"
    bound = {name for name, _, _ in _lib.SIGNATURES}
    assert set(header_symbols()) == bound, "ctypes signatures out of sync with the header"


def test_registry_covers_reference_kernels_with_push_lengths():
    from spirv_inference_amd import kernel_names, lib
    names = set(kernel_names())
    for k, n in REFERENCE_PUSH.items():
        assert k in names, f"reference kernel {k} not registered"
        assert lib().shp_kernel_push_count(k.encode()) == n, k
    assert lib().shp_kernel_push_count(b"not_a_kernel") < 0


def test_oracle_covers_every_registered_kernel(orc):
    from spirv_inference_amd import kernel_names
    assert set(kernel_names()) <= set(orc.kernel_names())


def test_no_device_fails_closed():
    """Without a GPU the context cannot be created and the error says so (no fallback)."""
    from spirv_inference_amd import Context, ShpError
    try:
        import torch
        if torch.cuda.is_available():
            pytest.skip("a GPU is present")
    except ImportError:
        pass
    with pytest.raises(ShpError, match="NO_DEVICE"):
        Context("any")


def test_product_does_not_link_the_oracle():
    from spirv_inference_amd import _lib
    blob = _lib.LIB_PATH.read_bytes()
    assert b"liboracle" not in blob and b"orc_run_kernel" not in blob
    src = "\n".join(p.read_text() for p in (ROOT / "spirv_inference_amd").rglob("*.py"))
    assert "import oracle" not in src and "from oracle" not in src
