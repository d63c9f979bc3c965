"""MI355X-native (gfx950) operator kernels for the SPIRV_INFERENCE dispatch surface.

The HIP kernels and the C ABI live in libspirv_hip.so (built from csrc/ by build.py);
this package is the Python-side host mirror used by tests and the benchmark.
"""
from ._lib import ShpError, lib  # noqa: F401
from .runtime import (Context, DeviceTensor, KernelOutput, KernelRun, f32_bits,  # noqa: F401
                      groups, kernel_names, run_kernel)

__all__ = ["Context", "DeviceTensor", "KernelOutput", "KernelRun", "ShpError", "f32_bits",
           "groups", "kernel_names", "lib", "run_kernel"]
