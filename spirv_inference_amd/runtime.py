"""Host-side mirror of the reference's dispatch surface on top of the C ABI.

`run_kernel(device_selector, KernelRun)` keeps the signature and meaning of
tflite_loader::vulkan::run_kernel (source/tflite_loader/src/vulkan.rs:27-44): the kernel
is chosen by the reference's name, driven by its i32 push vector, host buffers in and a
`KernelOutput` (values + device identity + elapsed_ms) out.  `Context` adds what the
reference lacks: device-resident tensors and asynchronous launches on one stream.
"""
from __future__ import annotations

import ctypes as C
import dataclasses
from typing import Optional, Sequence

import numpy as np

from ._lib import ACT, Epilogue, RunInfo, check, lib


@dataclasses.dataclass
class KernelRun:
    """vulkan.rs:27-36 with the SPIR-V bytes replaced by the kernel name."""
    label: str
    kernel: str
    input0: np.ndarray
    input1: np.ndarray
    output_elements: int
    dispatch_x: int
    push: Sequence[int]


@dataclasses.dataclass
class KernelOutput:
    """vulkan.rs:18-25."""
    values: np.ndarray
    device_name: str
    vendor_id: int
    device_id: int
    elapsed_ms: float


def groups(elements: int, local_size: int) -> int:
    """vulkan.rs:38-40."""
    return -(-elements // local_size)


def f32_bits(x: float) -> int:
    """The i32 push-constant encoding of an f32 (e.g. leaky_relu alpha, scheduler.rs:114-117)."""
    return int(np.array([x], dtype=np.float32).view(np.int32)[0])


def _push(push: Sequence[int]):
    arr = (C.c_int32 * max(1, len(push)))(*[int(p) for p in push])
    return arr, len(push)


class DeviceTensor:
    """A hipMalloc'd fp32 (or int32) buffer owned by a Context."""

    def __init__(self, ctx: "Context", n: int, dtype=np.float32, ptr: Optional[int] = None,
                 owned: bool = True):
        self.ctx, self.n, self.dtype, self.owned = ctx, int(n), np.dtype(dtype), owned
        if ptr is None:
            p = C.c_void_p()
            check(lib().shp_alloc(ctx.handle, max(4, self.n * self.dtype.itemsize), C.byref(p)),
                  "shp_alloc")
            ptr = p.value
        self.ptr = int(ptr)

    @property
    def nbytes(self) -> int:
        return self.n * self.dtype.itemsize

    def upload(self, arr: np.ndarray) -> "DeviceTensor":
        a = np.ascontiguousarray(arr, dtype=self.dtype).reshape(-1)
        if a.size != self.n:
            raise ValueError(f"upload of {a.size} elements into a tensor of {self.n}")
        check(lib().shp_upload(self.ctx.handle, self.ptr, a.ctypes.data, a.nbytes), "shp_upload")
        return self

    def download(self) -> np.ndarray:
        out = np.empty(self.n, dtype=self.dtype)
        check(lib().shp_download(self.ctx.handle, out.ctypes.data, self.ptr, out.nbytes),
              "shp_download")
        return out

    def free(self) -> None:
        if self.owned and self.ptr:
            check(lib().shp_free(self.ctx.handle, self.ptr), "shp_free")
        self.ptr = 0


class Context:
    """One device + one stream (shp_ctx)."""

    def __init__(self, selector: str = "any"):
        h = C.c_void_p()
        check(lib().shp_create(selector.encode(), C.byref(h)), "shp_create")
        self.handle = h.value
        info = RunInfo()
        check(lib().shp_device_info(self.handle, C.byref(info)), "shp_device_info")
        self.device_name = info.device_name.decode()
        self.vendor_id = info.vendor_id
        self.device_id = info.device_id

    def close(self) -> None:
        if self.handle:
            lib().shp_destroy(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    # -- memory
    def tensor(self, arr: np.ndarray, dtype=np.float32) -> DeviceTensor:
        a = np.asarray(arr, dtype=dtype)
        return DeviceTensor(self, a.size, dtype).upload(a)

    def empty(self, n: int, dtype=np.float32) -> DeviceTensor:
        return DeviceTensor(self, n, dtype)

    def fill_random(self, t: DeviceTensor, seed: int, tensor_id: int, kind: str = "normal",
                    a: float = 0.0, b: float = 1.0) -> DeviceTensor:
        check(lib().shp_fill_random(self.handle, t.ptr, t.n, seed, tensor_id,
                                    0 if kind == "uniform" else 1, a, b), "shp_fill_random")
        return t

    def sync(self) -> None:
        check(lib().shp_sync(self.handle), "shp_sync")

    # -- dispatch
    def launch(self, kernel: str, in0, in1, out: DeviceTensor, push: Sequence[int],
               out_elems: Optional[int] = None, bias=None, residual=None, act: str | int = 0,
               alpha: float = 0.0) -> None:
        """Asynchronous device-pointer launch (shp_launch / shp_launch_ex)."""
        arr, n = _push(push)
        p0 = in0.ptr if in0 is not None else None
        p1 = in1.ptr if in1 is not None else None
        oe = out.n if out_elems is None else out_elems
        act_code = ACT[act] if isinstance(act, str) else int(act)
        if bias is None and residual is None and act_code == 0:
            rc = lib().shp_launch(self.handle, kernel.encode(), p0, p1, out.ptr, arr, n, oe)
        else:
            epi = Epilogue(bias.ptr if bias is not None else None,
                           residual.ptr if residual is not None else None, act_code, alpha)
            rc = lib().shp_launch_ex(self.handle, kernel.encode(), p0, p1, out.ptr, arr, n, oe,
                                     C.byref(epi))
        check(rc, f"launch {kernel}")

    # -- captured launch sequences
    def capture_begin(self) -> None:
        """Record (instead of run) the launches made on this context until capture_end()."""
        check(lib().shp_capture_begin(self.handle), "shp_capture_begin")

    def capture_end(self) -> "Graph":
        g = C.c_void_p()
        check(lib().shp_capture_end(self.handle, C.byref(g)), "shp_capture_end")
        return Graph(g.value)

    def run_kernel(self, spec: KernelRun) -> KernelOutput:
        """Synchronous host-to-host call with the semantics of vulkan.rs:42-44."""
        a0 = np.ascontiguousarray(spec.input0, dtype=np.float32).reshape(-1)
        a1 = np.ascontiguousarray(spec.input1, dtype=np.float32).reshape(-1)
        out = np.zeros(spec.output_elements, dtype=np.float32)
        arr, n = _push(spec.push)
        info = RunInfo()
        rc = lib().shp_run_kernel(self.handle, spec.kernel.encode(), a0.ctypes.data, a0.size,
                                  a1.ctypes.data, a1.size, out.ctypes.data, out.size, arr, n,
                                  spec.dispatch_x, C.byref(info))
        check(rc, f"run_kernel {spec.label}")
        return KernelOutput(out, info.device_name.decode(), info.vendor_id, info.device_id,
                            info.elapsed_ms)

    def tune(self, key: str, value: int) -> None:
        """Planner override for this context's dense launches (shp_tune; 0 = automatic)."""
        check(lib().shp_tune(self.handle, key.encode(), int(value)), "shp_tune")

    # -- timing (KernelOutput.elapsed_ms per launch, accumulated per kernel name)
    def timing(self, enable: bool) -> None:
        check(lib().shp_timing_enable(self.handle, 1 if enable else 0), "shp_timing_enable")

    def timing_reset(self) -> None:
        check(lib().shp_timing_reset(self.handle), "shp_timing_reset")

    def timing_report(self) -> dict:
        out, i = {}, 0
        name = C.create_string_buffer(128)
        ms, cnt = C.c_double(), C.c_uint64()
        while True:
            rc = lib().shp_timing_entry(self.handle, i, name, 128, C.byref(ms), C.byref(cnt))
            if rc != 0:
                break
            out[name.value.decode()] = (ms.value, cnt.value)
            i += 1
        return out

    def timing_launches(self) -> list[tuple[str, float]]:
        """Every timed launch since the last reset, in issue order: (kernel, elapsed ms)."""
        n = C.c_uint64()
        check(lib().shp_timing_launch_count(self.handle, C.byref(n)), "shp_timing_launch_count")
        name = C.create_string_buffer(128)
        ms = C.c_double()
        out = []
        for i in range(n.value):
            check(lib().shp_timing_launch(self.handle, i, name, 128, C.byref(ms)),
                  "shp_timing_launch")
            out.append((name.value.decode(), ms.value))
        return out


class Graph:
    """A recorded launch sequence (shp_graph): launch() replays it on the context stream."""

    def __init__(self, handle: int):
        self.handle = handle

    def launch(self) -> None:
        check(lib().shp_graph_launch(self.handle), "shp_graph_launch")

    def destroy(self) -> None:
        if self.handle:
            lib().shp_graph_destroy(self.handle)
            self.handle = None


def kernel_names() -> list[str]:
    h = lib()
    return [h.shp_kernel_name(i).decode() for i in range(h.shp_kernel_count())]


def run_kernel(device_selector: str, spec: KernelRun) -> KernelOutput:
    """Free-function form of vulkan.rs:42 (creates a context per call, as the reference
    creates a Vulkan device per call; prefer a long-lived Context)."""
    with Context(device_selector) as ctx:
        return ctx.run_kernel(spec)
