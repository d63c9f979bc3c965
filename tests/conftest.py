import pathlib
import sys

import numpy as np
import pytest

ROOT = pathlib.Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

GOLDEN = ROOT / "tests" / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture(scope="session")
def orc():
    import oracle
    if not oracle.LIB_PATH.exists():
        oracle.build()
    return oracle


@pytest.fixture(scope="session")
def ctx():
    """One HIP context for the whole GPU session (the product library, no fallback)."""
    from spirv_inference_amd import Context
    c = Context("any")
    yield c
    c.close()


def raw_f32(path) -> np.ndarray:
    return np.fromfile(path, dtype="<f4")


def ulp_diff(a, b) -> np.ndarray:
    """ULP distance as in chained_graph_runtime/src/main.rs:809-819 (ordered ints)."""
    def ordered(x):
        i = np.asarray(x, np.float32).view(np.int32).astype(np.int64)
        return np.where(i < 0, -(i & 0x7FFFFFFF), i)
    return np.abs(ordered(a) - ordered(b))


def assert_close(actual, expected, atol=1e-4, rtol=1e-4, what=""):
    """The build's per-op gate: |a - e| <= atol + rtol * |e| (fp32)."""
    a = np.asarray(actual, np.float64).reshape(-1)
    e = np.asarray(expected, np.float64).reshape(-1)
    assert a.shape == e.shape, f"{what}: shape {a.shape} vs {e.shape}"
    assert np.all(np.isfinite(a)), f"{what}: non-finite output"
    err = np.abs(a - e)
    bad = err > atol + rtol * np.abs(e)
    if bad.any():
        i = int(np.argmax(err - (atol + rtol * np.abs(e))))
        raise AssertionError(
            f"{what}: {int(bad.sum())}/{a.size} outside atol={atol} rtol={rtol}; "
            f"max_abs={err.max():.3e} at {i}: got {a[i]!r} want {e[i]!r}")
