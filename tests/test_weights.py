"""Readers of the reference's raw-f32 parameter files (CPU; no device needed)."""
import numpy as np
import pytest

from spirv_inference_amd import weights as W


def test_read_input_list_resolves_relative_paths(tmp_path):
    # `--inputs-f32` form: comma-separated, empty entries skipped (xla_hlo/src/main.rs:35-42)
    (tmp_path / "list.txt").write_text("a/p0.raw.f32,a/p1.raw.f32,,\n")
    assert W.read_input_list(tmp_path / "list.txt") == [tmp_path / "a/p0.raw.f32",
                                                       tmp_path / "a/p1.raw.f32"]
    assert W.read_input_list(tmp_path / "list.txt", base="/x") == [
        __import__("pathlib").Path("/x/a/p0.raw.f32"), __import__("pathlib").Path("/x/a/p1.raw.f32")]


def test_read_raw_f32_little_endian_and_shape_checked(tmp_path):
    x = np.arange(12, dtype="<f4") * 0.5
    x.tofile(tmp_path / "w.raw.f32")
    y = W.read_raw_f32(tmp_path / "w.raw.f32", (3, 4))
    assert y.shape == (3, 4) and y.tobytes() == x.tobytes()
    with pytest.raises(ValueError):
        W.read_raw_f32(tmp_path / "w.raw.f32", (5, 4))
    (tmp_path / "odd.raw.f32").write_bytes(b"\0" * 6)
    with pytest.raises(ValueError):
        W.read_raw_f32(tmp_path / "odd.raw.f32")


def test_rope_check_matches_export_llama_tables():
    hd, S, theta = 64, 16, 10000.0
    inv = 1.0 / (theta ** (np.arange(0, hd, 2, dtype=np.float32) / hd))
    emb = np.concatenate([np.outer(np.arange(S, dtype=np.float32), inv)] * 2, axis=-1)
    W._check_rope(np.cos(emb), np.sin(emb), hd, theta)  # export_llama.py:116-124 tables pass
    with pytest.raises(ValueError):
        W._check_rope(np.cos(emb), np.sin(emb), hd, 500000.0)
