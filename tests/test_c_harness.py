"""The C++ single-op harness tests/c_ops/b1_linear_hip (the reference's
tests/c_ops/test_b1_linear.cpp command line and file formats, on the
MI355X library).  Argument handling runs without a GPU; the parity cases
(marked gpu) compare its out.bin with the oracle on the same inputs."""
import subprocess
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
EXE = ROOT / "tests" / "c_ops" / "_build" / "b1_linear_hip"


def run(*args, timeout=120):
    if not EXE.exists():
        pytest.skip("harness not built (make -C tests/c_ops)")
    return subprocess.run([str(EXE), *map(str, args)], capture_output=True, text=True, timeout=timeout)


def test_usage_without_arguments():
    r = run()
    assert r.returncode == 1
    assert "Usage" in r.stderr


def test_count_mismatch_rejected_before_device(tmp_path):
    np.zeros(10, np.float32).tofile(tmp_path / "act.bin")
    np.zeros(64 * 32, np.float32).tofile(tmp_path / "w.bin")
    r = run(tmp_path / "act.bin", tmp_path / "w.bin", tmp_path / "out.bin", 1, 64, 32)
    assert r.returncode == 1
    assert "expected act_count" in r.stderr


def test_bad_in_dim_rejected(tmp_path):
    r = run(tmp_path / "a", tmp_path / "w", tmp_path / "o", 1, 48, 32)
    assert r.returncode == 1


@pytest.mark.gpu
@pytest.mark.parametrize("batch,k,n,mode", [(1, 64, 32, "exact"), (5, 256, 40, "exact"),
                                             (5, 256, 40, "auto"), (200, 768, 600, "gemm"),
                                             (8, 3072, 96, "gemv")])
def test_harness_matches_oracle(tmp_path, oracle, batch, k, n, mode):
    rng = np.random.default_rng(batch * 1000 + k + n)
    act = rng.standard_normal((batch, k)).astype(np.float32)
    w = rng.standard_normal((n, k)).astype(np.float32)
    act.tofile(tmp_path / "act.bin")
    w.tofile(tmp_path / "weight.bin")
    print(f"harness {mode} batch={batch} in={k} out={n}", flush=True)
    r = run(tmp_path / "act.bin", tmp_path / "weight.bin", tmp_path / "out.bin", batch, k, n, mode)
    assert r.returncode == 0, r.stderr
    y = np.fromfile(tmp_path / "out.bin", dtype=np.float32).reshape(batch, n)
    raw = oracle.pack(w, order="sequential")   # the reference harness's writer
    if mode == "exact":
        want, _ = oracle.linear(act, raw, n, variant="scalar")
        assert np.array_equal(y.view(np.uint32), want.view(np.uint32))
    else:
        ref = oracle.linear_f64(act, raw, n)
        den = np.maximum(np.abs(ref), np.sqrt(np.mean(ref * ref)))
        assert np.max(np.abs(y - ref) / den) <= 1e-2
        cos = float((y.ravel().astype(np.float64) @ ref.ravel()) / (np.linalg.norm(y) * np.linalg.norm(ref)))
        assert cos >= 0.9999
    # the reference test's own gate (tests/c_ops/test_b1_linear.py): cosine
    # against the dequantised product
    deq = oracle.unpack(raw, n, k).astype(np.float64)
    ref_deq = act.astype(np.float64) @ deq.T
    cos = float((y.ravel().astype(np.float64) @ ref_deq.ravel()) / (np.linalg.norm(y) * np.linalg.norm(ref_deq)))
    assert cos > 0.9999
