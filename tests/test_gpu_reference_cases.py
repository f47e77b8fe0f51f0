"""The reference's own test cases for the B1_0 linear, through the HIP kernels.

Each case draws the inputs the reference's tests draw and asserts the gate
those tests assert, on the GPU in every mode that accepts the shape, and
through the ggml-style callback; then this build's bars against the oracle:
EXACT mode bit-identical to the oracle's scalar path, the FAST modes within
per element |y - ref| / max(|ref|, rms(ref)) <= 1e-2 and cosine >= 0.9999
of the oracle's AVX2 path and of the float64 product.

  * tests/c_ops/test_b1_linear.py:37-94: torch.manual_seed(42), act
    randn(1, 64), weight randn(32, 64), packed by the C++ writer of
    tests/c_ops/test_b1_linear.cpp:129-163 (a left-to-right block sum);
    gate: cos(out, act @ dequant(weight).T) > 0.9999, dequant with the
    unrounded fp32 block mean (:21-34).
  * tests/ops/test_all_ops.py:184-247: the same at batch 1, K = N = 3072.
  * tests/c_ops/test_webgpu_ops.cpp:69-133: srand(42), values
    (float)rand() / RAND_MAX * 2 - 1 in float arithmetic, batch 1, K = 64,
    N = 32, packed by its C++ writer (:29-45); gate: the GPU output against
    the CPU backend's (4 threads) on identical packed bytes, cos > 0.9999.
  * tests/fixtures/generate_fixtures.py:45-51 (b1_linear_ones): act = 1,
    weight = 0.5, batch 1, K = 32, N = 16 -> every output exactly 16.0.
"""
import ctypes
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

TOL_REL = 1e-2
TOL_COS = 0.9999
REF_GATE_COS = 0.9999  # the reference tests' own gate (strictly greater)
MODES = ("auto", "fast", "gemv", "gemm", "exact")


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def torch():
    import torch as t
    assert t.cuda.is_available(), "GPU tests need the MI355X"
    return t


@pytest.fixture(scope="module")
def b1(torch):
    import bonsai_b1
    bonsai_b1.load()
    return bonsai_b1


def cosine(a, b):
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    return float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b)))


def rel_to_rms(y, ref):
    ref = np.asarray(ref, dtype=np.float64)
    den = np.maximum(np.abs(ref), np.sqrt(np.mean(ref * ref)))
    return float(np.max(np.abs(np.asarray(y, np.float64) - ref) / den))


def torch_case(k, n):
    """torch.manual_seed(42); act = randn(1, k); weight = randn(n, k)."""
    import torch as t
    t.manual_seed(42)
    act = t.randn(1, k)
    weight = t.randn(n, k)
    return act.numpy().copy(), weight.numpy().copy()


def webgpu_case():
    """srand(42); 64 activations then 32 x 64 weights, each
    (float)rand() / RAND_MAX * 2 - 1 evaluated in float."""
    libc = ctypes.CDLL(None)
    libc.srand(42)
    raw = np.array([libc.rand() for _ in range(64 + 32 * 64)], dtype=np.int64)
    f = raw.astype(np.float32) / np.float32(2147483647) * np.float32(2) - np.float32(1)
    assert f.dtype == np.float32
    return f[:64].reshape(1, 64).copy(), f[64:].reshape(32, 64).copy()


def run_modes(torch, b1, act, packed_dev, n):
    """{mode: output} for every mode that takes the shape; the others must
    refuse it with ERR_ARG before launching anything."""
    from bonsai_b1 import capi
    a = torch.from_numpy(act).cuda()
    outs = {}
    for mode in MODES:
        try:
            y = b1.linear(a, packed_dev, n, mode=mode)
        except capi.B1Error as e:
            assert e.status == capi.ERR_ARG, (mode, e)
            say(f"  mode {mode}: shape refused (ERR_ARG)")
            continue
        torch.cuda.synchronize()
        outs[mode] = y.cpu().numpy()
    return outs


def run_callback(torch, b1, act, packed_dev, n):
    """The ggml-style callback (bonsai_b1_linear_f32_f32) over stand-in
    tensors, 4 ggml tasks as the reference's tests run the op."""
    from bonsai_b1 import capi
    m, k = act.shape

    class T(ctypes.Structure):
        pass
    T._fields_ = [("ne", ctypes.c_int64 * 4), ("nb", ctypes.c_size_t * 4),
                  ("src", ctypes.POINTER(T) * 2), ("data", ctypes.c_void_p)]
    a = torch.from_numpy(act).cuda()
    out = torch.full((m, n), 7.0, device="cuda")
    ta, tw, td = T(), T(), T()
    ta.ne[:] = [k, m, 1, 1]
    ta.nb[:] = [4, 4 * k, 4 * k * m, 4 * k * m]
    ta.data = a.data_ptr()
    tw.ne[:] = [packed_dev.numel(), 1, 1, 1]
    tw.data = packed_dev.data_ptr()
    td.ne[:] = [n, m, 1, 1]
    td.nb[:] = [4, 4 * n, 4 * n * m, 4 * n * m]
    td.src[0] = ctypes.pointer(ta)
    td.src[1] = ctypes.pointer(tw)
    td.data = out.data_ptr()
    ud = capi.B1LinearUserData(capi.MAGIC, k, n)
    lib = b1.load()
    torch.cuda.synchronize()
    for ith in (1, 2, 3, 0):
        lib.bonsai_b1_linear_f32_f32(ctypes.byref(td), ith, 4, ctypes.byref(ud))
    torch.cuda.synchronize()
    return out.cpu().numpy()


def check_outputs(outs, ref_gate, scalar, avx2, f64, what):
    for mode, y in outs.items():
        c_gate = cosine(y, ref_gate)
        say(f"  {what} {mode}: cos vs the reference's expectation {c_gate:.10f}")
        assert np.isfinite(y).all(), (what, mode)
        assert c_gate > REF_GATE_COS, (what, mode, c_gate)
        if mode == "exact":
            assert np.array_equal(y.view(np.uint32), scalar.view(np.uint32)), (what, mode)
            continue
        for ref, name in ((avx2, "avx2"), (f64, "f64")):
            r, c = rel_to_rms(y, ref), cosine(y, ref)
            assert r <= TOL_REL and c >= TOL_COS, (what, mode, name, r, c)


@pytest.mark.parametrize("k,n", [(64, 32), (3072, 3072)])
def test_torch_seed42_cases(torch, b1, oracle, k, n):
    """tests/c_ops/test_b1_linear.py:37-94 (K=64, N=32) and
    tests/ops/test_all_ops.py:184-247 (K=N=3072): the GPU quantizer writes
    the reference writers' bytes from the float weights, then every mode
    passes the reference's cosine gate and this build's bars."""
    import torch as t
    act, weight = torch_case(k, n)
    wd = t.from_numpy(weight).cuda()
    for order in ("numpy", "sequential"):
        got = b1.quantize_f32(wd, order=order)
        torch.cuda.synchronize()
        assert np.array_equal(got.cpu().numpy(), oracle.pack(weight, order=order)), order
    # the C binary of tests/c_ops/ packs with its sequential block sum
    packed = b1.quantize_f32(wd, order="sequential")
    raw = packed.cpu().numpy()
    expected = act.astype(np.float64) @ oracle.dequant_unrounded(weight).astype(np.float64).T
    scalar, bad = oracle.linear(act, raw, n, variant="scalar", nth=4)
    avx2, bad2 = oracle.linear(act, raw, n, variant="avx2", nth=4)
    assert bad == 0 and bad2 == 0
    f64 = oracle.linear_f64(act, raw, n)
    flat = packed.reshape(-1)
    outs = run_modes(torch, b1, act, flat, n)
    assert {"auto", "exact", "gemv", "gemm"} <= set(outs), sorted(outs)
    outs["callback"] = run_callback(torch, b1, act, flat, n)
    check_outputs(outs, expected, scalar, avx2, f64, f"seed42 K={k} N={n}")


def test_webgpu_srand42_case(torch, b1, oracle):
    """tests/c_ops/test_webgpu_ops.cpp:69-133: the GPU op against the CPU
    op (the oracle's AVX2 restatement at 4 ggml tasks) on identical packed
    bytes from the test's own C++ writer (sequential block sum)."""
    import torch as t
    act, weight = webgpu_case()
    packed = b1.quantize_f32(t.from_numpy(weight).cuda(), order="sequential")
    torch.cuda.synchronize()
    raw = packed.cpu().numpy()
    assert np.array_equal(raw, oracle.pack(weight, order="sequential"))
    cpu, bad = oracle.linear(act, raw, 32, variant="avx2", nth=4)
    scalar, _ = oracle.linear(act, raw, 32, variant="scalar", nth=4)
    assert bad == 0
    f64 = oracle.linear_f64(act, raw, 32)
    outs = run_modes(torch, b1, act, packed.reshape(-1), 32)
    outs["callback"] = run_callback(torch, b1, act, packed.reshape(-1), 32)
    # the reference gate compares GPU and CPU outputs on the same bytes
    check_outputs(outs, cpu, scalar, cpu, f64, "srand42 K=64 N=32")


def test_b1_linear_ones_fixture(torch, b1, oracle):
    """tests/fixtures/generate_fixtures.py:45-51: act = ones(1, 32), weight =
    0.5 * ones(16, 32): scale 0.5, every sign bit set, every output exactly
    16.0 in every mode that takes K = 32 (EXACT, and AUTO / FAST, which run
    EXACT there) and through the callback.  The same block repeated to
    K = 3072 and batch 8 and 256 reaches the small-M kernel and the MFMA
    GEMM: exactly 16.0 * 96 = 1536.0 (every partial sum is an integer
    multiple of 0.5 below 2^11, exact in fp16 products and fp32 sums)."""
    import torch as t
    act = np.ones((1, 32), np.float32)
    weight = np.full((16, 32), 0.5, np.float32)
    packed = b1.quantize_f32(t.from_numpy(weight).cuda())
    torch.cuda.synchronize()
    raw = packed.cpu().numpy()
    assert np.array_equal(raw, oracle.pack(weight))
    outs = run_modes(torch, b1, act, packed.reshape(-1), 16)
    assert {"auto", "exact"} <= set(outs), sorted(outs)
    outs["callback"] = run_callback(torch, b1, act, packed.reshape(-1), 16)
    for mode, y in outs.items():
        say(f"  ones {mode}: {np.unique(y)}")
        assert np.all(y == 16.0), mode
    wide = b1.quantize_f32(t.full((512, 3072), 0.5, device="cuda")).reshape(-1)
    for m in (8, 256):
        outs = run_modes(torch, b1, np.ones((m, 3072), np.float32), wide, 512)
        assert {"gemv", "gemm", "exact"} & set(outs)
        for mode, y in outs.items():
            say(f"  ones M={m} K=3072 {mode}: {np.unique(y)}")
            assert np.all(y == 1536.0), (m, mode)
