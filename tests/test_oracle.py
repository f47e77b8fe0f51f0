"""Pins the CPU oracle (oracle/) before anything is checked against it.

Each oracle function is checked against something it does not itself
compute: exhaustive IEEE conversions, numpy's own rounding, closed-form
answers, an fp64 brute force, the reference tests' own seeded inputs and
gates, and the committed golden fixtures.  All CPU; no GPU needed.
"""
import ctypes

import numpy as np
import pytest

from bonsai_b1 import synth


def rel_to_rms(y, ref):
    ref = np.asarray(ref, dtype=np.float64)
    den = np.maximum(np.abs(ref), np.sqrt(np.mean(ref * ref)))
    return np.max(np.abs(np.asarray(y, np.float64) - ref) / den)


def cosine(a, b):
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    return float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b)))


# ------------------------------------------------------------ fp16 ------

def test_fp16_to_fp32_exhaustive(oracle):
    """All 65536 binary16 patterns vs numpy's half->float (exact IEEE)."""
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = oracle.fp16_to_fp32_bits(h)
    want = h.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))
    # spot values that a wrong exponent bias or subnormal path would break
    assert oracle.lib().b1o_fp16_to_fp32(0x3C00) == 1.0
    assert oracle.lib().b1o_fp16_to_fp32(0x0001) == 2.0 ** -24
    assert oracle.lib().b1o_fp16_to_fp32(0x7BFF) == 65504.0
    assert oracle.lib().b1o_fp16_to_fp32(0x8400) == -(2.0 ** -14)


def test_fp32_to_fp16_rne(oracle):
    """Round-to-nearest-even vs numpy astype(float16), incl. ties/edges."""
    rng = np.random.default_rng(1)
    x = (rng.standard_normal(4000) * np.exp2(rng.integers(-30, 18, 4000))).astype(np.float32)
    edges = np.array([0.0, -0.0, 65504.0, 65519.996, 65520.0, -65520.0, 1e9,
                      2.0 ** -24, 2.0 ** -25, 2.0 ** -25 * 1.0000001, 3 * 2.0 ** -26,
                      2.0 ** -14, 2.0 ** -14 * (1 - 2.0 ** -11), 1 + 2.0 ** -11,
                      1 + 3 * 2.0 ** -11, np.inf, -np.inf, 0.005, 0.05], dtype=np.float32)
    # exact halfway points between consecutive fp16 values (ties to even)
    ties = ((np.arange(0x3C00, 0x3C40, dtype=np.uint16).view(np.float16).astype(np.float64)
             + 2.0 ** -11)).astype(np.float32)
    x = np.concatenate([x, edges, ties])
    got = oracle.fp32_to_fp16_bits(x)
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


# ---------------------------------------------------- pack / unpack -----

@pytest.mark.parametrize("dist", ["normal", "uniform", "ties", "zeros"])
def test_c_pack_equals_numpy_quantize(oracle, dist):
    """C packer == numpy restatement of convert_to_b1_0_packed.py:21-43."""
    rng = np.random.default_rng(7)
    n, k = 24, 256
    if dist == "normal":
        w = rng.standard_normal((n, k)).astype(np.float32)
    elif dist == "uniform":
        w = rng.uniform(-1, 1, (n, k)).astype(np.float32)
    elif dist == "ties":  # few distinct magnitudes -> many exact fp16 ties
        w = (rng.integers(-3, 4, (n, k)) * 0.0009765625).astype(np.float32)
    else:
        w = np.zeros((n, k), np.float32)
        w[::2, ::3] = -0.0
    assert np.array_equal(oracle.pack(w), oracle.quantize_b1_0(w))


@pytest.mark.parametrize("dist", ["normal", "wide", "ties", "zeros"])
def test_c_pack_seq_equals_cumsum(oracle, dist):
    """Sequential-order writer (tests/c_ops/test_b1_linear.cpp:129-163):
    scale = fp16(left-to-right float32 sum of |w| / 32); numpy's cumsum over
    float32 is that left-to-right sum, so it pins the order independently."""
    rng = np.random.default_rng(8)
    n, k = 24, 256
    if dist == "normal":
        w = rng.standard_normal((n, k)).astype(np.float32)
    elif dist == "wide":  # magnitudes over many binades: order-sensitive sums
        w = (rng.standard_normal((n, k)) * 2.0 ** rng.integers(-20, 20, (n, k))).astype(np.float32)
    elif dist == "ties":
        w = (rng.integers(-3, 4, (n, k)) * 0.0009765625).astype(np.float32)
    else:
        w = np.zeros((n, k), np.float32)
        w[::2, ::3] = -0.0
    blocks = np.abs(w).reshape(n, k // 32, 32)
    seq = np.cumsum(blocks, axis=-1, dtype=np.float32)[..., -1] / np.float32(32)
    want = oracle.quantize_b1_0(w).reshape(n, k // 32, 6).copy()
    want[:, :, 0:2] = seq.astype(np.float16).view(np.uint8).reshape(n, k // 32, 2)
    assert np.array_equal(oracle.pack(w, order="sequential"), want.reshape(n, -1))


def test_pack_orders_differ_at_ties(oracle):
    """The two reference writers disagree by one fp16 ulp on a few blocks in
    10^5 (fp32 sums of different order straddling an fp16 rounding tie), so
    the order has to be a parameter of any writer that claims bit parity."""
    rng = np.random.default_rng(9)
    w = rng.standard_normal((1000, 3200)).astype(np.float32)
    a, b = oracle.pack(w), oracle.pack(w, order="sequential")
    diff = (a != b).reshape(1000, 100, 6)
    assert diff.any()
    assert not diff[:, :, 2:].any()                       # sign words never differ
    sa = a.reshape(1000, 100, 6)[:, :, :2].copy().view("<u2")[..., 0].astype(np.int32)
    sb = b.reshape(1000, 100, 6)[:, :, :2].copy().view("<u2")[..., 0].astype(np.int32)
    assert np.abs(sa - sb).max() == 1                     # by one fp16 ulp


def test_pack_unpack_roundtrip(oracle):
    """pack(unpack(P)) == P for every block with scale > 0, both readers agree."""
    n, k = 40, 512
    raw = synth.packed_weights(n, k, seed=3)
    wd = oracle.dequantize_b1_0(raw, n, k)
    assert np.array_equal(oracle.unpack(raw, n, k).view(np.uint32), wd.view(np.uint32))
    assert np.array_equal(oracle.quantize_b1_0(wd), raw)
    assert np.array_equal(oracle.pack(wd), raw)


def test_layout_closed_form(oracle):
    """Byte layout on a hand-built block: scale bytes first, then the sign word LE."""
    w = np.full((1, 32), -0.25, np.float32)
    w[0, [0, 9, 31]] = 0.25          # bits 0, 9, 31 set
    raw = oracle.pack(w)[0]
    assert int(raw[0]) | (int(raw[1]) << 8) == 0x3400          # fp16(0.25)
    word = int(raw[2]) | (int(raw[3]) << 8) | (int(raw[4]) << 16) | (int(raw[5]) << 24)
    assert word == (1 << 0) | (1 << 9) | (1 << 31)
    # zero maps to +scale (w >= 0), src/.. convert_to_b1_0_packed.py:35
    z = np.zeros((1, 32), np.float32)
    assert oracle.pack(z)[0].tolist() == [0, 0, 0xFF, 0xFF, 0xFF, 0xFF]


def test_reference_scheme_row(oracle):
    """Hand-written 64-weight row of the reference test
    (tests/ops/test_b1_linear.py:86-127): scale = mean|w| per block, signs."""
    row = np.array([
        0.5, -0.3, 0.8, -0.2, 1.0, -0.1, 0.4, -0.6, 0.7, -0.9, 0.2, -0.4, 0.3, -0.8, 0.1, -0.5,
        0.6, -0.7, 0.9, -0.2, 0.4, -1.0, 0.8, -0.3, 0.5, -0.6, 0.2, -0.9, 0.7, -0.4, 0.3, -0.1,
        0.2, -0.5, 0.7, -0.3, 0.9, -0.1, 0.4, -0.6, 0.8, -0.2, 0.5, -0.7, 0.3, -0.9, 0.1, -0.4,
        0.6, -0.8, 0.2, -0.5, 0.7, -0.3, 0.9, -0.1, 0.4, -0.6, 0.8, -0.2, 0.5, -0.7, 0.3, -0.9],
        dtype=np.float32)[None, :]
    raw = oracle.pack(row)
    wd = oracle.unpack(raw, 1, 64)
    for b in range(2):
        blk = row[0, 32 * b:32 * (b + 1)]
        want = float(np.float16(np.mean(np.abs(blk))))
        assert abs(float(np.abs(wd[0, 32 * b])) - want) == 0.0
        assert abs(want - float(np.mean(np.abs(blk)))) < 1e-3 * want   # fp16 rounding only
    assert np.array_equal(np.sign(wd[0]), np.where(row[0] >= 0, 1.0, -1.0))


# ------------------------------------------------------ matmul value ----

@pytest.mark.parametrize("variant", ["scalar", "avx2"])
def test_b1_linear_ones_closed_form(oracle, variant):
    """tests/fixtures/generate_fixtures.py:45-51: act = 1, W = 0.5 -> 16.0."""
    act = np.ones((1, 32), np.float32)
    raw = oracle.pack(np.full((16, 32), 0.5, np.float32))
    out, bad = oracle.linear(act, raw, 16, variant=variant, nth=4)
    assert bad == 0
    assert np.all(out == 16.0)


@pytest.mark.parametrize("variant", ["scalar", "avx2"])
def test_known_answers(oracle, variant):
    m, k, n = 6, 128, 12
    act = synth.activations(m, k, seed=11)
    raw = synth.packed_weights(n, k, seed=12)
    r3 = raw.reshape(n, k // 32, 6)
    scales = r3[:, :, 0:2].copy().view(np.float16)[..., 0].astype(np.float32)

    # one-hot activation -> +-scale of the block holding that element
    for i in (0, 17, 33, 127):
        e = np.zeros((1, k), np.float32)
        e[0, i] = 1.0
        out, _ = oracle.linear(e, raw, n, variant=variant)
        bit = (r3[:, i // 32, 2 + (i % 32) // 8] >> (i % 8)) & 1
        assert np.array_equal(out[0], np.where(bit == 1, scales[:, i // 32], -scales[:, i // 32]))

    # complemented sign words -> exact negation
    base, _ = oracle.linear(act, raw, n, variant=variant)
    comp = raw.copy().reshape(n, k // 32, 6)
    comp[:, :, 2:6] ^= 0xFF
    neg, _ = oracle.linear(act, comp.reshape(n, -1), n, variant=variant)
    assert np.array_equal(neg, -base)

    # all bits set, one block -> scale * sequential sum of a
    allset = raw.copy().reshape(n, k // 32, 6)
    allset[:, :, 2:6] = 0xFF
    a1 = act[:, :32].copy()
    out, _ = oracle.linear(a1, allset[:, :1, :].reshape(n, 6).copy(), n, variant="scalar")
    seq = np.zeros(m, np.float32)
    for i in range(32):
        seq = (seq + a1[:, i]).astype(np.float32)
    assert np.array_equal(out, (seq[:, None] * scales[None, :, 0]).astype(np.float32))

    # zero scale -> exactly zero output
    z = raw.copy().reshape(n, k // 32, 6)
    z[:, :, 0:2] = 0
    out, _ = oracle.linear(act, z.reshape(n, -1), n, variant=variant)
    assert np.all(out == 0.0)

    # linearity: power-of-two scaling is exact
    out2, _ = oracle.linear(act * 2.0, raw, n, variant=variant)
    assert np.array_equal(out2, 2.0 * base)


@pytest.mark.parametrize("variant", ["scalar", "avx2"])
def test_vs_fp64_bruteforce(oracle, variant):
    """fp32 result within the worst-case fp32 summation bound of fp64."""
    m, k, n = 9, 1024, 37
    act = synth.activations(m, k, seed=21)
    raw = synth.packed_weights(n, k, seed=22)
    out, _ = oracle.linear(act, raw, n, variant=variant, nth=3)
    ref = oracle.linear_f64(act, raw, n)
    assert np.array_equal(oracle.linear_f64_c(act, raw, n), ref) or \
        np.allclose(oracle.linear_f64_c(act, raw, n), ref, rtol=1e-12, atol=1e-12)
    wd = np.abs(oracle.dequantize_b1_0(raw, n, k)).astype(np.float64)
    mag = np.abs(act).astype(np.float64) @ wd.T            # sum |s a|
    bound = (k + 2) * 2.0 ** -24 * mag
    assert np.all(np.abs(out - ref) <= bound)
    # a dropped block (the smallest plausible slip) is far outside that bound
    assert np.max(np.abs(out - ref)) < 0.05 * np.min(mag / (k / 32))


def test_avx2_bit_exact_vs_lane_model(oracle):
    """C AVX2 restatement == lane-by-lane numpy model of :116-192."""
    m, k, n = 7, 256, 16            # nth=4 -> 4 full 4-row tiles per task
    act = synth.activations(m, k, seed=31)
    raw = synth.packed_weights(n, k, seed=32)
    out, _ = oracle.linear(act, raw, n, variant="avx2", nth=4)
    assert np.array_equal(out, oracle.avx2_lane_model(act, raw, n))


def test_avx2_remainder_rows_use_scalar(oracle):
    """Rows outside full 4-row tiles (:204-236) use the scalar order."""
    m, k, n = 5, 192, 10            # nth=3 -> tasks of 4, 4, 2 rows
    act = synth.activations(m, k, seed=41)
    raw = synth.packed_weights(n, k, seed=42)
    avx, _ = oracle.linear(act, raw, n, variant="avx2", nth=3)
    sca, _ = oracle.linear(act, raw, n, variant="scalar", nth=3)
    assert np.array_equal(avx[:, 8:10], sca[:, 8:10])
    assert np.array_equal(avx[:, :8], oracle.avx2_lane_model(act, raw[:8], 8))


@pytest.mark.parametrize("nth", [1, 3, 4, 7, 64])
def test_thread_split_does_not_change_scalar(oracle, nth):
    m, k, n = 3, 128, 29
    act = synth.activations(m, k, seed=51)
    raw = synth.packed_weights(n, k, seed=52)
    a, _ = oracle.linear(act, raw, n, variant="scalar", nth=1)
    b, _ = oracle.linear(act, raw, n, variant="scalar", nth=nth)
    assert np.array_equal(a, b)


def test_nonfinite_reported(oracle):
    """The reference aborts on non-finite outputs; the oracle counts them."""
    m, k, n = 2, 64, 8
    act = synth.activations(m, k, seed=61)
    raw = synth.packed_weights(n, k, seed=62)
    act_nan = act.copy()
    act_nan[1, 5] = np.nan
    for v in ("scalar", "avx2"):
        _, bad = oracle.linear(act_nan, raw, n, variant=v)
        assert bad == n                      # row 1 is NaN in every column
    inf_scale = raw.copy().reshape(n, 2, 6)
    inf_scale[3, 1, 0:2] = [0x00, 0x7C]      # +Inf fp16 scale in row 3
    for v in ("scalar", "avx2"):
        _, bad = oracle.linear(act, inf_scale.reshape(n, -1), n, variant=v)
        assert bad == m


# -------------------------------------- the reference tests' own inputs ----

def _torch_inputs(seed, batch, k, n):
    torch = pytest.importorskip("torch")
    torch.manual_seed(seed)
    act = torch.randn(batch, k).numpy()
    w = torch.randn(n, k).numpy()
    return act, w


@pytest.mark.parametrize("case", [(1, 64, 32), (1, 3072, 3072)])
def test_reference_cosine_gates(oracle, case):
    """tests/c_ops/test_b1_linear.py:37-94 (M=1,K=64,N=32) and
    tests/ops/test_all_ops.py:184-247 (M=1,K=N=3072): torch seed 42, output
    vs act @ dequant(W).T (fp32 mean, unrounded) with cos > 0.9999."""
    batch, k, n = case
    act, w = _torch_inputs(42, batch, k, n)
    raw = oracle.pack(w)
    expected = act.astype(np.float64) @ oracle.dequant_unrounded(w).astype(np.float64).T
    for v in ("scalar", "avx2"):
        out, bad = oracle.linear(act, raw, n, variant=v)
        assert bad == 0
        assert cosine(out, expected) > 0.9999
        # tighter than the reference gate: only the fp16 scale rounding differs
        assert rel_to_rms(out, expected) < 2e-3


def test_reference_webgpu_gate_inputs(oracle):
    """tests/c_ops/test_webgpu_ops.cpp:69-133: srand(42), U(-1,1) via glibc
    rand(), M=1, K=64, N=32, its C-twin packer (:29-45).  The oracle output
    agrees with the fp64 dequantised product to cos > 0.9999."""
    libc = ctypes.CDLL(None)
    libc.srand(42)
    RAND_MAX = 2147483647
    vals = np.array([libc.rand() for _ in range(64 + 32 * 64)], dtype=np.float64)
    vals = (vals / RAND_MAX * 2 - 1).astype(np.float32)
    act = vals[:64].reshape(1, 64)
    w = vals[64:].reshape(32, 64)
    raw = oracle.pack(w)
    out, bad = oracle.linear(act, raw, 32, variant="avx2", nth=4)
    assert bad == 0
    assert cosine(out, oracle.linear_f64(act, raw, 32)) > 0.9999


# ------------------------------------------------------ golden fixtures ----

def test_golden_fixtures_reproduce(oracle):
    """The committed fixtures (tests/golden/*.npz) are reproduced bit-exactly:
    inputs by the seeded generator, outputs by the scalar and AVX2 paths."""
    from tests.golden import make_golden
    cases = make_golden.load_all()
    assert cases, "no golden fixtures committed"
    for name, c in cases.items():
        m, k, n = c["act"].shape[0], c["act"].shape[1], int(c["n"])
        assert np.array_equal(c["act"], synth.activations(m, k, int(c["seed_a"])))
        assert np.array_equal(c["w"], synth.packed_weights(n, k, int(c["seed_w"])))
        sc, _ = oracle.linear(c["act"], c["w"], n, variant="scalar", nth=4)
        av, _ = oracle.linear(c["act"], c["w"], n, variant="avx2", nth=4)
        assert np.array_equal(sc, c["y_scalar"]), name
        assert np.array_equal(av, c["y_avx2"]), name
        assert np.allclose(oracle.linear_f64(c["act"], c["w"], n), c["y_f64"], rtol=0, atol=1e-9), name


# ------------------------------------------- LayerNorm + modulation, SwiGLU ----

def test_norm_mod_closed_forms(oracle):
    """oracle.norm_mod (ggml_norm + x_n * (scale + 1) + shift,
    src/diffuser_graph.cpp:347-352) against what the mathematics fixes:
    float64 LayerNorm within fp32 rounding; a constant row normalises to
    exactly 0, so the output is exactly `shift`; scale = -1 gives exactly
    `shift`; scale = shift = 0 leaves rows of mean 0 and variance
    1 - eps / (var + eps) up to rounding; an affine change a x + b of a row
    (a > 0) leaves the normalised row unchanged up to rounding."""
    rng = np.random.default_rng(71)
    h = 3072
    x = (rng.standard_normal((6, h)) * 3 + 1.5).astype(np.float32)
    sc = rng.standard_normal(h).astype(np.float32) * 0.1
    sh = rng.standard_normal(h).astype(np.float32) * 0.1
    y = oracle.norm_mod(x, sc, sh)
    ref = oracle.norm_mod_f64(x, sc, sh)
    assert np.max(np.abs(y - ref)) < 5e-6
    xc = np.full((2, h), 3.25, np.float32)
    assert np.array_equal(oracle.norm_mod(xc, sc, sh), np.broadcast_to(sh, (2, h)))
    assert np.array_equal(oracle.norm_mod(x, np.full(h, -1, np.float32), sh), np.broadcast_to(sh, x.shape))
    z = np.zeros(h, np.float32)
    n0 = oracle.norm_mod(x, z, z).astype(np.float64)
    assert np.all(np.abs(n0.mean(axis=1)) < 1e-6)
    assert np.all(np.abs(n0.var(axis=1) - 1) < 1e-5)
    n1 = oracle.norm_mod((x * np.float32(4.0) + np.float32(-7.0)).astype(np.float32), z, z)
    assert np.max(np.abs(n1 - n0)) < 2e-5
    # a plausible mistake: eps outside the square root
    wrong = (x - x.mean(1, keepdims=True)) / (np.sqrt(x.var(1, keepdims=True)) + 1e-2)
    assert np.max(np.abs(oracle.norm_mod(x, z, z, eps=1e-2) - wrong)) > 1e-4


def test_pack_act_words_layout(oracle):
    """Word 16 j + d of a row holds elements 32 j + d (low half) and
    32 j + d + 16 (high half), each fp16 RNE (numpy astype(float16))."""
    a = np.arange(2 * 64, dtype=np.float32).reshape(2, 64) / 8
    w = oracle.pack_act_words(a)
    h = a.astype(np.float16).view(np.uint16).astype(np.uint32)
    assert w.shape == (2, 32)
    assert w[1, 16 + 3] == h[1, 32 + 3] | (h[1, 32 + 3 + 16] << 16)
    assert w[0, 0] == h[0, 0] | (h[0, 16] << 16)


def test_swiglu_f64_definition(oracle):
    """[gate | value] -> silu(gate) * value (the reference's own statement,
    tests/ops/test_all_ops.py:29-45): silu(0) = 0, silu(x) -> x for large x,
    and the halves are not swapped (value 0 gives 0 whatever the gate)."""
    y = np.array([[0.0, 20.0, -20.0, 1.0, 5.0, 2.0, 3.0, 0.0]])
    out = oracle.swiglu_f64(y)
    assert out.shape == (1, 4)
    assert out[0, 0] == 0.0
    assert abs(out[0, 1] - 20.0 * 2.0) < 1e-6
    assert abs(out[0, 2]) < 1e-6
    assert out[0, 3] == 0.0


def test_swiglu_f64_against_torch(oracle):
    """swiglu_f64 against an independent implementation: torch's silu in
    float64 on the gate half times the value half."""
    import torch
    rng = np.random.default_rng(11)
    y = rng.standard_normal((7, 64)) * 4
    want = (torch.nn.functional.silu(torch.from_numpy(y[:, :32])) * torch.from_numpy(y[:, 32:])).numpy()
    assert np.allclose(oracle.swiglu_f64(y), want, rtol=1e-14, atol=1e-300)


def test_gelu_tanh_f64_pinned(oracle):
    """gelu_tanh_f64 against torch's gelu(approximate="tanh") in float64,
    and within the tanh approximation's known distance (< 5e-4 absolute on
    this range) of the exact erf GELU; closed forms at 0 and the tails.  A
    wrong constant (0.0447 for 0.044715, or sqrt(pi/2) for sqrt(2/pi))
    fails the first check."""
    import torch
    from scipy.special import erf
    x = np.linspace(-8, 8, 4001)
    got = oracle.gelu_tanh_f64(x)
    want = torch.nn.functional.gelu(torch.from_numpy(x), approximate="tanh").numpy()
    assert np.allclose(got, want, rtol=1e-13, atol=1e-15)
    exact = 0.5 * x * (1.0 + erf(x / np.sqrt(2.0)))
    assert np.max(np.abs(got - exact)) < 5e-4
    assert oracle.gelu_tanh_f64(np.array([0.0]))[0] == 0.0
    assert abs(oracle.gelu_tanh_f64(np.array([30.0]))[0] - 30.0) < 1e-12
    assert abs(oracle.gelu_tanh_f64(np.array([-30.0]))[0]) < 1e-12
    bad = 0.5 * x * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (x + 0.0447 * x ** 3)))
    assert not np.allclose(bad, want, rtol=1e-13, atol=1e-15)
