"""GPU checks of the fused GEMM epilogues (bonsai_b1_linear_epi_f32,
bonsai_b1_linear_packed_f16_epi) against the same linear without them.

Bars:
  gate-residual : out = residual + gate * y is one fp32 multiply and one fp32
                  add per element, so it must equal numpy's float32
                  residual + gate * y bit for bit, y being the library's own
                  plain linear output (the fused GEMM computes the same y).
  SwiGLU        : out = silu(y[:, :H]) * y[:, H:] with silu = x / (1 + e^-x)
                  in fp32 through the device expf; against the same formula
                  in float64 on the library's y, |out - ref| <= 1e-6 *
                  max(|ref|, 1e-30) + 1e-30 per element (expf and the fp32
                  divide round within a few ulp).  The composition is also
                  checked against the float64 oracle to the FAST bar.
Paths: the packed GEMM with the epilogue fused (M > 16, K % 384 == 0), and
the separate pass after the GEMV (M <= 16), after EXACT mode and after the
fused-conversion GEMM (K % 384 != 0).
The activation producer (LayerNorm + modulation, fp32 or packed fp16) is
checked bit for bit against the oracle's restatement.
"""
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

SILU_TOL = 1e-6


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


def plain_linear(torch, b1, a, w, n, mode):
    """The linear without an epilogue, as the fused-epilogue GEMM computes
    it: a workspace that holds the packing only (m*k fp16 values and m row
    scales, each area rounded up to 256 bytes) keeps the GEMM unsplit along
    K (a split sums the K ranges in another order)."""
    m, k = a.shape
    ws = torch.empty((m * k * 2 + 255) // 256 * 256 + (m * 4 + 255) // 256 * 256, dtype=torch.uint8,
                     device="cuda")
    return b1.linear(a, w, n, mode=mode, workspace=ws)


CASES = [  # (m, k, n, mode): fused packed GEMM, ragged, GEMV pass, EXACT pass, conversion-GEMM pass
    (256, 768, 1024, "auto"),
    (200, 768, 640, "auto"),
    (4608, 3072, 3072, "auto"),
    (8, 3072, 512, "auto"),
    (64, 384, 128, "exact"),
    (200, 640, 576, "gemm"),
]


@pytest.mark.parametrize("m,k,n,mode", CASES)
def test_gate_residual_bit_exact(torch, b1, m, k, n, mode):
    from bonsai_b1 import synth
    say(f"gate-residual ({m},{k},{n}) {mode}")
    a = synth.device_activations(m, k, 61)
    w = synth.device_packed_weights(n, k, 62)
    gate = torch.randn(n, device="cuda")
    res = torch.randn((m, n + 8), device="cuda")[:, :n]
    y = plain_linear(torch, b1, a, w, n, mode)
    out = b1.linear_epi(a, w, n, "gate_residual", gate=gate, residual=res, mode=mode)
    torch.cuda.synchronize()
    want = res.cpu().numpy() + gate.cpu().numpy()[None, :] * y.cpu().numpy()   # float32 ops
    got = out.cpu().numpy()
    say(f"  mismatching elements: {int((got.view(np.uint32) != want.view(np.uint32)).sum())}")
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    # in place: the residual is the output (h = h + gate * y)
    h = res.clone()
    b1.linear_epi(a, w, n, "gate_residual", gate=gate, residual=h, out=h, mode=mode)
    torch.cuda.synchronize()
    assert np.array_equal(h.cpu().numpy().view(np.uint32), want.view(np.uint32))


def _swiglu64(y, h):
    y = y.astype(np.float64)
    g, v = y[:, :h], y[:, h:2 * h]
    return g / (1.0 + np.exp(-g)) * v


@pytest.mark.parametrize("m,k,n,mode", CASES)
def test_swiglu_matches_float64(torch, b1, oracle, m, k, n, mode):
    from bonsai_b1 import synth
    h = n // 2
    if h % 32:
        pytest.skip("H % 32 != 0")
    say(f"swiglu ({m},{k},{n}) {mode}")
    a = synth.device_activations(m, k, 63)
    w = synth.device_packed_weights(n, k, 64)
    y = plain_linear(torch, b1, a, w, n, mode)
    out = torch.full((m, h + 4), 7.0, device="cuda")
    b1.linear_epi(a, w, n, "swiglu", out=out[:, :h], mode=mode)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert bool((got[:, h:] == 7.0).all()), "columns past H untouched"
    ref = _swiglu64(y.cpu().numpy(), h)
    err = np.abs(got[:, :h] - ref) / (np.maximum(np.abs(ref), 1e-30))
    bad = np.abs(got[:, :h] - ref) > SILU_TOL * np.maximum(np.abs(ref), 1e-30) + 1e-30
    say(f"  max rel err {float(err.max()):.3e}, {int(bad.sum())} beyond the bar")
    assert not bad.any()
    if m * n * k <= 3e9:
        # the whole composition against the float64 oracle, FAST bar
        yo = oracle.linear_f64(a.cpu().numpy(), w.cpu().numpy().reshape(n, -1), n)
        ro = _swiglu64(yo, h)
        den = np.maximum(np.abs(ro), np.sqrt(np.mean(ro * ro)))
        r = float(np.max(np.abs(got[:, :h] - ro) / den))
        say(f"  vs oracle rel_to_rms {r:.3e}")
        assert r <= (1e-2 if mode != "exact" else 1e-5)


def test_packed_entry_matches_f32_entry(torch, b1):
    """bonsai_b1_linear_packed_f16_epi on the packed activations gives what
    bonsai_b1_linear_epi_f32 gives (same kernels), for both epilogues."""
    from bonsai_b1 import synth
    m, k, n = 300, 1152, 1536
    a = synth.device_activations(m, k, 65)
    w = synth.device_packed_weights(n, k, 66)
    gate = torch.randn(n, device="cuda")
    res = torch.randn((m, n), device="cuda")
    packed = b1.pack_act_f16(a)
    for kind, kw in (("gate_residual", {"gate": gate, "residual": res}), ("swiglu", {})):
        ref = b1.linear_epi(a, w, n, kind, **kw)
        got = b1.linear_packed_f16_epi(packed, w, k, n, m, kind, **kw)
        torch.cuda.synchronize()
        assert torch.equal(got, ref), kind


def test_epilogue_counts_linear_outputs(torch, b1):
    """The non-finite counter counts the linear's outputs y (the values the
    reference's abort checks), fused or not: a NaN activation row poisons n
    of them, before SwiGLU halves the columns."""
    from bonsai_b1 import synth
    for m, mode in ((256, "auto"), (8, "auto")):
        k, n = 768, 512
        act = synth.activations(m, k, 67)
        act[3, 5] = np.nan
        a = torch.from_numpy(act).cuda()
        w = synth.device_packed_weights(n, k, 68)
        for kind, kw in (("gate_residual", {"gate": torch.ones(n, device="cuda"),
                                            "residual": torch.zeros((m, n), device="cuda")}),
                         ("swiglu", {})):
            ctr = torch.zeros(1, dtype=torch.int32, device="cuda")
            b1.linear_epi(a, w, n, kind, mode=mode, nonfinite=ctr, **kw)
            torch.cuda.synchronize()
            assert int(ctr.item()) == n, (m, kind)


# ---------------------------------------------- LayerNorm + modulation (A) --

# (4608 rows: more work-groups than one round of the grid holds; 2051 x
# 1536: a ragged row count at a shorter row)
@pytest.mark.parametrize("rows,h", [(4096, 3072), (4608, 3072), (2051, 1536), (37, 3072), (5, 12288), (3, 96)])
def test_norm_mod_matches_oracle(torch, b1, oracle, rows, h):
    """bonsai_b1_norm_mod_f32 against the oracle's restatement of ggml_norm
    + modulation, bit for bit; the _pack form against the oracle's fp16 pack
    of the same values; and a linear fed by the packed form equals the
    linear of the fp32 form (the pack pass it replaces)."""
    rng = np.random.default_rng(81)
    x = (rng.standard_normal((rows, h)) * 2 + 0.5).astype(np.float32)
    x[0, :] = 1.75                       # constant row: var = 0, out = shift
    sc = (rng.standard_normal(h) * 0.2).astype(np.float32)
    sh = (rng.standard_normal(h) * 0.2).astype(np.float32)
    xd = torch.from_numpy(x).cuda()
    scd, shd = torch.from_numpy(sc).cuda(), torch.from_numpy(sh).cuda()
    y = b1.norm_mod(xd, scd, shd, eps=1e-6)
    packed = b1.norm_mod(xd, scd, shd, eps=1e-6, packed=True)
    torch.cuda.synchronize()
    want = oracle.norm_mod(x, sc, sh, eps=1e-6)
    got = y.cpu().numpy()
    nbad = int((got.view(np.uint32) != want.view(np.uint32)).sum())
    say(f"  norm_mod ({rows},{h}): {nbad} mismatching, max |diff| {float(np.abs(got - want).max()):.3e}")
    assert nbad == 0
    words = packed.cpu().numpy().view(np.uint32).reshape(rows, h // 2)
    assert np.array_equal(words, oracle.pack_act_words(want))
    if h % 384 == 0 and rows > 16:
        from bonsai_b1 import synth
        n = 512
        w = synth.device_packed_weights(n, h, 82)
        a = b1.linear(y, w, n, mode="gemm")     # split along K as the packed entry splits
        c = b1.linear_packed_f16(packed, w, h, n, rows)
        torch.cuda.synchronize()
        assert torch.equal(a, c)


def test_epilogue_graph_replay(torch, b1):
    """The fused SwiGLU and gate-residual linears captured in a HIP graph with
    the caller's workspace give the eager result on every replay (the
    gate-residual writes a fresh output each time: out != residual)."""
    from bonsai_b1 import synth
    m, k, n = 512, 3072, 2048
    a = synth.device_activations(m, k, 71)
    w = synth.device_packed_weights(n, k, 72)
    gate = torch.randn(n, device="cuda")
    res = torch.randn((m, n), device="cuda")
    ws = torch.empty(max(b1.linear_epi_workspace_bytes(m, k, n, "swiglu"),
                         b1.linear_epi_workspace_bytes(m, k, n, "gate_residual")), dtype=torch.uint8, device="cuda")
    ref_g = b1.linear_epi(a, w, n, "swiglu", workspace=ws).clone()
    ref_r = b1.linear_epi(a, w, n, "gate_residual", gate=gate, residual=res, workspace=ws).clone()
    og = torch.empty((m, n // 2), device="cuda")
    orr = torch.empty((m, n), device="cuda")
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        b1.linear_epi(a, w, n, "swiglu", out=og, workspace=ws)
        b1.linear_epi(a, w, n, "gate_residual", gate=gate, residual=res, out=orr, workspace=ws)
    for i in range(3):
        og.fill_(float(i))
        orr.fill_(float(i))
        b1.linear(a * 0.25, w, n)       # unrelated eager work between replays
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(og, ref_g) and torch.equal(orr, ref_r), f"replay {i}"


def test_two_streams_own_workspaces(torch, b1):
    """Calls on two streams with library-owned workspaces run concurrently
    without sharing a packing buffer: each stream's results equal the
    serial ones."""
    from bonsai_b1 import synth
    m, k, n = 1024, 3072, 4096
    a1 = synth.device_activations(m, k, 73)
    a2 = synth.device_activations(m, k, 74)
    w = synth.device_packed_weights(n, k, 75)
    r1 = b1.linear(a1, w, n)
    r2 = b1.linear(a2, w, n)
    torch.cuda.synchronize()
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    o1 = torch.empty((m, n), device="cuda")
    o2 = torch.empty((m, n), device="cuda")
    for _ in range(3):
        with torch.cuda.stream(s1):
            b1.linear(a1, w, n, out=o1)
        with torch.cuda.stream(s2):
            b1.linear(a2, w, n, out=o2)
        torch.cuda.synchronize()
        assert torch.equal(o1, r1) and torch.equal(o2, r2)


@pytest.mark.parametrize("mode", ["auto", "exact"])
def test_batch_with_epilogues_matches_single_calls(torch, b1, mode):
    """bonsai_b1_linear_batch_epi == the same ops one by one through
    bonsai_b1_linear_epi_f32 (bit for bit: same kernels): a double-block
    feed-forward (FF-in + SwiGLU, FF-out + in-place gate-residual), a plain
    op, and small-batch ops whose epilogues run as a separate pass."""
    from bonsai_b1 import synth
    m, d, hid = 256, 768, 1536
    x = synth.device_activations(m, d, 101)
    w_in = synth.device_packed_weights(2 * hid, d, 102)
    w_out = synth.device_packed_weights(d, hid, 103)
    w_p = synth.device_packed_weights(640, d, 104)
    gate = torch.randn(d, device="cuda")
    h0 = torch.randn((m, d), device="cuda")
    xs = synth.device_activations(8, d, 105)
    hs0 = torch.randn((8, d), device="cuda")
    dw = b1.device_weights
    act, h, plain = torch.empty((m, hid), device="cuda"), h0.clone(), torch.empty((m, 640), device="cuda")
    acts, hs = torch.empty((8, hid), device="cuda"), hs0.clone()
    ops = [(x, dw(w_in, d, 2 * hid), act, "swiglu"),
           (act, dw(w_out, hid, d), h, ("gate_residual", gate, h)),
           (x, dw(w_p, d, 640), plain),
           (xs, dw(w_in, d, 2 * hid), acts, "swiglu"),
           (acts, dw(w_out, hid, d), hs, ("gate_residual", gate, hs))]
    b1.linear_batch(ops, mode=mode)
    r_act = b1.linear_epi(x, w_in, 2 * hid, "swiglu", mode=mode)
    r_h = h0.clone()
    b1.linear_epi(r_act, w_out, d, "gate_residual", gate=gate, residual=r_h, out=r_h, mode=mode)
    r_plain = b1.linear(x, w_p, 640, mode=mode)
    r_acts = b1.linear_epi(xs, w_in, 2 * hid, "swiglu", mode=mode)
    r_hs = hs0.clone()
    b1.linear_epi(r_acts, w_out, d, "gate_residual", gate=gate, residual=r_hs, out=r_hs, mode=mode)
    torch.cuda.synchronize()
    for got, ref, name in ((act, r_act, "ff_in"), (h, r_h, "ff_out"), (plain, r_plain, "plain"),
                           (acts, r_acts, "ff_in small"), (hs, r_hs, "ff_out small")):
        assert torch.equal(got, ref), name
