"""The 16x16x32-MFMA tile GEMMs (b1_gemm16_kernel, 144 x 384 and 128 x 384).

The packed GEMM runs one of them for full-tile shapes whose 128 x 512 tiles
would quantise worse on the CUs (M % 144 or M % 128 == 0, N % 384 == 0,
K % 384 == 0, no split along K, fewer rounds counted in 128 x 512 tiles:
on 256 CUs e.g. 288 x 384 -> 768, 1440 x 1152 -> 3072 and the Flux shapes
M = 4608 with N = 3072, 9216, 12288 or 21504 take 144 x 384 tiles; 512 x
384 -> 768, 2048 x 768 -> 4608 and the Klein image shapes M = 4096 with
N = 3072, 9216 or 18432 take 128 x 384 tiles).  Checked here on such
shapes, through the fp32, packed and epilogue entries:

  * the FAST bar against the float64 oracle (per element
    |y - ref| / max(|ref|, rms(ref)) <= 1e-2 and cosine >= 0.9999);
  * the same bits on repeated launches, and from the fp32 entry and from
    pack + the packed entry (one kernel, one summation order);
  * the gate-residual epilogue bit for bit against residual + gate * y in
    fp32 (multiply, then add) on the same y, also in place;
  * range-safe row scales (rows beyond the fp16 range) row by row against
    the oracle, and the non-finite count;
  * an output row stride that is not a multiple of 4 (the scalar-store
    path): the same bits as the aligned call.
"""
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

TOL_REL = 1e-2
TOL_COS = 0.9999
SHAPES144 = [(288, 384, 768), (1440, 1152, 3072), (4608, 3072, 3072)]
SHAPES128 = [(512, 384, 768), (2048, 768, 4608), (4096, 3072, 9216)]
SHAPES = SHAPES144 + SHAPES128


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


def rel_to_rms(y, ref):
    ref = np.asarray(ref, dtype=np.float64)
    den = np.maximum(np.abs(ref), np.sqrt(np.mean(ref * ref)))
    return float(np.max(np.abs(np.asarray(y, np.float64) - ref) / den))


def cosine(a, b):
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    return float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b)))


def sampled_rows(m):
    return np.unique(np.concatenate([np.arange(min(m, 40)), np.linspace(0, m - 1, 40).astype(int),
                                     [m - 1]]))


def check_rows(y, a, w, n, rows, what, oracle):
    ref = oracle.linear_f64(a[rows].cpu().numpy(), w.cpu().numpy(), n)
    got = y[rows].cpu().numpy()
    r, c = rel_to_rms(got, ref), cosine(got, ref)
    say(f"  {what}: rel_to_rms={r:.3e} cos={c:.8f} over {len(rows)} rows")
    assert r <= TOL_REL and c >= TOL_COS, what


@pytest.mark.parametrize("m,k,n", SHAPES)
def test_tiles16_against_oracle_and_entries(torch, b1, oracle, m, k, n):
    from bonsai_b1 import synth
    say(f"tiles16 {(m, k, n)}")
    a = synth.device_activations(m, k, 201)
    w = synth.device_packed_weights(n, k, 202)
    y = b1.linear(a, w, n)
    torch.cuda.synchronize()
    check_rows(y, a, w, n, sampled_rows(m), "fp32 entry", oracle)
    for run in range(4):
        yy = b1.linear(a, w, n)
        torch.cuda.synchronize()
        assert torch.equal(yy, y), f"launch {run}"
    pa = b1.pack_act_f16(a)
    yp = b1.linear_packed_f16(pa, w, k, n, m)
    torch.cuda.synchronize()
    assert torch.equal(yp, y), "pack + packed entry"
    # an output row stride that is not a multiple of 4: scalar stores
    big = torch.full((m, n + 1), 7.0, device="cuda")
    b1.linear(a, w, n, out=big[:, :n])
    torch.cuda.synchronize()
    assert torch.equal(big[:, :n], y), "scalar-store path"
    assert bool((big[:, n] == 7.0).all())


@pytest.mark.parametrize("m,k,n", SHAPES144[:2] + SHAPES128[:2])
def test_tiles16_swiglu_scalar_store(torch, b1, m, k, n):
    """The fused SwiGLU epilogue into rows whose stride is not a multiple
    of 4 (element stores, the owner waves' block layout) gives the bits of
    the aligned call, which equal silu(gate) * value over the plain GEMM's
    columns as the separate epilogue pass computes them."""
    from bonsai_b1 import synth
    say(f"tiles16 swiglu scalar stores ({m},{k},{n})")
    h = n // 2
    a = synth.device_activations(m, k, 211)
    w = synth.device_packed_weights(n, k, 212)
    pa = b1.pack_act_f16(a)
    want = b1.linear_packed_f16_epi(pa, w, k, n, m, "swiglu")
    odd = torch.full((m, h + 1), 7.0, device="cuda")
    b1.linear_packed_f16_epi(pa, w, k, n, m, "swiglu", out=odd[:, :h])
    torch.cuda.synchronize()
    assert torch.equal(odd[:, :h], want), "scalar-store path"
    assert bool((odd[:, h] == 7.0).all())


@pytest.mark.parametrize("m,k,n", SHAPES144[:2] + SHAPES128[:2])
def test_tiles16_gate_residual(torch, b1, m, k, n):
    """out = residual + gate * y, fused, equals the fp32 multiply then add on
    the plain y; in place (residual = out) too."""
    from bonsai_b1 import synth
    a = synth.device_activations(m, k, 203)
    w = synth.device_packed_weights(n, k, 204)
    g = torch.Generator(device="cuda").manual_seed(205)
    gate = 0.1 * torch.randn(n, device="cuda", generator=g)
    res = torch.randn((m, n), device="cuda", generator=g)
    pa = b1.pack_act_f16(a)
    y = b1.linear_packed_f16(pa, w, k, n, m)
    torch.cuda.synchronize()
    want = res + gate * y
    got = b1.linear_packed_f16_epi(pa, w, k, n, m, "gate_residual", gate=gate, residual=res)
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    h = res.clone()
    b1.linear_packed_f16_epi(pa, w, k, n, m, "gate_residual", gate=gate, residual=h, out=h)
    torch.cuda.synchronize()
    assert torch.equal(h, want), "in place"
    # from fp32 activations through the epilogue entry (pack + fused GEMM)
    got2 = b1.linear_epi(a, w, n, "gate_residual", gate=gate, residual=res)
    torch.cuda.synchronize()
    assert torch.equal(got2, want), "fp32 epilogue entry"


@pytest.mark.parametrize("m,k,n", [(1440, 1152, 3072), (2048, 768, 4608)])
def test_tiles16_rows_beyond_fp16_and_nonfinite(torch, b1, oracle, m, k, n):
    from bonsai_b1 import synth
    a = synth.device_activations(m, k, 206)
    a[5] *= 3.0e5
    a[777] *= -2.0e6
    w = synth.device_packed_weights(n, k, 207)
    nf = torch.zeros(1, dtype=torch.int32, device="cuda")
    y = b1.linear(a, w, n, nonfinite=nf)
    torch.cuda.synchronize()
    assert int(nf.item()) == 0
    for r in (5, 777):
        check_rows(y, a, w, n, np.array([r]), f"row {r} beyond fp16", oracle)
    check_rows(y, a, w, n, sampled_rows(m), "other rows", oracle)
    # an infinite scale in column 1000's block 7: that column of every row
    wr = w.view(n, k // 32, 6).clone()
    wr[1000, 7, 0:2] = torch.tensor([0x00, 0x7C], dtype=torch.uint8)
    nf.zero_()
    yb = b1.linear(a, wr.view(-1), n, nonfinite=nf)
    torch.cuda.synchronize()
    bad = int((~torch.isfinite(yb)).sum())
    say(f"  non-finite outputs {bad}, counted {int(nf.item())}")
    assert bad == m and int(nf.item()) == m
    assert bool(torch.isfinite(torch.cat([yb[:, :1000], yb[:, 1001:]], 1)).all())
