"""FAST mode on activations beyond the fp16 range, the library workspace
under graph capture, and one answer from the fp32 and packed entries.

The reference sums any finite fp32 activation in fp32
(src/b1_0_kernel.h:117-134,218-228).  FAST mode rounds activations to fp16,
whose largest finite value is 65504; the fp32 entry points therefore pack a
row whose largest |a| would overflow (>= 65520) times 2^-e and multiply its
outputs by 2^e (the packed GEMM, split-K, grouped small-M ops of a batch,
the fused epilogues), and, where a kernel converts activations itself (the
small-M kernel, GEMMs without a workspace), compute such rows again in
EXACT arithmetic.

Bars:
  * every path: each row within the FAST bar of the float64 oracle,
    relative to that row's own rms (a row of 1e6 would otherwise hide the
    others), cosine >= 0.9999, and no non-finite output counted;
  * the paths that recompute a row exactly give EXACT mode's bits for it;
  * rows within the fp16 range keep the bits of the plain packing (the
    same kernels on the unscaled rows).
"""
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

TOL_REL = 1e-2
TOL_COS = 0.9999


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


# rows beyond the fp16 range (index: what is planted); all finite
BIG_ROWS = {1: "whole row x 1e5", 2: "one element 1e6", 3: "one element -3e5",
            5: "exactly 65520 (rounds to inf in fp16)", 6: "row x 1e37"}


def big_activations(m, k, seed):
    """N(0,1) activations with the rows of BIG_ROWS planted (m >= 8)."""
    rng = np.random.default_rng(seed)
    a = rng.standard_normal((m, k)).astype(np.float32)
    a[1] *= np.float32(1e5)
    a[2, 7] = 1e6
    a[3, k - 1] = -3e5
    a[4, 0] = 65500.0                  # within range: rounds to 65504
    a[5, 3] = 65520.0
    a[6] *= np.float32(1e37)
    return a


def assert_rows_close(y, ref, what):
    """Each row against the float64 oracle relative to its own rms."""
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    rms = np.sqrt(np.mean(ref * ref, axis=1, keepdims=True))
    r = float(np.max(np.abs(y - ref) / np.maximum(np.abs(ref), rms)))
    c = min(float(y[i] @ ref[i] / (np.linalg.norm(y[i]) * np.linalg.norm(ref[i]))) for i in range(len(y)))
    say(f"  {what}: worst row rel_to_rms={r:.3e} min row cos={c:.8f}")
    assert np.isfinite(y).all(), what
    assert r <= TOL_REL, what
    assert c >= TOL_COS, what


# (m, k, n, mode, workspace): "lib" = the library's own, None = a too-small
# caller workspace (the kernels that convert activations themselves)
PATHS = [
    (2048, 768, 4608, "auto", "lib"),     # packed GEMM, unsplit (192 tiles of 128 x 384)
    (256, 3072, 3072, "auto", "lib"),     # packed GEMM split along K (C1)
    (8, 3072, 4096, "auto", "lib"),       # small-M kernel: exact rows inside it
    (16, 768, 640, "gemm", "lib"),        # GEMM tile for a few rows
    (300, 768, 600, "gemm", None),        # fused-conversion GEMM + exact rows
    (16, 6144, 1000, "gemv", None),       # small-M, two K passes, ragged N
    (8, 3328, 1000, "gemv", None),        # small-M over fp32 rows staged in LDS, ragged second K pass
    (12, 448, 96, "auto", "lib"),         # K % 256 != 0: small-M + fix-up kernel
    (200, 448, 320, "auto", "lib"),       # K % 384 != 0: fused-conversion GEMM + exact rows
]


@pytest.mark.parametrize("m,k,n,mode,ws", PATHS)
def test_activations_beyond_fp16(torch, b1, oracle, m, k, n, mode, ws):
    from bonsai_b1 import synth
    say(f"beyond fp16 ({m},{k},{n}) {mode} workspace={ws}")
    act = big_activations(m, k, m + k + n)
    raw = synth.packed_weights(n, k, 77)
    a = torch.from_numpy(act).cuda()
    w = torch.from_numpy(raw.ravel()).cuda()
    nf = torch.zeros(1, dtype=torch.int32, device="cuda")
    small = torch.empty(16, dtype=torch.uint8, device="cuda")
    y = b1.linear(a, w, n, mode=mode, nonfinite=nf, workspace=small if ws is None else None)
    ye = b1.linear(a, w, n, mode="exact")
    torch.cuda.synchronize()
    y, ye = y.cpu().numpy(), ye.cpu().numpy()
    assert int(nf.item()) == 0, "non-finite outputs counted"
    assert_rows_close(y, oracle.linear_f64(act, raw, n), f"({m},{k},{n}) {mode}")
    converting = ws is None or (mode != "gemm" and m <= 16) or k % 384 != 0
    if converting:
        for r in BIG_ROWS:
            assert np.array_equal(y[r].view(np.uint32), ye[r].view(np.uint32)), f"row {r} ({BIG_ROWS[r]}) not exact"
    # the rows within range are untouched by the scaling: the same call with
    # the planted rows zeroed gives them the same bits
    plain = act.copy()
    plain[list(BIG_ROWS)] = 0.0
    yp = b1.linear(torch.from_numpy(plain).cuda(), w, n, mode=mode, workspace=small if ws is None else None)
    torch.cuda.synchronize()
    keep = [i for i in range(m) if i not in BIG_ROWS]
    assert np.array_equal(yp.cpu().numpy()[keep].view(np.uint32), y[keep].view(np.uint32)), "rows within range changed"


def test_inf_activation_stays_non_finite(torch, b1, oracle):
    """An inf activation is not scaled away: its row's outputs are
    non-finite in every mode (the reference's fp32 sums are too, and it
    aborts), and the counter reports them."""
    from bonsai_b1 import synth
    m, k, n = 64, 768, 512
    act = synth.activations(m, k, 9)
    act[10, 5] = np.inf
    raw = synth.packed_weights(n, k, 10)
    a = torch.from_numpy(act).cuda()
    w = torch.from_numpy(raw.ravel()).cuda()
    for mode in ("auto", "gemm", "exact"):
        nf = torch.zeros(1, dtype=torch.int32, device="cuda")
        y = b1.linear(a, w, n, mode=mode, nonfinite=nf)
        torch.cuda.synchronize()
        y = y.cpu().numpy()
        say(f"  inf activation, {mode}: {int(nf.item())} counted")
        assert not np.isfinite(y[10]).any()
        assert np.isfinite(np.delete(y, 10, axis=0)).all()
        assert int(nf.item()) == n


def test_epilogues_beyond_fp16(torch, b1, oracle):
    """The fused epilogues apply the row scale before their own arithmetic:
    gate-residual and SwiGLU on rows beyond the fp16 range, against the
    float64 composition."""
    from bonsai_b1 import synth
    m, k, n = 256, 3072, 1024
    act = big_activations(m, k, 5)
    act[6] /= np.float32(1e30)   # keep SwiGLU's products finite (1e7 range)
    raw = synth.packed_weights(n, k, 78)
    a = torch.from_numpy(act).cuda()
    w = torch.from_numpy(raw.ravel()).cuda()
    gate = torch.randn(n, device="cuda")
    res = torch.randn((m, n), device="cuda")
    out = b1.linear_epi(a, w, n, "gate_residual", gate=gate, residual=res)
    sw = b1.linear_epi(a, w, n, "swiglu")
    torch.cuda.synchronize()
    y64 = oracle.linear_f64(act, raw, n)
    d = out.cpu().numpy().astype(np.float64) - res.cpu().numpy()
    assert_rows_close(d, gate.cpu().numpy()[None, :].astype(np.float64) * y64, "gate-residual")
    assert_rows_close(sw.cpu().numpy(), oracle.swiglu_f64(y64), "SwiGLU")


def test_callback_beyond_fp16(torch, b1, oracle):
    """The ggml-style callback over activations beyond the fp16 range runs
    to completion (the reference's fp32 path gives finite outputs there, so
    it must not abort) and matches the oracle."""
    import ctypes
    from bonsai_b1 import capi, synth
    m, k, n = 64, 3072, 768
    act = big_activations(m, k, 6)
    raw = synth.packed_weights(n, k, 79)
    lib = b1.load()
    W = b1.Weights(raw, k, n)
    a = torch.from_numpy(act).cuda()
    out = torch.empty((m, n), device="cuda")
    torch.cuda.synchronize()

    class T(ctypes.Structure):
        pass
    T._fields_ = [("ne", ctypes.c_int64 * 4), ("nb", ctypes.c_size_t * 4),
                  ("src", ctypes.POINTER(T) * 2), ("data", ctypes.c_void_p)]
    ta, tw, td = T(), T(), T()
    ta.ne[:] = [k, m, 1, 1]
    ta.nb[:] = [4, 4 * k, 4 * k * m, 4 * k * m]
    ta.data = a.data_ptr()
    tw.ne[:] = [W.c.nbytes, 1, 1, 1]
    tw.data = W.c.data
    td.ne[:] = [n, m, 1, 1]
    td.nb[:] = [4, 4 * n, 4 * n * m, 4 * n * m]
    td.src[0] = ctypes.pointer(ta)
    td.src[1] = ctypes.pointer(tw)
    td.data = out.data_ptr()
    ud = capi.B1LinearUserData(capi.MAGIC, k, n)
    lib.bonsai_b1_linear_f32_f32(ctypes.byref(td), 0, 4, ctypes.byref(ud))
    torch.cuda.synchronize()
    assert_rows_close(out.cpu().numpy(), oracle.linear_f64(act, raw, n), "callback")
    W.free()


# -------------------------------------------- library workspace and graphs --

def test_pinned_workspace_survives_growth(torch, b1):
    """A graph captured with the library's workspace keeps its buffer: an
    eager call that needs a larger one on the same stream afterwards gets a
    new buffer instead of freeing the captured one.  Every replay equals
    the eager result, and so do eager calls interleaved with the replays."""
    from bonsai_b1 import synth
    s = torch.cuda.Stream()
    k, n = 3072, 4096
    a_small = synth.device_activations(512, k, 81)
    a_big = synth.device_activations(4096, k, 82)
    w = synth.device_packed_weights(n, k, 83)
    with torch.cuda.stream(s):
        ref_small = b1.linear(a_small, w, n)          # the stream's first workspace
        y = torch.empty((512, n), device="cuda")
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            b1.linear(a_small, w, n, out=y)           # pins that workspace
        ref_big = b1.linear(a_big, w, n)              # grows: a new buffer
        torch.cuda.synchronize()
        for i in range(3):
            y.fill_(float(i))
            g.replay()
            big = b1.linear(a_big, w, n)
            torch.cuda.synchronize()
            say(f"  replay {i}: small max |diff| {float((y - ref_small).abs().max()):.3e}, "
                f"big max |diff| {float((big - ref_big).abs().max()):.3e}")
            assert torch.equal(y, ref_small), f"replay {i}"
            assert torch.equal(big, ref_big), f"eager call {i}"
    del g
    torch.cuda.synchronize()


def test_packed_small_m_group_under_capture_without_workspace(torch, b1):
    """A batch of small-M ops on one 12-token input (a grouped run would read
    a range-safe packing) captured on a stream the library has never seen
    and with no caller workspace: a capture allocates nothing, so the ops
    run one by one instead of failing.  Every replay equals the single
    calls, with eager calls between the replays."""
    from bonsai_b1 import synth
    m, k = 12, 3072
    ns = (1024, 640, 384)
    x = synth.device_activations(m, k, 84)
    ws = [synth.device_packed_weights(n, k, 85 + i) for i, n in enumerate(ns)]
    refs = [b1.linear(x, w, n) for w, n in zip(ws, ns)]
    outs = [torch.empty((m, n), device="cuda") for n in ns]
    ops = [(x, b1.device_weights(w, k, n), o) for w, n, o in zip(ws, ns, outs)]
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            b1.linear_batch(ops)
    torch.cuda.synchronize()
    other = synth.device_activations(300, k, 88)
    for i in range(3):
        for o in outs:
            o.fill_(float(i + 1))
        b1.linear(other, ws[0], ns[0])
        g.replay()
        torch.cuda.synchronize()
        for j, (o, r) in enumerate(zip(outs, refs)):
            assert torch.equal(o, r), f"replay {i}, op {j}"
    del g
    torch.cuda.synchronize()


# ----------------------------------------------- one entry, one answer ---

@pytest.mark.parametrize("m,k,n", [(256, 3072, 3072), (512, 9216, 3072), (37, 15360, 384)])
def test_packed_entry_splits_like_fp32_entry(torch, b1, m, k, n):
    """bonsai_b1_linear_packed_f16 splits along K exactly as
    bonsai_b1_linear_f32 does for the same shape (the library's workspace
    or the caller's), so the two entries agree bit for bit."""
    from bonsai_b1 import synth
    say(f"packed entry split ({m},{k},{n})")
    a = synth.device_activations(m, k, 91)
    w = synth.device_packed_weights(n, k, 92)
    ref = b1.linear(a, w, n)
    packed = b1.pack_act_f16(a)
    y = b1.linear_packed_f16(packed, w, k, n, m)
    need = b1.linear_packed_workspace_bytes(m, k, n)
    assert need > 0, "this shape splits along K"
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    y2 = b1.linear_packed_f16(packed, w, k, n, m, workspace=ws)
    torch.cuda.synchronize()
    assert torch.equal(y, ref)
    assert torch.equal(y2, ref)


@pytest.mark.parametrize("m,k,n", [(256, 3072, 3072), (2048, 768, 4608), (8, 3072, 4096)])
def test_scaled_halves_equal_fp32_entry(torch, b1, m, k, n):
    """bonsai_b1_pack_act_f16_scaled + bonsai_b1_linear_packed_f16_scaled
    give bonsai_b1_linear_f32's FAST results bit for bit (split-K and
    unsplit GEMMs), on activations beyond the fp16 range too; small-M
    batches agree on rows within range (the fp32 entry computes the others
    in EXACT arithmetic: both within the FAST bar of the oracle).  On rows
    within range the scaled packing is bonsai_b1_pack_act_f16's, with
    scale 1."""
    from bonsai_b1 import synth
    act = big_activations(m, k, 13)
    a = torch.from_numpy(act).cuda()
    w = torch.from_numpy(synth.packed_weights(n, k, 14).ravel()).cuda()
    ref = b1.linear(a, w, n)
    packed, rs = b1.pack_act_f16_scaled(a)
    y = b1.linear_packed_f16_scaled(packed, rs, w, k, n, m)
    plain = b1.pack_act_f16(a)
    torch.cuda.synchronize()
    keep = [i for i in range(m) if i not in BIG_ROWS]
    if m > 16:
        assert torch.equal(y, ref)
    else:
        assert torch.equal(y[keep], ref[keep])
        ye = b1.linear(a, w, n, mode="exact")
        torch.cuda.synchronize()
        assert torch.equal(ref[list(BIG_ROWS)], ye[list(BIG_ROWS)])
        assert_rows_close(y.cpu().numpy(), ref.cpu().numpy().astype(np.float64), "scaled vs fp32 entry")
    scales = rs.cpu().numpy()
    assert bool((scales[keep] == 1.0).all())
    assert bool((scales[list(BIG_ROWS)] > 1.0).all())
    pk = packed.view(m, k * 2).cpu().numpy()
    assert np.array_equal(pk[keep], plain.view(m, k * 2).cpu().numpy()[keep])
